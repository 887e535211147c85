"""The five reference workloads at their full sizes on the GPU.

Where the oracle finishes in seconds the whole workload is compared with it
(tier-1, hex pie); otherwise the oracle checks a slice (single images of the
icosphere batch, 16 of the 4096 range-mode meshes, a down-scaled displaced
sphere), and the full-size run is checked through properties that do not
depend on size: batch independence (an image renders the same alone and in
its batch), peel-layer depth order, barycentric recomputation in float64 on
sampled pixels, and partition of unity of the interpolate gradient."""
import numpy as np
import pytest

import oracle as O
import scenes
from parity import (LOD_DELTA, assert_fwd_close, assert_grad_close, assert_grad_close_lod, dev, host,
                    lod_switch_mask, torch_dev)

pytestmark = pytest.mark.gpu


def _threads():
    O.set_threads(16)


def test_tier1_color_fit_256():
    """rasterize -> interpolate(colour) -> MSE against the target triangle's
    image, forward and backward (d_attr), N=1 at 256x256."""
    torch = torch_dev()
    from diffrast import DiffRast
    sc = scenes.tier1_triangle(H=256, W=256)
    pos, tri, attr = sc["pos"], sc["tri"], sc["attr"]
    rast_r, _ = O.rasterize(pos, tri, (256, 256), gradDB=False, max_per_tile=0)
    target, _ = O.interpolate(sc["target_attr"], rast_r, tri)
    a = dev(attr).requires_grad_(True)
    rast, _ = DiffRast.rasterize(dev(pos), dev(tri), (256, 256), gradDB=False)
    out, _ = DiffRast.interpolate(a, rast, dev(tri))
    np.testing.assert_array_equal(host(rast), rast_r)
    ref, _ = O.interpolate(attr, rast_r, tri)
    np.testing.assert_array_equal(host(out), ref)
    loss = torch.nn.functional.mse_loss(out, dev(target))
    loss.backward()
    g = (2.0 / ref.size) * (ref - target)
    d_attr, _, _ = O.interpolate_vjp(attr, rast_r, tri, g.astype(np.float32))
    assert_grad_close(host(a.grad), d_attr, "d_attr")


def test_hexpie_chain_4x512():
    """rasterize -> interpolate -> antialias (topology hash) -> MSE, backward
    to pos and the shared colour attribute, N=4 at 512x512."""
    torch = torch_dev()
    from diffrast import DiffRast
    _threads()
    sc = scenes.hex_pie(N=4, H=512, W=512)
    pos, tri, attr, target = sc["pos"], sc["tri"], sc["attr"], sc["target"]
    p = dev(pos).requires_grad_(True)
    a = dev(attr).requires_grad_(True)
    t = dev(tri)
    topo = DiffRast.antialiasConstructTopologyHash(t)
    rast, _ = DiffRast.rasterize(p, t, (512, 512), gradDB=False)
    col, _ = DiffRast.interpolate(a, rast, t)
    out = DiffRast.antialias(col, rast, p, t, topologyHash=topo)
    loss = torch.nn.functional.mse_loss(out, dev(target))
    loss.backward()

    rast_r, _ = O.rasterize(pos, tri, (512, 512), gradDB=False, max_per_tile=0)
    col_r, _ = O.interpolate(attr, rast_r, tri)
    topo_r = O.antialiasConstructTopologyHash(tri)
    np.testing.assert_array_equal(host(topo), topo_r)
    out_r = O.antialias(col_r, rast_r, pos, tri, topo_r)
    np.testing.assert_array_equal(host(rast), rast_r)
    np.testing.assert_array_equal(host(col), col_r)
    assert_fwd_close(host(out), out_r)
    g = ((2.0 / out_r.size) * (out_r - target)).astype(np.float32)
    d_col, d_pos_aa = O.antialias_vjp(col_r, rast_r, pos, tri, g, topo_r)
    d_attr, d_rast, _ = O.interpolate_vjp(attr, rast_r, tri, d_col)
    d_pos_r = O.rasterize_vjp(pos, tri, rast_r, d_rast) + d_pos_aa
    assert_grad_close(host(a.grad), d_attr, "d_attr")
    assert_grad_close(host(p.grad), d_pos_r, "d_pos")


def _ico_chain(DiffRast, torch, sc, sel):
    pos = dev(sc["pos"][sel]).requires_grad_(True)
    tri = dev(sc["tri"])
    attr = dev(sc["uv"]).requires_grad_(True)
    tex = dev(sc["tex"]).requires_grad_(True)
    topo = DiffRast.antialiasConstructTopologyHash(tri)
    H, W = sc["H"], sc["W"]
    rast, db = DiffRast.rasterize(pos, tri, (H, W), gradDB=True)
    uv, uv_da = DiffRast.interpolate(attr, rast, tri, rastDB=db, diffAttrs="all")
    col = DiffRast.texture(tex, uv, uvDA=uv_da, filterMode="linear-mipmap-linear",
                           boundaryMode="clamp")
    out = DiffRast.antialias(col, rast, pos, tri, topologyHash=topo)
    g = dev(sc["g"][sel])
    out.backward(g)
    return dict(rast=host(rast), db=host(db), uv=host(uv), uv_da=host(uv_da), col=host(col),
                out=host(out), d_pos=host(pos.grad), d_uv=host(attr.grad), d_tex=host(tex.grad))


def test_icosphere_chain_8x1024():
    """The benchmark workload at full size (8 x 1024^2, 81,920 triangles):
    image 0 against the oracle (forward and every gradient), and every image
    of the batch renders and differentiates as it does alone."""
    torch = torch_dev()
    from diffrast import DiffRast
    _threads()
    sc = scenes.textured_icosphere(N=8, H=1024, W=1024, level=6, tex_size=1024)
    rng = np.random.default_rng(5)
    sc["g"] = (rng.normal(size=(8, 1024, 1024, 4)) * 1e-3).astype(np.float32)
    full = _ico_chain(DiffRast, torch, sc, slice(0, 8))
    one = _ico_chain(DiffRast, torch, sc, slice(0, 1))
    # batch independence: image 0 alone == image 0 in the batch
    for k in ("rast", "db", "uv", "uv_da", "col", "out"):
        np.testing.assert_array_equal(full[k][:1], one[k], err_msg=k)
    assert_grad_close(full["d_pos"][:1], one["d_pos"], "d_pos batch vs alone")
    # image 0 against the oracle
    pos0, tri, uva, tex = sc["pos"][:1], sc["tri"], sc["uv"], sc["tex"]
    rast, db = O.rasterize(pos0, tri, (1024, 1024), max_per_tile=0)
    np.testing.assert_array_equal(one["rast"], rast)
    np.testing.assert_array_equal(one["db"], db)
    uv, uvda = O.interpolate(uva, rast, tri, rastDB=db, diffAttrs="all")
    np.testing.assert_array_equal(one["uv"], uv)
    np.testing.assert_array_equal(one["uv_da"], uvda)
    col = O.texture(tex, uv, uvDA=uvda, filterMode="linear-mipmap-linear", boundaryMode="clamp")
    assert_fwd_close(one["col"], col)
    topo = O.antialiasConstructTopologyHash(tri)
    out = O.antialias(col, rast, pos0, tri, topo)
    assert_fwd_close(one["out"], out)
    d_col, d_pos_aa = O.antialias_vjp(col, rast, pos0, tri, sc["g"][:1], topo)
    d_tex, d_uv, d_uvda, _ = O.texture_vjp(tex, uv, d_col, uvDA=uvda,
                                           filterMode="linear-mipmap-linear",
                                           boundaryMode="clamp")
    d_attr, d_rast, d_db = O.interpolate_vjp(uva, rast, tri, d_uv, rastDB=db, diffAttrs="all",
                                             d_out_da=d_uvda)
    d_pos = O.rasterize_vjp(pos0, tri, rast, d_rast, d_db) + d_pos_aa
    assert_grad_close(one["d_tex"], d_tex, "d_tex")
    assert_grad_close(one["d_uv"], d_attr, "d_uv attribute")
    assert_grad_close(one["d_pos"], d_pos, "d_pos")


def _bary64(pos, tri, rast, n, H, W, pix):
    """u, v, z of sampled pixels recomputed in float64 from their triangle."""
    h, w = pix // W, pix % W
    t = rast[h, w, 3].astype(np.int64) - 1
    P = pos[n][tri[t]].astype(np.float64)                 # [S,3,4]
    sx, sy, sz = P[..., 0] / P[..., 3], P[..., 1] / P[..., 3], P[..., 2] / P[..., 3]
    x = 2.0 * (w + 0.5) / W - 1.0
    y = 1.0 - 2.0 * (h + 0.5) / H
    area = (sx[:, 1] - sx[:, 0]) * (sy[:, 2] - sy[:, 0]) - (sx[:, 2] - sx[:, 0]) * (sy[:, 1] - sy[:, 0])
    e1 = (sx[:, 2] - x) * (sy[:, 0] - y) - (sx[:, 0] - x) * (sy[:, 2] - y)
    e2 = (sx[:, 0] - x) * (sy[:, 1] - y) - (sx[:, 1] - x) * (sy[:, 0] - y)
    u, v = e1 / area, e2 / area
    z = (1 - u - v) * sz[:, 0] + u * sz[:, 1] + v * sz[:, 2]
    return t, u, v, z


def test_displaced_sphere_peel_16x2048():
    """~1.3M triangles, N=16 at 2048^2, four depth-peeling layers, then
    interpolate (normal + RGB) forward and backward on the first layer.
    Properties at full size; the oracle on a down-scaled instance.  (The
    rasterize backward of this workload is test_displaced_sphere_d_pos.)"""
    torch = torch_dev()
    from diffrast import DiffRast
    _threads()
    H = W = 2048
    sc = scenes.displaced_sphere(N=16, H=H, W=W, level=8)
    pos, tri, attr = sc["pos"], sc["tri"], sc["attr"]
    p, t = dev(pos), dev(tri)
    layers, prev = [], None
    for _ in range(4):
        r, _ = DiffRast.rasterize(p, t, (H, W), gradDB=False, peelLayer=prev)
        layers.append(r)
        prev = r
    cov = [(r[..., 3] > 0) for r in layers]
    for k in range(3):
        # under a covered pixel the next layer lies strictly deeper; where the
        # previous layer is empty there is no constraint (Rasterize.swift:387-391)
        # and the pixel renders as in the first layer
        deeper = cov[k] & cov[k + 1]
        assert bool((layers[k + 1][..., 2][deeper] > layers[k][..., 2][deeper]).all().item()), k
        free = ~cov[k]
        assert bool((layers[k + 1][free] == layers[0][free]).all().item()), k
    assert int((cov[0] & cov[1]).sum().item()) > 0
    rng = np.random.default_rng(8)
    for k in range(2):
        r0 = host(layers[k][0])
        covered = np.flatnonzero(r0[..., 3].ravel() > 0)
        assert covered.size > 0
        pix = rng.choice(covered, size=min(4096, covered.size), replace=False)
        tt, u, v, z = _bary64(pos, tri, r0, 0, H, W, pix)
        rr = r0.reshape(-1, 4)[pix]
        # triangles of ~2 pixels: the fp32 edge functions the reference
        # evaluates lose a few bits to cancellation against float64
        np.testing.assert_allclose(rr[:, 0], u, atol=2e-3)
        np.testing.assert_allclose(rr[:, 1], v, atol=2e-3)
        np.testing.assert_allclose(rr[:, 2], z, atol=2e-5)
        assert (u > -1e-4).all() and (v > -1e-4).all() and (u + v < 1 + 1e-4).all()

    a = dev(attr).requires_grad_(True)
    out, _ = DiffRast.interpolate(a, layers[0], t)
    g = torch.randn(out.shape, device=out.device) * 1e-3
    out.backward(g)
    # partition of unity: every covered pixel's weights sum to one
    c0 = cov[0].unsqueeze(-1)
    want = (g.double() * c0).sum(dim=(0, 1, 2))
    got = a.grad.double().sum(dim=(0, 1))
    np.testing.assert_allclose(host(got), host(want), rtol=1e-4, atol=1e-6)
    # sampled pixels: out = weights . vertex attributes, in float64
    r0 = host(layers[0][0])
    covered = np.flatnonzero(r0[..., 3].ravel() > 0)
    pix = rng.choice(covered, size=4096, replace=False)
    rr = r0.reshape(-1, 4)[pix]
    tv = tri[rr[:, 3].astype(np.int64) - 1]
    A = attr[0].astype(np.float64)
    u, v = rr[:, 0:1].astype(np.float64), rr[:, 1:2].astype(np.float64)
    want = (1 - u - v) * A[tv[:, 0]] + u * A[tv[:, 1]] + v * A[tv[:, 2]]
    np.testing.assert_allclose(host(out[0]).reshape(-1, 6)[pix], want, rtol=1e-5, atol=1e-6)

    # the same mesh, down-scaled, against the oracle: two layers + interpolate
    small = scenes.displaced_sphere(N=1, H=256, W=256, level=8)
    sp, st, sa = small["pos"], small["tri"], small["attr"]
    r_prev, o_prev = None, None
    for _ in range(2):
        r, _ = DiffRast.rasterize(dev(sp), dev(st), (256, 256), gradDB=False, peelLayer=r_prev)
        ro, _ = O.rasterize(sp, st, (256, 256), gradDB=False, peelLayer=o_prev, max_per_tile=0)
        np.testing.assert_array_equal(host(r), ro)
        r_prev, o_prev = r, ro
    a2 = dev(sa).requires_grad_(True)
    out2, _ = DiffRast.interpolate(a2, r_prev, dev(st))
    ref2, _ = O.interpolate(sa, o_prev, st)
    np.testing.assert_array_equal(host(out2), ref2)
    g2 = rng.normal(size=ref2.shape).astype(np.float32)
    out2.backward(dev(g2))
    d_attr2, _, _ = O.interpolate_vjp(sa, o_prev, st, g2)
    assert_grad_close(host(a2.grad), d_attr2, "d_attr (down-scaled)")


def _peel_chain(DiffRast, p, t, a, H, W, layers, gs):
    """layers x rasterize(peel) -> interpolate each layer -> sum <out, g>;
    returns the layers' rast (forward values)."""
    prev, loss, rs = None, 0.0, []
    for k in range(layers):
        r, _ = DiffRast.rasterize(p, t, (H, W), gradDB=False, peelLayer=prev)
        out, _ = DiffRast.interpolate(a, r, t)
        loss = loss + (out * gs[k]).sum()
        rs.append(r.detach())
        prev = r.detach()
    loss.backward()
    return rs


def test_displaced_sphere_d_pos():
    """The displaced-sphere workload's backward to pos: four peel layers ->
    interpolate -> sum of <out, g> -> rasterize VJP of every layer (d_pos by
    atomics on ~655k vertices).  Down-scaled (1 x 256^2, same mesh) the whole
    chain is checked against the oracle; at full size (16 x 2048^2) through
    properties: finite, a zero z channel (interpolate passes no depth
    gradient), no gradient on vertices of triangles no layer shows, and
    image 0 alone equal to image 0 in its batch."""
    torch = torch_dev()
    from diffrast import DiffRast
    _threads()
    rng = np.random.default_rng(44)
    small = scenes.displaced_sphere(N=1, H=256, W=256, level=8)
    sp, st, sa = small["pos"], small["tri"], small["attr"]
    gs = [rng.normal(size=(1, 256, 256, sa.shape[-1])).astype(np.float32) for _ in range(4)]
    p = dev(sp).requires_grad_(True)
    a = dev(sa).requires_grad_(True)
    rs = _peel_chain(DiffRast, p, dev(st), a, 256, 256, 4, [dev(g) for g in gs])
    want = np.zeros_like(sp)
    o_prev = None
    for k in range(4):
        ro, _ = O.rasterize(sp, st, (256, 256), gradDB=False, peelLayer=o_prev, max_per_tile=0)
        np.testing.assert_array_equal(host(rs[k]), ro)
        _, d_rast, _ = O.interpolate_vjp(sa, ro, st, gs[k])
        want += O.rasterize_vjp(sp, st, ro, d_rast, None)
        o_prev = ro
    assert_grad_close(host(p.grad), want, "d_pos (down-scaled, 4 layers)")

    H = W = 2048
    sc = scenes.displaced_sphere(N=16, H=H, W=W, level=8)
    pos, tri, attr = sc["pos"], sc["tri"], sc["attr"]
    t = dev(tri)
    gfull = [torch.randn((16, H, W, attr.shape[-1]), device="cuda") * 1e-3 for _ in range(4)]
    p = dev(pos).requires_grad_(True)
    a = dev(attr).requires_grad_(True)
    rs = _peel_chain(DiffRast, p, t, a, H, W, 4, gfull)
    d_pos = p.grad.detach()
    assert bool(torch.isfinite(d_pos).all().item())
    assert bool((d_pos[..., 2] == 0).all().item())
    assert bool((d_pos[..., :2] != 0).any().item())
    # vertices of no shown triangle get nothing (image 0)
    shown = np.zeros(tri.shape[0], bool)
    for r in rs:
        ids = host(r[0, ..., 3]).astype(np.int64).ravel()
        shown[ids[ids > 0] - 1] = True
    touched = np.zeros(pos.shape[1], bool)
    touched[tri[shown].ravel()] = True
    assert not host(d_pos[0])[~touched].any()
    # image 0 alone equals image 0 in the batch
    p0 = dev(pos[:1]).requires_grad_(True)
    a0 = dev(attr[:1]).requires_grad_(True)
    _peel_chain(DiffRast, p0, t, a0, H, W, 4, [g[:1] for g in gfull])
    assert_grad_close(host(p0.grad[0]), host(d_pos[0]), "d_pos image 0 alone vs batch")


_hw = (np.arange(256, dtype=np.float32) + 0.5) / 256
ENV = np.stack([np.ones((256, 256), np.float32), np.repeat(1 - 2 * _hw[:, None], 256, 1),
                np.repeat(1 - 2 * _hw[None, :], 256, 0)], -1).astype(np.float32)


def test_range_batch_cube_4096():
    """Range mode: 4096 meshes of 512 triangles in one [V,4] buffer at
    256^2, per-pixel directions and their screen derivatives interpolated and
    looked up in a shared 6x512^2x3 cube map with the trilinear filter and a
    per-pixel bias map U[-1,1] (the cube + mip + bias extension), forward and
    backward to the cube map, the directions and pos.  Meshes 0..15 against
    the oracle (forward, d_cube, the direction gradient and its derivatives'
    gradient, then d_dir-attribute and d_pos through interpolate and the
    range-mode rasterize VJP with rast_db); the full batch against those
    meshes rendered alone."""
    torch = torch_dev()
    from diffrast import DiffRast
    _threads()
    sc = scenes.range_batch(N=4096, T_per=512, H=256, W=256)
    pos, tri, ranges, d = sc["pos"], sc["tri"], sc["ranges"], sc["dir"]
    rng = np.random.default_rng(9)
    cube = rng.random((1, 6, 512, 512, 3)).astype(np.float32)
    bias = rng.uniform(-1, 1, size=(4096, 256, 256)).astype(np.float32)

    def run(rows):
        p = dev(pos).requires_grad_(True)
        attr = dev(d).requires_grad_(True)
        tex = dev(cube).requires_grad_(True)
        rast, db = DiffRast.rasterize(p, dev(tri), (256, 256), gradDB=True,
                                      ranges=torch.as_tensor(ranges[rows]))
        dirs, dirs_da = DiffRast.interpolate(attr, rast, dev(tri), rastDB=db, diffAttrs="all")
        # empty pixels interpolate to the zero vector, which has no cube face
        # (NaN in the reference too): they look up the environment through
        # the +x face, one direction per pixel
        bg = (rast[..., 3:4] == 0).float()
        dirs = dirs + bg * torch.as_tensor(ENV, device=bg.device)
        col = DiffRast.texture(tex, dirs, uvDA=dirs_da, filterMode="linear-mipmap-linear",
                               boundaryMode="cube", mipLevelBiasMap=dev(bias[rows]),
                               dirGrad=True)
        dirs.retain_grad()
        dirs_da.retain_grad()
        g = torch.ones_like(col) * 1e-3
        (col * g).sum().backward()
        return rast, dirs, dirs_da, col, p, attr, tex

    rast, dirs, dirs_da, col, p, attr, tex = run(slice(0, 4096))
    t = rast[..., 3].reshape(4096, -1).long() - 1
    lo = torch.as_tensor(ranges[:, 0], device=t.device)[:, None]
    assert bool(((t < 0) | ((t >= lo) & (t < lo + 512))).all().item())
    assert bool(torch.isfinite(tex.grad).all().item()) and bool(torch.isfinite(p.grad).all().item())
    r16, d16, da16, c16, p16, a16, tex16 = run(slice(0, 16))
    np.testing.assert_array_equal(host(rast[:16]), host(r16))
    np.testing.assert_array_equal(host(dirs[:16]), host(d16))
    np.testing.assert_array_equal(host(col[:16]), host(c16))
    # the first 16 meshes' vertices only receive gradients from their images
    nt, nv = 16 * 512, 16 * 512 * 3
    assert_grad_close(host(p.grad[:nv]), host(p16.grad[:nv]), "d_pos (batch independence)")
    # meshes 0..15 against the oracle (their triangles and vertices come first)
    rr, rdb = O.rasterize(pos[:nv], tri[:nt], (256, 256), gradDB=True, ranges=ranges[:16],
                          max_per_tile=0)
    np.testing.assert_array_equal(host(r16), rr)
    dr, dda = O.interpolate(d[:nv], rr, tri[:nt], rastDB=rdb, diffAttrs="all")
    dr = dr + (rr[..., 3:4] == 0).astype(np.float32) * ENV
    np.testing.assert_array_equal(host(d16), dr)
    np.testing.assert_array_equal(host(da16), dda)
    cr = O.texture(cube, dr, uvDA=dda, filterMode="linear-mipmap-linear", boundaryMode="cube",
                   mipLevelBiasMap=bias[:16])
    assert_fwd_close(host(c16), cr)
    g = np.full(cr.shape, 1e-3, np.float32)
    vjp = lambda b: O.texture_vjp(cube, dr, g, uvDA=dda, filterMode="linear-mipmap-linear",
                                  boundaryMode="cube", mipLevelBias=b,
                                  mipLevelBiasMap=bias[:16], dirGrad=True)
    d_tex, d_dir, d_dda, _ = vjp(0.0)
    assert_grad_close(host(tex16.grad), d_tex, "d_cube")
    # the direction gradient and its derivatives' gradient, then through
    # interpolate and the range-mode rasterize VJP (with rast_db) to pos.
    # The oracle's chain continues from the GPU's d_dir / d_dirDA, so a LOD
    # switch pixel (evaluated on either side) is not counted twice.
    lo, hi = vjp(-LOD_DELTA), vjp(LOD_DELTA)
    sw = lod_switch_mask(d_dir, lo[1], hi[1]) | lod_switch_mask(d_dda, lo[2], hi[2])
    assert_grad_close_lod(host(d16.grad), d_dir, sw, lo[1], hi[1], "d_dir")
    assert_grad_close_lod(host(da16.grad), d_dda, sw, lo[2], hi[2], "d_dirDA")
    d_attr, d_rast, d_rdb = O.interpolate_vjp(d[:nv], rr, tri[:nt], host(d16.grad), rastDB=rdb,
                                              diffAttrs="all", d_out_da=host(da16.grad))
    assert_grad_close(host(a16.grad[:nv]), d_attr, "d_dir attribute")
    d_pos = O.rasterize_vjp(pos[:nv], tri[:nt], rr, d_rast, d_rdb, ranges=ranges[:16])
    assert_grad_close(host(p16.grad[:nv]), d_pos, "d_pos")
