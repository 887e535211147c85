"""antialias on the GPU against the CPU oracle: topology hash bit-exact
(and equal to the O(T^2) brute force), forward within the forward
tolerance, d_color (gathered here, scattered by the reference) and d_pos
within the gradient tolerance."""
import numpy as np
import pytest

import oracle as O
import scenes
from parity import assert_fwd_close, assert_grad_close, dev, host, torch_dev
from test_oracle_antialias import brute_topology

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("case", ["icosphere", "random", "nonmanifold", "single"])
def test_topology(case):
    torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(3)
    if case == "icosphere":
        _, tri = scenes.icosphere(6)
    elif case == "random":
        tri = rng.integers(0, 500, size=(20000, 3)).astype(np.int32)
    elif case == "nonmanifold":
        tri = np.array([[0, 1, 2], [0, 1, 3], [0, 1, 4], [1, 2, 3]], np.int32)
    else:
        tri = np.array([[0, 1, 2]], np.int32)
    got = host(DiffRast.antialiasConstructTopologyHash(dev(tri)))
    ref = O.antialiasConstructTopologyHash(tri)
    np.testing.assert_array_equal(got, ref)
    if tri.shape[0] <= 20000 and case != "icosphere":
        np.testing.assert_array_equal(got, brute_topology(tri))


def aa_scene(kind):
    if kind == "hexpie":
        sc = scenes.hex_pie(N=3, H=96, W=80)
        return sc["pos"], sc["tri"], 96, 80
    if kind == "icosphere":
        sc = scenes.textured_icosphere(N=2, H=128, W=144, level=4, tex_size=8)
        return sc["pos"], sc["tri"], 128, 144
    if kind == "quad":
        pos = np.array([[-0.45, 0.55, 0, 1], [0.55, 0.55, 0, 1], [0.55, -0.45, 0, 1],
                        [-0.45, -0.45, 0, 1]], np.float32)[None]
        return pos, np.array([[0, 1, 2], [0, 2, 3]], np.int32), 4, 4
    sc = scenes.tier1_triangle(H=61, W=47)
    return sc["pos"], sc["tri"], 61, 47


@pytest.mark.parametrize("kind", ["hexpie", "icosphere", "quad", "tier1"])
@pytest.mark.parametrize("C", [1, 2, 3, 4, 5])
def test_antialias(kind, C):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(C + len(kind))
    pos, tri, H, W = aa_scene(kind)
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N = pos.shape[0]
    color = rng.random((N, H, W, C)).astype(np.float32)
    c = dev(color).requires_grad_(True)
    p = dev(pos).requires_grad_(True)
    out = DiffRast.antialias(c, dev(rast), p, dev(tri))
    ref = O.antialias(color, rast, pos, tri)
    assert_fwd_close(host(out), ref)
    assert (host(out) != color).any()
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_color, d_pos = O.antialias_vjp(color, rast, pos, tri, g)
    assert_grad_close(host(c.grad), d_color, "d_color")
    assert_grad_close(host(p.grad), d_pos, "d_pos")
    assert (host(p.grad)[..., 2] == 0).all()


def test_antialias_unaligned_rows():
    """Color rows that are not 16-byte aligned take the any-C kernel."""
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(11)
    pos, tri, H, W = aa_scene("tier1")
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N = pos.shape[0]
    color = rng.random((N, H, W, 4)).astype(np.float32)
    buf = torch.empty(color.size + 1, device="cuda")
    c = buf[1:].view(color.shape)
    c.copy_(dev(color))
    assert c.data_ptr() % 16 != 0
    out = DiffRast.antialias(c, dev(rast), dev(pos), dev(tri))
    assert_fwd_close(host(out), O.antialias(color, rast, pos, tri))


@pytest.mark.parametrize("C", [4, 3])
def test_antialias_dense_edges(C):
    """Triangles of a few pixels: about 40% of the pixels blend, up to ~220
    of a 16x16 tile's 256, most in more than one direction, so some tiles
    hold more partial blends than the d_pos queue (256) and the overflow
    path runs too."""
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(21 + C)
    sc = scenes.textured_icosphere(N=2, H=128, W=128, level=5, tex_size=8)
    pos, tri, H, W = sc["pos"], sc["tri"], 128, 128
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N = pos.shape[0]
    color = rng.random((N, H, W, C)).astype(np.float32)
    ref = O.antialias(color, rast, pos, tri)
    blended = (ref != color).any(-1).sum(axis=(1, 2))
    assert blended.min() > 4000, blended
    c = dev(color).requires_grad_(True)
    p = dev(pos).requires_grad_(True)
    out = DiffRast.antialias(c, dev(rast), p, dev(tri))
    assert_fwd_close(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_color, d_pos = O.antialias_vjp(color, rast, pos, tri, g)
    assert_grad_close(host(c.grad), d_color, "d_color")
    assert_grad_close(host(p.grad), d_pos, "d_pos")


def aa_abi(color, rast, pos, tri, g, masked):
    """Forward and backward straight through the C ABI: dr_antialias_fwd /
    dr_antialias_bwd, or dr_antialias_fwd_save / dr_antialias_bwd_saved
    (the forward keeps state, the blend mask first, that the backward
    reads).  Returns out, the blend mask as [N, H, W] (or None), d_color,
    d_pos."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast import DiffRast
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    N, H, W, C = color.shape
    V, T = pos.shape[1], tri.shape[0]
    c, r, p, t = dev(color), dev(rast), dev(pos), dev(tri)
    topo = DiffRast.antialiasConstructTopologyHash(t)
    out = torch.empty_like(c)
    d_color = torch.empty_like(c)
    d_pos = torch.empty_like(p)
    gd = dev(g)
    if masked:
        mask = torch.full((lib.dr_antialias_saved_bytes(N, H, W, T),), 0xAA, dtype=torch.uint8,
                          device="cuda")
        L.check(lib.dr_antialias_fwd_save(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), N, H, W,
                                          C, V, T, _ptr(out), _ptr(mask), _stream()))
        L.check(lib.dr_antialias_bwd_saved(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo),
                                           _ptr(gd), _ptr(mask), N, H, W, C, V, T, _ptr(d_color),
                                           _ptr(d_pos), 0, _stream()))
    else:
        mask = None
        L.check(lib.dr_antialias_fwd(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), N, H, W, C, V,
                                     T, _ptr(out), _stream()))
        L.check(lib.dr_antialias_bwd(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), _ptr(gd), N, H,
                                     W, C, V, T, _ptr(d_color), _ptr(d_pos), 0, _stream()))
    if mask is not None:  # the header's byte order -> [N, H, W]
        h, w = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
        nty, ntx = -(-H // 16), -(-W // 16)
        idx = ((h // 16) * ntx + w // 16) * 256 + ((h % 16) // 8 * 2 + (w % 16) // 8) * 64 + \
            (h % 8) * 8 + w % 8
        m = host(mask)
        mask = np.stack([m[n * nty * ntx * 256 + idx] for n in range(N)])
    return host(out), mask, host(d_color), host(d_pos)


@pytest.mark.parametrize("scene", ["dense", "icosphere", "hexpie"])
def test_antialias_mask_abi(scene):
    """Both backward entry points against the oracle on the same inputs; the
    forward's blend mask marks exactly the pixels that blend (random
    colours, so a blend changes the pixel), in a tile-border-heavy scene
    too.  The unmasked backward's d_pos queue overflows in the dense scene."""
    torch_dev()
    rng = np.random.default_rng(5)
    if scene == "dense":
        sc = scenes.textured_icosphere(N=2, H=128, W=128, level=5, tex_size=8)
        pos, tri, H, W = sc["pos"], sc["tri"], 128, 128
    else:
        pos, tri, H, W = aa_scene(scene)
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N = pos.shape[0]
    color = rng.random((N, H, W, 4)).astype(np.float32)
    ref = O.antialias(color, rast, pos, tri)
    g = rng.normal(size=ref.shape).astype(np.float32)
    d_color, d_pos = O.antialias_vjp(color, rast, pos, tri, g)
    for masked in (False, True):
        out, mask, dc, dp = aa_abi(color, rast, pos, tri, g, masked)
        assert_fwd_close(out, ref)
        assert_grad_close(dc, d_color, f"d_color masked={masked}")
        assert_grad_close(dp, d_pos, f"d_pos masked={masked}")
        if masked:
            assert mask.max() < 16
            np.testing.assert_array_equal(mask != 0, (ref != color).any(-1))


def test_antialias_saved_mask_superset():
    """The backward re-derives every queued pair's blend weight, so a blend
    mask with every bit set (also on pixels next to nothing, next to the
    image border, or on empty pixels) gives the same gradients, and no mask
    content can send a record or vertex read out of range."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast import DiffRast
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    rng = np.random.default_rng(9)
    pos, tri, H, W = aa_scene("tier1")  # ragged 61 x 47, mostly empty pixels
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N, V, T, C = pos.shape[0], pos.shape[1], tri.shape[0], 4
    color = rng.random((N, H, W, C)).astype(np.float32)
    g = rng.normal(size=color.shape).astype(np.float32)
    d_color, d_pos = O.antialias_vjp(color, rast, pos, tri, g)
    c, r, p, t, gd = dev(color), dev(rast), dev(pos), dev(tri), dev(g)
    topo = DiffRast.antialiasConstructTopologyHash(t)
    out = torch.empty_like(c)
    saved = torch.empty(lib.dr_antialias_saved_bytes(N, H, W, T), dtype=torch.uint8, device="cuda")
    L.check(lib.dr_antialias_fwd_save(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), N, H, W, C,
                                      V, T, _ptr(out), _ptr(saved), _stream()))
    mask_bytes = N * (-(-H // 16)) * (-(-W // 16)) * 256
    saved[:mask_bytes].fill_(0xFF)
    dc, dp = torch.empty_like(c), torch.empty_like(p)
    L.check(lib.dr_antialias_bwd_saved(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), _ptr(gd),
                                       _ptr(saved), N, H, W, C, V, T, _ptr(dc), _ptr(dp), 0,
                                       _stream()))
    assert_grad_close(host(dc), d_color, "d_color, full mask")
    assert_grad_close(host(dp), d_pos, "d_pos, full mask")


def test_antialias_saved_ids_stay_in_bounds():
    """The saved state's triangle ids (int32 in the blend mask's pixel order,
    after the mask) equal rast's; ids outside [0, T) read as empty, as rast
    ids do, so garbage there, with every mask bit set, changes the gradients
    but sends no record or vertex read out of range."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast import DiffRast
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    rng = np.random.default_rng(11)
    pos, tri, H, W = aa_scene("tier1")  # ragged 61 x 47
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N, V, T, C = pos.shape[0], pos.shape[1], tri.shape[0], 4
    color = rng.random((N, H, W, C)).astype(np.float32)
    g = rng.normal(size=color.shape).astype(np.float32)
    c, r, p, t, gd = dev(color), dev(rast), dev(pos), dev(tri), dev(g)
    topo = DiffRast.antialiasConstructTopologyHash(t)
    out = torch.empty_like(c)
    saved = torch.empty(lib.dr_antialias_saved_bytes(N, H, W, T), dtype=torch.uint8, device="cuda")
    L.check(lib.dr_antialias_fwd_save(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), N, H, W, C,
                                      V, T, _ptr(out), _ptr(saved), _stream()))
    nty, ntx = -(-H // 16), -(-W // 16)
    mask_bytes = N * nty * ntx * 256
    ids = saved[mask_bytes:5 * mask_bytes].view(torch.int32)
    h, w = np.meshgrid(np.arange(H), np.arange(W), indexing="ij")
    idx = ((h // 16) * ntx + w // 16) * 256 + ((h % 16) // 8 * 2 + (w % 16) // 8) * 64 + \
        (h % 8) * 8 + w % 8
    got = host(ids)
    got = np.stack([got[n * nty * ntx * 256 + idx] for n in range(N)])
    want = rast[..., 3].astype(np.int64) - 1  # rast ids are triangle + 1, 0 = empty
    np.testing.assert_array_equal(got, want)
    assert (want >= 0).any() and (want < 0).any()
    ids.copy_(torch.randint(-2 ** 31, 2 ** 31 - 1, ids.shape, dtype=torch.int32, device="cuda"))
    ids[::7] = torch.arange(ids[::7].numel(), dtype=torch.int32, device="cuda") % max(T, 1)
    saved[:mask_bytes].fill_(0xFF)
    dc, dp = torch.empty_like(c), torch.empty_like(p)
    L.check(lib.dr_antialias_bwd_saved(_ptr(c), _ptr(r), _ptr(p), _ptr(t), _ptr(topo), _ptr(gd),
                                       _ptr(saved), N, H, W, C, V, T, _ptr(dc), _ptr(dp), 0,
                                       _stream()))
    torch.cuda.synchronize()
    assert np.isfinite(host(dc)).all()


def test_straight_edge_blend_weights():
    """The blend weight by value on the GPU: straight silhouette edges
    crossing every pixel row or column at exact sub-pixel positions
    (Antialias.swift:274-309).  Coverage from the GPU rasterizer, and the
    forward of DiffRast.antialias and of both C-ABI forward entry points
    with a one-hot coverage colour, equal the closed form
    beta = 0.5 - |x_e - (q + 0.5)| bit for bit; the gradients match the
    oracle."""
    torch_dev()
    from diffrast import DiffRast
    from test_oracle_antialias import straight_edge_expect
    H = W = 64
    sc = scenes.straight_edges(H, W)
    pos, tri, beta = sc["pos"], sc["tri"], sc["beta"]
    rast, _ = DiffRast.rasterize(dev(pos), dev(tri), (H, W), gradDB=False)
    rast = host(rast)
    cov = (rast[..., 3] > 0).astype(np.float32)
    np.testing.assert_array_equal(cov, sc["cov"])
    color = np.stack([cov, 1.0 - cov], -1)
    expect = straight_edge_expect(color, cov, beta)
    out = DiffRast.antialias(dev(color), dev(rast), dev(pos), dev(tri))
    np.testing.assert_array_equal(host(out), expect)
    g = np.random.default_rng(11).normal(size=color.shape).astype(np.float32)
    d_color, d_pos = O.antialias_vjp(color, rast, pos, tri, g)
    for masked in (False, True):
        o, mask, dc, dp = aa_abi(color, rast, pos, tri, g, masked)
        np.testing.assert_array_equal(o, expect)
        assert_grad_close(dc, d_color, f"d_color masked={masked}")
        assert_grad_close(dp, d_pos, f"d_pos masked={masked}")
        if masked:
            np.testing.assert_array_equal(mask != 0, beta > 0)
