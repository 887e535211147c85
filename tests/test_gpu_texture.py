"""texture on the GPU against the CPU oracle, every filter x boundary mode,
shared and per-image textures, C in {1,2,3,4,5}, mip bias (scalar and
per-pixel), cube maps.  Forward within the forward tolerance (the LOD's
log2 may differ by an ulp between CPU and GPU, so mip modes are compared
with tolerance); d_uv and the scatter-added d_tex within the gradient
tolerance; d_uvDA / d_biasMap within it off the pixels on a mip-level
switch (parity.lod_switch_mask), which must be under 1% of all."""
import numpy as np
import pytest

import oracle as O
from parity import (LOD_DELTA, assert_fwd_close, assert_grad_close, assert_grad_close_lod, dev, host,
                    lod_switch_mask, torch_dev)

pytestmark = pytest.mark.gpu

FILTERS = ["nearest", "linear", "linear-mipmap-nearest", "linear-mipmap-linear"]
BOUNDS = ["wrap", "clamp", "zero"]


def inputs(rng, N, Nt, Ht, Wt, C, Hi, Wi):
    tex = rng.random((Nt, Ht, Wt, C)).astype(np.float32)
    uv = rng.uniform(-0.3, 1.3, size=(N, Hi, Wi, 2)).astype(np.float32)
    uv[:, :3] = 0.0  # a band of "background" pixels sampling one texel (hotspot)
    da = (rng.normal(size=(N, Hi, Wi, 4)) * rng.choice([0.001, 0.02, 0.2, 2.0],
                                                       size=(N, Hi, Wi, 1))).astype(np.float32)
    da[:, :3] = 0.0
    return tex, uv, da


@pytest.mark.parametrize("filt", FILTERS)
@pytest.mark.parametrize("bnd", BOUNDS)
@pytest.mark.parametrize("C,Nt", [(4, 1), (3, 2), (1, 2), (5, 1), (2, 1)])
def test_texture(filt, bnd, C, Nt):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(FILTERS.index(filt) * 100 + BOUNDS.index(bnd) * 10 + C * 2 + Nt)
    N, Ht, Wt, Hi, Wi = 2, 32, 64, 37, 45
    tex, uv, da = inputs(rng, N, Nt, Ht, Wt, C, Hi, Wi)
    mip = "mipmap" in filt
    t = dev(tex).requires_grad_(True)
    u = dev(uv).requires_grad_(True)
    d = dev(da).requires_grad_(True) if mip else None
    out = DiffRast.texture(t, u, uvDA=d, filterMode=filt, boundaryMode=bnd)
    ref = O.texture(tex, uv, uvDA=da if mip else None, filterMode=filt, boundaryMode=bnd)
    if mip:
        assert_fwd_close(host(out), ref)
    else:
        np.testing.assert_array_equal(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_uv, d_da, _ = O.texture_vjp(tex, uv, g, uvDA=da if mip else None, filterMode=filt,
                                         boundaryMode=bnd)
    assert tuple(t.grad.shape) == tex.shape
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    assert_grad_close(host(u.grad), d_uv, "d_uv")
    if mip:
        lo, hi = (O.texture_vjp(tex, uv, g, uvDA=da, filterMode=filt, boundaryMode=bnd,
                                mipLevelBias=b)[2] for b in (-LOD_DELTA, LOD_DELTA))
        assert_grad_close_lod(host(d.grad), d_da, lod_switch_mask(d_da, lo, hi), lo, hi, "d_uvDA")


@pytest.mark.parametrize("filt", ["linear-mipmap-linear", "linear-mipmap-nearest"])
def test_mip_bias(filt):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(5)
    tex, uv, da = inputs(rng, 2, 1, 64, 64, 4, 31, 33)
    bm = rng.uniform(-1, 1, size=(2, 31, 33)).astype(np.float32)
    t = dev(tex).requires_grad_(True)
    u = dev(uv).requires_grad_(True)
    d = dev(da).requires_grad_(True)
    b = dev(bm).requires_grad_(True)
    out = DiffRast.texture(t, u, uvDA=d, filterMode=filt, boundaryMode="clamp",
                           mipLevelBias=0.5, mipLevelBiasMap=b)
    ref = O.texture(tex, uv, uvDA=da, filterMode=filt, boundaryMode="clamp",
                    mipLevelBias=0.5, mipLevelBiasMap=bm)
    assert_fwd_close(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_uv, d_da, d_bm = O.texture_vjp(tex, uv, g, uvDA=da, filterMode=filt,
                                            boundaryMode="clamp", mipLevelBias=0.5,
                                            mipLevelBiasMap=bm)
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    assert_grad_close(host(u.grad), d_uv, "d_uv")
    lo, hi = (O.texture_vjp(tex, uv, g, uvDA=da, filterMode=filt, boundaryMode="clamp",
                            mipLevelBias=0.5 + b, mipLevelBiasMap=bm) for b in (-LOD_DELTA, LOD_DELTA))
    sw = lod_switch_mask(d_da, lo[2], hi[2]) | lod_switch_mask(d_bm, lo[3], hi[3])
    assert_grad_close_lod(host(d.grad), d_da, sw, lo[2], hi[2], "d_uvDA")
    assert_grad_close_lod(host(b.grad), d_bm, sw, lo[3], hi[3], "d_biasMap")


@pytest.mark.parametrize("C,Nt", [(3, 1), (1, 2), (4, 2)])
def test_cube(C, Nt):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(C)
    N, Ht, Wt, Hi, Wi = 2, 16, 16, 19, 23
    tex = rng.random((Nt, 6, Ht, Wt, C)).astype(np.float32)
    dirs = rng.normal(size=(N, Hi, Wi, 3)).astype(np.float32)
    t = dev(tex).requires_grad_(True)
    u = dev(dirs).requires_grad_(True)
    out = DiffRast.texture(t, u, boundaryMode="cube")
    ref = O.texture(tex, dirs, boundaryMode="cube")
    np.testing.assert_array_equal(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_dir, _, _ = O.texture_vjp(tex, dirs, g, boundaryMode="cube")
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    np.testing.assert_array_equal(host(u.grad), 0)


def test_construct_mip():
    torch = torch_dev()
    from diffrast import DiffRast
    tex = np.random.default_rng(0).random((2, 64, 32, 3)).astype(np.float32)
    got = DiffRast.textureConstructMip(dev(tex))
    ref = O.textureConstructMip(tex)
    assert len(got) == len(ref) == 6
    for a, b in zip(got, ref):
        np.testing.assert_array_equal(host(a), b)
    got = DiffRast.textureConstructMip(dev(tex), maxLevel=2)
    assert [tuple(l.shape) for l in got] == [(2, 64, 32, 3), (2, 32, 16, 3), (2, 16, 8, 3)]


def test_fixture_parity(fixtures):
    """ParityTests.swift:92-111 on the GPU: nvdiffrast's texture outputs."""
    torch_dev()
    from diffrast import DiffRast
    tex = np.zeros((1, 8, 8, 3), np.float32)
    for y in range(8):
        for x in range(8):
            tex[0, y, x] = [x / 7, y / 7, (x + y) / 14]
    out = DiffRast.texture(dev(tex), dev(fixtures["uv"]), boundaryMode="clamp")
    assert np.abs(host(out) - fixtures["tex_bilinear"]).max() <= 1e-5
    out = DiffRast.texture(dev(tex), dev(fixtures["uv"]), uvDA=dev(fixtures["uv_da"]),
                           filterMode="linear-mipmap-linear", boundaryMode="clamp")
    assert np.abs(host(out) - fixtures["tex_trilinear"]).max() <= 1e-4


@pytest.mark.parametrize("filt", ["linear-mipmap-linear", "linear-mipmap-nearest", "linear"])
@pytest.mark.parametrize("bnd", ["clamp", "wrap"])
def test_smooth_lod_ramp(filt, bnd):
    """A smooth uv field whose LOD rises across the image (~1.1 to ~3.2), so
    16x16 tiles hold one, two or three levels and waves of one tile start on
    different levels; a background band samples one texel."""
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(7)
    N, Hi, Wi, Ht, Wt, C = 2, 96, 112, 256, 256, 4
    x = (np.arange(Wi, dtype=np.float32) + 0.5)[None, :] * np.ones((Hi, 1), np.float32)
    y = (np.arange(Hi, dtype=np.float32) + 0.5)[:, None] * np.ones((1, Wi), np.float32)
    u = 2.0 * (x / Wi) ** 2 + 0.01
    v = y / Hi * 0.8 + 0.1
    uv = np.stack([u, v], -1)[None].repeat(N, 0).astype(np.float32)
    da = np.stack([4.0 * x / Wi ** 2, np.zeros_like(x), np.zeros_like(x),
                   np.full_like(x, 0.8 / Hi)], -1)[None].repeat(N, 0).astype(np.float32)
    uv[:, :, :5] = 0.0
    da[:, :, :5] = 0.0
    tex = rng.random((1, Ht, Wt, C)).astype(np.float32)
    mip = "mipmap" in filt
    t = dev(tex).requires_grad_(True)
    uu = dev(uv).requires_grad_(True)
    d = dev(da).requires_grad_(True) if mip else None
    out = DiffRast.texture(t, uu, uvDA=d, filterMode=filt, boundaryMode=bnd)
    ref = O.texture(tex, uv, uvDA=da if mip else None, filterMode=filt, boundaryMode=bnd)
    assert_fwd_close(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_uv, d_da, _ = O.texture_vjp(tex, uv, g, uvDA=da if mip else None, filterMode=filt,
                                         boundaryMode=bnd)
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    assert_grad_close(host(uu.grad), d_uv, "d_uv")
    if mip:
        lo, hi = (O.texture_vjp(tex, uv, g, uvDA=da, filterMode=filt, boundaryMode=bnd,
                                mipLevelBias=b)[2] for b in (-LOD_DELTA, LOD_DELTA))
        assert_grad_close_lod(host(d.grad), d_da, lod_switch_mask(d_da, lo, hi), lo, hi, "d_uvDA")


def test_cached_pyramid():
    # texture(..., mip=textureConstructMip(tex)) reuses the pyramid: the same
    # outputs and gradients as a pyramid built in the call, and a copied
    # (unpacked) list gives the same again
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(11)
    tex, uv, da = inputs(rng, 2, 1, 64, 32, 4, 29, 31)
    outs = []
    for mode in ("built", "cached", "copied"):
        t = dev(tex).requires_grad_(True)
        u = dev(uv).requires_grad_(True)
        d = dev(da).requires_grad_(True)
        mip = None
        if mode != "built":
            mip = DiffRast.textureConstructMip(t.detach())
            if mode == "copied":
                mip = [lv.clone() for lv in mip]
        out = DiffRast.texture(t, u, uvDA=d, filterMode="linear-mipmap-linear",
                               boundaryMode="clamp", mip=mip)
        g = dev(np.linspace(-1, 1, out.numel(), dtype=np.float32).reshape(out.shape))
        (out * g).sum().backward()
        outs.append([host(x) for x in (out, t.grad, u.grad, d.grad)])
    for k in (1, 2):
        np.testing.assert_array_equal(outs[k][0], outs[0][0])
        for a, b in zip(outs[k][1:], outs[0][1:]):
            assert_grad_close(a, b)


def test_cached_pyramid_fewer_levels():
    # a pyramid of 4 levels caps the LOD at 3: a large footprint samples the
    # 8x8 box means of level 3 (at texel centres, exactly one texel)
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(12)
    tex = rng.random((1, 32, 32, 3)).astype(np.float32)
    td = dev(tex)
    mip = DiffRast.textureConstructMip(td, maxLevel=3)
    assert len(mip) == 4
    iy, ix = np.meshgrid(np.arange(4), np.arange(4), indexing="ij")
    uv = np.stack([(ix + 0.5) / 4, (iy + 0.5) / 4], -1).astype(np.float32)[None]
    da = np.tile(np.array([1.0, 0.0, 0.0, 1.0], np.float32), (1, 4, 4, 1))
    out = DiffRast.texture(td, dev(uv), uvDA=dev(da), filterMode="linear-mipmap-linear",
                           boundaryMode="clamp", mip=mip)
    want = tex.astype(np.float64).reshape(1, 4, 8, 4, 8, 3).mean(axis=(2, 4))
    np.testing.assert_allclose(host(out), want, rtol=1e-6, atol=1e-6)
    with pytest.raises(ValueError):
        DiffRast.texture(dev(tex), dev(uv), uvDA=dev(da), filterMode="linear-mipmap-linear",
                         mip=[dev(tex), dev(tex)])


def test_cached_pyramid_stale():
    # a pyramid whose texture was changed in place (an optimizer step) or
    # that belongs to another tensor is refused; a rebuilt one is accepted
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(13)
    tex, uv, da = inputs(rng, 1, 1, 32, 32, 4, 9, 11)
    t = dev(tex).requires_grad_(True)
    kw = dict(uvDA=dev(da), filterMode="linear-mipmap-linear", boundaryMode="clamp")
    mip = DiffRast.textureConstructMip(t.detach())
    DiffRast.texture(t, dev(uv), mip=mip, **kw)
    with torch.no_grad():
        t.add_(0.5)
    with pytest.raises(ValueError, match="modified in place"):
        DiffRast.texture(t, dev(uv), mip=mip, **kw)
    with pytest.raises(ValueError, match="another texture"):
        DiffRast.texture(dev(tex), dev(uv), mip=DiffRast.textureConstructMip(t.detach()), **kw)
    mip = DiffRast.textureConstructMip(t.detach())
    out = DiffRast.texture(t, dev(uv), mip=mip, **kw)
    ref = O.texture(tex + np.float32(0.5), uv, uvDA=da, filterMode="linear-mipmap-linear",
                    boundaryMode="clamp")
    assert_fwd_close(host(out), ref)


@pytest.mark.parametrize("C", [4, 5])
def test_level_above_2g_elements(C):
    """A texture level of more than 2^31 floats (C = 4: the windowed
    backward, sides up to 32767; C = 5: the tiled backward): texel offsets
    are formed in 64 bits (32 bits where a level stays below 2^32 floats).
    16 pixels sample the last 8x8 texels; their outputs and gradients equal
    those of the same texels as a texture of their own (the pixels' uv
    rescaled, so the bilinear fractions differ by the rounding of u * W),
    and d_tex is zero away from them."""
    torch = torch_dev()
    from diffrast import DiffRast
    S = 23200 if C == 4 else 20800
    assert S * S * C > 2 ** 31
    gen = torch.Generator(device="cuda").manual_seed(C)
    tex = torch.rand((1, S, S, C), device="cuda", generator=gen).requires_grad_(True)
    rng = np.random.default_rng(C)
    x = rng.uniform(S - 7.5, S - 0.5, size=(1, 4, 4, 2))   # texel-space sample points
    uv = dev((x / S).astype(np.float32))
    g = dev(rng.standard_normal((1, 4, 4, C)).astype(np.float32))
    uv_big = uv.detach().clone().requires_grad_(True)
    out = DiffRast.texture(tex, uv_big, filterMode="linear", boundaryMode="clamp")
    d_tex, d_uv = torch.autograd.grad(out, [tex, uv_big], g)
    corner = host(d_tex[0, S - 8:, S - 8:, :]).copy()
    far = host(d_tex[0, :64, :64, :]).copy()
    got_out, got_duv = host(out).copy(), host(d_uv).copy()
    crop = tex.detach()[:, S - 8:, S - 8:, :].contiguous().requires_grad_(True)
    del tex, d_tex, out
    torch.cuda.empty_cache()
    uv_c = dev(((x - (S - 8)) / 8).astype(np.float32)).requires_grad_(True)
    ref = DiffRast.texture(crop, uv_c, filterMode="linear", boundaryMode="clamp")
    r_tex, r_uv = torch.autograd.grad(ref, [crop, uv_c], g)
    np.testing.assert_allclose(got_out, host(ref), rtol=0, atol=2e-3)
    np.testing.assert_allclose(corner, host(r_tex)[0], rtol=0, atol=5e-3 * float(np.abs(host(g)).max()))
    # d_uv scales with the texture size (u * S against u' * 8); the sample
    # points differ by up to S * 2^-24 texels between the two, so the
    # differences are held to 2e-3 of the largest component
    r_duv = host(r_uv) * (S / 8.0)
    np.testing.assert_allclose(got_duv, r_duv, rtol=0, atol=2e-3 * float(np.abs(r_duv).max()))
    assert not far.any()
