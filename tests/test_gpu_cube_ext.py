"""GPU: the cube-map extension (mip filters, scalar and per-pixel bias, the
direction gradient) against the oracle's restatement of it (pinned in
tests/test_oracle_cube_ext.py by reduction to the reference's 2D trilinear
and cube bilinear, and by finite differences).  Forward within the forward
tolerance (the LOD's log2 may differ by an ulp between CPU and GPU); the
scatter-added d_tex within the gradient tolerance, and d_dir, d_dirDA and
d_biasMap within it off the pixels on a mip-level switch
(parity.lod_switch_mask), which must be under 1% of all."""
import numpy as np
import pytest

import oracle as O
from parity import (LOD_DELTA, assert_fwd_close, assert_grad_close, assert_grad_close_lod, dev, host,
                    lod_switch_mask, torch_dev)

pytestmark = pytest.mark.gpu


def cube_inputs(rng, N, Nt, S, C, Hi, Wi):
    tex = rng.random((Nt, 6, S, S, C)).astype(np.float32)
    dirs = rng.normal(size=(N, Hi, Wi, 3)).astype(np.float32)
    dd = (rng.normal(size=(N, Hi, Wi, 6)) * rng.choice([0.001, 0.01, 0.05, 0.3],
                                                       size=(N, Hi, Wi, 1))).astype(np.float32)
    return tex, dirs, dd


@pytest.mark.parametrize("filt", ["linear-mipmap-linear", "linear-mipmap-nearest"])
@pytest.mark.parametrize("C,Nt", [(3, 1), (4, 2), (1, 1), (5, 2)])
def test_cube_mip(filt, C, Nt):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(C * 10 + Nt + (0 if "linear-mipmap-linear" == filt else 100))
    N, S, Hi, Wi = 2, 32, 21, 27
    tex, dirs, dd = cube_inputs(rng, N, Nt, S, C, Hi, Wi)
    bm = rng.uniform(-1, 1, size=(N, Hi, Wi)).astype(np.float32)
    t = dev(tex).requires_grad_(True)
    u = dev(dirs).requires_grad_(True)
    d = dev(dd).requires_grad_(True)
    b = dev(bm).requires_grad_(True)
    out = DiffRast.texture(t, u, uvDA=d, filterMode=filt, boundaryMode="cube",
                           mipLevelBias=0.25, mipLevelBiasMap=b, dirGrad=True)
    ref = O.texture(tex, dirs, uvDA=dd, filterMode=filt, boundaryMode="cube", mipLevelBias=0.25,
                    mipLevelBiasMap=bm)
    assert_fwd_close(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_dir, d_dd, d_bm = O.texture_vjp(tex, dirs, g, uvDA=dd, filterMode=filt,
                                             boundaryMode="cube", mipLevelBias=0.25,
                                             mipLevelBiasMap=bm, dirGrad=True)
    assert tuple(t.grad.shape) == tex.shape
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    lo, hi = (O.texture_vjp(tex, dirs, g, uvDA=dd, filterMode=filt, boundaryMode="cube",
                            mipLevelBias=0.25 + b, mipLevelBiasMap=bm, dirGrad=True)
              for b in (-LOD_DELTA, LOD_DELTA))
    sw = (lod_switch_mask(d_dir, lo[1], hi[1]) | lod_switch_mask(d_dd, lo[2], hi[2]) |
          lod_switch_mask(d_bm, lo[3], hi[3]))
    assert_grad_close_lod(host(u.grad), d_dir, sw, lo[1], hi[1], "d_dir")
    assert_grad_close_lod(host(d.grad), d_dd, sw, lo[2], hi[2], "d_dirDA")
    assert_grad_close_lod(host(b.grad), d_bm, sw, lo[3], hi[3], "d_biasMap")


def test_cube_mip_shared_footprints():
    """Rows of pixels on one direction share their footprints on both
    levels: whole rows go through the backward's wave grouping (the
    per-wave accumulator and the grouped atomics) instead of the table."""
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(77)
    N, S, C, Hi, Wi = 1, 32, 3, 20, 40
    tex, dirs, dd = cube_inputs(rng, N, 1, S, C, Hi, Wi)
    dirs[:, 3:9] = np.array([1.0, 0.3, -0.2], np.float32)
    dd[:, 3:9] = np.float32(0.02)
    bm = rng.uniform(-1, 1, size=(N, Hi, Wi)).astype(np.float32)
    bm[:, 3:9] = 0.0
    t = dev(tex).requires_grad_(True)
    out = DiffRast.texture(t, dev(dirs), uvDA=dev(dd), filterMode="linear-mipmap-linear",
                           boundaryMode="cube", mipLevelBias=0.25, mipLevelBiasMap=dev(bm))
    ref = O.texture(tex, dirs, uvDA=dd, filterMode="linear-mipmap-linear", boundaryMode="cube",
                    mipLevelBias=0.25, mipLevelBiasMap=bm)
    assert_fwd_close(host(out), ref)
    g = rng.normal(size=ref.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex = O.texture_vjp(tex, dirs, g, uvDA=dd, filterMode="linear-mipmap-linear",
                          boundaryMode="cube", mipLevelBias=0.25, mipLevelBiasMap=bm)[0]
    assert_grad_close(host(t.grad), d_tex, "d_tex")


def test_cube_mip_without_dir_grad():
    # the default keeps the reference's zero direction gradient
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(7)
    tex, dirs, dd = cube_inputs(rng, 1, 1, 16, 3, 9, 11)
    u = dev(dirs).requires_grad_(True)
    d = dev(dd).requires_grad_(True)
    out = DiffRast.texture(dev(tex), u, uvDA=d, filterMode="linear-mipmap-linear",
                           boundaryMode="cube")
    out.sum().backward()
    np.testing.assert_array_equal(host(u.grad), 0)
    assert host(d.grad).any()


@pytest.mark.parametrize("C,Nt", [(3, 1), (2, 2)])
def test_cube_linear_dir_grad(C, Nt):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(20 + C)
    N, S, Hi, Wi = 2, 16, 13, 17
    tex, dirs, _ = cube_inputs(rng, N, Nt, S, C, Hi, Wi)
    t = dev(tex).requires_grad_(True)
    u = dev(dirs).requires_grad_(True)
    out = DiffRast.texture(t, u, boundaryMode="cube", dirGrad=True)
    np.testing.assert_array_equal(host(out), O.texture(tex, dirs, boundaryMode="cube"))
    g = rng.normal(size=out.shape).astype(np.float32)
    (out * dev(g)).sum().backward()
    d_tex, d_dir, _, _ = O.texture_vjp(tex, dirs, g, boundaryMode="cube", dirGrad=True)
    assert_grad_close(host(t.grad), d_tex, "d_tex")
    assert_grad_close(host(u.grad), d_dir, "d_dir")


def test_cube_mip_face_reduces_to_2d():
    """Directions on face +X with x = 1: the cube trilinear equals the 2D
    trilinear of that face (clamp), on the GPU too."""
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(9)
    cube = rng.random((1, 6, 32, 32, 4)).astype(np.float32)
    uv = (rng.integers(40, 4056, size=(1, 15, 17, 2)) / 4096.0).astype(np.float32)
    da = (rng.normal(size=(1, 15, 17, 4)) * 0.05).astype(np.float32)
    dirs = np.stack([np.ones_like(uv[..., 0]), 1 - 2 * uv[..., 1], 1 - 2 * uv[..., 0]], -1)
    dd = np.stack([np.zeros_like(da[..., 0])] * 2 + [-2 * da[..., 2], -2 * da[..., 3],
                                                     -2 * da[..., 0], -2 * da[..., 1]], -1)
    a = DiffRast.texture(dev(cube), dev(dirs.astype(np.float32)), uvDA=dev(dd.astype(np.float32)),
                         filterMode="linear-mipmap-linear", boundaryMode="cube")
    b = DiffRast.texture(dev(cube[:, 0]), dev(uv), uvDA=dev(da),
                         filterMode="linear-mipmap-linear", boundaryMode="clamp")
    np.testing.assert_array_equal(host(a), host(b))
