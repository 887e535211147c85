"""DR_ACCUMULATE through the C ABI: every scatter-accumulated gradient
(d_pos of rasterize and antialias, d_attr, d_tex, d_color of antialias) is
added to what its buffer holds; the other outputs are overwritten."""
import ctypes

import numpy as np
import pytest

import scenes
from parity import assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu

ACC = 1


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s(torch):
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


@pytest.fixture(scope="module")
def chain():
    torch = torch_dev()
    from diffrast import DiffRast
    sc = scenes.textured_icosphere(N=2, H=72, W=88, level=3, tex_size=32)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    H, W = sc["H"], sc["W"]
    rast, db = DiffRast.rasterize(pos, tri, (H, W), gradDB=True)
    attr = dev(sc["uv"])
    uv, uvda = DiffRast.interpolate(attr, rast, tri, rastDB=db, diffAttrs="all")
    tex = dev(sc["tex"])
    topo = DiffRast.antialiasConstructTopologyHash(tri)
    color = DiffRast.texture(tex, uv, uvDA=uvda, filterMode="linear-mipmap-linear",
                             boundaryMode="clamp")
    return dict(torch=torch, pos=pos, tri=tri, H=H, W=W, rast=rast, db=db, attr=attr, uv=uv,
                uvda=uvda, tex=tex, topo=topo, color=color.contiguous())


def _twice(run, outs, acc_mask, rng):
    """run(flags) fills `outs`; returns (fresh results, results with priors,
    priors)."""
    import torch
    run(0)
    torch.cuda.synchronize()
    fresh = [host(o).copy() for o in outs]
    priors = [rng.normal(size=o.shape).astype(np.float32) for o in outs]
    for o, p in zip(outs, priors):
        o.copy_(dev(p))
    run(ACC)
    torch.cuda.synchronize()
    got = [host(o) for o in outs]
    for f, g, p, a in zip(fresh, got, priors, acc_mask):
        assert_grad_close(g, f + p if a else f)


def test_rasterize_bwd_accumulate(chain):
    from diffrast import _lib
    lib, c = _lib.load(), chain
    torch = c["torch"]
    rng = np.random.default_rng(1)
    N, V = c["pos"].shape[:2]
    d_rast = dev(rng.normal(size=c["rast"].shape).astype(np.float32))
    d_db = dev(rng.normal(size=c["db"].shape).astype(np.float32))
    d_pos = torch.empty_like(c["pos"])
    run = lambda fl: _lib.check(lib.dr_rasterize_bwd(
        _p(c["pos"]), V * 4, _p(c["tri"]), _p(c["rast"]), _p(d_rast), _p(d_db), N, V,
        c["tri"].shape[0], c["H"], c["W"], _p(d_pos), fl, _s(torch)))
    _twice(run, [d_pos], [True], rng)


def test_interpolate_bwd_accumulate(chain):
    from diffrast import _lib
    lib, c = _lib.load(), chain
    torch = c["torch"]
    rng = np.random.default_rng(2)
    N = c["rast"].shape[0]
    V, A = c["attr"].shape
    d_out = dev(rng.normal(size=c["uv"].shape).astype(np.float32))
    d_da = dev(rng.normal(size=c["uvda"].shape).astype(np.float32))
    d_attr = torch.empty_like(c["attr"])
    d_rast = torch.empty_like(c["rast"])
    d_db = torch.empty_like(c["db"])
    run = lambda fl: _lib.check(lib.dr_interpolate_bwd(
        _p(c["attr"]), 0, _p(c["rast"]), _p(c["db"]), _p(c["tri"]), None, A, _p(d_out),
        _p(d_da), N, c["H"], c["W"], V, c["tri"].shape[0], A, _p(d_attr), 0, _p(d_rast), _p(d_db),
        fl, _s(torch)))
    _twice(run, [d_attr, d_rast, d_db], [True, False, False], rng)


def test_texture_bwd_accumulate(chain):
    from diffrast import _lib
    lib, c = _lib.load(), chain
    torch = c["torch"]
    rng = np.random.default_rng(3)
    tex = c["tex"]
    Nt, Ht, Wt, C = tex.shape
    lh, lw = (ctypes.c_int32 * 32)(), (ctypes.c_int32 * 32)()
    L = lib.dr_texture_mip_levels(Ht, Wt, -1, lh, lw)
    pyr = torch.empty(max(1, lib.dr_texture_mip_size(Nt, Ht, Wt, C, L)), device=tex.device)
    _lib.check(lib.dr_texture_build_mip(_p(tex), Nt, Ht, Wt, C, L, _p(pyr), _s(torch)))
    N, Hi, Wi = c["uv"].shape[:3]
    d_out = dev(rng.normal(size=(N, Hi, Wi, C)).astype(np.float32))
    d_tex = torch.empty_like(tex)
    d_uv = torch.empty_like(c["uv"])
    d_uvda = torch.empty_like(c["uvda"])
    run = lambda fl: _lib.check(lib.dr_texture_bwd(
        _p(tex), _p(pyr), Nt, Ht, Wt, C, L, _p(c["uv"]), _p(c["uvda"]), None, 0.0, 3, 1, N,
        Hi, Wi, _p(d_out), _p(d_tex), _p(d_uv), _p(d_uvda), None, fl, _s(torch)))
    _twice(run, [d_tex, d_uv, d_uvda], [True, False, False], rng)


@pytest.mark.parametrize("C", [4, 2, 5])
def test_antialias_bwd_accumulate(chain, C):
    from diffrast import _lib
    lib, c = _lib.load(), chain
    torch = c["torch"]
    rng = np.random.default_rng(4 + C)
    N, V = c["pos"].shape[:2]
    T = c["tri"].shape[0]
    H, W = c["H"], c["W"]
    color = dev(rng.random((N, H, W, C)).astype(np.float32))
    d_out = dev(rng.normal(size=(N, H, W, C)).astype(np.float32))
    d_color = torch.empty_like(color)
    d_pos = torch.empty_like(c["pos"])
    run = lambda fl: _lib.check(lib.dr_antialias_bwd(
        _p(color), _p(c["rast"]), _p(c["pos"]), _p(c["tri"]), _p(c["topo"]), _p(d_out), N, H,
        W, C, V, T, _p(d_color), _p(d_pos), fl, _s(torch)))
    _twice(run, [d_color, d_pos], [True, True], rng)


@pytest.mark.parametrize("C", [4, 3, 5])
def test_antialias_bwd_saved_accumulate(chain, C):
    """The same through dr_antialias_fwd_save / dr_antialias_bwd_saved (C 3
    and 5 take the other kernel instantiations), and the saved pair's
    gradients equal the plain pair's."""
    from diffrast import _lib
    lib, c = _lib.load(), chain
    torch = c["torch"]
    rng = np.random.default_rng(40 + C)
    N, V = c["pos"].shape[:2]
    T = c["tri"].shape[0]
    H, W = c["H"], c["W"]
    color = dev(rng.random((N, H, W, C)).astype(np.float32))
    d_out = dev(rng.normal(size=(N, H, W, C)).astype(np.float32))
    out = torch.empty_like(color)
    saved = torch.empty(lib.dr_antialias_saved_bytes(N, H, W, T), dtype=torch.uint8,
                        device="cuda")
    _lib.check(lib.dr_antialias_fwd_save(_p(color), _p(c["rast"]), _p(c["pos"]), _p(c["tri"]),
                                         _p(c["topo"]), N, H, W, C, V, T, _p(out), _p(saved),
                                         _s(torch)))
    d_color = torch.empty_like(color)
    d_pos = torch.empty_like(c["pos"])
    run = lambda fl: _lib.check(lib.dr_antialias_bwd_saved(
        _p(color), _p(c["rast"]), _p(c["pos"]), _p(c["tri"]), _p(c["topo"]), _p(d_out),
        _p(saved), N, H, W, C, V, T, _p(d_color), _p(d_pos), fl, _s(torch)))
    _twice(run, [d_color, d_pos], [True, True], rng)
    plain_c = torch.empty_like(color)
    plain_p = torch.empty_like(c["pos"])
    _lib.check(lib.dr_antialias_bwd(_p(color), _p(c["rast"]), _p(c["pos"]), _p(c["tri"]),
                                    _p(c["topo"]), _p(d_out), N, H, W, C, V, T, _p(plain_c),
                                    _p(plain_p), 0, _s(torch)))
    run(0)
    assert_grad_close(host(d_color), host(plain_c), "d_color saved vs plain")
    assert_grad_close(host(d_pos), host(plain_p), "d_pos saved vs plain")
