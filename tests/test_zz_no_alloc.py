"""dr_texture_bwd_noalloc, the texture backward that allocates nothing,
against dr_texture_bwd through the C ABI on the same inputs: several calls
in a row on one GPU (the fixed array keeps the previous call's contents),
the later ones smaller, 2D trilinear with and without a bias map and the
cube extension; a pyramid above the fixed array is rejected before any
work is queued.  Per-pixel gradients (d_uv, d_uvDA, d_biasMap) are written
by the same kernels and must be identical; d_tex within the scatter-add
tolerance (atomic order)."""
import ctypes

import numpy as np
import pytest

from parity import assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu

LINEAR_MIPMAP_LINEAR, CLAMP, WRAP, CUBE = 3, 1, 0, 3


def _case(rng, N, Nt, S, C, Hi, Wi, cube, bias_map):
    tex = rng.random((Nt, 6, S, S, C) if cube else (Nt, S, S, C)).astype(np.float32)
    if cube:
        uv = rng.normal(size=(N, Hi, Wi, 3)).astype(np.float32)
        da = (rng.normal(size=(N, Hi, Wi, 6)) * 0.05).astype(np.float32)
    else:
        uv = rng.uniform(-0.2, 1.2, size=(N, Hi, Wi, 2)).astype(np.float32)
        uv[:, :2] = 0.0  # background rows on one texel
        da = (rng.normal(size=(N, Hi, Wi, 4)) * rng.choice([0.001, 0.02, 0.3],
                                                           size=(N, Hi, Wi, 1))).astype(np.float32)
    bm = rng.uniform(-1, 1, size=(N, Hi, Wi)).astype(np.float32) if bias_map else None
    g = rng.normal(size=(N, Hi, Wi, C)).astype(np.float32)
    return tex, uv, da, bm, g


def _run(fn_name, tex, uv, da, bm, g, cube, boundary, flags):
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    N, Hi, Wi = uv.shape[:3]
    Nt, C = tex.shape[0], tex.shape[-1]
    S = tex.shape[-2]
    L_levels = lib.dr_texture_mip_levels(S, S, -1, None, None)
    faces = Nt * 6 if cube else Nt
    td = dev(tex)
    pyr = torch.empty(max(lib.dr_texture_mip_size(faces, S, S, C, L_levels), 1), device="cuda")
    L.check(lib.dr_texture_build_mip(_ptr(td), faces, S, S, C, L_levels, _ptr(pyr), _stream()))
    uvd, dad, gd = dev(uv), dev(da), dev(g)
    bmd = dev(bm) if bm is not None else None
    d_tex = torch.full(tex.shape, 7.0, device="cuda")  # overwritten (zeroed first)
    d_uv = torch.full(uv.shape, 7.0, device="cuda")
    d_da = torch.full(da.shape, 7.0, device="cuda")
    d_bm = torch.full(bm.shape, 7.0, device="cuda") if bm is not None else None
    fn = getattr(lib, fn_name)
    L.check(fn(_ptr(td), _ptr(pyr), Nt, S, S, C, L_levels, _ptr(uvd), _ptr(dad), _ptr(bmd), 0.25,
               LINEAR_MIPMAP_LINEAR, boundary, N, Hi, Wi, _ptr(gd), _ptr(d_tex), _ptr(d_uv),
               _ptr(d_da), _ptr(d_bm), flags, _stream()))
    torch.cuda.synchronize()
    return [host(d_tex), host(d_uv), host(d_da), None if d_bm is None else host(d_bm)]


CASES = [  # N, Nt, S, C, Hi, Wi, cube, bias map, boundary, flags
    (2, 1, 256, 4, 64, 80, False, False, CLAMP, 0),
    (1, 1, 64, 3, 33, 41, False, True, WRAP, 0),
    (2, 2, 32, 3, 19, 23, True, True, CUBE, 2),   # DR_CUBE_DIR_GRAD
    (1, 1, 16, 1, 9, 11, False, False, CLAMP, 0),
]


def test_texture_bwd_noalloc_matches():
    rng = np.random.default_rng(99)
    for k, (N, Nt, S, C, Hi, Wi, cube, bias, bnd, flags) in enumerate(CASES):
        args = _case(rng, N, Nt, S, C, Hi, Wi, cube, bias)
        ref = _run("dr_texture_bwd", *args, cube, bnd, flags)
        got = _run("dr_texture_bwd_noalloc", *args, cube, bnd, flags)
        assert_grad_close(got[0], ref[0], f"d_tex case {k}")
        for a, b, what in zip(got[1:], ref[1:], ("d_uv", "d_uvDA", "d_biasMap")):
            if b is not None:
                np.testing.assert_array_equal(a, b, err_msg=f"{what} case {k}")


def test_texture_bwd_noalloc_rejects_large_pyramid():
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    S, C = 4096, 4  # levels 1.. of a 4096^2 RGBA texture: 22.4M floats > 8M
    L_levels = lib.dr_texture_mip_levels(S, S, -1, None, None)
    assert lib.dr_texture_mip_size(1, S, S, C, L_levels) > L.DR_TEXTURE_BWD_NOALLOC_FLOATS
    tex = torch.zeros((1, S, S, C), device="cuda")
    pyr = torch.zeros(lib.dr_texture_mip_size(1, S, S, C, L_levels), device="cuda")
    uv = torch.zeros((1, 8, 8, 2), device="cuda")
    da = torch.zeros((1, 8, 8, 4), device="cuda")
    g = torch.zeros((1, 8, 8, C), device="cuda")
    d_tex = torch.zeros_like(tex)
    rc = lib.dr_texture_bwd_noalloc(_ptr(tex), _ptr(pyr), 1, S, S, C, L_levels, _ptr(uv), _ptr(da),
                                    None, 0.0, LINEAR_MIPMAP_LINEAR, CLAMP, 1, 8, 8, _ptr(g),
                                    _ptr(d_tex), None, None, None, 0, _stream())
    assert rc == L.DR_ERR_ARGUMENT
    assert b"above the fixed" in lib.dr_get_last_error()
    torch.cuda.synchronize()
