"""dr_texture_bwd_noalloc, the texture backward that allocates nothing,
against dr_texture_bwd through the C ABI on the same inputs: several calls
in a row on one GPU (the fixed array keeps the previous call's contents),
the later ones smaller, 2D trilinear with and without a bias map and the
cube extension; it takes no device memory where dr_texture_bwd grows the
library's scratch; a pyramid above the fixed array (2D or cube) is
rejected before any work is queued, leaving d_tex untouched.  Per-pixel
gradients (d_uv, d_uvDA, d_biasMap) are written by the same kernels and
must be identical; d_tex within the scatter-add tolerance (atomic
order)."""
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


def _bufs(tex, uv, da, bm, g, cube):
    """Device copies of the inputs, the pyramid and the gradient outputs."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    Nt, C, S = tex.shape[0], tex.shape[-1], tex.shape[-2]
    L_levels = lib.dr_texture_mip_levels(S, S, -1, None, None)
    faces = Nt * 6 if cube else Nt
    b = dict(tex=dev(tex), uv=dev(uv), da=dev(da), g=dev(g), L=L_levels,
             bm=dev(bm) if bm is not None else None,
             pyr=torch.empty(max(lib.dr_texture_mip_size(faces, S, S, C, L_levels), 1),
                             device="cuda"),
             d_tex=torch.empty(tex.shape, device="cuda"), d_uv=torch.empty(uv.shape, device="cuda"),
             d_da=torch.empty(da.shape, device="cuda"),
             d_bm=torch.empty(bm.shape, device="cuda") if bm is not None else None)
    L.check(lib.dr_texture_build_mip(_ptr(b["tex"]), faces, S, S, C, L_levels, _ptr(b["pyr"]),
                                     _stream()))
    return b


def _call(fn_name, b, boundary, flags):
    """One call of fn_name on the buffers; the outputs are first set to 7
    (the call overwrites them: d_tex is zeroed first)."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    for k in ("d_tex", "d_uv", "d_da", "d_bm"):
        if b[k] is not None:
            b[k].fill_(7.0)
    N, Hi, Wi = b["uv"].shape[:3]
    Nt, C, S = b["tex"].shape[0], b["tex"].shape[-1], b["tex"].shape[-2]
    L.check(getattr(lib, fn_name)(
        _ptr(b["tex"]), _ptr(b["pyr"]), Nt, S, S, C, b["L"], _ptr(b["uv"]), _ptr(b["da"]),
        _ptr(b["bm"]), 0.25, LINEAR_MIPMAP_LINEAR, boundary, N, Hi, Wi, _ptr(b["g"]),
        _ptr(b["d_tex"]), _ptr(b["d_uv"]), _ptr(b["d_da"]), _ptr(b["d_bm"]), flags, _stream()))
    torch.cuda.synchronize()


def _run(fn_name, tex, uv, da, bm, g, cube, boundary, flags):
    b = _bufs(tex, uv, da, bm, g, cube)
    _call(fn_name, b, boundary, flags)
    return [host(b["d_tex"]), host(b["d_uv"]), host(b["d_da"]),
            None if b["d_bm"] is None else host(b["d_bm"])]


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


def test_texture_bwd_noalloc_takes_no_device_memory():
    """Device memory free before and after a call on buffers allocated
    beforehand: dr_texture_bwd, with the library's scratch released first,
    grows it by the pyramid gradient (levels 1.. of a 1024^2 RGBA texture,
    5.6 MB); the allocation-free entry point, after the same release,
    takes none."""
    torch = torch_dev()
    import diffrast._lib as L
    lib = L.load()
    b = _bufs(*_case(np.random.default_rng(7), 1, 1, 1024, 4, 64, 64, False, False), False)
    _call("dr_texture_bwd_noalloc", b, CLAMP, 0)  # code objects loaded
    used = {}
    for fn in ("dr_texture_bwd", "dr_texture_bwd_noalloc"):
        L.check(lib.dr_release_scratch())
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        _call(fn, b, CLAMP, 0)
        used[fn] = free0 - torch.cuda.mem_get_info()[0]
    assert used["dr_texture_bwd"] >= 4 << 20, used  # the scratch is visible here
    assert used["dr_texture_bwd_noalloc"] <= 0, used


@pytest.mark.parametrize("cube", [False, True])
def test_texture_bwd_noalloc_rejects_large_pyramid(cube):
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    # levels 1.. of a 4096^2 RGBA texture (22.4M floats), or of six 1024^2
    # five-channel faces (10.5M): above the fixed array's 8M
    S, C = (1024, 5) if cube else (4096, 4)
    faces = 6 if cube else 1
    L_levels = lib.dr_texture_mip_levels(S, S, -1, None, None)
    assert lib.dr_texture_mip_size(faces, S, S, C, L_levels) > L.DR_TEXTURE_BWD_NOALLOC_FLOATS
    shape = (1, 6, S, S, C) if cube else (1, S, S, C)
    tex = torch.zeros(shape, device="cuda")
    pyr = torch.zeros(lib.dr_texture_mip_size(faces, S, S, C, L_levels), device="cuda")
    uv = torch.zeros((1, 8, 8, 3 if cube else 2), device="cuda")
    da = torch.zeros((1, 8, 8, 6 if cube else 4), device="cuda")
    g = torch.zeros((1, 8, 8, C), device="cuda")
    d_tex = torch.full(shape, 7.0, device="cuda")
    rc = lib.dr_texture_bwd_noalloc(_ptr(tex), _ptr(pyr), 1, S, S, C, L_levels, _ptr(uv), _ptr(da),
                                    None, 0.0, LINEAR_MIPMAP_LINEAR, CUBE if cube else CLAMP, 1, 8,
                                    8, _ptr(g), _ptr(d_tex), None, None, None, 0, _stream())
    assert rc == L.DR_ERR_ARGUMENT
    assert b"above the fixed" in lib.dr_get_last_error()
    torch.cuda.synchronize()
    assert bool((d_tex == 7.0).all().item())  # nothing was queued
