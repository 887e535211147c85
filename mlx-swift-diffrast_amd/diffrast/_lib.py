"""ctypes binding of libdiffrast_mi355x.so (the C ABI in include/diffrast_mi355x.h).

There is no fallback: if the library is missing or cannot be loaded, every
op raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libdiffrast_mi355x.so")

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_u = ctypes.c_uint
_f = ctypes.c_float

# Every exported function and its argument types, in header order.
SIGNATURES = {
    "dr_abi_version": ([], _i),
    "dr_get_last_error": ([], ctypes.c_char_p),
    "dr_release_scratch": ([], _i),
    "dr_profile_enable": ([_i], _i),
    "dr_profile_select": ([ctypes.c_char_p], _i),
    "dr_profile_reset": ([], _i),
    "dr_profile_report": ([ctypes.c_char_p, _i], _i),
    "dr_rasterize_fwd": ([_p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p, _p], _i),
    "dr_rasterize_fwd_ex": ([_p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p, _i, _p], _i),
    "dr_rasterize_fwd_again": ([_p, _i64, _p, _p, _p, _i, _i, _i, _i, _i, _p, _p, _i, _p], _i),
    "dr_rasterize_tile_counts": ([_p, _i64, _p, _p, _i, _i, _i, _i, _i, _p, _p, _p], _i),
    "dr_rasterize_reserve": ([_i, _i, _i, _i, _i, _i, _p], _i),
    "dr_rasterize_bwd": ([_p, _i64, _p, _p, _p, _p, _i, _i, _i, _i, _i, _p, _u, _p], _i),
    "dr_interpolate_fwd": ([_p, _i64, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _i, _p, _p, _p],
                           _i),
    "dr_interpolate_bwd": ([_p, _i64, _p, _p, _p, _p, _i, _p, _p, _i, _i, _i, _i, _i, _i, _p, _i64,
                            _p, _p, _u, _p], _i),
    "dr_texture_mip_levels": ([_i, _i, _i, _p, _p], _i),
    "dr_texture_mip_size": ([_i, _i, _i, _i, _i], _i64),
    "dr_texture_build_mip": ([_p, _i, _i, _i, _i, _i, _p, _p], _i),
    "dr_texture_fwd": ([_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _f, _i, _i, _i, _i, _i, _p, _p],
                       _i),
    "dr_texture_bwd": ([_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _f, _i, _i, _i, _i, _i, _p, _p,
                        _p, _p, _p, _u, _p], _i),
    "dr_texture_bwd_noalloc": ([_p, _p, _i, _i, _i, _i, _i, _p, _p, _p, _f, _i, _i, _i, _i, _i,
                                _p, _p, _p, _p, _p, _u, _p], _i),
    "dr_antialias_topology": ([_p, _i, _p, _p], _i),
    "dr_antialias_fwd": ([_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p], _i),
    "dr_antialias_bwd": ([_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _u, _p], _i),
    "dr_antialias_saved_bytes": ([_i, _i, _i, _i], _i64),
    "dr_antialias_fwd_save": ([_p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _p], _i),
    "dr_antialias_bwd_saved": ([_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _i, _i, _p, _p, _u,
                                _p], _i),
    "dr_mse_loss": ([_p, _p, _i64, _p, _p, _p], _i),
    "dr_adam_step": ([_p, _p, _p, _p, _p, _p, _i64, _i, _f, _f, _f, _f, _p], _i),
}

DR_OK, DR_ERR_ARGUMENT, DR_ERR_HIP, DR_ERR_MEMORY, DR_ERR_CAPTURE = 0, 1, 2, 3, 4
DR_ACCUMULATE = 1
DR_CUBE_DIR_GRAD = 2
DR_RASTERIZE_BWD_REUSE = 4
DR_TEXTURE_BWD_NOALLOC_FLOATS = 8 * 1024 * 1024
ABI_VERSION = 1

_lib = None


def load():
    """Loads the library once; raises if it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"diffrast: {LIB_PATH} is not built (run `make -C mlx-swift-diffrast_amd`)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if lib.dr_abi_version() != ABI_VERSION:
        raise RuntimeError("diffrast: ABI version mismatch")
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc == DR_OK:
        return
    msg = (_lib.dr_get_last_error() or b"").decode(errors="replace")
    if rc == DR_ERR_ARGUMENT:
        raise ValueError(msg)
    raise RuntimeError(f"diffrast error {rc}: {msg}")


def profile_report():
    """{kernel: {"count": launches, "total_ms": ms}} of the launches timed
    since dr_profile_reset while dr_profile_enable(1) was on."""
    lib = load()
    n = lib.dr_profile_report(None, 0)
    if n < 0:
        raise RuntimeError("dr_profile_report failed")
    buf = ctypes.create_string_buffer(n + 1)
    lib.dr_profile_report(buf, n + 1)
    out = {}
    for line in buf.value.decode().splitlines():
        name, cnt, ms = line.split()
        out[name] = {"count": int(cnt), "total_ms": float(ms)}
    return out
