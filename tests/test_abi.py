"""The C-ABI library loads on a machine without a GPU and exports every
function include/diffrast_mi355x.h declares; host-only entry points work and
argument errors come back as codes, not crashes.  CPU only."""
import ctypes
import os
import re

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "diffrast_mi355x.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(dr_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_entry_points():
    names = declared_functions()
    for n in ("dr_rasterize_fwd", "dr_rasterize_bwd", "dr_interpolate_fwd", "dr_interpolate_bwd",
              "dr_texture_fwd", "dr_texture_bwd", "dr_texture_build_mip", "dr_antialias_fwd",
              "dr_antialias_bwd", "dr_antialias_topology"):
        assert n in names


def test_library_exports_every_declared_symbol():
    import diffrast._lib as L
    assert os.path.exists(L.LIB_PATH), "build the library first (make -C mlx-swift-diffrast_amd)"
    lib = ctypes.CDLL(L.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # the Python binding declares exactly the header's functions
    assert sorted(L.SIGNATURES) == declared_functions()


def test_host_entry_points():
    import diffrast._lib as L
    lib = L.load()
    assert lib.dr_abi_version() == 1
    lh = (ctypes.c_int32 * 32)()
    lw = (ctypes.c_int32 * 32)()
    # Texture.swift:153-159: 1024^2 -> 11 levels; odd sizes stop; maxLevel caps
    assert lib.dr_texture_mip_levels(1024, 1024, -1, lh, lw) == 11
    assert (lh[10], lw[10]) == (1, 1)
    assert lib.dr_texture_mip_levels(12, 8, -1, lh, lw) == 3
    assert [lh[i] for i in range(3)] == [12, 6, 3]
    assert lib.dr_texture_mip_levels(8, 8, 2, lh, lw) == 3
    assert lib.dr_texture_mip_size(1, 4, 4, 1, 3) == 4 + 1
    assert lib.dr_texture_mip_size(2, 8, 8, 3, 4) == 2 * 3 * (16 + 4 + 1)


def test_argument_errors_are_codes():
    import diffrast._lib as L
    lib = L.load()
    # null tensors are rejected before any HIP call
    rc = lib.dr_rasterize_fwd(None, 0, None, None, None, 1, 3, 1, 4, 4, None, None, None)
    assert rc == L.DR_ERR_ARGUMENT
    assert b"rasterize" in lib.dr_get_last_error()
    rc = lib.dr_interpolate_fwd(None, 0, None, None, None, None, 0, 1, 2, 2, 3, 1, 2, None, None,
                                None)
    assert rc == L.DR_ERR_ARGUMENT
    with pytest.raises(ValueError):
        L.check(rc)
