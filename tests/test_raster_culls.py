"""The pixel-parallel rasterizer's conservative culls (edge_excludes,
depth_excludes in mlx-swift-diffrast_amd/csrc/raster_tests.h, the header the
kernels include) against the per-pixel test they skip (test_tri): a host
build of the same functions, fuzzed with adversarial triangles and quadrant
boxes (tests/raster_culls.cpp), must find no culled candidate that passes
the per-pixel test at a pixel centre of its box, and both culls must fire.
CPU only."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "mlx-swift-diffrast_amd", "csrc")


def test_culls_never_drop_a_covering_candidate(tmp_path):
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("needs g++")
    exe = tmp_path / "raster_culls"
    subprocess.run([cxx, "-O2", "-std=c++17", "-ffp-contract=off", "-Wall", "-Wno-unknown-pragmas",
                    "-I", CSRC, "-o", str(exe), os.path.join(HERE, "raster_culls.cpp")], check=True)
    r = subprocess.run([str(exe), "400000"], capture_output=True, text=True)
    assert r.returncode == 0, r.stdout + r.stderr
    m = re.search(r"edge: (\d+) tested, (\d+) culled \((\d+) with.*depth: (\d+) tested, (\d+) culled",
                  r.stdout)
    assert m, r.stdout
    edge_tested, edge_culled, through, depth_tested, depth_culled = map(int, m.groups())
    assert edge_culled > 0.1 * edge_tested and through > 0
    assert depth_culled > 0.05 * depth_tested
