"""The oracle's cube-map extension (mip filters, per-pixel bias and the
direction gradient; the reference samples cube maps bilinearly only and
returns a zero direction gradient, Texture.swift:75-76, 196-198).  Pinned by
reduction to the reference's own paths and by finite differences.  CPU only."""
import numpy as np
import pytest

import oracle as O

TRI = "linear-mipmap-linear"


def face0_dirs(uv, uv_da):
    """Directions on face +X (x = 1) whose face (u, v) and screen
    derivatives are exactly uv and uv_da: sc = -z = 2u - 1, tc = -y = 2v - 1."""
    u, v = uv[..., 0], uv[..., 1]
    d = np.stack([np.ones_like(u), 1.0 - 2.0 * v, 1.0 - 2.0 * u], -1).astype(np.float32)
    ux, uy, vx, vy = (uv_da[..., i] for i in range(4))
    dd = np.stack([np.zeros_like(ux), np.zeros_like(ux), -2 * vx, -2 * vy, -2 * ux, -2 * uy],
                  -1).astype(np.float32)
    return d, dd


def grid_uv(rng, N, H, W):
    # multiples of 1/4096: 2u - 1 and back are exact
    return (rng.integers(40, 4056, size=(N, H, W, 2)) / 4096.0).astype(np.float32)


@pytest.mark.parametrize("filt", [TRI, "linear-mipmap-nearest"])
def test_face_reduces_to_2d_trilinear(filt):
    rng = np.random.default_rng(1)
    cube = rng.random((1, 6, 16, 16, 3)).astype(np.float32)
    uv = grid_uv(rng, 2, 5, 7)
    da = (rng.normal(size=(2, 5, 7, 4)) * rng.choice([0.002, 0.02, 0.2], (2, 5, 7, 1))
          ).astype(np.float32)
    d, dd = face0_dirs(uv, da)
    out = O.texture(cube, d, uvDA=dd, filterMode=filt, boundaryMode="cube")
    ref = O.texture(cube[:, 0], uv, uvDA=da, filterMode=filt, boundaryMode="clamp")
    np.testing.assert_array_equal(out, ref)
    g = rng.normal(size=out.shape).astype(np.float32)
    d_tex, d_dir, d_dd, _ = O.texture_vjp(cube, d, g, uvDA=dd, filterMode=filt,
                                          boundaryMode="cube", dirGrad=True)
    r_tex, r_uv, r_da, _ = O.texture_vjp(cube[:, 0], uv, g, uvDA=da, filterMode=filt,
                                         boundaryMode="clamp")
    np.testing.assert_array_equal(d_tex[:, 0], r_tex)
    assert not d_tex[:, 1:].any()
    # z = 1 - 2u, y = 1 - 2v: d/dz = -d/du / 2, d/dy = -d/dv / 2 (x also
    # carries the LOD's dependence on the direction)
    np.testing.assert_allclose(d_dir[..., 2], -0.5 * r_uv[..., 0], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(d_dir[..., 1], -0.5 * r_uv[..., 1], rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(d_dd[..., [4, 5, 2, 3]], -0.5 * r_da, rtol=1e-6, atol=1e-7)


def test_single_level_is_the_reference_cube():
    rng = np.random.default_rng(2)
    cube = rng.random((2, 6, 8, 8, 2)).astype(np.float32)
    d = rng.normal(size=(2, 6, 5, 3)).astype(np.float32)
    ref = O.texture(cube, d, boundaryMode="cube")
    g = rng.normal(size=ref.shape).astype(np.float32)
    r_tex, r_dir, _, _ = O.texture_vjp(cube, d, g, boundaryMode="cube")
    assert not r_dir.any()                       # the reference: d_dir = 0
    e_tex, e_dir, _, _ = O.texture_vjp(cube, d, g, boundaryMode="cube", dirGrad=True)
    np.testing.assert_array_equal(e_tex, r_tex)  # same d_tex, sequential order
    assert e_dir.any()
    # a 1x1-level pyramid (8x8 faces, lod forced to 0) samples like bilinear
    tiny = np.full((2, 6, 5, 6), 1e-7, np.float32)
    out = O.texture(cube, d, uvDA=tiny, filterMode=TRI, boundaryMode="cube")
    np.testing.assert_array_equal(out, ref)


def _fd(loss, x, eps=1e-3):
    g = np.zeros_like(x, dtype=np.float64)
    flat = x.reshape(-1)
    for i in range(flat.size):
        xp = flat.copy(); xp[i] += eps
        xm = flat.copy(); xm[i] -= eps
        g.reshape(-1)[i] = (loss(xp.reshape(x.shape)) - loss(xm.reshape(x.shape))) / (2 * eps)
    return g


# one direction per face, away from the face edges; footprints between levels
DIRS = np.array([[[[0.9, 0.21, -0.33], [-0.8, 0.27, 0.18], [0.23, 0.85, -0.29]],
                  [[-0.31, -0.9, 0.17], [0.26, -0.22, 0.95], [0.19, 0.31, -0.8]]]], np.float32)


@pytest.mark.parametrize("target", ["tex", "dir", "dd", "biasMap"])
def test_gradcheck(target):
    rng = np.random.default_rng(0xC0BE)
    # smooth faces so the FD step stays within one bilinear cell's curvature
    yy, xx = np.meshgrid(np.linspace(0, 1, 16), np.linspace(0, 1, 16), indexing="ij")
    base = np.stack([np.sin(3 * xx + 2 * yy), np.cos(2 * xx - yy)], -1)
    cube = np.stack([base * (1 + 0.2 * f) + 0.1 * f for f in range(6)])[None].astype(np.float32)
    dd = (rng.normal(size=(1, 2, 3, 6)) * 0.08).astype(np.float32)
    bm = np.array([[[0.2, -0.1, 0.05], [0.1, -0.25, 0.3]]], np.float32)
    w = rng.normal(size=(1, 2, 3, 2)).astype(np.float32)
    use_bm = target == "biasMap"

    def loss(t, d, e, m):
        return (O.texture(t, d, uvDA=e, filterMode=TRI, boundaryMode="cube",
                          mipLevelBiasMap=m if use_bm else None).astype(np.float64) * w).sum()

    d_tex, d_dir, d_dd, d_bm = O.texture_vjp(cube, DIRS, w, uvDA=dd, filterMode=TRI,
                                             boundaryMode="cube",
                                             mipLevelBiasMap=bm if use_bm else None,
                                             dirGrad=True)
    got, fd = {
        "tex": (d_tex, lambda: _fd(lambda x: loss(x, DIRS, dd, bm), cube)),
        "dir": (d_dir, lambda: _fd(lambda x: loss(cube, x, dd, bm), DIRS, eps=2e-4)),
        "dd": (d_dd, lambda: _fd(lambda x: loss(cube, DIRS, x, bm), dd)),
        "biasMap": (d_bm, lambda: _fd(lambda x: loss(cube, DIRS, dd, x), bm)),
    }[target]
    ref = fd()
    np.testing.assert_allclose(got, ref, atol=8e-3 * max(1.0, np.abs(ref).max()))
