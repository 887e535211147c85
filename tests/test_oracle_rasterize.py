"""Pins the CPU oracle's rasterize against the reference's own known answers
(Tests/MLXDiffRastTests/RasterizeTests.swift), a brute-force full-triangle
scan (no bins), finite differences, and the nvdiffrast fixture after the
convention remap of CONVENTIONS.md.  CPU only."""
import numpy as np
import pytest

import oracle as O
import scenes

FULL_TRI = np.array([[-1, 1, 0, 1], [-1, -1, 0, 1], [1, 1, 0, 1]], np.float32)[None]
TRI1 = np.array([[0, 1, 2]], np.int32)


def test_single_triangle_covers_image():
    # RasterizeTests.swift:11-51
    rast, db = O.rasterize(FULL_TRI, TRI1, (2, 2), gradDB=False)
    assert rast.shape == (1, 2, 2, 4) and db.shape == (1, 2, 2, 0)
    f = rast.reshape(-1)
    np.testing.assert_allclose(f[0:4], [0.25, 0.25, 0.0, 1.0], atol=1e-5)
    assert f[(0 * 2 + 0) * 4 + 3] == 1.0
    assert f[(0 * 2 + 1) * 4 + 3] == 1.0  # on the edge -> inside (inclusive rule)
    assert f[(1 * 2 + 0) * 4 + 3] == 1.0
    assert f[(1 * 2 + 1) * 4 + 3] == 0.0


def test_depth_test_picks_front_triangle():
    # RasterizeTests.swift:54-86
    p = np.concatenate([FULL_TRI[0].copy(), FULL_TRI[0].copy()])
    p[0:3, 2] = 0.5
    p[3:6, 2] = -0.5
    tri = np.array([[0, 1, 2], [3, 4, 5]], np.int32)
    rast, _ = O.rasterize(p[None], tri, (2, 2), gradDB=False)
    f = rast.reshape(-1, 4)
    covered = f[:, 3] != 0
    assert covered.any()
    np.testing.assert_allclose(f[covered, 2], -0.5, atol=1e-5)
    assert (f[covered, 3] == 2.0).all()


def test_pixels_outside_triangle_are_zero():
    # RasterizeTests.swift:89-107
    p = np.array([[-1, 1, 0, 1], [-0.5, 1, 0, 1], [-1, 0.5, 0, 1]], np.float32)[None]
    rast, _ = O.rasterize(p, TRI1, (4, 4), gradDB=False)
    assert (rast[0, 3, 3] == 0).all()


def test_rast_db_analytic():
    # RasterizeTests.swift:119-143: (du/dx, du/dy, dv/dx, dv/dy) = (0, .5, .5, 0)
    _, db = O.rasterize(FULL_TRI, TRI1, (2, 2))
    f = db.reshape(-1, 4)
    for pix in (0, 1, 2):
        np.testing.assert_allclose(f[pix], [0.0, 0.5, 0.5, 0.0], atol=1e-5)
    np.testing.assert_array_equal(f[3], 0)


def test_rasterize_into_interpolate_da():
    # RasterizeTests.swift:148-169
    rast, db = O.rasterize(FULL_TRI, TRI1, (2, 2))
    attr = np.array([0, 2, 4], np.float32).reshape(1, 3, 1)
    _, da = O.interpolate(attr, rast, TRI1, rastDB=db, diffAttrs="all")
    assert da.shape == (1, 2, 2, 2)
    np.testing.assert_allclose(da.reshape(-1)[:2], [2.0, 1.0], atol=1e-5)


def test_rasterize_into_interpolate_partition_of_unity():
    # RasterizeTests.swift:364-394
    rast, _ = O.rasterize(FULL_TRI, TRI1, (2, 2), gradDB=False)
    attr = np.eye(3, dtype=np.float32)[None]
    out, _ = O.interpolate(attr, rast, TRI1)
    s = out.reshape(-1, 3).sum(1)
    cov = rast.reshape(-1, 4)[:, 3] > 0
    np.testing.assert_allclose(s, np.where(cov, 1.0, 0.0), atol=1e-5)


def test_peel_layers():
    # RasterizeTests.swift:253-306
    p = np.array([[-2, 2, -0.5, 1], [-2, -2, -0.5, 1], [2, 2, -0.5, 1],
                  [-2, 2, 0.5, 1], [-2, -2, 0.5, 1], [2, 2, 0.5, 1]], np.float32)[None]
    tri = np.array([[0, 1, 2], [3, 4, 5]], np.int32)
    l0, _ = O.rasterize(p, tri, (2, 2), gradDB=False)
    c0 = l0[..., 3] > 0
    assert c0.any()
    np.testing.assert_allclose(l0[..., 2][c0], -0.5, atol=1e-5)
    assert (l0[..., 3][c0] == 1).all()
    l1, _ = O.rasterize(p, tri, (2, 2), gradDB=False, peelLayer=l0)
    c1 = l1[..., 3] > 0
    assert c1.any()
    np.testing.assert_allclose(l1[..., 2][c1], 0.5, atol=1e-5)
    assert (l1[..., 3][c1] == 2).all()
    l2, _ = O.rasterize(p, tri, (2, 2), gradDB=False, peelLayer=l1)
    assert (l2[..., 3] == 0).all()


def test_range_mode_selects_per_batch_triangles():
    # RasterizeTests.swift:312-360
    pos = np.array([[-1, 1, 0, 1], [-1, -1, 0, 1], [1, 1, 0, 1],
                    [1, 1, 0.5, 1], [-1, -1, 0.5, 1], [1, -1, 0.5, 1]], np.float32)
    tri = np.array([[0, 1, 2], [3, 4, 5]], np.int32)
    ranges = np.array([[0, 1], [1, 1]], np.int32)
    rast, _ = O.rasterize(pos, tri, (2, 2), gradDB=False, ranges=ranges)
    assert rast.shape == (2, 2, 2, 4)
    assert set(np.unique(rast[0, ..., 3])) <= {0.0, 1.0}
    assert set(np.unique(rast[1, ..., 3])) <= {0.0, 2.0}
    assert (rast[0, ..., 3] == 1).any() and (rast[1, ..., 3] == 2).any()


def _brute_force(pos, tri, H, W):
    """Every triangle against every pixel, no binning: the same per-pixel
    arithmetic as the reference body (Rasterize.swift:412-463), so any
    difference can only come from the tile-bin candidate lists."""
    f = np.float32
    N = pos.shape[0]
    out = np.zeros((N, H, W, 4), np.float32)
    for n in range(N):
        p = pos[n]
        w = p[:, 3]
        s = (p[:, :3] / w[:, None]).astype(np.float32)
        pw = np.arange(W, dtype=np.float32)
        ph = np.arange(H, dtype=np.float32)
        ndc_x = (f(2.0) * (pw + f(0.5)) / f(W) - f(1.0)).astype(np.float32)[None, :]
        ndc_y = (f(1.0) - f(2.0) * (ph + f(0.5)) / f(H)).astype(np.float32)[:, None]
        best_z = np.full((H, W), 1e30, np.float32)
        best = np.zeros((H, W, 4), np.float32)
        for t, (i0, i1, i2) in enumerate(tri):
            if w[i0] <= 0 or w[i1] <= 0 or w[i2] <= 0:
                continue
            sx0, sy0, sz0 = s[i0]
            sx1, sy1, sz1 = s[i1]
            sx2, sy2, sz2 = s[i2]
            area = f((sx1 - sx0) * (sy2 - sy0) - (sx2 - sx0) * (sy1 - sy0))
            if area == 0:
                continue
            e0 = (sx1 - ndc_x) * (sy2 - ndc_y) - (sx2 - ndc_x) * (sy1 - ndc_y)
            e1 = (sx2 - ndc_x) * (sy0 - ndc_y) - (sx0 - ndc_x) * (sy2 - ndc_y)
            e2 = (sx0 - ndc_x) * (sy1 - ndc_y) - (sx1 - ndc_x) * (sy0 - ndc_y)
            inv = f(1.0) / area
            bw, u, v = e0 * inv, e1 * inv, e2 * inv
            z = (bw * sz0 + u * sz1) + v * sz2
            ok = ((e0 * area) >= 0) & ((e1 * area) >= 0) & ((e2 * area) >= 0)
            ok &= (ndc_x >= min(sx0, sx1, sx2)) & (ndc_x <= max(sx0, sx1, sx2))
            ok &= (ndc_y >= min(sy0, sy1, sy2)) & (ndc_y <= max(sy0, sy1, sy2))
            ok &= (z >= -1) & (z <= 1) & (z < best_z)
            best_z = np.where(ok, z, best_z)
            best[..., 0] = np.where(ok, u, best[..., 0])
            best[..., 1] = np.where(ok, v, best[..., 1])
            best[..., 2] = np.where(ok, z, best[..., 2])
            best[..., 3] = np.where(ok, f(t + 1), best[..., 3])
        out[n] = best
    return out


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_binned_equals_brute_force(seed):
    rng = np.random.default_rng(100 + seed)
    T, H, W = 40, 37, 53  # ragged sizes: partial tiles on both axes
    xyz = rng.uniform(-1.3, 1.3, size=(2, 3 * T, 3)).astype(np.float32)
    w = rng.uniform(0.6, 1.6, size=(2, 3 * T, 1)).astype(np.float32)
    pos = np.concatenate([xyz * w, w], 2)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    ref = _brute_force(pos, tri, H, W)
    np.testing.assert_array_equal(rast[..., 3], ref[..., 3])
    np.testing.assert_array_equal(rast, ref)


def test_overflow_semantics():
    # Rasterize.swift:165-171: more than 128 triangles in a tile are silently
    # dropped by the reference; max_per_tile=0 keeps all of them.  Stack 200
    # full-screen triangles, the last one nearest, so the reference's
    # truncation makes a different triangle win.
    T = 200
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T, 1))
    p[:, 2] = np.repeat(np.linspace(0.9, -0.9, T), 3)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    st = {}
    r128, _ = O.rasterize(p[None], tri, (16, 16), gradDB=False, stats=st)
    rall, _ = O.rasterize(p[None], tri, (16, 16), gradDB=False, max_per_tile=0)
    assert st["max_tile_count"] == T and st["overflow_tiles"] == 1
    assert (r128[..., 3] == 128).all()
    assert (rall[..., 3] == T).all()


def _fd(loss, x, eps=1e-3):
    g = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        xp = flat.copy(); xp[i] += eps
        xm = flat.copy(); xm[i] -= eps
        g.reshape(-1)[i] = (loss(xp.reshape(x.shape)) - loss(xm.reshape(x.shape))) / (2 * eps)
    return g


@pytest.mark.parametrize("use_db", [False, True])
def test_gradcheck_rasterize(use_db):
    # RasterizeTests.swift:181-246
    N, H, W = 1, 2, 2
    pos0 = np.array([[-3, 3, 0.0, 1], [-3, -3, 0.1, 1], [3, 0, -0.1, 1]], np.float32)[None]
    i = np.arange(N * H * W * 4)
    w_r = np.where(i % 4 == 3, 0.0, (1 + i % 7) * 0.1).astype(np.float32).reshape(N, H, W, 4)
    w_db = ((2 + i % 5) * 0.05 if use_db else 0 * i).astype(np.float32).reshape(N, H, W, 4)

    def loss(p):
        r, db = O.rasterize(p, TRI1, (H, W), gradDB=use_db)
        val = (r.astype(np.float64) * w_r).sum()
        if use_db:
            val += (db.astype(np.float64) * w_db).sum()
        return val

    rast, _ = O.rasterize(pos0, TRI1, (H, W), gradDB=use_db)
    g = O.rasterize_vjp(pos0, TRI1, rast, w_r, w_db if use_db else None)
    np.testing.assert_allclose(g, _fd(loss, pos0), atol=5e-3)


def test_nvdiffrast_fixture_after_remap(fixtures):
    """CONVENTIONS.md:17-72: flip image y, map nvdiffrast (u,v)=(w0,w1) to
    this library's (u,v)=(w1,w2).  All vertices have w=1, so nvdiffrast's
    perspective-correct barycentrics equal the screen-space ones; pixels
    that both libraries cover must agree.  Edge pixels may differ because
    nvdiffrast's fill rule is not inclusive."""
    pos = np.array([[-0.7, 0.8, 0.0, 1.0], [0.8, 0.7, 0.1, 1.0], [0.7, -0.8, 0.2, 1.0],
                    [-0.8, -0.7, 0.0, 1.0]], np.float32)[None]
    tri = np.array([[0, 1, 2], [0, 2, 3]], np.int32)
    rast, db = O.rasterize(pos, tri, (16, 16))
    nv = fixtures["rast"][:, ::-1]
    nvdb = fixtures["rast_db"][:, ::-1]
    both = (rast[..., 3] > 0) & (nv[..., 3] > 0)
    same = both & (rast[..., 3] == nv[..., 3])
    assert same.sum() >= 0.97 * max(both.sum(), 1)
    assert (rast[..., 3] > 0).sum() >= 0.97 * (nv[..., 3] > 0).sum()
    my_u = nv[..., 1]
    my_v = 1.0 - nv[..., 0] - nv[..., 1]
    np.testing.assert_allclose(rast[..., 0][same], my_u[same], atol=2e-5)
    np.testing.assert_allclose(rast[..., 1][same], my_v[same], atol=2e-5)
    np.testing.assert_allclose(rast[..., 2][same], nv[..., 2][same], atol=2e-5)
    # rast_db: my u = nv.v, my v = 1 - nv.u - nv.v; the y flip negates d/dy.
    exp = np.stack([nvdb[..., 2], -nvdb[..., 3],
                    -(nvdb[..., 0] + nvdb[..., 2]), (nvdb[..., 1] + nvdb[..., 3])], -1)
    np.testing.assert_allclose(db[same], exp[same], atol=2e-5)


def test_icosphere_tile_occupancy():
    """At the textured-icosphere workload (level-6 sphere, 1024^2) the
    silhouette tiles hold up to ~200 candidate triangles, above the
    reference's 128-entry bins (Rasterize.swift:165-171).  The reference then
    drops triangles in atomic (nondeterministic) order; this build keeps all
    of them.  The parity tests therefore compare against the oracle with
    max_per_tile=0, and this test records how much the truncation changes."""
    sc = scenes.textured_icosphere(N=1)
    st = {}
    r128, _ = O.rasterize(sc["pos"], sc["tri"], (1024, 1024), gradDB=False, stats=st)
    rall, _ = O.rasterize(sc["pos"], sc["tri"], (1024, 1024), gradDB=False, max_per_tile=0)
    assert st["overflow_tiles"] > 0 and st["max_tile_count"] > 128
    changed = (r128[..., 3] != rall[..., 3]).sum()
    covered = (rall[..., 3] > 0).sum()
    assert 0 < changed < 0.02 * covered


def test_tile_counts_closed_form():
    # one triangle over the top-left quadrant of a 64x64 image: pixel AABB
    # x, y in [0, 31] (px = (ndc+1)*W/2 - 0.5), i.e. tiles (0..1, 0..1);
    # a second one behind the camera (w < 0) and a degenerate one add nothing
    pos = np.array([[-1, 1, 0, 1], [-1, 0, 0, 1], [0, 1, 0, 1],
                    [-1, 1, 0, -1], [1, 1, 0, -1], [0, 0, 0, -1],
                    [0, 0, 0, 1], [0.5, 0.5, 0, 1], [1, 1, 0, 1]], np.float32)[None]
    tri = np.arange(9, dtype=np.int32).reshape(3, 3)
    c = O.rasterize_tile_counts(pos, tri, (64, 64))
    want = np.zeros((1, 4, 4), np.int32)
    want[0, :2, :2] = 1
    np.testing.assert_array_equal(c, want)
    # counts agree with the forward's bin statistics
    st = {}
    O.rasterize(pos, tri, (64, 64), stats=st)
    assert st["max_tile_count"] == c.max() and st["pairs"] == c.sum()
