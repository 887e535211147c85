"""Pins the CPU oracle's antialias against the reference's known answers
(Tests/MLXDiffRastTests/AntialiasTests.swift), an O(T^2) topology brute
force with its symmetry invariant, and finite differences.  CPU only."""
import numpy as np
import pytest

import oracle as O
import scenes

TRI1 = np.array([[0, 1, 2]], np.int32)


def test_topology_shared_edge():
    # AntialiasTests.swift:11-36
    h = O.antialiasConstructTopologyHash(np.array([[0, 1, 2], [1, 2, 3]], np.int32))
    np.testing.assert_array_equal(h, [[1, -1, -1], [-1, -1, 0]])


def test_topology_single_triangle():
    # AntialiasTests.swift:38-42
    np.testing.assert_array_equal(O.antialiasConstructTopologyHash(TRI1), [[-1, -1, -1]])


def test_topology_non_manifold():
    # AntialiasTests.swift:47-71
    h = O.antialiasConstructTopologyHash(np.array([[0, 1, 2], [0, 1, 3], [0, 1, 4]], np.int32))
    np.testing.assert_array_equal(h[:, 2], -2)
    np.testing.assert_array_equal(h[:, :2], -1)


def brute_topology(tri):
    """O(T^2) edge matching: edge k of t is the one opposite vertex k."""
    T = tri.shape[0]
    keys = {}
    for t in range(T):
        v = tri[t]
        for k, (a, b) in enumerate(((v[1], v[2]), (v[2], v[0]), (v[0], v[1]))):
            keys.setdefault((min(a, b), max(a, b)), []).append((t, k))
    out = np.full((T, 3), -1, np.int32)
    for users in keys.values():
        if len(users) == 2:
            (t0, k0), (t1, k1) = users
            out[t0, k0], out[t1, k1] = t1, t0
        elif len(users) > 2:
            for t, k in users:
                out[t, k] = -2
    return out


@pytest.mark.parametrize("case", ["icosphere", "random", "fan"])
def test_topology_brute_force_and_symmetry(case):
    rng = np.random.default_rng(5)
    if case == "icosphere":
        _, tri = scenes.icosphere(3)
    elif case == "random":
        tri = rng.integers(0, 30, size=(200, 3)).astype(np.int32)
    else:
        tri = np.array([[0, i, i + 1] for i in range(1, 9)] + [[0, 9, 1], [0, 1, 2]], np.int32)
    h = O.antialiasConstructTopologyHash(tri)
    np.testing.assert_array_equal(h, brute_topology(tri))
    for t in range(tri.shape[0]):
        for k in range(3):
            s = h[t, k]
            if s >= 0:
                assert t in h[s]
    if case == "icosphere":
        assert (h >= 0).all()  # closed manifold: every edge has one neighbour


def test_no_silhouette_is_identity():
    # AntialiasTests.swift:78-87
    color = np.arange(18, dtype=np.float32).reshape(1, 3, 3, 2)
    out = O.antialias(color, np.zeros((1, 3, 3, 4), np.float32), np.zeros((1, 3, 4), np.float32),
                      TRI1)
    np.testing.assert_array_equal(out, color)


FULL = np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32)[None]
TILT = np.array([[-3, 3, 0, 1], [-3, -2.7, 0, 1], [2.7, 3, 0, 1]], np.float32)[None]


def test_fully_covered_is_identity():
    # AntialiasTests.swift:91-107
    color = np.array([1, 2, 3, 4], np.float32).reshape(1, 2, 2, 1)
    rast, _ = O.rasterize(FULL, TRI1, (2, 2), gradDB=False)
    np.testing.assert_array_equal(O.antialias(color, rast, FULL, TRI1), color)


def test_silhouette_blends():
    # AntialiasTests.swift:112-173
    H = W = 4
    rast, _ = O.rasterize(TILT, TRI1, (H, W), gradDB=False)
    color = (10 * (1 + np.arange(16))).astype(np.float32).reshape(1, H, W, 1)
    out = O.antialias(color, rast, TILT, TRI1)
    cov = rast[0, ..., 3] > 0
    found = False
    for h in range(H):
        for w in range(W):
            nb = [(h, w + 1), (h + 1, w), (h, w - 1), (h - 1, w)]
            mixed = any(0 <= a < H and 0 <= b < W and cov[a, b] != cov[h, w] for a, b in nb)
            if mixed and abs(out[0, h, w, 0] - color[0, h, w, 0]) > 1e-4:
                found = True
    assert found
    for h in range(1, H - 1):
        for w in range(1, W - 1):
            blk = rast[0, h - 1:h + 2, w - 1:w + 2, 3]
            if (blk == rast[0, h, w, 3]).all():
                assert abs(out[0, h, w, 0] - color[0, h, w, 0]) < 1e-5


def _fd(loss, x, eps=1e-3):
    g = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        xp = flat.copy(); xp[i] += eps
        xm = flat.copy(); xm[i] -= eps
        g.reshape(-1)[i] = (loss(xp.reshape(x.shape)) - loss(xm.reshape(x.shape))) / (2 * eps)
    return g


def test_gradcheck_color():
    # AntialiasTests.swift:176-213
    H = W = 4
    C = 2
    rast, _ = O.rasterize(TILT, TRI1, (H, W), gradDB=False)
    topo = O.antialiasConstructTopologyHash(TRI1)
    color = (np.arange(32, dtype=np.float32) * 0.3 + 1).reshape(1, H, W, C)
    w = ((1 + np.arange(32) % 7) * 0.1).astype(np.float32).reshape(1, H, W, C)
    loss = lambda c: (O.antialias(c, rast, TILT, TRI1, topo).astype(np.float64) * w).sum()
    d_color, _ = O.antialias_vjp(color, rast, TILT, TRI1, w, topo)
    np.testing.assert_allclose(d_color, _fd(loss, color), atol=5e-3)


QUAD = np.array([[-0.45, 0.55, 0, 1], [0.55, 0.55, 0, 1], [0.55, -0.45, 0, 1],
                 [-0.45, -0.45, 0, 1]], np.float32)[None]
QTRI = np.array([[0, 1, 2], [0, 2, 3]], np.int32)


def test_gradcheck_pos():
    # AntialiasTests.swift:238-279
    H = W = 4
    C = 2
    topo = O.antialiasConstructTopologyHash(QTRI)
    rast, _ = O.rasterize(QUAD, QTRI, (H, W), gradDB=False)
    color = (np.arange(32, dtype=np.float32) * 0.3 + 1).reshape(1, H, W, C)
    w = ((1 + np.arange(32) % 5) * 0.1).astype(np.float32).reshape(1, H, W, C)
    loss = lambda p: (O.antialias(color, rast, p, QTRI, topo).astype(np.float64) * w).sum()
    _, d_pos = O.antialias_vjp(color, rast, QUAD, QTRI, w, topo)
    np.testing.assert_allclose(d_pos, _fd(loss, QUAD), atol=5e-3)
    np.testing.assert_array_equal(d_pos[..., 2], 0)  # no z term
    assert np.abs(d_pos).max() > 1e-5  # AntialiasTests.swift:283-297


def test_alpha_range():
    """Every blend weight lies in (0, 0.5] (the smaller of two cuts)."""
    sc = scenes.hex_pie(N=1, H=64, W=64)
    rast, _ = O.rasterize(sc["pos"], sc["tri"], (64, 64), gradDB=False)
    color = np.zeros((1, 64, 64, 1), np.float32)
    # out - color = sum_dir alpha * (cn - cp): probe each alpha with a
    # colour that is 1 on one neighbour only.
    color[0, ::2, ::2, 0] = 1.0
    out = O.antialias(color, rast, sc["pos"], sc["tri"])
    delta = np.abs(out - color)
    assert delta.max() <= 2.0 + 1e-6
    assert (delta > 0).any()


def test_straight_edge_blend_weights():
    """The blend weight by value (Antialias.swift:274-309): a straight
    silhouette edge crossing every pixel row (images 0, 1) or column
    (images 2, 3) at a known sub-pixel position x_e blends exactly the pixel
    q = floor(x_e) holding the crossing, by beta = 0.5 - |x_e - (q + 0.5)|,
    towards its neighbour across the edge; no other pixel changes.  Every
    quantity is exact in fp32, so the oracle must equal the closed form
    bit for bit (a half-pixel shift of the endpoints, a blend of the other
    pixel of the pair or a cut measured from the wrong side all fail)."""
    H = W = 64
    sc = scenes.straight_edges(H, W)
    pos, tri, beta = sc["pos"], sc["tri"], sc["beta"]
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False)
    cov = (rast[..., 3] > 0).astype(np.float32)
    np.testing.assert_array_equal(cov, sc["cov"])
    color = np.stack([cov, 1.0 - cov], -1)  # one-hot coverage
    out = O.antialias(color, rast, pos, tri)
    np.testing.assert_array_equal(out, straight_edge_expect(color, cov, beta))
    assert (beta > 0).sum() == 4 * 64 and np.unique(beta[beta > 0]).size == 6


def straight_edge_expect(color, cov, beta):
    """The closed form: the blended pixel moves towards the other side of
    the edge by beta (the colour is one-hot coverage)."""
    sign = np.where(cov > 0, -1.0, 1.0)
    return (color + (sign * beta)[..., None] * np.array([1.0, -1.0])).astype(np.float32)
