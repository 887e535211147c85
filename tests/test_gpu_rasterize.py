"""rasterize on the GPU (through the C ABI) against the CPU oracle: tri_id,
coverage, barycentrics, z and rast_db bit-exact; d_pos within the
scatter-add tolerance.  Cases: the reference's known answers, random and
ragged scenes, the workload scenes, range mode, depth peeling, a tile whose
list exceeds the reference's 128 entries."""
import numpy as np
import pytest

import oracle as O
import scenes
from parity import assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu


def run(pos, tri, H, W, gradDB=True, ranges=None, peel=None):
    torch = torch_dev()
    from diffrast import DiffRast
    p = dev(pos).requires_grad_(True)
    r, db = DiffRast.rasterize(p, dev(tri), (H, W), gradDB=gradDB,
                               ranges=None if ranges is None else torch.as_tensor(ranges),
                               peelLayer=None if peel is None else dev(peel))
    return p, r, db


def check_fwd(pos, tri, H, W, gradDB=True, ranges=None, peel=None):
    _, r, db = run(pos, tri, H, W, gradDB, ranges, peel)
    rr, rdb = O.rasterize(pos, tri, (H, W), gradDB=gradDB, ranges=ranges, peelLayer=peel,
                          max_per_tile=0)
    r = host(r)
    np.testing.assert_array_equal(r[..., 3], rr[..., 3])   # tri_id + coverage
    np.testing.assert_array_equal(r, rr)                   # u, v, z bit-exact
    if gradDB:
        np.testing.assert_array_equal(host(db), rdb)
    else:
        assert tuple(db.shape) == r.shape[:3] + (0,)
    return r


def test_known_answers():
    pos = np.array([[-1, 1, 0, 1], [-1, -1, 0, 1], [1, 1, 0, 1]], np.float32)[None]
    tri = np.array([[0, 1, 2]], np.int32)
    r = check_fwd(pos, tri, 2, 2)
    np.testing.assert_allclose(r.reshape(-1)[:4], [0.25, 0.25, 0, 1], atol=1e-6)
    assert r[0, 1, 1, 3] == 0 and r[0, 0, 1, 3] == 1


@pytest.mark.parametrize("seed,H,W", [(0, 37, 53), (1, 64, 64), (2, 100, 17), (3, 1, 300)])
def test_random_triangles(seed, H, W):
    rng = np.random.default_rng(seed)
    T = 300
    xyz = rng.uniform(-1.3, 1.3, size=(3, 3 * T, 3)).astype(np.float32)
    w = rng.uniform(0.4, 1.6, size=(3, 3 * T, 1)).astype(np.float32)
    w[0, :5] = -0.5  # some triangles behind the camera
    pos = np.concatenate([xyz * w, w], 2)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    check_fwd(pos, tri, H, W, gradDB=True)
    check_fwd(pos, tri, H, W, gradDB=False)


def test_equal_depth_ties_pick_lowest_index():
    # 40 identical full-screen triangles: every pixel must report triangle 0
    # (the reference keeps the first of its bin order; this build defines
    # it as the lowest index).
    base = np.array([[-3, 3, 0.2, 1], [-3, -3, 0.2, 1], [3, 0, 0.2, 1]], np.float32)
    pos = np.tile(base, (40, 1))[None]
    tri = np.arange(120, dtype=np.int32).reshape(40, 3)
    r = check_fwd(pos, tri, 20, 20)
    assert (r[..., 3] == 1).all()


def test_deep_tile_beyond_128():
    T = 300
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T, 1))
    p[:, 2] = np.repeat(np.linspace(0.9, -0.9, T), 3)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    r = check_fwd(p[None], tri, 16, 16)
    assert (r[..., 3] == T).all()


def tile_counts(pos, tri, H, W, ranges=None):
    torch = torch_dev()
    from diffrast import DiffRast
    got = host(DiffRast.rasterizeTileCounts(
        dev(pos), dev(tri), (H, W), ranges=None if ranges is None else torch.as_tensor(ranges)))
    ref = O.rasterize_tile_counts(pos, tri, (H, W), ranges=ranges)
    np.testing.assert_array_equal(got, ref)
    return got


def test_tile_counts():
    # the reference's bins[tile, 0], bit-exact: random (some behind the
    # camera, some degenerate), a tile past the reference's 128, range mode
    rng = np.random.default_rng(7)
    T = 400
    xyz = rng.uniform(-1.3, 1.3, size=(2, 3 * T, 3)).astype(np.float32)
    w = rng.uniform(0.4, 1.6, size=(2, 3 * T, 1)).astype(np.float32)
    w[0, :5] = -0.5
    xyz[1, 30:33] = xyz[1, 30]       # zero area
    pos = np.concatenate([xyz * w, w], 2)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    c = tile_counts(pos, tri, 61, 45)
    assert c.shape == (2, 4, 3)
    T2 = 300
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T2, 1))
    tri2 = np.arange(3 * T2, dtype=np.int32).reshape(T2, 3)
    c = tile_counts(p[None], tri2, 40, 40)
    assert (c == T2).all() and c.max() > 128      # every tile past the reference's limit
    sc = scenes.range_batch(N=24, T_per=40)
    tile_counts(sc["pos"], sc["tri"], 48, 40, ranges=sc["ranges"])
    tile_counts(sc["pos"], sc["tri"], 33, 35,
                ranges=np.array([[0, 80], [30, 20], [900, 5000], [5, 0]], np.int32))
    from diffrast import _lib
    lib = _lib.load()
    import ctypes
    torch = torch_dev()
    pd, td = dev(p[None]), dev(tri2)
    out = torch.empty((1, 3, 3), dtype=torch.int32, device="cuda")
    mx = ctypes.c_int64(-1)
    _lib.check(lib.dr_rasterize_tile_counts(pd.data_ptr(), 3 * T2 * 4, td.data_ptr(), None, 1,
                                            3 * T2, T2, 40, 40, out.data_ptr(), ctypes.byref(mx),
                                            torch.cuda.current_stream().cuda_stream))
    assert mx.value == T2


def test_range_mode():
    sc = scenes.range_batch(N=24, T_per=40)
    r = check_fwd(sc["pos"], sc["tri"], 48, 40, ranges=sc["ranges"])
    t = r[..., 3].reshape(24, -1)
    for n in range(24):
        ids = np.unique(t[n][t[n] > 0]) - 1
        assert ((ids >= n * 40) & (ids < n * 40 + 40)).all()
    # ranges that overlap, run past T or are empty
    ranges = np.array([[0, 80], [30, 20], [900, 5000], [5, 0]], np.int32)
    check_fwd(sc["pos"], sc["tri"], 33, 35, ranges=ranges)


@pytest.mark.parametrize("gradDB", [False, True])
def test_peel_layers(gradDB):
    """Three depth-peeling layers, with and without rast_db (the reference's
    default is gradDB = true, Rasterize.swift:48), forward bit-exact and each
    layer's d_pos against the oracle."""
    torch = torch_dev()
    sc = scenes.textured_icosphere(N=2, H=96, W=96, level=3, tex_size=8)
    pos, tri = sc["pos"], sc["tri"]
    rng = np.random.default_rng(21)
    prev = None
    for layer in range(3):
        cur = check_fwd(pos, tri, 96, 96, gradDB=gradDB, peel=prev)
        # a closed sphere has two layers (front and back); the third is empty
        assert (cur[..., 3] > 0).any() == (layer < 2), layer
        p, r, db = run(pos, tri, 96, 96, gradDB, peel=prev)
        g = rng.normal(size=tuple(r.shape)).astype(np.float32)
        gdb = rng.normal(size=tuple(r.shape)).astype(np.float32) if gradDB else None
        loss = (r * dev(g)).sum()
        if gradDB:
            loss = loss + (db * dev(gdb)).sum()
        loss.backward()
        ref = O.rasterize_vjp(pos, tri, cur, g, gdb)
        assert_grad_close(host(p.grad), ref, f"d_pos layer {layer}")
        prev = cur


@pytest.mark.parametrize("name", ["tier1", "hexpie", "icosphere"])
def test_workload_scenes(name):
    if name == "tier1":
        sc = scenes.tier1_triangle(H=256, W=256)
        check_fwd(sc["pos"], sc["tri"], 256, 256, gradDB=False)
    elif name == "hexpie":
        sc = scenes.hex_pie(N=4, H=512, W=512)
        check_fwd(sc["pos"], sc["tri"], 512, 512, gradDB=False)
    else:
        sc = scenes.textured_icosphere(N=2, H=1024, W=1024, tex_size=8)
        check_fwd(sc["pos"], sc["tri"], 1024, 1024, gradDB=True)


@pytest.mark.parametrize("gradDB", [False, True])
@pytest.mark.parametrize("name", ["random", "hexpie", "icosphere", "range"])
def test_backward(name, gradDB):
    torch = torch_dev()
    rng = np.random.default_rng(11)
    ranges = None
    if name == "random":
        T = 200
        xyz = rng.uniform(-1.2, 1.2, size=(2, 3 * T, 3)).astype(np.float32)
        w = rng.uniform(0.5, 1.5, size=(2, 3 * T, 1)).astype(np.float32)
        pos = np.concatenate([xyz * w, w], 2)
        tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
        H, W = 45, 61
    elif name == "hexpie":
        sc = scenes.hex_pie(N=2, H=256, W=256)
        pos, tri, H, W = sc["pos"], sc["tri"], 256, 256
    elif name == "icosphere":
        sc = scenes.textured_icosphere(N=1, H=512, W=512, level=5, tex_size=8)
        pos, tri, H, W = sc["pos"], sc["tri"], 512, 512
    else:
        sc = scenes.range_batch(N=6, T_per=30)
        pos, tri, ranges, H, W = sc["pos"], sc["tri"], sc["ranges"], 40, 40
    p, r, db = run(pos, tri, H, W, gradDB, ranges)
    g = rng.normal(size=tuple(r.shape)).astype(np.float32)
    gdb = rng.normal(size=tuple(r.shape)).astype(np.float32) if gradDB else None
    loss = (r * dev(g)).sum()
    if gradDB:
        loss = loss + (db * dev(gdb)).sum()
    loss.backward()
    rr = host(r)
    ref = O.rasterize_vjp(pos, tri, rr, g, gdb, ranges=ranges)
    assert_grad_close(host(p.grad), ref, f"d_pos {name}")


def test_tile_capacity_overflow():
    """Per-tile list capacity comes from the largest count seen so far: a
    fresh scratch sized on a sparse scene, then a tile with 300 candidates,
    must take the full-scan path and still match; later calls (capacity
    raised from the read-back count) match too."""
    torch = torch_dev()
    from diffrast import _lib
    torch.cuda.synchronize()
    assert _lib.load().dr_release_scratch() == 0
    sc = scenes.tier1_triangle(H=32, W=32)
    check_fwd(sc["pos"], sc["tri"], 32, 32)
    T = 300
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T, 1))
    p[:, 2] = np.repeat(np.linspace(0.9, -0.9, T), 3)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    for _ in range(3):
        r = check_fwd(p[None], tri, 32, 32)
        assert (r[..., 3] == T).all()
        torch.cuda.synchronize()


def test_backward_ignores_foreign_triangle_ids():
    """A rast whose triangle ids lie outside [0, T) (not one this mesh's
    forward wrote) adds nothing at those pixels and reads nothing out of
    bounds: d_pos equals that of the same rast with those pixels empty."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    rng = np.random.default_rng(17)
    sc = scenes.hex_pie(N=2, H=64, W=64)
    pos, tri, H, W = sc["pos"], sc["tri"], 64, 64
    rast, _ = O.rasterize(pos, tri, (H, W), gradDB=False, max_per_tile=0)
    N, V, T = pos.shape[0], pos.shape[1], tri.shape[0]
    bad = rng.random((N, H, W)) < 0.3
    foreign = rast.copy()
    foreign[..., 3][bad] = T + 1 + rng.integers(0, 1 << 20, size=int(bad.sum()))
    emptied = rast.copy()
    emptied[bad] = 0.0
    # every device buffer stays referenced until the results are read back
    pd, td = dev(pos), dev(tri)
    g = dev(rng.normal(size=rast.shape).astype(np.float32))
    out = []
    for r in (foreign, emptied):
        rd = dev(r)
        d_pos = torch.empty((N, V, 4), device="cuda")
        L.check(lib.dr_rasterize_bwd(_ptr(pd), V * 4, _ptr(td), _ptr(rd), _ptr(g), None, N, V, T,
                                     H, W, _ptr(d_pos), 0, _stream()))
        out.append(host(d_pos))
    # same terms; only the order of the cross-tile fp32 atomics may differ
    assert_grad_close(out[0], out[1], "d_pos with foreign ids")


def test_many_tiles_binning_path():
    """An image of more than 16,384 tiles (16 x 262,160 pixels, 16,385
    tiles) takes the binning without LDS counters; the result is the same
    as the oracle's, including the tile counts."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast import DiffRast
    rng = np.random.default_rng(23)
    H, W, T = 16, 16 * 16385, 400
    xyz = rng.uniform(-1.1, 1.1, size=(1, 3 * T, 3)).astype(np.float32)
    xyz[..., 0] = np.repeat(rng.uniform(-1.0, 1.0, size=(1, T)), 3, axis=1) + \
        rng.uniform(-2e-3, 2e-3, size=(1, 3 * T))  # narrow triangles across the width
    pos = np.concatenate([xyz, np.ones((1, 3 * T, 1), np.float32)], 2).astype(np.float32)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    check_fwd(pos, tri, H, W, gradDB=True)
    counts = host(DiffRast.rasterizeTileCounts(dev(pos), dev(tri), (H, W)))
    np.testing.assert_array_equal(counts, O.rasterize_tile_counts(pos, tri, (H, W)))


def check_capped(pos, tri, H, W, cap, gradDB=True, ranges=None, peel=None):
    """maxPerTile = cap against the oracle's max_per_tile = cap (the
    reference's truncation with its appends in triangle order)."""
    torch = torch_dev()
    from diffrast import DiffRast
    r, db = DiffRast.rasterize(dev(pos), dev(tri), (H, W), gradDB=gradDB,
                               ranges=None if ranges is None else torch.as_tensor(ranges),
                               peelLayer=None if peel is None else dev(peel), maxPerTile=cap)
    rr, rdb = O.rasterize(pos, tri, (H, W), gradDB=gradDB, ranges=ranges, peelLayer=peel,
                          max_per_tile=cap)
    r = host(r)
    np.testing.assert_array_equal(r, rr)
    if gradDB:
        np.testing.assert_array_equal(host(db), rdb)
    return r


def test_capped_tile_overflow():
    """300 full-screen triangles per tile, nearest last: with a per-tile cap
    every pixel shows the cap's last triangle.  The first call after a
    sparse scene has list capacity below 300 (ordered full scan stopping at
    the cap); later calls sort the complete list in LDS or, above 1,024
    ids, take the same ordered scan."""
    torch = torch_dev()
    from diffrast import _lib
    torch.cuda.synchronize()
    assert _lib.load().dr_release_scratch() == 0
    sc = scenes.tier1_triangle(H=32, W=32)
    check_fwd(sc["pos"], sc["tri"], 32, 32)
    T = 300
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T, 1))
    p[:, 2] = np.repeat(np.linspace(0.9, -0.9, T), 3)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    for cap in (128, 128, 5, 1, 299, 300, 1024):
        r = check_capped(p[None], tri, 32, 32, cap)
        assert (r[..., 3] == min(cap, T)).all(), cap
        torch.cuda.synchronize()
    # 1,500 per tile: above the triangle-parallel kernel's 1,024-id sort, so
    # even a complete list takes the ordered scan that stops at the cap
    T2 = 1500
    p2 = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T2, 1))
    p2[:, 2] = np.repeat(np.linspace(0.9, -0.9, T2), 3)
    tri2 = np.arange(3 * T2, dtype=np.int32).reshape(T2, 3)
    for cap in (128, 128, 1024):
        r = check_capped(p2[None], tri2, 32, 32, cap)
        assert (r[..., 3] == cap).all(), cap
        torch.cuda.synchronize()
    # range mode: image 1 draws triangles [100, 300) and keeps [100, 228)
    ranges = np.array([[0, 300], [100, 200], [250, 10]], np.int32)
    r = check_capped(p, tri, 32, 32, 128, ranges=ranges)
    assert (r[0, ..., 3] == 128).all() and (r[1, ..., 3] == 228).all() and (r[2, ..., 3] == 260).all()


def test_capped_icosphere_1024():
    """The benchmark scene (level-6 icosphere, 1024^2) with the reference's
    128 per tile: tri_id, barycentrics, z and rast_db bit-exact against the
    oracle's truncating mode; the truncation changes some pixels."""
    torch = torch_dev()
    from diffrast import DiffRast
    O.set_threads(16)
    sc = scenes.textured_icosphere(N=2, H=1024, W=1024, tex_size=8)
    r = check_capped(sc["pos"], sc["tri"], 1024, 1024, 128)
    full, _ = DiffRast.rasterize(dev(sc["pos"]), dev(sc["tri"]), (1024, 1024))
    assert (host(full)[..., 3] != r[..., 3]).any()


@pytest.mark.parametrize("gradDB", [False, True])
def test_capped_peel(gradDB):
    sc = scenes.textured_icosphere(N=1, H=128, W=128, level=5, tex_size=8)
    prev = None
    for _ in range(2):
        prev = check_capped(sc["pos"], sc["tri"], 128, 128, 16, gradDB=gradDB, peel=prev)


def test_range_mode_does_not_wait():
    """A range-mode call returns while work queued before it still runs:
    its ranges go through pinned staging, not a host-waited copy."""
    torch = torch_dev()
    from diffrast import DiffRast
    sc = scenes.range_batch(N=64, T_per=40)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    ranges = torch.as_tensor(sc["ranges"])
    stream = torch.cuda.current_stream()

    def calls(sleep):
        waited = 0
        for _ in range(3):
            if sleep:
                torch.cuda._sleep(200_000_000)  # ~0.1 s of spinning on the stream
            r, _ = DiffRast.rasterize(pos, tri, (48, 40), ranges=ranges)
            waited += stream.query()  # True: the stream drained before the call returned
        return r, waited

    # the same calls once first: the library sizes its scratch, and torch's
    # allocator caches the output blocks (a fresh device allocation may wait)
    calls(False)
    torch.cuda.synchronize()
    r, waited = calls(True)
    torch.cuda.synchronize()
    assert waited == 0
    rr, _ = O.rasterize(sc["pos"], sc["tri"], (48, 40), ranges=sc["ranges"], max_per_tile=0)
    np.testing.assert_array_equal(host(r), rr)


def _setup_launches(fn):
    """fn() with the library's launch timing on: how many triangle-setup
    passes (k_setup) it ran."""
    import diffrast._lib as L
    import torch
    lib = L.load()
    torch.cuda.synchronize()
    lib.dr_profile_reset()
    lib.dr_profile_enable(1)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        lib.dr_profile_enable(0)
    return L.profile_report().get("k_setup", {}).get("count", 0)


@pytest.mark.parametrize("gradDB", [False, True])
def test_peel_reuses_setup(gradDB):
    """Peel layers of one pos tensor: the layers after the first reuse the
    triangle setup and tile lists of the call before (one k_setup for three
    layers); every layer bit-exact against the oracle, and d_pos of the
    three layers against the oracle's."""
    torch = torch_dev()
    from diffrast import DiffRast
    sc = scenes.textured_icosphere(N=2, H=96, W=96, level=3, tex_size=8)
    pos, tri = sc["pos"], sc["tri"]
    p, t = dev(pos).requires_grad_(True), dev(tri)
    rng = np.random.default_rng(5)
    out = {}

    def layers():
        prev, prev_host, loss, ref = None, None, 0, np.zeros_like(pos)
        for _ in range(3):
            r, db = DiffRast.rasterize(p, t, (96, 96), gradDB=gradDB, peelLayer=prev)
            rr, rdb = O.rasterize(pos, tri, (96, 96), gradDB=gradDB, peelLayer=prev_host,
                                  max_per_tile=0)
            np.testing.assert_array_equal(host(r), rr)
            if gradDB:
                np.testing.assert_array_equal(host(db), rdb)
            g = rng.normal(size=rr.shape).astype(np.float32)
            loss = loss + (r * dev(g)).sum()
            ref += O.rasterize_vjp(pos, tri, rr, g, None)
            prev, prev_host = r.detach(), rr
        out["loss"], out["ref"] = loss, ref

    assert _setup_launches(layers) == 1
    out["loss"].backward()
    assert_grad_close(host(p.grad), out["ref"], "d_pos of the peel layers")


def test_peel_after_in_place_update_recomputes():
    """pos changed in place between two layers (a new autograd version): the
    second layer does its own setup and matches the oracle on the new pos."""
    torch = torch_dev()
    from diffrast import DiffRast
    sc = scenes.textured_icosphere(N=2, H=96, W=96, level=3, tex_size=8)
    pos, tri = sc["pos"], sc["tri"]
    p, t = dev(pos), dev(tri)
    r1, _ = DiffRast.rasterize(p, t, (96, 96), gradDB=False)
    p[..., 0] += 0.05
    moved = pos.copy()
    moved[..., 0] += np.float32(0.05)
    np.testing.assert_array_equal(host(p), moved)
    n = _setup_launches(lambda: DiffRast.rasterize(p, t, (96, 96), gradDB=False, peelLayer=r1))
    assert n == 1
    r2, _ = DiffRast.rasterize(p, t, (96, 96), gradDB=False, peelLayer=r1)
    rr, _ = O.rasterize(moved, tri, (96, 96), gradDB=False, peelLayer=host(r1), max_per_tile=0)
    np.testing.assert_array_equal(host(r2), rr)


def test_rasterize_again_abi():
    """dr_rasterize_fwd_again through the C-ABI: after a call with the same
    arguments it reuses that call's setup (one k_setup for both calls); with
    other arguments (here another resolution) it does the full work; every
    result bit-exact against the oracle."""
    import ctypes
    torch = torch_dev()
    import diffrast._lib as L
    lib = L.load()
    sc = scenes.textured_icosphere(N=2, H=64, W=80, level=3, tex_size=8)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    N, V, T = pos.shape[0], pos.shape[1], tri.shape[0]
    P = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())
    S = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    res = []

    def fwd(fn, H, W, peel=None):
        r = torch.empty((N, H, W, 4), device="cuda")
        db = torch.empty((N, H, W, 4), device="cuda")
        L.check(fn(P(pos), V * 4, P(tri), None, P(peel), N, V, T, H, W, P(r), P(db), 0, S))
        res.append((H, W, peel, r, db))
        return r

    def calls():
        r1 = fwd(lib.dr_rasterize_fwd_ex, 64, 80)
        fwd(lib.dr_rasterize_fwd_again, 64, 80, peel=r1)    # reuses the first call
        r3 = fwd(lib.dr_rasterize_fwd_again, 48, 40)        # another size: full work
        fwd(lib.dr_rasterize_fwd_again, 48, 40, peel=r3)    # reuses the third

    assert _setup_launches(calls) == 2
    for H, W, peel, r, db in res:
        rr, rdb = O.rasterize(sc["pos"], sc["tri"], (H, W), gradDB=True,
                              peelLayer=None if peel is None else host(peel), max_per_tile=0)
        np.testing.assert_array_equal(host(r), rr)
        np.testing.assert_array_equal(host(db), rdb)


def _raster_kernels(fn):
    """fn() with the library's launch timing on: the forward kernels it ran."""
    import diffrast._lib as L
    import torch
    lib = L.load()
    torch.cuda.synchronize()
    lib.dr_profile_reset()
    lib.dr_profile_enable(1)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        lib.dr_profile_enable(0)
    rep = L.profile_report()
    return {k for k in ("k_raster", "k_raster_px") if rep.get(k, {}).get("count", 0)}


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["small", "large"])
def test_forward_kernel_choice(kind):
    """Small triangles (a fine mesh) run the triangle-parallel forward,
    large ones (two triangles over the whole image) the pixel-parallel one,
    chosen from the previous call's tiles per triangle; both match the
    oracle bit for bit, with and without rast_db and a peel layer."""
    torch = torch_dev()
    from diffrast import DiffRast
    H = W = 128
    if kind == "small":
        sc = scenes.textured_icosphere(N=2, H=H, W=W, level=4, tex_size=8)
        pos, tri = sc["pos"], sc["tri"]
    else:
        quad = np.array([[-0.9, -0.8, 0.1, 1.0], [0.95, -0.9, 0.3, 1.0],
                         [0.9, 0.85, 0.5, 1.0], [-0.85, 0.9, 0.2, 1.0]], np.float32)
        pos = np.stack([quad, quad[[1, 2, 3, 0]] * np.float32([1, 1, 0.5, 1])])
        tri = np.array([[0, 1, 2], [0, 2, 3]], np.int32)
    p, t = dev(pos), dev(tri)
    want = "k_raster" if kind == "small" else "k_raster_px"
    for _ in range(2):  # the second call sees the first call's statistics
        ran = _raster_kernels(lambda: DiffRast.rasterize(p, t, (H, W), gradDB=True))
    assert ran == {want}
    rast, db = DiffRast.rasterize(p, t, (H, W), gradDB=True)
    rr, rdb = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    np.testing.assert_array_equal(host(rast), rr)
    np.testing.assert_array_equal(host(db), rdb)
    r2, _ = DiffRast.rasterize(p, t, (H, W), gradDB=False, peelLayer=rast)
    rr2, _ = O.rasterize(pos, tri, (H, W), gradDB=False, peelLayer=rr, max_per_tile=0)
    np.testing.assert_array_equal(host(r2), rr2)


def test_capped_large_triangles_pixel_parallel():
    """300 full-screen triangles over 64 tiles each take the pixel-parallel
    forward; with a per-tile cap (ranked in LDS, or the ordered full scan
    while the list capacity is short) every pixel shows the cap's last
    triangle, bit-exact against the oracle."""
    torch = torch_dev()
    from diffrast import DiffRast, _lib
    torch.cuda.synchronize()
    assert _lib.load().dr_release_scratch() == 0
    sc = scenes.tier1_triangle(H=128, W=128)
    check_fwd(sc["pos"], sc["tri"], 128, 128)  # a short list capacity first
    T = 300
    p = np.tile(np.array([[-3, 3, 0, 1], [-3, -3, 0, 1], [3, 0, 0, 1]], np.float32), (T, 1))
    p[:, 2] = np.repeat(np.linspace(0.9, -0.9, T), 3)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    for cap in (128, 128, 5, 300, 0):
        if cap:
            r = check_capped(p[None], tri, 128, 128, cap)
            assert (r[..., 3] == min(cap, T)).all(), cap
        else:
            check_fwd(p[None], tri, 128, 128)
        torch.cuda.synchronize()
    ran = _raster_kernels(lambda: DiffRast.rasterize(dev(p[None]), dev(tri), (128, 128),
                                                     maxPerTile=16))
    assert ran == {"k_raster_px"}


def _launches(fn, names):
    """fn() with the library's launch timing on: launches of each kernel."""
    import diffrast._lib as L
    import torch
    lib = L.load()
    torch.cuda.synchronize()
    lib.dr_profile_reset()
    lib.dr_profile_enable(1)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        lib.dr_profile_enable(0)
    rep = L.profile_report()
    return {k: rep.get(k, {}).get("count", 0) for k in names}


def _bwd_case(rng, pos, tri, H, W, ranges=None):
    """A forward whose loss weights rast and rast_db with fixed random
    cotangents; returns (pos leaf, loss, oracle d_pos)."""
    from diffrast import DiffRast
    p = dev(pos).requires_grad_(True)
    r, db = DiffRast.rasterize(p, dev(tri), (H, W), gradDB=True,
                               ranges=None if ranges is None else torch_dev().as_tensor(ranges))
    g = rng.normal(size=tuple(r.shape)).astype(np.float32)
    gdb = rng.normal(size=tuple(r.shape)).astype(np.float32)
    loss = (r * dev(g)).sum() + (db * dev(gdb)).sum()
    ref = O.rasterize_vjp(pos, tri, host(r), g, gdb, ranges=ranges)
    return p, loss, ref


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["icosphere", "range"])
def test_backward_reuses_forward_records(name):
    """Once a backward has used per-triangle records, later forwards write
    them with their setup and the backward of the last forward on the
    stream skips k_rbwd_rec; a backward of an earlier forward (another
    forward ran since) recomputes them.  Every d_pos matches the oracle."""
    rng = np.random.default_rng(5)
    ranges = None
    if name == "icosphere":
        sc = scenes.textured_icosphere(N=2, H=256, W=256, level=4, tex_size=8)
        pos, tri, H, W = sc["pos"], sc["tri"], 256, 256
    else:
        sc = scenes.range_batch(N=4, T_per=6)
        pos, tri, ranges, H, W = sc["pos"], sc["tri"], sc["ranges"], 96, 96
    names = ("k_rbwd_rec", "k_raster_bwd")
    import diffrast._lib as L
    import torch
    torch.cuda.synchronize()
    assert L.load().dr_release_scratch() == 0  # a fresh stream state: no records asked for yet
    # a first step: its backward computes the records (and asks for them)
    p, loss, ref = _bwd_case(rng, pos, tri, H, W, ranges)
    assert _launches(loss.backward, names) == {"k_rbwd_rec": 1, "k_raster_bwd": 1}
    assert_grad_close(host(p.grad), ref, "d_pos first step")
    # the next step's backward reuses what its forward stored
    p, loss, ref = _bwd_case(rng, pos, tri, H, W, ranges)
    assert _launches(loss.backward, names) == {"k_rbwd_rec": 0, "k_raster_bwd": 1}
    assert_grad_close(host(p.grad), ref, "d_pos with the forward's records")
    # two forwards, backwards in reverse order: the last forward's backward
    # reuses, the earlier one's recomputes (its records were overwritten)
    pos2 = pos.copy()
    pos2[..., 0] += 0.01 * pos2[..., 3]
    pa, la, ra = _bwd_case(rng, pos, tri, H, W, ranges)
    pb, lb, rb = _bwd_case(rng, pos2, tri, H, W, ranges)
    assert _launches(lb.backward, names) == {"k_rbwd_rec": 0, "k_raster_bwd": 1}
    assert _launches(la.backward, names) == {"k_rbwd_rec": 1, "k_raster_bwd": 1}
    assert_grad_close(host(pb.grad), rb, "d_pos of the last forward")
    assert_grad_close(host(pa.grad), ra, "d_pos of the earlier forward")
    # backwards in call order: the earlier one recomputes into the slot, so
    # the last one may not take the slot as its forward's either
    pa, la, ra = _bwd_case(rng, pos, tri, H, W, ranges)
    pb, lb, rb = _bwd_case(rng, pos2, tri, H, W, ranges)
    assert _launches(la.backward, names) == {"k_rbwd_rec": 1, "k_raster_bwd": 1}
    assert _launches(lb.backward, names) == {"k_rbwd_rec": 1, "k_raster_bwd": 1}
    assert_grad_close(host(pa.grad), ra, "d_pos of the earlier forward, first")
    assert_grad_close(host(pb.grad), rb, "d_pos of the last forward, second")


@pytest.mark.gpu
def test_backward_reuse_flag_abi_checks_its_inputs():
    """DR_RASTERIZE_BWD_REUSE through the C-ABI: the library takes the
    forward's stored records only for the pos and tri that forward drew; a
    backward that passes the flag with another pos buffer gets its own
    records (k_rbwd_rec runs) and that pos's d_pos."""
    import ctypes
    torch = torch_dev()
    import diffrast._lib as L
    lib = L.load()
    torch.cuda.synchronize()
    assert lib.dr_release_scratch() == 0
    sc = scenes.textured_icosphere(N=2, H=256, W=256, level=4, tex_size=8)
    posa = sc["pos"]
    posb = posa.copy()
    posb[..., 1] += 0.02 * posb[..., 3]
    pa, pb, tri = dev(posa), dev(posb), dev(sc["tri"])
    N, V, T, H, W = pa.shape[0], pa.shape[1], tri.shape[0], 256, 256
    P = lambda x: None if x is None else ctypes.c_void_p(x.data_ptr())
    S = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rng = np.random.default_rng(8)
    g = rng.normal(size=(N, H, W, 4)).astype(np.float32)
    gdb = rng.normal(size=(N, H, W, 4)).astype(np.float32)
    dg, ddb = dev(g), dev(gdb)

    def fwd(p):
        r = torch.empty((N, H, W, 4), device="cuda")
        db = torch.empty((N, H, W, 4), device="cuda")
        L.check(lib.dr_rasterize_fwd_ex(P(p), V * 4, P(tri), None, None, N, V, T, H, W, P(r),
                                        P(db), 0, S))
        return r

    def bwd(p, r, flags):
        d = torch.empty_like(p)
        L.check(lib.dr_rasterize_bwd(P(p), V * 4, P(tri), P(r), P(dg), P(ddb), N, V, T, H, W,
                                     P(d), flags, S))
        return d

    names = ("k_rbwd_rec",)
    ra = fwd(pa)
    bwd(pa, ra, 0)                                  # asks later forwards for the records
    ra = fwd(pa)                                    # stores them
    rb = fwd(pb)                                    # stores pos b's instead
    out = {}
    # the flag with pos a after pos b's forward: the stored records are b's
    assert _launches(lambda: out.setdefault("a", bwd(pa, ra, L.DR_RASTERIZE_BWD_REUSE)),
                     names) == {"k_rbwd_rec": 1}
    rb = fwd(pb)                                    # pos b's records again
    assert _launches(lambda: out.setdefault("b", bwd(pb, rb, L.DR_RASTERIZE_BWD_REUSE)),
                     names) == {"k_rbwd_rec": 0}
    for key, pos, r in (("a", posa, ra), ("b", posb, rb)):
        ref = O.rasterize_vjp(pos, sc["tri"], host(r), g, gdb)
        assert_grad_close(host(out[key]), ref, f"d_pos {key}")


@pytest.mark.gpu
def test_backward_small_triangles_with_forward_records():
    """Triangles averaging under 8 pixels: a backward builds each pixel's
    triangle values itself, but once a backward has run, the forward stores
    the per-triangle records and the next backward reads them (all four
    peel layers of one pos qualify).  d_pos matches the oracle both ways."""
    import diffrast._lib as L
    import torch
    from diffrast import DiffRast
    torch.cuda.synchronize()
    assert L.load().dr_release_scratch() == 0
    sc = scenes.textured_icosphere(N=2, H=64, W=64, level=5, tex_size=8)
    pos, tri, H, W = sc["pos"], sc["tri"], 64, 64
    assert 2 * tri.shape[0] * 8 > 2 * H * W  # below 8 pixels per triangle
    rng = np.random.default_rng(21)
    for step in range(2):
        p = dev(pos).requires_grad_(True)
        t = dev(tri)
        layers, prev, loss, refs = [], None, 0.0, []
        for _ in range(2):
            r, db = DiffRast.rasterize(p, t, (H, W), gradDB=True, peelLayer=prev)
            g = rng.normal(size=tuple(r.shape)).astype(np.float32)
            gdb = rng.normal(size=tuple(r.shape)).astype(np.float32)
            loss = loss + (r * dev(g)).sum() + (db * dev(gdb)).sum()
            refs.append(O.rasterize_vjp(pos, tri, host(r), g, gdb))
            prev = r.detach()
        loss.backward()
        assert_grad_close(host(p.grad), refs[0] + refs[1], f"d_pos step {step}")


@pytest.mark.gpu
def test_pixel_parallel_depth_cull_keeps_ties():
    """The pixel-parallel forward drops a candidate for an 8x8 quadrant when
    its smallest depth over the quadrant's pixel centres (less a margin over
    the fp32 rounding) lies above every pixel's best depth so far.  Exact
    duplicates (the lower index keeps the pixel) and copies a few ulps
    nearer or farther in depth, taken in random and in near-to-far order,
    stay bit-exact against the oracle, forward, rast_db and a peeled layer."""
    torch = torch_dev()
    from diffrast import DiffRast
    H, W = 128, 96
    rng = np.random.default_rng(57)
    base = rng.uniform(-1.3, 1.3, size=(120, 3, 2)).astype(np.float32)
    bz = rng.uniform(-0.9, 0.9, size=(120, 3)).astype(np.float32)
    pick = rng.choice(120, size=80, replace=False)
    xy = np.concatenate([base, base[pick]], 0)
    z = np.concatenate([bz, bz[pick]], 0)
    for i, k in enumerate(range(160, 200)):  # near ties: 1-3 ulps either way
        step = (i % 3) + 1
        toward = np.float32(-2.0) if i % 2 else np.float32(2.0)
        for _ in range(step):
            z[k] = np.nextafter(z[k], toward)
    T = xy.shape[0]
    order = [np.arange(T), np.argsort(z.mean(1))]  # image 1: near to far
    pos = np.stack([np.concatenate([xy[o], z[o][..., None], np.ones((T, 3, 1), np.float32)],
                                   -1).reshape(-1, 4) for o in order]).astype(np.float32)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    p, t = dev(pos), dev(tri)
    for _ in range(2):  # the second call sees the first call's statistics
        ran = _raster_kernels(lambda: DiffRast.rasterize(p, t, (H, W), gradDB=True))
    assert ran == {"k_raster_px"}
    rast, db = DiffRast.rasterize(p, t, (H, W), gradDB=True)
    rr, rdb = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    np.testing.assert_array_equal(host(rast), rr)
    np.testing.assert_array_equal(host(db), rdb)
    assert (rr[..., 3] > 0).mean() > 0.9
    r2, _ = DiffRast.rasterize(p, t, (H, W), gradDB=False, peelLayer=rast)
    rr2, _ = O.rasterize(pos, tri, (H, W), gradDB=False, peelLayer=rr, max_per_tile=0)
    np.testing.assert_array_equal(host(r2), rr2)


def test_pixel_parallel_edge_cull_keeps_boundary_pixels():
    """The pixel-parallel forward drops a candidate for an 8x8 quadrant only
    when one of its edges keeps every pixel centre there outside (with a
    margin over the fp32 rounding).  Large triangles whose vertices sit on
    pixel centres put edges exactly through centres (e = 0 counts as
    inside): the result is still bit-exact against the oracle."""
    torch = torch_dev()
    from diffrast import DiffRast
    H, W, T = 128, 96, 96
    rng = np.random.default_rng(31)
    ix = rng.integers(0, W, size=(2, 3 * T))
    iy = rng.integers(0, H, size=(2, 3 * T))
    x = (2.0 * (ix.astype(np.float32) + np.float32(0.5)) / np.float32(W) - 1.0).astype(np.float32)
    y = (1.0 - 2.0 * (iy.astype(np.float32) + np.float32(0.5)) / np.float32(H)).astype(np.float32)
    z = rng.uniform(-0.9, 0.9, size=(2, 3 * T)).astype(np.float32)
    pos = np.stack([x, y, z, np.ones_like(x)], -1).astype(np.float32)
    tri = np.arange(3 * T, dtype=np.int32).reshape(T, 3)
    p, t = dev(pos), dev(tri)
    for _ in range(2):  # the second call sees the first call's statistics
        ran = _raster_kernels(lambda: DiffRast.rasterize(p, t, (H, W), gradDB=True))
    assert ran == {"k_raster_px"}
    rast, db = DiffRast.rasterize(p, t, (H, W), gradDB=True)
    rr, rdb = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    np.testing.assert_array_equal(host(rast), rr)
    np.testing.assert_array_equal(host(db), rdb)
    r2, _ = DiffRast.rasterize(p, t, (H, W), gradDB=False, peelLayer=rast)
    rr2, _ = O.rasterize(pos, tri, (H, W), gradDB=False, peelLayer=rr, max_per_tile=0)
    np.testing.assert_array_equal(host(r2), rr2)


def _fill_launches(fn):
    """fn() with the library's launch timing on: {binning fill kind: launches}."""
    import diffrast._lib as L
    import torch
    lib = L.load()
    torch.cuda.synchronize()
    lib.dr_profile_reset()
    lib.dr_profile_enable(1)
    try:
        fn()
        torch.cuda.synchronize()
    finally:
        lib.dr_profile_enable(0)
    rep = L.profile_report()
    return {k: rep.get(k, {}).get("count", 0) for k in ("k_bin_fill", "k_bin_fill_bal")}


@pytest.mark.parametrize("kind", ["one", "range", "capped", "small"])
def test_balanced_binning(kind):
    """A few large triangles per image (4 tiles each or more on average,
    counted by the first call on a stream or read back from an earlier one):
    the binning deals the (triangle, tile) pairs out evenly over the
    workgroup (k_bin_fill_bal); the lists it builds rasterize bit-exactly as
    the oracle's, uncapped and with the reference's per-tile limit (whose
    ranking needs complete lists).  Small triangles keep one triangle per
    thread (k_bin_fill)."""
    torch_dev()
    from diffrast import _lib
    assert _lib.load().dr_release_scratch() == 0  # no statistics from earlier calls
    if kind == "one":  # one triangle over most of a 256^2 image
        sc = scenes.tier1_triangle(H=256, W=256)
        pos, tri, ranges, H, W = sc["pos"], sc["tri"], None, 256, 256
    elif kind == "small":  # ~1 tile per triangle
        sc = scenes.textured_icosphere(N=2, H=128, W=128, level=4, tex_size=8)
        pos, tri, ranges, H, W = sc["pos"], sc["tri"], None, 128, 128
    else:  # 24 images of 96 random triangles, most of them over most tiles
        sc = scenes.range_batch(N=24, T_per=96, H=80, W=112)  # (at most 256 per image)
        pos, tri, ranges, H, W = sc["pos"], sc["tri"], sc["ranges"], 80, 112
    for call in range(3):
        if kind == "capped":
            n = _fill_launches(lambda: check_capped(pos, tri, H, W, 32, ranges=ranges))
        else:
            n = _fill_launches(lambda: check_fwd(pos, tri, H, W, ranges=ranges))
        if kind == "small":
            assert n == {"k_bin_fill": 1, "k_bin_fill_bal": 0}, (call, n)
        else:
            assert n == {"k_bin_fill": 0, "k_bin_fill_bal": 1}, (call, n)
