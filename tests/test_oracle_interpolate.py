"""Pins the CPU oracle's interpolate against the reference's known answers
(Tests/MLXDiffRastTests/InterpolateTests.swift), finite differences, and the
nvdiffrast fixture (interp_out, interp_out_da, d_attr) after the
convention remap of CONVENTIONS.md.  CPU only."""
import numpy as np
import pytest

import oracle as O

TRI1 = np.array([[0, 1, 2]], np.int32)


def test_forward_constant_barys():
    # InterpolateTests.swift:11-38
    attr = np.array([[i, i + 1, i + 2] for i in range(3)], np.float32)[None]
    rast = np.tile(np.array([0.25, 0.5, 0.0, 1.0], np.float32), (1, 2, 2, 1))
    out, da = O.interpolate(attr, rast, TRI1)
    assert out.shape == (1, 2, 2, 3) and da.shape == (1, 2, 2, 0)
    np.testing.assert_allclose(out.reshape(-1, 3), np.tile([1.25, 2.25, 3.25], (4, 1)), atol=1e-5)


def test_empty_pixels_are_zero():
    # InterpolateTests.swift:40-52
    attr = np.ones((1, 3, 2), np.float32)
    rast = np.array([0, 0, 0, 0, 0, 0, 0, 1], np.float32).reshape(1, 1, 2, 4)
    out, _ = O.interpolate(attr, rast, TRI1)
    np.testing.assert_array_equal(out.reshape(-1), [0, 0, 1, 1])


def test_range_mode_broadcasts_across_batch():
    # InterpolateTests.swift:57-71
    attr = np.array([10, 20, 30, 40, 50, 60], np.float32).reshape(3, 2)
    rast = np.array([0, 0, 0, 1, 1, 0, 0, 1], np.float32).reshape(2, 1, 1, 4)
    out, _ = O.interpolate(attr, rast, TRI1)
    np.testing.assert_array_equal(out.reshape(-1), [10, 20, 30, 40])


def test_forward_da_matches_analytic():
    # InterpolateTests.swift:78-99
    attr = np.array([1, 2, 4, 5, 7, 8], np.float32).reshape(1, 3, 2)
    rast = np.array([0.1, 0.2, 0.0, 1.0], np.float32).reshape(1, 1, 1, 4)
    db = np.array([0.5, -0.25, 0.125, 1.0], np.float32).reshape(1, 1, 1, 4)
    _, da = O.interpolate(attr, rast, TRI1, rastDB=db, diffAttrs="all")
    assert da.shape == (1, 1, 1, 4)
    np.testing.assert_allclose(da.reshape(-1), [2.25, 5.25, 2.25, 5.25], atol=1e-5)


def test_diff_attrs_indices_matches_all_subset():
    # InterpolateTests.swift:106-131
    attr = np.arange(1, 10, dtype=np.float32).reshape(1, 3, 3)
    rast = np.array([0.2, 0.3, 0.0, 1.0], np.float32).reshape(1, 1, 1, 4)
    db = np.array([0.5, 0.1, -0.2, 0.3], np.float32).reshape(1, 1, 1, 4)
    _, a = O.interpolate(attr, rast, TRI1, rastDB=db, diffAttrs="all")
    _, b = O.interpolate(attr, rast, TRI1, rastDB=db, diffAttrs=[0, 2])
    assert b.shape == (1, 1, 1, 4)
    a, b = a.reshape(-1), b.reshape(-1)
    np.testing.assert_allclose(b, [a[0], a[1], a[4], a[5]], atol=1e-6)


def test_shape_errors():
    attr = np.ones((1, 3, 2), np.float32)
    rast = np.zeros((1, 2, 2, 4), np.float32)
    with pytest.raises(ValueError):
        O.interpolate(attr, rast, TRI1, diffAttrs="all")  # rastDB missing
    with pytest.raises(ValueError):
        O.interpolate(attr, rast, TRI1, rastDB=rast, diffAttrs=[5])


def _fd(loss, x, eps=1e-3, skip=None):
    g = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        if skip is not None and skip(i):
            continue
        xp = flat.copy(); xp[i] += eps
        xm = flat.copy(); xm[i] -= eps
        g.reshape(-1)[i] = (loss(xp.reshape(x.shape)) - loss(xm.reshape(x.shape))) / (2 * eps)
    return g


def _setup(rng, A, da, H=2, W=2):
    us = rng.uniform(0.05, 0.45, size=H * W)
    vs = rng.uniform(0.05, 0.45, size=H * W)
    rast = np.stack([us, vs, np.zeros(H * W), np.ones(H * W)], 1).astype(np.float32)
    rast = rast.reshape(1, H, W, 4)
    attr = rng.normal(size=(1, 3, A)).astype(np.float32)
    db = rng.normal(size=(1, H, W, 4)).astype(np.float32) if da else None
    return attr, rast, db


@pytest.mark.parametrize("target", ["attr", "rast", "rastDB"])
@pytest.mark.parametrize("diff", [None, "all", [1, 3]])
def test_gradcheck(target, diff):
    # InterpolateTests.swift:133-312 (basic, DA, .indices)
    if target == "rastDB" and diff is None:
        pytest.skip("no rastDB dependence without diffAttrs")
    rng = np.random.default_rng(7)
    A = 4 if isinstance(diff, list) else 2
    attr, rast, db = _setup(rng, A, diff is not None)
    K = A if diff == "all" else (len(diff) if diff else 0)
    w_out = rng.normal(size=(1, 2, 2, A)).astype(np.float32)
    w_da = rng.normal(size=(1, 2, 2, 2 * K)).astype(np.float32)

    def loss_of(a, r, d):
        o, od = O.interpolate(a, r, TRI1, rastDB=d, diffAttrs=diff)
        v = (o.astype(np.float64) * w_out).sum()
        if diff is not None:
            v += (od.astype(np.float64) * w_da).sum()
        return v

    d_attr, d_rast, d_db = O.interpolate_vjp(attr, rast, TRI1, w_out, rastDB=db, diffAttrs=diff,
                                             d_out_da=w_da if diff is not None else None)
    if target == "attr":
        np.testing.assert_allclose(d_attr, _fd(lambda x: loss_of(x, rast, db), attr), atol=5e-3)
    elif target == "rast":
        skip = lambda i: i % 4 >= 2
        fd = _fd(lambda x: loss_of(attr, x, db), rast, skip=skip)
        np.testing.assert_array_equal(d_rast[..., 2:], 0)
        np.testing.assert_allclose(d_rast[..., :2], fd[..., :2], atol=5e-3)
    else:
        np.testing.assert_allclose(d_db, _fd(lambda x: loss_of(attr, rast, x), db), atol=5e-3)


def _nv_to_mine(nv_rast, nv_db):
    """CONVENTIONS.md:17-72: y flip, (u,v) = (nv.v, 1 - nv.u - nv.v)."""
    r = nv_rast[:, ::-1].copy()
    d = nv_db[:, ::-1].copy()
    mine = np.stack([r[..., 1], 1 - r[..., 0] - r[..., 1], r[..., 2], r[..., 3]], -1)
    mdb = np.stack([d[..., 2], -d[..., 3], -(d[..., 0] + d[..., 2]), d[..., 1] + d[..., 3]], -1)
    return mine.astype(np.float32), mdb.astype(np.float32)


ATTR = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 0]], np.float32)[None]
TRI2 = np.array([[0, 1, 2], [0, 2, 3]], np.int32)


def test_nvdiffrast_fixture_interp(fixtures):
    """nvdiffrast's interp outputs, given its own rast converted to this
    library's convention: the physical barycentric weights are the same, so
    the interpolated attributes and their screen derivatives must match."""
    rast, db = _nv_to_mine(fixtures["rast"], fixtures["rast_db"])
    out, da = O.interpolate(ATTR, rast, TRI2, rastDB=db, diffAttrs="all")
    np.testing.assert_allclose(out, fixtures["interp_out"][:, ::-1], atol=2e-6)
    nv_da = fixtures["interp_out_da"][:, ::-1].copy()
    nv_da[..., 1::2] *= -1  # y flip negates d/dy
    np.testing.assert_allclose(da, nv_da, atol=2e-6)


def test_nvdiffrast_fixture_d_attr(fixtures):
    rast, db = _nv_to_mine(fixtures["rast"], fixtures["rast_db"])
    co = fixtures["co_interp_out"][:, ::-1].copy()
    co_da = fixtures["co_interp_out_da"][:, ::-1].copy()
    co_da[..., 1::2] *= -1
    d_attr, _, _ = O.interpolate_vjp(ATTR, rast, TRI2, co, rastDB=db, diffAttrs="all",
                                     d_out_da=co_da)
    np.testing.assert_allclose(d_attr, fixtures["d_attr_from_interp"], rtol=1e-5, atol=1e-5)
