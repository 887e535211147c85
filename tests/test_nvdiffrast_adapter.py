"""The nvdiffrast-convention conversions (CONVENTIONS.md:17-72 of the
reference) on the CPU: exact inverses of each other, and nvdiffrast's own
fixture outputs reproduced from the oracle's outputs through them."""
import numpy as np
import pytest

import oracle as O

torch = pytest.importorskip("torch")
from diffrast.nvdiffrast import rast_from_nvdiffrast, rast_to_nvdiffrast  # noqa: E402

POS = np.array([[-0.7, 0.8, 0.0, 1.0], [0.8, 0.7, 0.1, 1.0], [0.7, -0.8, 0.2, 1.0],
                [-0.8, -0.7, 0.0, 1.0]], np.float32)[None]
TRI = np.array([[0, 1, 2], [0, 2, 3]], np.int32)
ATTR = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 0]], np.float32)[None]


def test_round_trip():
    rng = np.random.default_rng(0)
    w = rng.dirichlet([1, 1, 1], size=(2, 9, 7)).astype(np.float32)
    rast = np.concatenate([w[..., 1:], rng.random((2, 9, 7, 1), dtype=np.float32),
                           rng.integers(0, 4, (2, 9, 7, 1)).astype(np.float32)], -1)
    rast[rast[..., 3] == 0] = 0.0
    db = rng.normal(size=(2, 9, 7, 4)).astype(np.float32)
    db[rast[..., 3] == 0] = 0.0
    nv, nvdb = rast_to_nvdiffrast(torch.tensor(rast), torch.tensor(db))
    # nvdiffrast's (u, v) = (w0, w1), image flipped, empty pixels zero
    cov = rast[..., 3] > 0
    np.testing.assert_allclose(nv.numpy()[:, ::-1][..., 0][cov], w[..., 0][cov], atol=1e-6)
    np.testing.assert_array_equal(nv.numpy()[:, ::-1][..., 1], rast[..., 0])
    assert (nv.numpy()[:, ::-1][~cov] == 0).all()
    back, backdb = rast_from_nvdiffrast(nv, nvdb)
    np.testing.assert_allclose(back.numpy(), rast, atol=1e-6)
    np.testing.assert_allclose(backdb.numpy(), db, atol=1e-5)


def test_fixture_rast_from_oracle(fixtures):
    """The oracle's rast / rast_db in nvdiffrast's convention equal
    nvdiffrast's fixture where both cover the pixel with the same triangle
    (w = 1 everywhere, so the barycentrics agree; edge pixels follow
    different fill rules)."""
    rast, db = O.rasterize(POS, TRI, (16, 16))
    nv, nvdb = (t.numpy() for t in rast_to_nvdiffrast(torch.tensor(rast), torch.tensor(db)))
    ref, refdb = fixtures["rast"], fixtures["rast_db"]
    same = (nv[..., 3] > 0) & (nv[..., 3] == ref[..., 3])
    assert same.sum() >= 0.97 * (ref[..., 3] > 0).sum()
    np.testing.assert_allclose(nv[same], ref[same], atol=2e-5)
    np.testing.assert_allclose(nvdb[same], refdb[same], atol=2e-5)


def test_fixture_interp_through_conversion(fixtures):
    """nvdiffrast's rast converted to this library's convention, fed to the
    oracle's interpolate, reproduces nvdiffrast's interp_out after the
    inverse image flip."""
    mine, mdb = rast_from_nvdiffrast(torch.tensor(fixtures["rast"]),
                                     torch.tensor(fixtures["rast_db"]))
    out, da = O.interpolate(ATTR, mine.numpy(), TRI, rastDB=mdb.numpy(), diffAttrs="all")
    np.testing.assert_allclose(out[:, ::-1], fixtures["interp_out"], atol=2e-6)
    da = da[:, ::-1].copy()
    da[..., 1::2] *= -1
    np.testing.assert_allclose(da, fixtures["interp_out_da"], atol=2e-6)
