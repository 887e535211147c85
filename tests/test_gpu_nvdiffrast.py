"""GPU: nvdiffrast's functional API (diffrast.nvdiffrast) on the inputs of
the reference's nvdiffrast fixture (scripts/diffrast_fixtures.py:23-54),
compared with nvdiffrast's outputs in nvdiffrast's own conventions."""
import numpy as np
import pytest

from parity import dev, host, torch_dev

pytestmark = pytest.mark.gpu

POS = np.array([[-0.7, 0.8, 0.0, 1.0], [0.8, 0.7, 0.1, 1.0], [0.7, -0.8, 0.2, 1.0],
                [-0.8, -0.7, 0.0, 1.0]], np.float32)[None]
TRI = np.array([[0, 1, 2], [0, 2, 3]], np.int32)
ATTR = np.array([[1, 0, 0], [0, 1, 0], [0, 0, 1], [1, 1, 0]], np.float32)[None]
TEX8 = np.array([[[x / 7, y / 7, (x + y) / 14] for x in range(8)] for y in range(8)],
                np.float32)[None]


def test_rasterize(fixtures):
    torch_dev()
    import diffrast.nvdiffrast as dr
    ctx = dr.RasterizeCudaContext()
    rast, db = dr.rasterize(ctx, dev(POS), dev(TRI), [16, 16])
    rast, db = host(rast), host(db)
    ref, refdb = fixtures["rast"], fixtures["rast_db"]
    same = (rast[..., 3] > 0) & (rast[..., 3] == ref[..., 3])
    assert same.sum() >= 0.97 * (ref[..., 3] > 0).sum()
    np.testing.assert_allclose(rast[same], ref[same], atol=2e-5)
    np.testing.assert_allclose(db[same], refdb[same], atol=2e-5)
    assert (rast[rast[..., 3] == 0] == 0).all()        # empty pixels are zero
    _, nodb = dr.rasterize(ctx, dev(POS), dev(TRI), [16, 16], grad_db=False)
    assert nodb.shape[-1] == 0


def test_interpolate_and_gradients(fixtures):
    """interp_out / interp_out_da and the three backward outputs, given
    nvdiffrast's own rast: same physical barycentrics, so they must agree."""
    torch = torch_dev()
    import diffrast.nvdiffrast as dr
    rast = dev(fixtures["rast"]).requires_grad_(True)
    db = dev(fixtures["rast_db"]).requires_grad_(True)
    attr = dev(ATTR).requires_grad_(True)
    out, da = dr.interpolate(attr, rast, dev(TRI), rast_db=db, diff_attrs="all")
    np.testing.assert_allclose(host(out), fixtures["interp_out"], atol=2e-6)
    np.testing.assert_allclose(host(da), fixtures["interp_out_da"], atol=2e-6)
    (out * dev(fixtures["co_interp_out"])).sum().backward(retain_graph=True)
    (da * dev(fixtures["co_interp_out_da"])).sum().backward()
    np.testing.assert_allclose(host(attr.grad), fixtures["d_attr_from_interp"], rtol=1e-5,
                               atol=1e-5)
    cov = fixtures["rast"][..., 3] > 0
    np.testing.assert_allclose(host(rast.grad)[cov][:, :2],
                               fixtures["d_rast_from_interp"][cov][:, :2], rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(host(db.grad)[cov], fixtures["d_rast_db_from_interp"][cov],
                               rtol=1e-5, atol=1e-5)


def test_texture(fixtures):
    torch_dev()
    import diffrast.nvdiffrast as dr
    tex = dev(TEX8).requires_grad_(True)
    uv = dev(fixtures["uv"]).requires_grad_(True)
    out = dr.texture(tex, uv, filter_mode="linear", boundary_mode="clamp")
    assert np.abs(host(out) - fixtures["tex_bilinear"]).max() <= 1e-5
    (out * dev(fixtures["co_tex"])).sum().backward()
    np.testing.assert_allclose(host(tex.grad), fixtures["d_tex_from_bilinear"], rtol=1e-5,
                               atol=1e-4)
    np.testing.assert_allclose(host(uv.grad), fixtures["d_uv_from_bilinear"], rtol=1e-4,
                               atol=1e-5)
    out = dr.texture(dev(TEX8), dev(fixtures["uv"]), uv_da=dev(fixtures["uv_da"]),
                     filter_mode="auto", boundary_mode="clamp")
    assert np.abs(host(out) - fixtures["tex_trilinear"]).max() <= 1e-4
    t8 = dev(TEX8)
    mip = dr.texture_construct_mip(t8)
    out2 = dr.texture(t8, dev(fixtures["uv"]), uv_da=dev(fixtures["uv_da"]), mip=mip,
                      filter_mode="linear-mipmap-linear", boundary_mode="clamp")
    np.testing.assert_array_equal(host(out2), host(out))


def test_antialias_is_the_flipped_library_op():
    """antialias in nvdiffrast's conventions is this library's antialias on
    the flipped images (the reference's silhouette rule, not nvdiffrast's)."""
    torch = torch_dev()
    import diffrast.nvdiffrast as dr
    from diffrast import DiffRast
    rng = np.random.default_rng(3)
    pos = dev(POS)
    rast_nv, _ = dr.rasterize(None, pos, dev(TRI), [16, 16])
    color = dev(rng.random((1, 16, 16, 3), dtype=np.float32))
    p1 = pos.clone().requires_grad_(True)
    out = dr.antialias(color, rast_nv, p1, dev(TRI), pos_gradient_boost=2.0)
    rast_mine, _ = DiffRast.rasterize(pos, dev(TRI), (16, 16))
    p2 = pos.clone().requires_grad_(True)
    ref = DiffRast.antialias(color.flip(1), rast_mine, p2, dev(TRI)).flip(1)
    np.testing.assert_array_equal(host(out), host(ref))
    g = dev(rng.normal(size=(1, 16, 16, 3)).astype(np.float32))
    (out * g).sum().backward()
    (ref * g).sum().backward()
    np.testing.assert_allclose(host(p1.grad), 2.0 * host(p2.grad), rtol=1e-5, atol=1e-6)
