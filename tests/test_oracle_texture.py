"""Pins the CPU oracle's texture against the reference's known answers
(Tests/MLXDiffRastTests/TextureTests.swift), the nvdiffrast fixture
(ParityTests.swift:92-111 plus the gradients the fixture holds), finite
differences and d_tex partition of unity.  CPU only."""
import numpy as np
import pytest

import oracle as O

T22 = np.array([10, 20, 30, 40], np.float32).reshape(1, 2, 2, 1)


def test_texel_centers():
    # TextureTests.swift:11-27
    uv = np.array([.25, .25, .75, .25, .25, .75, .75, .75], np.float32).reshape(1, 2, 2, 2)
    np.testing.assert_array_equal(O.texture(T22, uv).reshape(-1), [10, 20, 30, 40])


def test_center_is_mean():
    # TextureTests.swift:30-38
    uv = np.array([0.5, 0.5], np.float32).reshape(1, 1, 1, 2)
    np.testing.assert_allclose(O.texture(T22, uv).item(), 25, atol=1e-5)


def test_boundary_modes():
    # TextureTests.swift:41-71
    one = np.ones((1, 2, 2, 1), np.float32)
    uv5 = np.array([5.0, 5.0], np.float32).reshape(1, 1, 1, 2)
    assert abs(O.texture(one, uv5, boundaryMode="zero").item()) < 1e-6
    uv10 = np.array([10.0, 10.0], np.float32).reshape(1, 1, 1, 2)
    np.testing.assert_allclose(O.texture(T22, uv10, boundaryMode="clamp").item(), 40, atol=1e-6)
    a = O.texture(T22, np.array([0.4, 0.6], np.float32).reshape(1, 1, 1, 2), boundaryMode="wrap")
    b = O.texture(T22, np.array([1.4, 0.6], np.float32).reshape(1, 1, 1, 2), boundaryMode="wrap")
    np.testing.assert_allclose(a, b, atol=1e-5)


CUBE = np.array([10, 20, 30, 40, 50, 60], np.float32).reshape(1, 6, 1, 1, 1)
DIRS = np.array([[1, 0, 0], [-1, 0, 0], [0, 1, 0], [0, -1, 0], [0, 0, 1], [0, 0, -1]],
                np.float32).reshape(1, 1, 6, 3)


def test_cube_face_selection():
    # TextureTests.swift:78-101
    out = O.texture(CUBE, DIRS, boundaryMode="cube")
    assert out.shape == (1, 1, 6, 1)
    np.testing.assert_array_equal(out.reshape(-1), [10, 20, 30, 40, 50, 60])


def test_cube_gradient_picks_one_face():
    # TextureTests.swift:104-113
    d = np.array([0, 1, 0], np.float32).reshape(1, 1, 1, 3)
    d_tex, d_dir, _, _ = O.texture_vjp(np.zeros_like(CUBE), d, np.ones((1, 1, 1, 1), np.float32),
                                       boundaryMode="cube")
    np.testing.assert_array_equal(d_tex.reshape(-1), [0, 0, 1, 0, 0, 0])
    np.testing.assert_array_equal(d_dir, 0)


def test_mip_shapes_and_means():
    # TextureTests.swift:137-161
    lv = O.textureConstructMip(np.arange(16, dtype=np.float32).reshape(1, 4, 4, 1))
    assert [l.shape for l in lv] == [(1, 4, 4, 1), (1, 2, 2, 1), (1, 1, 1, 1)]
    np.testing.assert_allclose(lv[1].reshape(-1)[0], 2.5, atol=1e-6)
    np.testing.assert_allclose(lv[2].item(), 7.5, atol=1e-6)
    lv = O.textureConstructMip(np.zeros((1, 8, 8, 1), np.float32), maxLevel=2)
    assert [l.shape for l in lv] == [(1, 8, 8, 1), (1, 4, 4, 1), (1, 2, 2, 1)]
    # odd dims stop the pyramid (Texture.swift:153)
    lv = O.textureConstructMip(np.zeros((1, 12, 8, 1), np.float32))
    assert [l.shape[1:3] for l in lv] == [(12, 8), (6, 4), (3, 2)]


TEX42 = (np.arange(32, dtype=np.float32) * 0.05).reshape(1, 4, 4, 2)
UV1 = np.array([0.42, 0.31], np.float32).reshape(1, 1, 1, 2)


def test_trilinear_at_lod0_is_bilinear():
    # TextureTests.swift:167-182
    da = np.full((1, 1, 1, 4), 1e-6, np.float32)
    b = O.texture(TEX42, UV1)
    t = O.texture(TEX42, UV1, uvDA=da, filterMode="linear-mipmap-linear")
    np.testing.assert_allclose(b, t, atol=1e-4)


def test_trilinear_at_max_lod_is_mean():
    # TextureTests.swift:187-196
    tex = np.ones((1, 4, 4, 1), np.float32)
    uv = np.array([0.5, 0.5], np.float32).reshape(1, 1, 1, 2)
    da = np.full((1, 1, 1, 4), 100, np.float32)
    np.testing.assert_allclose(O.texture(tex, uv, uvDA=da, filterMode="linear-mipmap-linear"),
                               1.0, atol=1e-6)


def test_nearest():
    # TextureTests.swift:215-244
    uv = np.array([0.3, 0.7], np.float32).reshape(1, 1, 1, 2)
    np.testing.assert_allclose(O.texture(T22, uv, filterMode="nearest").item(), 30, atol=1e-6)
    d_tex, d_uv, _, _ = O.texture_vjp(T22, uv, np.ones((1, 1, 1, 1), np.float32),
                                      filterMode="nearest")
    np.testing.assert_array_equal(d_tex.reshape(-1), [0, 0, 1, 0])
    np.testing.assert_array_equal(d_uv.reshape(-1), [0, 0])


def test_mip_nearest_equals_trilinear_at_integer_lod():
    # TextureTests.swift:251-268
    da = np.array([0.5, 0.0, 0.0, 0.5], np.float32).reshape(1, 1, 1, 4)
    t = O.texture(TEX42, UV1, uvDA=da, filterMode="linear-mipmap-linear")
    n = O.texture(TEX42, UV1, uvDA=da, filterMode="linear-mipmap-nearest")
    np.testing.assert_allclose(t, n, atol=1e-5)


def test_bias_map_equals_scaled_uvda():
    # TextureTests.swift:272-293
    uv = np.tile(UV1, (1, 2, 2, 1))
    da = np.tile(np.array([0.3, 0.1, 0.1, 0.3], np.float32), (1, 2, 2, 1))
    bm = np.array([0.5, -0.3, 1.0, -1.0], np.float32).reshape(1, 2, 2)
    a = O.texture(TEX42, uv, uvDA=da, filterMode="linear-mipmap-linear", mipLevelBiasMap=bm)
    s = O.texture(TEX42, uv, uvDA=(da * (2.0 ** bm)[..., None]).astype(np.float32),
                  filterMode="linear-mipmap-linear")
    np.testing.assert_allclose(a, s, atol=1e-5)


def test_scalar_bias_equals_scaled_uvda():
    # TextureTests.swift:298-315
    da = np.array([0.3, 0.1, 0.1, 0.3], np.float32).reshape(1, 1, 1, 4)
    a = O.texture(TEX42, UV1, uvDA=da, filterMode="linear-mipmap-linear", mipLevelBias=1.0)
    s = O.texture(TEX42, UV1, uvDA=da * 2, filterMode="linear-mipmap-linear")
    np.testing.assert_allclose(a, s, atol=1e-5)


def _fd(loss, x, eps=1e-3):
    g = np.zeros_like(x)
    flat = x.reshape(-1)
    for i in range(flat.size):
        xp = flat.copy(); xp[i] += eps
        xm = flat.copy(); xm[i] -= eps
        g.reshape(-1)[i] = (loss(xp.reshape(x.shape)) - loss(xm.reshape(x.shape))) / (2 * eps)
    return g


@pytest.mark.parametrize("target,boundary", [("tex", "wrap"), ("uv", "wrap"),
                                             ("tex", "clamp"), ("uv", "zero")])
def test_gradcheck_bilinear(target, boundary):
    # TextureTests.swift:117-131, 385-438
    rng = np.random.default_rng(0x7E27)
    tex = rng.normal(size=(1, 3, 3, 2)).astype(np.float32)
    uv = np.array([[[0.25 + 0.3 * pw, 0.30 + 0.25 * ph] for pw in range(2)] for ph in range(2)],
                  np.float32)[None]
    w = ((1 + np.arange(8) % 5) * 0.1).astype(np.float32).reshape(1, 2, 2, 2)
    loss = lambda t, u: (O.texture(t, u, boundaryMode=boundary).astype(np.float64) * w).sum()
    d_tex, d_uv, _, _ = O.texture_vjp(tex, uv, w, boundaryMode=boundary)
    if target == "tex":
        np.testing.assert_allclose(d_tex, _fd(lambda x: loss(x, uv), tex), atol=5e-3)
    else:
        np.testing.assert_allclose(d_uv, _fd(lambda x: loss(tex, x), uv), atol=5e-3)


@pytest.mark.parametrize("target", ["tex", "uv", "uvDA", "biasMap"])
def test_gradcheck_trilinear(target):
    # TextureTests.swift:200-210, 317-379 (biasMap: the MLX-op fold, :109-121)
    rng = np.random.default_rng(0x71117EAB)
    tex = rng.normal(size=(1, 4, 4, 2)).astype(np.float32)
    uv = np.array([[[0.32 + 0.27 * pw, 0.41 + 0.23 * ph] for pw in range(2)] for ph in range(2)],
                  np.float32)[None]
    da = (0.4 + 0.05 * (np.arange(16) % 3)).astype(np.float32).reshape(1, 2, 2, 4)
    bm = np.array([0.1, -0.2, 0.15, 0.05], np.float32).reshape(1, 2, 2)
    w = ((1 + np.arange(8) % 5) * 0.1).astype(np.float32).reshape(1, 2, 2, 2)
    use_bm = target == "biasMap"

    def loss(t, u, d, m):
        return (O.texture(t, u, uvDA=d, filterMode="linear-mipmap-linear",
                          mipLevelBiasMap=m if use_bm else None).astype(np.float64) * w).sum()

    d_tex, d_uv, d_da, d_bm = O.texture_vjp(tex, uv, w, uvDA=da, filterMode="linear-mipmap-linear",
                                            mipLevelBiasMap=bm if use_bm else None)
    got, fd = {
        "tex": (d_tex, lambda: _fd(lambda x: loss(x, uv, da, bm), tex)),
        "uv": (d_uv, lambda: _fd(lambda x: loss(tex, x, da, bm), uv)),
        "uvDA": (d_da, lambda: _fd(lambda x: loss(tex, uv, x, bm), da)),
        "biasMap": (d_bm, lambda: _fd(lambda x: loss(tex, uv, da, x), bm)),
    }[target]
    np.testing.assert_allclose(got, fd(), atol=8e-3)


TEX8 = np.zeros((1, 8, 8, 3), np.float32)
for y in range(8):
    for x in range(8):
        TEX8[0, y, x] = [x / 7, y / 7, (x + y) / 14]


def test_nvdiffrast_fixture_bilinear(fixtures):
    # ParityTests.swift:92-100 (asserted by the reference), plus the
    # backward outputs the fixture holds (same texture conventions).
    uv = fixtures["uv"]
    out = O.texture(TEX8, uv, boundaryMode="clamp")
    assert np.abs(out - fixtures["tex_bilinear"]).max() <= 1e-5
    d_tex, d_uv, _, _ = O.texture_vjp(TEX8, uv, fixtures["co_tex"], boundaryMode="clamp")
    np.testing.assert_allclose(d_tex, fixtures["d_tex_from_bilinear"], rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(d_uv, fixtures["d_uv_from_bilinear"], rtol=1e-4, atol=1e-5)


def test_nvdiffrast_fixture_trilinear(fixtures):
    # ParityTests.swift:102-111; the fixture's uv_da is tiny (LOD clamps to 0)
    uv, da = fixtures["uv"], fixtures["uv_da"]
    out = O.texture(TEX8, uv, uvDA=da, filterMode="linear-mipmap-linear", boundaryMode="clamp")
    assert np.abs(out - fixtures["tex_trilinear"]).max() <= 1e-4
    d_tex, d_uv, d_da, _ = O.texture_vjp(TEX8, uv, fixtures["co_tex"], uvDA=da,
                                         filterMode="linear-mipmap-linear", boundaryMode="clamp")
    np.testing.assert_allclose(d_tex, fixtures["d_tex_from_trilinear"], rtol=1e-5, atol=1e-4)
    np.testing.assert_allclose(d_uv, fixtures["d_uv_from_trilinear"], rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(d_da, fixtures["d_uvDA_from_trilinear"], atol=1e-6)


def test_partition_of_unity_clamp():
    rng = np.random.default_rng(3)
    tex = rng.random((1, 16, 16, 3)).astype(np.float32)
    uv = rng.uniform(-0.2, 1.2, size=(1, 9, 11, 2)).astype(np.float32)
    g = rng.random((1, 9, 11, 3)).astype(np.float32)
    for fm, da in (("linear", None),
                   ("linear-mipmap-linear", rng.uniform(0, 0.3, size=(1, 9, 11, 4)).astype(np.float32))):
        d_tex, _, _, _ = O.texture_vjp(tex, uv, g, uvDA=da, filterMode=fm, boundaryMode="clamp")
        np.testing.assert_allclose(d_tex.sum(axis=(0, 1, 2)), g.sum(axis=(0, 1, 2)), rtol=1e-5)
