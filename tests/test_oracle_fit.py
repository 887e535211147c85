"""The oracle's loss and Adam step (the inverse-rendering samples' pieces),
pinned against closed forms and torch.optim.Adam.  CPU only."""
import numpy as np
import pytest

import oracle as O


def test_mse_closed_form():
    # constant difference c: loss c^2, gradient 2c/n everywhere
    n = 1 << 12
    out = np.full(n, 0.75, np.float32)
    tgt = np.full(n, 0.25, np.float32)
    loss, g = O.mse_loss(out, tgt)
    assert loss == np.float32(0.25)
    assert np.all(g == np.float32(2 * 0.5 / n))
    # sign: the gradient points from target to out
    loss, g = O.mse_loss(tgt, out)
    assert np.all(g == np.float32(-2 * 0.5 / n))


def test_mse_matches_float64_mean():
    rng = np.random.default_rng(3)
    a = rng.random((3, 17, 5), dtype=np.float32)
    b = rng.random((3, 17, 5), dtype=np.float32)
    loss, g = O.mse_loss(a, b)
    ref = np.mean((a.astype(np.float64) - b) ** 2)
    assert abs(float(loss) - ref) <= 1e-6 * ref
    np.testing.assert_allclose(g, 2.0 * (a.astype(np.float64) - b) / a.size, rtol=1e-6)
    assert g.shape == a.shape


def test_adam_first_step_is_signed_lr():
    # t = 1 from zero state: m_hat = g, v_hat = g^2, so the step is lr * sign(g)
    rng = np.random.default_rng(0)
    p = rng.standard_normal(257).astype(np.float32)
    g = rng.standard_normal(257).astype(np.float32)
    z = np.zeros_like(p)
    p1, m, v = O.adam_step(p, g, z, z, 1, lr=0.05)
    np.testing.assert_allclose(p1, p - 0.05 * np.sign(g), atol=2e-6)
    # (1 - beta) is taken in fp32, as the reference's Float arithmetic does
    np.testing.assert_allclose(m, (1.0 - float(np.float32(0.9))) * g.astype(np.float64), rtol=1e-6)
    np.testing.assert_allclose(v, (1.0 - float(np.float32(0.999))) * g.astype(np.float64) ** 2,
                               rtol=1e-6)


def test_adam_matches_torch_adam():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    p0 = rng.standard_normal(1000).astype(np.float32)
    tp = torch.tensor(p0, requires_grad=True)
    opt = torch.optim.Adam([tp], lr=0.015, betas=(0.9, 0.999), eps=1e-8)
    p, m, v = p0.copy(), np.zeros_like(p0), np.zeros_like(p0)
    for t in range(1, 31):
        g = rng.standard_normal(1000).astype(np.float32) * np.float32(10.0 ** (t % 3 - 1))
        tp.grad = torch.tensor(g)
        opt.step()
        p, m, v = O.adam_step(p, g, m, v, t, lr=0.015)
    np.testing.assert_allclose(p, tp.detach().numpy(), rtol=1e-5, atol=1e-6)


def test_adam_mask_freezes_components():
    rng = np.random.default_rng(2)
    p = rng.standard_normal((1, 4, 4)).astype(np.float32)
    g = rng.standard_normal((1, 4, 4)).astype(np.float32)
    mask = np.tile(np.array([1, 1, 0, 0], np.float32), 4).reshape(1, 4, 4)
    z = np.zeros_like(p)
    p1, m, v = O.adam_step(p, g, z, z, 1, lr=0.01, mask=mask)
    assert np.array_equal(p1[..., 2:], p[..., 2:])
    assert np.all(p1[..., :2] != p[..., :2])


def test_bias_correction_power_is_correctly_rounded():
    # beta^t rounded once to fp32 (float64 pow, then one rounding, agrees
    # away from ties); numpy's fp32 power differs at 0.9^4
    for b in (0.9, 0.999, 0.95):
        for t in range(1, 400):
            assert O._pow_f32(np.float32(b), t) == np.float32(float(np.float32(b)) ** t), (b, t)
    assert O._pow_f32(np.float32(0.9), 4) == np.float32(0.6560999)
