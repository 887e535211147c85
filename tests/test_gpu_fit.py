"""GPU: the loss and Adam kernels against the oracle, and the reference's
three inverse-rendering samples converging to the README's anchors
(README.md:69-75: colour fit 0.028 -> 0, pose fit 0.034 -> 0.0007, mesh
fit 0.034 -> 0.0002)."""
import numpy as np
import pytest

import oracle as O
from parity import dev, host, torch_dev

pytestmark = pytest.mark.gpu


def _call_mse(torch, out, target, with_grad=True):
    from diffrast import _lib
    lib = _lib.load()
    loss = torch.empty((), device=out.device, dtype=torch.float32)
    d = torch.empty_like(out) if with_grad else None
    _lib.check(lib.dr_mse_loss(out.data_ptr(), target.data_ptr(), out.numel(), loss.data_ptr(),
                               None if d is None else d.data_ptr(),
                               torch.cuda.current_stream().cuda_stream))
    return loss, d


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (4096, 0), (4096, 1), (1000003, 0),
                                      (1000003, 3)])
def test_mse_loss_kernel(n, offset):
    torch = torch_dev()
    rng = np.random.default_rng(n + offset)
    a = rng.random(n + offset, dtype=np.float32)
    b = rng.random(n + offset, dtype=np.float32)
    ta, tb = dev(a)[offset:], dev(b)[offset:]       # offset: unaligned (scalar path)
    loss, d = _call_mse(torch, ta, tb)
    ref_loss, ref_d = O.mse_loss(a[offset:], b[offset:])
    assert abs(float(loss) - float(ref_loss)) <= 1e-6 * float(ref_loss)
    assert np.array_equal(host(d), ref_d)           # elementwise: bit-exact
    # the loss alone, and the same value again (fixed summation order)
    loss2, _ = _call_mse(torch, ta, tb, with_grad=False)
    assert float(loss2) == float(loss)


def test_mse_loss_autograd():
    torch = torch_dev()
    from diffrast.fit import mse_loss
    rng = np.random.default_rng(5)
    a = dev(rng.random((2, 8, 8, 3), dtype=np.float32)).requires_grad_(True)
    b = dev(rng.random((2, 8, 8, 3), dtype=np.float32))
    loss = mse_loss(a, b)
    (3.0 * loss).backward()
    ref = 3.0 * 2.0 * (host(a).astype(np.float64) - host(b)) / a.numel()
    np.testing.assert_allclose(host(a.grad), ref, rtol=1e-6, atol=1e-12)
    with pytest.raises(ValueError):
        mse_loss(a, b[:1])


@pytest.mark.parametrize("n,masked", [(1, False), (4099, False), (4099, True), (300000, True)])
def test_adam_kernel_bit_exact(n, masked):
    torch = torch_dev()
    from diffrast.fit import Adam
    rng = np.random.default_rng(n)
    p = rng.standard_normal(n).astype(np.float32)
    mask = (rng.random(n) < 0.5).astype(np.float32) if masked else None
    opt = Adam((n,), learningRate=0.015)
    tp = dev(p)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    for t in range(1, 6):
        g = (rng.standard_normal(n) * 10.0 ** (t % 3 - 1)).astype(np.float32)
        tp = opt.step(tp, dev(g), None if mask is None else dev(mask))
        p, m, v = O.adam_step(p, g, m, v, t, lr=0.015, mask=mask)
        assert np.array_equal(host(tp), p), f"step {t}"
        assert np.array_equal(host(opt.m), m) and np.array_equal(host(opt.v), v)


def test_adam_in_place():
    torch = torch_dev()
    from diffrast import _lib
    lib = _lib.load()
    rng = np.random.default_rng(9)
    p = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    tp, tg = dev(p), dev(g)
    tm, tv = torch.zeros_like(tp), torch.zeros_like(tp)
    s = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.dr_adam_step(tp.data_ptr(), tg.data_ptr(), None, tm.data_ptr(), tv.data_ptr(),
                                tp.data_ptr(), 1000, 1, 0.01, 0.9, 0.999, 1e-8, s))
    ref, _, _ = O.adam_step(p, g, np.zeros_like(p), np.zeros_like(p), 1, lr=0.01)
    assert np.array_equal(host(tp), ref)
    assert lib.dr_adam_step(tp.data_ptr(), tg.data_ptr(), None, tm.data_ptr(), tv.data_ptr(),
                            tp.data_ptr(), 1000, 0, 0.01, 0.9, 0.999, 1e-8, s) == \
        _lib.DR_ERR_ARGUMENT


def _oracle_first_loss(sc):
    """The sample's first loss from the oracle's renders of the same scene."""
    tri, S = host(sc.tri), sc.size

    def render(param):
        if sc.kind == "color":
            rast, _ = O.rasterize(host(sc.pos), tri, (S, S), gradDB=False)
            return O.interpolate(param, rast, tri)[0]
        rast, _ = O.rasterize(param, tri, (S, S), gradDB=False)
        col, _ = O.interpolate(host(sc.attr), rast, tri)
        return O.antialias(col, rast, param, tri)

    loss, _ = O.mse_loss(render(host(sc.init)), render(host(sc.target)))
    return float(loss)


# README.md:73-75: (first loss, final loss).  The mesh sample's quoted first
# loss (0.034) is not what MeshFitExample/main.swift renders as written
# (start radius 0.42 at (0.13, -0.09), 96x96): the oracle gives 0.0484, so
# that sample's first loss is checked against the oracle only.
ANCHORS = {"color": (0.028, 1e-6), "pose": (0.034, 0.0007), "mesh": (None, 0.0002)}


@pytest.mark.parametrize("name", ["color", "pose", "mesh"])
def test_sample_converges(name):
    torch_dev()
    from diffrast import fit
    sc = getattr(fit, name + "_scene")()
    res = fit.run(sc)
    first, final = ANCHORS[name]
    print(f"{name}: first {res.losses[0]:.6f} final {res.losses[-1]:.6f}", flush=True)
    assert len(res.losses) == sc.steps and all(np.isfinite(res.losses))
    ref_first = _oracle_first_loss(sc)
    assert abs(res.losses[0] - ref_first) <= 1e-5 * ref_first
    if first is not None:
        # the README quotes rounded figures (pose: 0.0334 renders as 0.034)
        assert abs(res.losses[0] - first) <= 0.001
    # every gradient is order-independent (d_pos summed in fp64 across
    # workgroups), so each sample converges to one fixed final loss
    # (mesh: 0.000153 against the README's 0.0002)
    assert res.losses[-1] <= final
    if sc.kind == "pose":
        d = host(res.param - res.target)[0, :, :2]
        print(f"{name}: max vertex offset {np.abs(d).max():.4f} NDC", flush=True)
        assert np.abs(d).max() < 0.1
        # z and w are frozen by the gradient mask
        assert np.array_equal(host(res.param)[..., 2:], host(sc.init)[..., 2:])


def test_mesh_fit_is_deterministic():
    """d_pos (rasterize and antialias backward) is summed in fp64 across
    workgroups and rounded once, the loss in a fixed order and Adam
    elementwise: two runs of the mesh sample give the same losses and the
    same final vertices, bit for bit."""
    torch_dev()
    from diffrast import fit
    runs = [fit.run(fit.mesh_scene()) for _ in range(2)]
    print(f"mesh: final {runs[0].losses[-1]:.8f}", flush=True)
    assert runs[0].losses == runs[1].losses
    assert np.array_equal(host(runs[0].param), host(runs[1].param))


@pytest.mark.parametrize("name", ["color", "pose", "mesh"])
def test_graph_loop_matches_eager(name):
    """The samples' default loop replays one captured step (loss and
    gradient) and updates the parameter in place; the eager loop calls
    every op each step.  Same kernels on the same data: the pose samples'
    gradients are order-independent (fp64 sums), so their losses and
    final vertices agree bit for bit; the colour sample's d_attr is added in
    fp32 across workgroups in a varying order, so its losses agree to 1e-5."""
    torch_dev()
    from diffrast import fit
    sc = getattr(fit, name + "_scene")()
    eager = fit.run(sc, steps=40, graph=False)
    graph = fit.run(sc, steps=40, graph=True)
    print(f"{name}: eager {eager.losses[-1]:.8f} graph {graph.losses[-1]:.8f}", flush=True)
    if sc.kind == "pose":
        assert graph.losses == eager.losses
        assert np.array_equal(host(graph.param), host(eager.param))
    else:
        np.testing.assert_allclose(graph.losses, eager.losses, rtol=1e-5, atol=1e-9)
        np.testing.assert_allclose(host(graph.param), host(eager.param), rtol=1e-5, atol=1e-7)


def test_adam_step_in_place_matches_step():
    torch = torch_dev()
    from diffrast.fit import Adam
    rng = np.random.default_rng(3)
    p = dev(rng.standard_normal((1, 7, 4)).astype(np.float32))
    g = dev(rng.standard_normal((1, 7, 4)).astype(np.float32))
    mask = dev(np.tile(np.float32([1, 1, 0, 0]), 7).reshape(1, 7, 4))
    a, b = Adam(p.shape, learningRate=0.01), Adam(p.shape, learningRate=0.01)
    ref = a.step(p, g, mask)
    q = p.clone()
    b.step_(q, g, mask)
    assert np.array_equal(host(q), host(ref))
    assert b.t == a.t == 1
    with pytest.raises(ValueError):
        b.step_(q[..., :2].clone(), g[..., :2].clone())
