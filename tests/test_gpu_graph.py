"""HIP graph capture of whole steps (torch.cuda.graph over the op wrappers,
which call the C ABI on the capturing stream).  Once every call has run on
the capturing stream, a captured step allocates nothing and waits for
nothing, and every replay equals the eager step: the forward outputs and
the loss bit for bit, the gradients within the gradient tolerance (d_attr
and d_pos are scatter-added across workgroups in an order that varies from
run to run, eager or replayed), for the tier-1 colour fit (rasterize ->
interpolate -> MSE -> d_attr) and the hex-pie chain with antialias (-> d_pos
and d_attr).
Replays alternate with eager steps and host synchronisation.  A call that
would allocate or wait while its stream is captured is refused with
DR_ERR_CAPTURE, and dr_rasterize_reserve spares the first forward its
wait."""
import numpy as np
import pytest

import scenes
from parity import assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu


def _mse(out, target, loss):
    import torch
    import diffrast._lib as L
    from diffrast.ops import _stream
    d_out = torch.empty_like(out)
    L.check(L.load().dr_mse_loss(out.data_ptr(), target.data_ptr(), out.numel(), loss.data_ptr(),
                                 d_out.data_ptr(), _stream()))
    out.backward(d_out)


def _tier1():
    import torch
    from diffrast import DiffRast
    sc = scenes.tier1_triangle(H=256, W=256)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    attr = dev(sc["attr"]).requires_grad_(True)
    r, _ = DiffRast.rasterize(pos, tri, (256, 256), gradDB=False)
    target = DiffRast.interpolate(dev(sc["target_attr"]), r, tri)[0].detach()
    loss = torch.zeros((), device="cuda")

    def step():
        attr.grad = None
        rast, _ = DiffRast.rasterize(pos, tri, (256, 256), gradDB=False)
        out, _ = DiffRast.interpolate(attr, rast, tri)
        _mse(out, target, loss)
        return {"rast": rast, "out": out, "loss": loss, "d_attr": attr.grad}
    return step


def _hexpie():
    import torch
    from diffrast import DiffRast
    sc = scenes.hex_pie(N=4, H=512, W=512)
    pos = dev(sc["pos"]).requires_grad_(True)
    attr = dev(sc["attr"]).requires_grad_(True)
    tri = dev(sc["tri"])
    target = dev(sc["target"])
    topo = DiffRast.antialiasConstructTopologyHash(tri)
    loss = torch.zeros((), device="cuda")

    def step():
        pos.grad = attr.grad = None
        rast, _ = DiffRast.rasterize(pos, tri, (512, 512), gradDB=False)
        col, _ = DiffRast.interpolate(attr, rast, tri)
        out = DiffRast.antialias(col, rast, pos, tri, topologyHash=topo)
        _mse(out, target, loss)
        return {"rast": rast, "out": out, "loss": loss, "d_pos": pos.grad, "d_attr": attr.grad}
    return step


def ctypes_stream(s):
    import ctypes
    return ctypes.c_void_p(s.cuda_stream)


def _snapshot(res):
    return {k: host(v).copy() for k, v in res.items()}


@pytest.mark.parametrize("scene", ["tier1", "hexpie"])
def test_graph_replay_matches_eager(scene):
    torch = torch_dev()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        step = _tier1() if scene == "tier1" else _hexpie()
        for _ in range(3):  # every call once on the capturing stream: scratch sized
            step()
        s.synchronize()
        ref = _snapshot(step())
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=s):
            static = step()
        for rep in range(3):
            g.replay()
            s.synchronize()
            got = _snapshot(static)
            for k in ("rast", "out", "loss"):
                np.testing.assert_array_equal(got[k], ref[k], err_msg=f"{k} replay {rep}")
            for k in ("d_attr", "d_pos"):
                if k in ref:
                    assert_grad_close(got[k], ref[k], f"{k} replay {rep}")
            eager = _snapshot(step())  # eager work between replays
            np.testing.assert_array_equal(eager["out"], ref["out"])
            s.synchronize()


def test_capture_refuses_allocation():
    """On a stream the library has not seen, the first rasterize would
    allocate its scratch and count its tiles: under capture it is refused
    with DR_ERR_CAPTURE and nothing is launched."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _ptr
    lib = L.load()
    sc = scenes.tier1_triangle(H=64, W=64)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    rast = torch.empty((1, 64, 64, 4), device="cuda")
    s = torch.cuda.Stream()
    g = torch.cuda.CUDAGraph()
    rc = None
    with torch.cuda.stream(s):
        g.capture_begin()
        try:
            rast.zero_()  # the graph is not empty
            rc = lib.dr_rasterize_fwd(_ptr(pos), 3 * 4, _ptr(tri), None, None, 1, 3, 1, 64, 64,
                                      _ptr(rast), None, ctypes_stream(s))
        finally:
            g.capture_end()
    assert rc == L.DR_ERR_CAPTURE
    assert b"captured into a HIP graph" in lib.dr_get_last_error()


def test_reserve_spares_the_first_wait():
    """After dr_rasterize_reserve on a fresh stream, the first forward
    returns while work queued before it still runs (no tile count is waited
    for), and its output equals an unreserved stream's."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast import DiffRast
    lib = L.load()
    sc = scenes.textured_icosphere(N=2, H=128, W=128, level=4, tex_size=8)
    pos, tri = dev(sc["pos"]), dev(sc["tri"])
    ref, _ = DiffRast.rasterize(pos, tri, (128, 128))
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    with torch.cuda.stream(s):
        V, T = sc["pos"].shape[1], sc["tri"].shape[0]
        L.check(lib.dr_rasterize_reserve(2, V, T, 128, 128, 64, ctypes_stream(s)))
        out = torch.empty_like(ref)  # torch's block allocated before the timed call
        db = torch.empty_like(ref)
        s.synchronize()
        torch.cuda._sleep(200_000_000)  # ~0.1 s of spinning on the stream
        from diffrast.ops import _ptr
        L.check(lib.dr_rasterize_fwd(_ptr(pos), V * 4, _ptr(tri), None, None, 2, V, T, 128, 128,
                                     _ptr(out), _ptr(db), ctypes_stream(s)))
        waited = s.query()
        s.synchronize()
    assert not waited
    np.testing.assert_array_equal(host(out), host(ref))
