"""interpolate on the GPU against the CPU oracle: forward (basic and DA)
bit-exact, d_rast / d_rast_db bit-exact (no scatter), d_attr within the
scatter-add tolerance.  Instanced, shared [V,A] and [1,V,A] attributes,
.all and .indices, empty pixels, ragged sizes."""
import numpy as np
import pytest

import oracle as O
import scenes
from parity import assert_fwd_close, assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu


def scene(kind, rng):
    if kind == "icosphere":
        sc = scenes.textured_icosphere(N=2, H=256, W=320, level=4, tex_size=8)
        pos, tri, H, W = sc["pos"], sc["tri"], 256, 320
    elif kind == "hexpie":
        sc = scenes.hex_pie(N=3, H=77, W=131)
        pos, tri, H, W = sc["pos"], sc["tri"], 77, 131
    else:  # 2,048 tiles on 7 vertices: d_attr summed through its copies
        sc = scenes.hex_pie(N=2, H=512, W=512)
        pos, tri, H, W = sc["pos"], sc["tri"], 512, 512
    rast, db = O.rasterize(pos, tri, (H, W), max_per_tile=0)
    return pos, tri, rast, db


@pytest.mark.parametrize("kind", ["icosphere", "hexpie", "hexpie512"])
@pytest.mark.parametrize("A,diff,layout", [
    (2, None, "inst"), (2, "all", "shared"), (3, None, "one"), (3, "all", "inst"),
    (4, [1, 3], "shared"), (6, None, "inst"), (5, "all", "one"), (5, [4, 0, 4], "inst")])
def test_interpolate(kind, A, diff, layout):
    torch = torch_dev()
    from diffrast import DiffRast
    rng = np.random.default_rng(A * 7 + len(kind))
    pos, tri, rast, db = scene(kind, rng)
    N, H, W, _ = rast.shape
    V = pos.shape[1]
    shape = {"inst": (N, V, A), "shared": (V, A), "one": (1, V, A)}[layout]
    attr = rng.normal(size=shape).astype(np.float32)
    a = dev(attr).requires_grad_(True)
    r = dev(rast).requires_grad_(True)
    d = dev(db).requires_grad_(True)
    out, out_da = DiffRast.interpolate(a, r, dev(tri), rastDB=d if diff else None, diffAttrs=diff)
    ro, rda = O.interpolate(attr, rast, tri, rastDB=db if diff else None, diffAttrs=diff)
    np.testing.assert_array_equal(host(out), ro)
    assert_fwd_close(host(out), ro)
    if diff:
        np.testing.assert_array_equal(host(out_da), rda)
    else:
        assert tuple(out_da.shape) == (N, H, W, 0)
    g = rng.normal(size=ro.shape).astype(np.float32)
    loss = (out * dev(g)).sum()
    gda = None
    if diff:
        gda = rng.normal(size=rda.shape).astype(np.float32)
        loss = loss + (out_da * dev(gda)).sum()
    loss.backward()
    d_attr, d_rast, d_db = O.interpolate_vjp(attr, rast, tri, g, rastDB=db if diff else None,
                                             diffAttrs=diff, d_out_da=gda)
    assert tuple(a.grad.shape) == attr.shape
    assert_grad_close(host(a.grad), d_attr, "d_attr")
    assert_fwd_close(host(r.grad), d_rast, "d_rast")
    if diff:
        assert_fwd_close(host(d.grad), d_db, "d_rast_db")


def test_empty_and_constant():
    torch_dev()
    from diffrast import DiffRast
    # InterpolateTests.swift:11-52
    attr = np.array([[i, i + 1, i + 2] for i in range(3)], np.float32)[None]
    rast = np.tile(np.array([0.25, 0.5, 0.0, 1.0], np.float32), (1, 2, 2, 1))
    out, _ = DiffRast.interpolate(dev(attr), dev(rast), dev(np.array([[0, 1, 2]], np.int32)))
    np.testing.assert_allclose(host(out).reshape(-1, 3), np.tile([1.25, 2.25, 3.25], (4, 1)),
                               atol=1e-6)
    rast = np.array([0, 0, 0, 0, 0, 0, 0, 1], np.float32).reshape(1, 1, 2, 4)
    out, _ = DiffRast.interpolate(dev(np.ones((1, 3, 2), np.float32)), dev(rast),
                                  dev(np.array([[0, 1, 2]], np.int32)))
    np.testing.assert_array_equal(host(out).reshape(-1), [0, 0, 1, 1])


def test_errors():
    torch_dev()
    from diffrast import DiffRast
    attr = dev(np.ones((1, 3, 2), np.float32))
    rast = dev(np.zeros((1, 2, 2, 4), np.float32))
    tri = dev(np.array([[0, 1, 2]], np.int32))
    with pytest.raises(ValueError):
        DiffRast.interpolate(attr, rast, tri, diffAttrs="all")
    with pytest.raises(ValueError):
        DiffRast.interpolate(attr, rast, tri, rastDB=rast, diffAttrs=[2])
    with pytest.raises(ValueError):
        DiffRast.interpolate(dev(np.ones((3, 3, 2), np.float32)), rast, tri)


def test_small_d_attr_copies_accumulate():
    """A d_attr of 7 shared rows over 2,048 tiles is summed through copies;
    DR_ACCUMULATE adds the call's sum to the buffer, and a second plain
    call overwrites it (the copies are left zero between calls)."""
    import ctypes
    torch = torch_dev()
    from diffrast import _lib
    lib = _lib.load()
    rng = np.random.default_rng(5)
    pos, tri, rast, db = scene("hexpie512", rng)
    N, H, W, _ = rast.shape
    V, A = pos.shape[1], 3
    attr = rng.normal(size=(V, A)).astype(np.float32)
    g = rng.normal(size=(N, H, W, A)).astype(np.float32)
    ref, _, _ = O.interpolate_vjp(attr, rast, tri, g)
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    ta, tr, tt, tg = dev(attr), dev(rast), dev(tri), dev(g)
    d_attr = torch.full((V, A), 1.5, device="cuda")
    d_rast = torch.empty_like(tr)
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    run = lambda fl: _lib.check(lib.dr_interpolate_bwd(
        p(ta), 0, p(tr), None, p(tt), None, 0, p(tg), None, N, H, W, V, tri.shape[0], A,
        p(d_attr), 0, p(d_rast), None, fl, st))
    run(1)  # accumulate onto 1.5
    assert_grad_close(host(d_attr) - 1.5, ref, "accumulated d_attr")
    run(0)
    assert_grad_close(host(d_attr), ref, "d_attr after the accumulate call")
    run(0)
    assert_grad_close(host(d_attr), ref, "d_attr, second plain call")
