"""Out-of-range indices never send a kernel out of range: a triangle with a
vertex id outside [0, V) is not drawn and gets no gradient (rasterize,
interpolate, antialias and their backward passes); a rast whose triangle
ids lie outside [0, T) reads as empty in interpolate and the backward passes;
a diff_idx entry outside [0, A) gives zero derivatives.  (The reference
reads out of range in these cases; these are the library's declared
semantics.)"""
import numpy as np
import pytest

import oracle as O
import scenes
from parity import assert_fwd_close, assert_grad_close, dev, host, torch_dev

pytestmark = pytest.mark.gpu


def _scene():
    sc = scenes.hex_pie(N=2, H=64, W=80)
    return sc["pos"], sc["tri"], 64, 80


def test_rasterize_skips_triangles_with_foreign_vertices():
    torch = torch_dev()
    from diffrast import DiffRast
    pos, tri, H, W = _scene()
    V = pos.shape[1]
    bad, fixed = tri.copy(), tri.copy()
    bad[1] = [0, V + 5, 2]
    bad[3] = [-7, 1, 2]
    fixed[[1, 3]] = 0  # degenerate: zero area, not drawn
    p = dev(pos).requires_grad_(True)
    r, db = DiffRast.rasterize(p, dev(bad), (H, W), gradDB=True)
    rr, rdb = O.rasterize(pos, fixed, (H, W), gradDB=True, max_per_tile=0)
    np.testing.assert_array_equal(host(r), rr)
    np.testing.assert_array_equal(host(db), rdb)
    rng = np.random.default_rng(2)
    g = rng.normal(size=rr.shape).astype(np.float32)
    (r * dev(g)).sum().backward()
    ref = O.rasterize_vjp(pos, fixed, rr, g, None)
    assert_grad_close(host(p.grad), ref, "d_pos")


def test_interpolate_foreign_ids_read_as_empty():
    torch = torch_dev()
    from diffrast import DiffRast
    pos, tri, H, W = _scene()
    V, T = pos.shape[1], tri.shape[0]
    rng = np.random.default_rng(3)
    rast, db = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    attr = rng.normal(size=(V, 3)).astype(np.float32)
    sel = rng.random(rast.shape[:3]) < 0.3
    foreign = rast.copy()
    foreign[..., 3][sel] = T + 1 + rng.integers(0, 1000, size=int(sel.sum()))
    emptied = rast.copy()
    emptied[sel] = 0.0
    outs = []
    for r in (foreign, emptied):
        a = dev(attr).requires_grad_(True)
        rd = dev(r).requires_grad_(True)
        dbd = dev(db).requires_grad_(True)
        out, out_da = DiffRast.interpolate(a, rd, dev(tri), rastDB=dbd, diffAttrs="all")
        g = np.random.default_rng(4).normal(size=tuple(out.shape)).astype(np.float32)
        gd = np.random.default_rng(5).normal(size=tuple(out_da.shape)).astype(np.float32)
        ((out * dev(g)).sum() + (out_da * dev(gd)).sum()).backward()
        outs.append([host(out), host(out_da), host(a.grad), host(rd.grad), host(dbd.grad)])
    np.testing.assert_array_equal(outs[0][0], outs[1][0])
    np.testing.assert_array_equal(outs[0][1], outs[1][1])
    assert_grad_close(outs[0][2], outs[1][2], "d_attr")
    np.testing.assert_array_equal(outs[0][3], outs[1][3])
    np.testing.assert_array_equal(outs[0][4], outs[1][4])


@pytest.mark.parametrize("A,diff", [(6, None), (3, "all"), (5, None)])
def test_interpolate_foreign_vertex_ids_read_as_empty(A, diff):
    """Pixels of a triangle with a vertex id outside [0, V) interpolate to
    zero and add no gradient, whatever shares their wave (the forward reads
    every slot's vertex rows before checking any)."""
    torch = torch_dev()
    from diffrast import DiffRast
    pos, tri, H, W = _scene()
    V, T = pos.shape[1], tri.shape[0]
    rast, db = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    bad = tri.copy()
    bad[1] = [0, V + 5, 2]
    bad[3] = [-7, 1, 2]
    ids = rast[..., 3].astype(np.int64) - 1
    emptied, db_e = rast.copy(), db.copy()
    hit = (ids == 1) | (ids == 3)
    assert hit.any() and (~hit & (ids >= 0)).any()
    emptied[hit] = 0.0
    rng = np.random.default_rng(6 + A)
    attr = rng.normal(size=(V, A)).astype(np.float32)
    a = dev(attr).requires_grad_(True)
    rd = dev(rast).requires_grad_(True)
    dbd = dev(db).requires_grad_(True)
    out, out_da = DiffRast.interpolate(a, rd, dev(bad), rastDB=dbd if diff else None,
                                       diffAttrs=diff)
    ro, rda = O.interpolate(attr, emptied, tri, rastDB=db_e if diff else None, diffAttrs=diff)
    np.testing.assert_array_equal(host(out), ro)
    if diff:
        np.testing.assert_array_equal(host(out_da), rda)
    g = rng.normal(size=ro.shape).astype(np.float32)
    loss = (out * dev(g)).sum()
    gda = None
    if diff:
        gda = rng.normal(size=rda.shape).astype(np.float32)
        loss = loss + (out_da * dev(gda)).sum()
    loss.backward()
    d_attr, d_rast, _ = O.interpolate_vjp(attr, emptied, tri, g, rastDB=db_e if diff else None,
                                          diffAttrs=diff, d_out_da=gda)
    assert_grad_close(host(a.grad), d_attr, "d_attr")
    assert_fwd_close(host(rd.grad), d_rast, "d_rast")


def test_interpolate_diff_idx_out_of_range():
    torch = torch_dev()
    from diffrast import DiffRast
    import diffrast._lib as L
    from diffrast.ops import _ptr, _stream
    lib = L.load()
    pos, tri, H, W = _scene()
    V, T = pos.shape[1], tri.shape[0]
    N = pos.shape[0]
    rng = np.random.default_rng(6)
    rast, db = O.rasterize(pos, tri, (H, W), gradDB=True, max_per_tile=0)
    attr = rng.normal(size=(V, 3)).astype(np.float32)
    idx = np.array([2, 7, -1, 0], np.int32)  # entries 1 and 2 name no attribute
    ad, rd, dbd, td, idd = dev(attr), dev(rast), dev(db), dev(tri), dev(idx)
    out = torch.empty((N, H, W, 3), device="cuda")
    out_da = torch.empty((N, H, W, 8), device="cuda")
    L.check(lib.dr_interpolate_fwd(_ptr(ad), 0, _ptr(rd), _ptr(dbd), _ptr(td), _ptr(idd), 4, N, H,
                                   W, V, T, 3, _ptr(out), _ptr(out_da), _stream()))
    _, ref_da = O.interpolate(attr, rast, tri, rastDB=db, diffAttrs=[2, 0])
    got = host(out_da)
    assert_fwd_close(got[..., [0, 1, 6, 7]], ref_da)
    assert (got[..., 2:6] == 0).all()


def test_antialias_triangle_with_foreign_vertex():
    """Never blends, and the gradients stay finite."""
    torch = torch_dev()
    from diffrast import DiffRast
    pos, tri, H, W = _scene()
    V = pos.shape[1]
    bad = tri.copy()
    bad[1] = [0, V + 5, 2]
    rng = np.random.default_rng(7)
    p = dev(pos).requires_grad_(True)
    r, _ = DiffRast.rasterize(p, dev(bad), (H, W), gradDB=False)
    color = dev(rng.random((pos.shape[0], H, W, 4)).astype(np.float32)).requires_grad_(True)
    out = DiffRast.antialias(color, r, p, dev(bad))
    out.backward(dev(rng.normal(size=tuple(out.shape)).astype(np.float32)))
    assert np.isfinite(host(out)).all()
    assert np.isfinite(host(color.grad)).all() and np.isfinite(host(p.grad)).all()


def test_triangle_count_above_32bit_indexing_is_refused():
    """tri is indexed as t * 3 + k in 32 bits: a call with more than
    715,827,882 triangles is refused before any work is queued (the tensors
    here are small; nothing reads them)."""
    torch = torch_dev()
    import diffrast._lib as L
    from diffrast.ops import _stream
    lib = L.load()
    T = 715827883
    buf = torch.zeros(64, device="cuda")
    itri = torch.zeros(64, dtype=torch.int32, device="cuda")
    p, t = buf.data_ptr(), itri.data_ptr()
    rc = lib.dr_rasterize_fwd(p, 12, t, None, None, 1, 3, T, 8, 8, p, None, _stream())
    assert rc == L.DR_ERR_ARGUMENT and b"715827882" in lib.dr_get_last_error()
    rc = lib.dr_interpolate_fwd(p, 0, p, None, t, None, 0, 1, 8, 8, 3, T, 1, p, None, _stream())
    assert rc == L.DR_ERR_ARGUMENT and b"715827882" in lib.dr_get_last_error()
    rc = lib.dr_antialias_topology(t, T, t, _stream())
    assert rc == L.DR_ERR_ARGUMENT and b"715827882" in lib.dr_get_last_error()
    rc = lib.dr_antialias_fwd(p, p, p, t, t, 1, 8, 8, 1, 3, T, p, _stream())
    assert rc == L.DR_ERR_ARGUMENT and b"715827882" in lib.dr_get_last_error()
    torch.cuda.synchronize()
