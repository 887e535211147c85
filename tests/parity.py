"""Shared helpers of the GPU parity tests.

Tolerances (the contract the HIP kernels are held to, versus the CPU
oracle on identical inputs):
  * integer / index outputs (tri_id, coverage, topology): bit-exact;
  * forward floats: |got - ref| <= 1e-5 * |ref| + 1e-6;
  * gradients accumulated by scatter-add (summation order differs):
    |got - ref| <= 1e-4 * |ref| + 1e-4 * max|ref|;
  * the mip filters' LOD-dependent gradients (d_uvDA, d_biasMap, the cube
    direction gradient) at the gradient tolerance; on pixels whose LOD sits
    on a switch (see lod_switch_mask), which must be rare, they must match
    the oracle on one side of the switch.
"""
import numpy as np
import pytest

FWD_RTOL, FWD_ATOL = 1e-5, 1e-6
GRAD_RTOL = 1e-4


def torch_dev():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("needs a ROCm GPU")
    return torch


def dev(x, dtype=None):
    import torch
    t = torch.as_tensor(np.ascontiguousarray(x))
    if dtype is not None:
        t = t.to(dtype)
    return t.cuda()


def host(t):
    return t.detach().cpu().numpy()


def assert_fwd_close(got, ref, what=""):
    np.testing.assert_allclose(got, ref, rtol=FWD_RTOL, atol=FWD_ATOL, err_msg=what)


def assert_grad_close(got, ref, what="", rtol=GRAD_RTOL):
    scale = float(np.abs(ref).max()) if np.size(ref) else 0.0
    np.testing.assert_allclose(got, ref, rtol=rtol, atol=rtol * scale + 1e-30, err_msg=what)


LOD_DELTA = 1e-5


def lod_switch_mask(ref, lo, hi, frac=0.25):
    """Pixels [N,H,W] whose oracle gradient jumps when the LOD moves by
    +-LOD_DELTA (lo / hi: the oracle's output with mipLevelBias lowered /
    raised by LOD_DELTA, which shifts the LOD by exactly that before the
    clamp).  These sit on a mip-level switch or at the ends of the LOD
    range where the reference zeroes d_uvDA (Texture.swift:1020-1024): a
    one-ulp difference between the CPU's and the GPU's log2 can move them
    to the other side.  A smooth dependence on the LOD moves an output by
    about LOD_DELTA relative, far below `frac` of the tolerance."""
    scale = float(np.abs(ref).max()) if np.size(ref) else 0.0
    d = np.abs(np.asarray(hi, np.float64) - np.asarray(lo, np.float64))
    if d.ndim > 3:
        d = d.reshape(d.shape[:3] + (-1,)).max(axis=-1)
    return d > frac * GRAD_RTOL * scale


def assert_grad_close_lod(got, ref, switch, lo, hi, what="", max_frac=0.01):
    """assert_grad_close on the pixels off a LOD switch.  A switch pixel
    (at most `max_frac` of all) must be finite and, over all its channels,
    match the oracle's value at the LOD it was evaluated at or at the LOD
    shifted by -+LOD_DELTA (`lo`, `hi`: the two sides of the switch), each at
    the gradient tolerance."""
    assert switch.mean() <= max_frac, f"{what}: {switch.mean():.4f} of pixels on a LOD switch"
    got = np.asarray(got)
    keep = ~switch
    scale = float(np.abs(ref).max()) if np.size(ref) else 0.0
    atol = GRAD_RTOL * scale + 1e-30
    np.testing.assert_allclose(got[keep], np.asarray(ref)[keep], rtol=GRAD_RTOL, atol=atol,
                               err_msg=what)
    g = got[switch].astype(np.float64)
    if g.size == 0:
        return
    assert np.isfinite(g).all(), f"{what}: non-finite gradient on a LOD switch pixel"
    ok = np.zeros(g.shape[:1], bool)
    for side in (ref, lo, hi):
        s = np.asarray(side, np.float64)[switch]
        close = np.abs(g - s) <= atol + GRAD_RTOL * np.abs(s)
        ok |= close.reshape(close.shape[0], -1).all(axis=1)
    assert ok.all(), (f"{what}: {(~ok).sum()} of {ok.size} LOD-switch pixels match neither "
                      "side of the switch")
