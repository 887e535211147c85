"""Shared helpers of the GPU parity tests.

Tolerances (the contract the HIP kernels are held to, versus the CPU
oracle on identical inputs):
  * integer / index outputs (tri_id, coverage, topology): bit-exact;
  * forward floats: |got - ref| <= 1e-5 * |ref| + 1e-6;
  * gradients accumulated by scatter-add (summation order differs):
    |got - ref| <= 1e-4 * |ref| + 1e-4 * max|ref|.
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
