"""Shared helpers for the GPU tests (device memory comes from torch: plumbing)."""
import os

import numpy as np

import oracle

# Relative tolerance of a GPU dot product against the oracle, scaled by
# sum_i |w_i x_i| of that output.  Both sides accumulate in f32 in different
# orders; the bar the hot path must meet is 1e-3.
MV_RTOL = 2e-5
# The batch-1 MFMA kernel against the oracle: the matrix cores' sums lose bits
# when one product dwarfs the others (measured ~3e-5 of sum |w x| with 1e4x
# outliers in a column), so activations with such outliers get this bound;
# still 10x inside the 1e-3 bar.
MFMA_RTOL = 1e-4


def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        raise RuntimeError("GPU tests need a visible GPU (torch.cuda.is_available() is False)")
    return torch


def to_dev(a):
    torch = torch_cuda()
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def stream():
    return torch_cuda().cuda.current_stream().cuda_stream


def sync():
    torch_cuda().cuda.synchronize()


def ncpu():
    return max(1, min(16, os.cpu_count() or 1))


def abs_dot_scale(kind, w, in_dim, out_dim, x):
    """sum_i |w_i x_i| per output row (float64), from the oracle's dequant."""
    W = oracle.dequant(kind, w, in_dim, out_dim)
    return np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64))


def assert_close_scaled(got, want, scale, rtol=MV_RTOL, what=""):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    bound = rtol * scale + 1e-30
    bad = np.nonzero(~(err <= bound))[0]
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size} outputs off; first [{i}] got {got[i]!r} want {want[i]!r} "
                             f"err {err[i]:.3e} bound {bound[i]:.3e} (max err/scale "
                             f"{np.max(err / np.maximum(scale, 1e-30)):.3e})")
    return float(np.max(err / np.maximum(scale, 1e-30))) if scale.size else 0.0
