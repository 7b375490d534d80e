"""The allocation-free batch-1 matvec (aspida_kq_matvec_packed_noalloc_dev):
through the C ABI, its outputs equal aspida_kq_matvec_packed_dev's bit for
bit on the same inputs, on two calls in a row with the second smaller (the
fixed scratch keeps the first call's contents), for launch splits that use
the scratch (tiles split over workgroups: counters and partial sums) and one
that does not; the first call's result also matches the oracle.  Shapes
beyond the fixed scratch are refused with -E2BIG."""
import errno

import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import synth
from gpu_helpers import abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev, torch_cuda

pytestmark = pytest.mark.gpu

# (kind, first (out, in), second (out, in)): the second call is smaller.
CASES = [
    (aa.Q4_K, (1000, 14336), (64, 14336)),     # MFMA, 64-row tiles split over 14 and 28 workgroups
    (aa.Q6_K, (2048, 8192), (1000, 14336)),    # MFMA, split 8 then 14
    (aa.Q8_0, (2048, 8192), (300, 4096)),      # vector kernel, split 4 then 8
    (aa.Q4_K, (4096, 4096), (300, 4096)),      # 16-row workgroups: no scratch used
]


def _packed(dev, kind, out_dim, in_dim, gen):
    torch = torch_cuda()
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    p = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
    dev.pack(kind, to_dev(w).data_ptr(), in_dim, out_dim, p.data_ptr(), stream())
    return w, p


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{aa.KIND_NAMES[c[0]]}_{c[1][0]}x{c[1][1]}_then_{c[2][0]}x{c[2][1]}")
def test_noalloc_matches_matvec_packed(case):
    torch = torch_cuda()
    dev = aa.DeviceOps()
    lib = dev.lib
    kind, first, second = case
    gen = synth.rng(4242 + kind + first[0])
    for n, (out_dim, in_dim) in enumerate((first, second)):
        w, p = _packed(dev, kind, out_dim, in_dim, gen)
        x = synth.activations_np(in_dim, gen)
        dx = to_dev(x)
        y_ref = torch.full((out_dim,), float("nan"), device="cuda")
        y_na = torch.full((out_dim,), float("nan"), device="cuda")
        st = stream()
        assert lib.aspida_kq_matvec_packed_dev(kind, p.data_ptr(), in_dim, out_dim, dx.data_ptr(),
                                               y_ref.data_ptr(), st) == 0
        assert lib.aspida_kq_matvec_packed_noalloc_dev(kind, p.data_ptr(), in_dim, out_dim, dx.data_ptr(),
                                                       y_na.data_ptr(), st) == 0
        sync()
        a, b = y_ref.cpu().numpy(), y_na.cpu().numpy()
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), \
            f"call {n}: {aa.KIND_NAMES[kind]} {out_dim}x{in_dim} differs from aspida_kq_matvec_packed_dev"
        if n == 0:
            want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
            assert_close_scaled(b, want, abs_dot_scale(kind, w, in_dim, out_dim, x), what="noalloc vs oracle")


def test_noalloc_rejects_shapes_beyond_scratch():
    torch = torch_cuda()
    lib = aa.DeviceOps().lib
    p = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    x = torch.zeros(4096, device="cuda")
    y = torch.full((16,), 7.0, device="cuda")
    # 4097 64-row tiles of arrival counters: beyond the 4096 the scratch holds.
    assert lib.aspida_kq_matvec_packed_noalloc_dev(aa.Q4_K, p.data_ptr(), 4096, 4097 * 64, x.data_ptr(),
                                                   y.data_ptr(), stream()) == -errno.E2BIG
    assert aa.LLMGpu().last_error() == -errno.E2BIG
    assert lib.aspida_kq_matvec_packed_noalloc_dev(aa.Q4_K, p.data_ptr(), 300, 64, x.data_ptr(), y.data_ptr(),
                                                   stream()) == -errno.EINVAL
    sync()
    assert torch.all(y == 7.0)   # nothing launched
