"""GPU parity of the K-quant dequantizer and batch-1 matvec against the CPU oracle.

Dequantization is bit-exact.  Matvec outputs match the oracle's QMatVec within
MV_RTOL (2e-5) times sum_i |w_i x_i| per output, through the reference ABI
(aspida_gpu_matvec, host pointers) and the device-pointer entry point, over
every kind, every launch layout, ragged row counts, one-super-block rows, the
benchmark shapes and scale fields holding +-0, subnormals, Inf and NaN.
"""
import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import synth
from gpu_helpers import abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev, torch_cuda

pytestmark = pytest.mark.gpu

KINDS = list(aa.KINDS)
NAME = {0: "q4k", 1: "q6k", 2: "q5k", 3: "q3k", 4: "q2k", 5: "q80"}


@pytest.fixture(scope="module")
def gpu():
    torch_cuda()
    g = aa.LLMGpu()
    yield g
    g.lib.aspida_kq_set_mv_config(0, 16)


@pytest.fixture(scope="module")
def dev():
    return aa.DeviceOps()


def _dequant_gpu(dev, kind, w, in_dim, out_dim):
    torch = torch_cuda()
    dw = to_dev(w)
    dst = torch.empty((out_dim, in_dim), dtype=torch.float32, device="cuda")
    dev.dequant(kind, dw.data_ptr(), in_dim, out_dim, dst.data_ptr(), stream())
    sync()
    return dst.cpu().numpy()


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_golden_bit_exact(kind, dev, golden):
    rnd = golden("kq_random.npz")
    blocks = rnd[f"{NAME[kind]}_blocks"]
    exp = rnd[f"{NAME[kind]}_expected"]
    got = _dequant_gpu(dev, kind, blocks.reshape(-1), 256, blocks.shape[0])
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
    kat = golden("kq_kat.npz")
    got = _dequant_gpu(dev, kind, kat[f"{NAME[kind]}_block"], 256, 1)[0]
    assert np.array_equal(got.view(np.uint32), kat[f"{NAME[kind]}_expected"].view(np.uint32))


@pytest.mark.parametrize("kind", KINDS)
def test_dequant_random_rows_bit_exact(kind, dev):
    gen = synth.rng(100 + kind)
    in_dim, out_dim = 2048, 96
    w = gen.integers(0, 256, aa.weight_bytes(kind, in_dim, out_dim), dtype=np.uint8)  # any f16 pattern
    got = _dequant_gpu(dev, kind, w, in_dim, out_dim)
    want = oracle.dequant(kind, w, in_dim, out_dim)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _check_mv(gpu, kind, out_dim, in_dim, seed, what, specials=False):
    gen = synth.rng(seed)
    if specials:
        w = gen.integers(0, 256, aa.weight_bytes(kind, in_dim, out_dim), dtype=np.uint8)
    else:
        w = synth.weight_np(kind, out_dim, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    y = gpu.matvec(w, kind, in_dim, out_dim, x)
    gpu.free_weight(w)
    want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
    scale = abs_dot_scale(kind, w, in_dim, out_dim, x)
    return assert_close_scaled(y, want, scale, what=what)


# Row lengths of 1..56 super-blocks exercise every stream shape: chunks of
# 16/8/4/2/1 super-blocks per wave, teams of 1..7 waves, idle lanes.
SMALL_SHAPES = [(1, 256), (3, 512), (67, 768), (130, 4096), (257, 2304), (33, 3328), (70, 8192),
                (41, 14336)]
CONFIGS = [(1, 16), (2, 16), (4, 16), (2, 4), (4, 64)]


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"R{c[0]}W{c[1]}")
@pytest.mark.parametrize("kind", KINDS)
def test_matvec_small_shapes_all_configs(kind, cfg, gpu):
    assert gpu.lib.aspida_kq_set_mv_config(*cfg) == 0
    try:
        for i, (out_dim, in_dim) in enumerate(SMALL_SHAPES):
            _check_mv(gpu, kind, out_dim, in_dim, 1000 * kind + i, f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")
    finally:
        gpu.lib.aspida_kq_set_mv_config(0, 16)


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_special_scales(kind, gpu):
    """Uniform random bytes everywhere: f16 scales include +-0, subnormals,
    Inf and NaN, which Aspida reads as +0.0."""
    _check_mv(gpu, kind, 64, 1024, 77 + kind, "specials", specials=True)


BENCH_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("shape", BENCH_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("kind", list(aa.KQUANTS))
def test_matvec_benchmark_shapes(kind, shape, gpu):
    out_dim, in_dim = shape
    r = _check_mv(gpu, kind, out_dim, in_dim, 5 + kind, f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")
    print(f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}: max |err| / sum|wx| = {r:.2e}")


def test_matvec_device_entry_point(dev):
    torch = torch_cuda()
    gen = synth.rng(21)
    kind, out_dim, in_dim = 0, 1000, 4096
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    dw, dx = to_dev(w), to_dev(x)
    dq = torch.empty(in_dim // 16, dtype=torch.float32, device="cuda")
    dy = torch.empty(out_dim, dtype=torch.float32, device="cuda")
    dev.xsum(dx.data_ptr(), in_dim, 1, dq.data_ptr(), stream())
    dev.matvec(kind, dw.data_ptr(), in_dim, out_dim, dx.data_ptr(), dq.data_ptr(), dy.data_ptr(), stream())
    sync()
    want = oracle.qmatvec(kind, w, in_dim, out_dim, x)
    assert_close_scaled(dy.cpu().numpy(), want, abs_dot_scale(kind, w, in_dim, out_dim, x), what="dev")
    # the group sums the kernels use are plain ascending sums of 16
    xq = x.reshape(-1, 16).astype(np.float64).sum(1)
    assert np.allclose(dq.cpu().numpy(), xq, rtol=1e-6, atol=1e-6)


def test_kind5_runs_q8_0_not_q2_k(gpu):
    """The reference sent kind 5 to its Q2_K kernel (gpu_matvec.cu:517)."""
    _check_mv(gpu, 5, 50, 1024, 31, "Q8_0 via kind 5")


def test_weight_cache_refresh_after_free(gpu):
    gen = synth.rng(41)
    kind, out_dim, in_dim = 0, 32, 512
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    y1 = gpu.matvec(w, kind, in_dim, out_dim, x)
    w[:] = synth.weight_np(kind, out_dim, in_dim, gen)   # same host address, new bytes
    y_stale = gpu.matvec(w, kind, in_dim, out_dim, x)    # served from the HBM mirror
    assert np.array_equal(y1, y_stale)
    gpu.free_weight(w)
    gpu.free_weight(w)                                   # idempotent
    y2 = gpu.matvec(w, kind, in_dim, out_dim, x)
    want = oracle.qmatvec(kind, w, in_dim, out_dim, x)
    assert_close_scaled(y2, want, abs_dot_scale(kind, w, in_dim, out_dim, x), what="after free")
    gpu.free_weight(w)


def test_errors_leave_nan_and_code(gpu):
    gpu.last_error()
    y = gpu.matvec(np.zeros(144, np.uint8), 0, 256, 4, np.ones(256, np.float32))
    assert np.all(np.isnan(y)) and gpu.last_error() != 0
    assert gpu.last_error() == 0
