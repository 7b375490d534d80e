"""GPU parity of the small-batch product (aspida_gpu_matmul: the MFMA kernels
for Q4_K / Q6_K, the vector-ALU kernel for other kinds; and the packed-layout
device form), the dense f32 matvec, concurrent callers, and the reference's
own GPU test harness (gpu/test_matvec.cu, built into oracle/_ref/) run
against this library as a drop-in.  Products match the oracle's QMatMul
within 2e-5 of sum_i |w_i x_i| per output."""
import os
import subprocess
import threading

import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import synth
from gpu_helpers import abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev, torch_cuda

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    torch_cuda()
    return aa.LLMGpu()


def _batched_scale(kind, w, in_dim, out_dim, X):
    W = np.abs(oracle.dequant(kind, w, in_dim, out_dim)).astype(np.float64)
    return np.abs(X.astype(np.float64)) @ W.T


@pytest.mark.parametrize("batch", [1, 2, 3, 8, 33, 64])
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K])
def test_matmul_config_batches(kind, batch, gpu):
    gen = synth.rng(500 + batch + kind)
    out_dim, in_dim = 1536, 4096
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = gpu.matmul(w, kind, in_dim, out_dim, X)
    gpu.free_weight(w)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} B={batch}")


# BASELINE config 2 at its exact shapes: Q4_K and Q6_K weights of 4096 x 4096
# and 14336 x 4096 times B = 2 ... 64 activation vectors, on the library's
# default kernel pick (the same entry point and plans as bench.py's
# small_batch table).  The whole product runs on the GPU; 96 of its rows
# (the first and last 32 and 32 spread between) are checked against the
# oracle's QMatVec per vector.
CONFIG2_ROWS = 32


def _sample_rows(out_dim, gen):
    mid = np.sort(gen.choice(np.arange(CONFIG2_ROWS, out_dim - CONFIG2_ROWS), CONFIG2_ROWS, replace=False))
    return np.concatenate([np.arange(CONFIG2_ROWS), mid, np.arange(out_dim - CONFIG2_ROWS, out_dim)])


@pytest.mark.parametrize("batch", [2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("shape", [(4096, 4096), (14336, 4096)], ids=["4096x4096", "14336x4096"])
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K], ids=["Q4_K", "Q6_K"])
def test_config2_exact_shapes_default_pick(kind, shape, batch):
    out_dim, in_dim = shape
    gen = synth.rng(1200 + batch + out_dim // 1024 + 7 * kind)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    rows = _sample_rows(out_dim, gen)
    rb = aa.weight_bytes(kind, in_dim, 1)
    wr = np.ascontiguousarray(w.reshape(out_dim, rb)[rows]).ravel()
    want = oracle.qmatmul(kind, wr, in_dim, rows.size, X, nthreads=ncpu())
    scale = _batched_scale(kind, wr, in_dim, rows.size, X)
    assert np.all(np.isfinite(Y))
    assert_close_scaled(Y[:, rows].ravel(), want.ravel(), scale.ravel(),
                        what=f"config 2 {aa.KIND_NAMES[kind]} {out_dim}x{in_dim} B={batch}")


# Shapes whose launches pad the batch to fewer vectors than the whole batch
# (Q6_K in steps of 32, a tail of 1 or 16): the workspace must hold each
# launch's finer column split (Qwen2-1.5B down, Qwen2-7B o).
@pytest.mark.parametrize("case", [(aa.Q6_K, 8960, 1536, 48), (aa.Q4_K, 3584, 3584, 65), (aa.Q6_K, 3584, 3584, 48),
                                  (aa.Q4_K, 3584, 3584, 48)], ids=lambda c: f"{aa.KIND_NAMES[c[0]]}_{c[1]}to{c[2]}_B{c[3]}")
def test_matmul_launch_paddings(case, gpu):
    kind, in_dim, out_dim, batch = case
    gen = synth.rng(550 + batch + in_dim)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = gpu.matmul(w, kind, in_dim, out_dim, X)
    gpu.free_weight(w)
    assert gpu.last_error() == 0
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} {in_dim}->{out_dim} B={batch}")


@pytest.mark.parametrize("kind", list(aa.KINDS))
def test_matmul_all_kinds(kind, gpu):
    gen = synth.rng(600 + kind)
    out_dim, in_dim, batch = 75, 1024, 5
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = gpu.matmul(w, kind, in_dim, out_dim, X)
    gpu.free_weight(w)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X)
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=aa.KIND_NAMES[kind])


def _packed_matmul(kind, w, X, in_dim, out_dim):
    torch = torch_cuda()
    dev = aa.DeviceOps()
    dw, dx = to_dev(w), to_dev(np.ascontiguousarray(X, np.float32))
    dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
    dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
    dy = torch.full((X.shape[0], out_dim), float("nan"), device="cuda")
    dev.matmul_packed(kind, dp.data_ptr(), in_dim, out_dim, X.shape[0], dx.data_ptr(), dy.data_ptr(), stream())
    sync()
    return dy.cpu().numpy()


def _packed_rows(kind, w, X, in_dim, out_dim):
    """The batch-1 packed matvec of every row of X (same packed image) on the
    VALU kernel, whose sums the multi-vector kernel reproduces bit for bit
    (Q4_K and Q6_K run batch 1 on MFMA by default)."""
    torch = torch_cuda()
    dev = aa.DeviceOps()
    dw = to_dev(w)
    dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
    dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
    out = []
    dev.set_mv_engine(1)
    try:
        for b in range(X.shape[0]):
            dx = to_dev(np.ascontiguousarray(X[b], np.float32))
            dy = torch.full((out_dim,), float("nan"), device="cuda")
            dev.matvec_packed(kind, dp.data_ptr(), in_dim, out_dim, dx.data_ptr(), dy.data_ptr(), stream())
            sync()
            out.append(dy.cpu().numpy())
    finally:
        dev.set_mv_engine(0)
    return np.stack(out)


# Multi-vector VALU product (the small-batch engine of the kinds without an
# MFMA kernel; forced here for Q4_K/Q6_K too): rows bit-identical to the
# batch-1 VALU kernel.  Ragged weight rows, one super-block column, tiles
# split over workgroups (ks > 1), columns per wave > 1, batches of 8 and one
# beyond (two launches).
MULTI_CASES = [(2, 130, 768), (3, 1000, 4096), (4, 64, 14336), (5, 64, 14336), (8, 300, 256), (8, 4096, 4096),
               (11, 200, 1024)]


@pytest.mark.parametrize("case", MULTI_CASES, ids=lambda c: f"B{c[0]}_{c[1]}x{c[2]}")
@pytest.mark.parametrize("kind", list(aa.KINDS))
def test_multi_vector_rows_bit_identical_to_matvec(kind, case):
    batch, out_dim, in_dim = case
    gen = synth.rng(700 + batch + kind * 7 + out_dim)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    dev = aa.DeviceOps()
    dev.set_mm_engine(1)
    try:
        Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    finally:
        dev.set_mm_engine(0)
    R = _packed_rows(kind, w, X, in_dim, out_dim)
    assert np.array_equal(Y.view(np.uint32), R.view(np.uint32)), "rows differ from the batch-1 kernel"
    want = oracle.qmatvec(kind, w, in_dim, out_dim, X[-1], nthreads=ncpu())
    assert_close_scaled(Y[-1], want, abs_dot_scale(kind, w, in_dim, out_dim, X[-1]), what="last row")


@pytest.mark.parametrize("kind", [aa.Q5_K, aa.Q8_0])
def test_multi_vector_chunks_beyond_eight(kind):
    """Kinds without MFMA run batches above 8 as launches of 8."""
    batch, out_dim, in_dim = 19, 200, 512
    gen = synth.rng(811 + kind)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    R = _packed_rows(kind, w, X, in_dim, out_dim)
    assert np.array_equal(Y.view(np.uint32), R.view(np.uint32))


# MFMA product (Q4_K, Q6_K): one and several 16-row activation blocks, ragged
# batch sizes, more than 64 rows (two launches), ragged weight rows, one
# workgroup per tile and tiles split over workgroups.
MFMA_CASES = [(2, 130, 768), (16, 64, 4096), (17, 1000, 4096), (33, 67, 2304), (64, 4096, 4096),
              (65, 300, 1024), (100, 128, 14336)]


@pytest.mark.parametrize("case", MFMA_CASES, ids=lambda c: f"B{c[0]}_{c[1]}x{c[2]}")
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K])
def test_mfma_matmul_matches_oracle(kind, case):
    batch, out_dim, in_dim = case
    gen = synth.rng(900 + batch + kind + out_dim)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} B={batch} {out_dim}x{in_dim}")


# Every small-batch engine on the Q4_K product (aspida_kq_set_mm_engine: the
# vector kernel, the 64-vector and the 16-vector MFMA kernels): batches below,
# at and above 16 (two 16-vector launches, one ragged), ragged weight rows,
# one column per wave and long column runs, tiles split over workgroups.
MM_ENGINE_CASES = [(2, 130, 768), (5, 64, 4096), (16, 1000, 4096), (17, 67, 2304), (40, 4096, 4096),
                   (9, 16448, 2048), (3, 256, 14336), (20, 12352, 512), (64, 12352, 256), (63, 300, 1024),
                   (2, 13000, 256), (4, 12352, 512), (48, 12352, 512), (61, 13000, 256),
                   (5, 32768, 4096)]  # 8192 (tile, column) pairs: the pick's 16-vector kernel


# Engine 4 is the one-pass kernel (kq_mmv.hip): 64-row tiles from 12352 rows
# (193 tiles), 16-row blocks below; up to 64 vectors in one launch, up to 4
# converted through LDS.  Engine 5
# runs up to 4 vectors per launch on the batch-1 16-row kernels.  Engine 6 is
# the wave-per-column kernel (kq_mmw.hip) where in_dim is a multiple of 1024
# (columns split over waves, workgroups and, for 12352 rows at 4096, column
# groups), the vector kernel elsewhere.  Engine 0 is the library's pick.
@pytest.mark.parametrize("engine", [0, 1, 2, 3, 4, 5, 6])
@pytest.mark.parametrize("case", MM_ENGINE_CASES, ids=lambda c: f"B{c[0]}_{c[1]}x{c[2]}")
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K], ids=["Q4_K", "Q6_K"])
def test_mm_engines_match_oracle(kind, case, engine):
    batch, out_dim, in_dim = case
    gen = synth.rng(950 + batch + out_dim)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    dev = aa.DeviceOps()
    dev.set_mm_engine(engine)
    try:
        Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    finally:
        dev.set_mm_engine(0)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"engine {engine} B={batch} {out_dim}x{in_dim}")


# Columns whose largest |x| is below 2^-102 take the largest activation scale
# (2^116, so that the lo plane's factor S 2^11 stays finite): tiny and mixed
# magnitudes through the matrix-core small-batch engines (4 the one-pass
# kernel, 6 the wave-per-column kernel, 0 the pick), one 64-row tile
# (columns split over workgroups) and several.
@pytest.mark.parametrize("engine", [0, 4, 6])
@pytest.mark.parametrize("case", [(16, 64, 4096), (40, 4096, 4096), (64, 12352, 512)],
                         ids=lambda c: f"B{c[0]}_{c[1]}x{c[2]}")
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K], ids=["Q4_K", "Q6_K"])
def test_mm_engines_tiny_activations(kind, case, engine):
    batch, out_dim, in_dim = case
    gen = synth.rng(1300 + batch + out_dim)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    X[0] *= np.float32(1e-33)                       # every column of vector 0 below 2^-102
    X[1, :256] *= np.float32(1e-33)                 # one column of vector 1
    X[2, 256:512] *= np.float32(3e4)                 # a large column
    Y = _engine_matmul(engine, kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert np.all(np.isfinite(Y))
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"engine {engine} tiny B={batch} {out_dim}x{in_dim}")


def _engine_matmul(engine, kind, w, X, in_dim, out_dim):
    dev = aa.DeviceOps()
    dev.set_mm_engine(engine)
    try:
        return _packed_matmul(kind, w, X, in_dim, out_dim)
    finally:
        dev.set_mm_engine(0)


# Decimal exponents of each activation row's magnitude; None = an all-zero
# row.  Up to 4 rows the one-pass kernel converts through LDS (kq_mmv.hip's
# staged build), 9 rows in registers.
ROW_SCALES = [[-30, -12, -3, 0, 0, 3, 12, 30, None], [-30, None, 30, 3], [30, -30]]


@pytest.mark.parametrize("engine", [0, 4, 5])
@pytest.mark.parametrize("exps", ROW_SCALES, ids=lambda e: f"B{len(e)}")
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K])
def test_mfma_matmul_row_scales(kind, exps, engine):
    """Activation rows spanning 1e-30..1e30 in magnitude (each row is split
    with its own power-of-two scale) and all-zero rows."""
    gen = synth.rng(77 + kind + len(exps))
    batch, out_dim, in_dim = len(exps), 192, 1024
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    X *= (10.0 ** np.array([0 if e is None else e for e in exps]))[:, None].astype(np.float32)
    zero = [i for i, e in enumerate(exps) if e is None]
    X[zero] = 0.0
    Y = _engine_matmul(engine, kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} scaled rows")
    assert np.all(Y[zero] == 0.0)


@pytest.mark.parametrize("engine", [0, 4, 5])
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K])
def test_mfma_matmul_special_scales(kind, engine):
    """Raw random bytes everywhere: f16 scales include +-0, subnormals, Inf and
    NaN, which Aspida reads as +0.0."""
    gen = synth.rng(88 + kind)
    batch, out_dim, in_dim = 4, 64, 1024
    w = gen.integers(0, 256, aa.weight_bytes(kind, in_dim, out_dim), dtype=np.uint8)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _engine_matmul(engine, kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} specials")


@pytest.mark.parametrize("kind", [aa.Q5_K, aa.Q3_K, aa.Q2_K, aa.Q8_0])
def test_packed_matmul_other_kinds(kind):
    gen = synth.rng(300 + kind)
    batch, out_dim, in_dim = 3, 70, 2048
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=aa.KIND_NAMES[kind])


def test_matmul_rows_equal_matvec(gpu):
    """gpu/test_matvec.cu:152: batched == per-row to ~1e-4 relative."""
    gen = synth.rng(7)
    kind, out_dim, in_dim, batch = aa.Q4_K, 512, 2048, 4
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = gpu.matmul(w, kind, in_dim, out_dim, X)
    rows = np.stack([gpu.matvec(w, kind, in_dim, out_dim, X[b]) for b in range(batch)])
    gpu.free_weight(w)
    assert np.max(np.abs(Y - rows)) <= 1e-4 * np.max(np.abs(rows))


def test_dense_matvec(gpu):
    gen = synth.rng(8)
    for out_dim, in_dim in ((128, 2048), (7, 130), (1000, 4096)):
        W = (gen.standard_normal((out_dim, in_dim)) * 0.02).astype(np.float32)
        x = synth.activations_np(in_dim, gen)
        y = gpu.dense_matvec(W, x)
        gpu.free_weight(W)
        want = oracle.dense_matvec(W, x)
        scale = np.abs(W).astype(np.float64) @ np.abs(x.astype(np.float64))
        assert_close_scaled(y, want, scale, what=f"dense {out_dim}x{in_dim}")


def test_concurrent_callers(gpu):
    """Several host threads calling the ABI at once (the CPU-MoE path calls
    MatVec from LLM_Pool workers, llm_moe.adb:249-271)."""
    gen = synth.rng(9)
    cases = []
    for t in range(8):
        kind = list(aa.KQUANTS)[t % 5]
        out_dim, in_dim = 300 + 17 * t, 1024
        w = synth.weight_np(kind, out_dim, in_dim, gen)
        x = synth.activations_np(in_dim, gen)
        cases.append((kind, w, in_dim, out_dim, x))
    results = [None] * len(cases)

    def work(i):
        kind, w, in_dim, out_dim, x = cases[i]
        outs = [gpu.matvec(w, kind, in_dim, out_dim, x) for _ in range(20)]
        results[i] = outs

    threads = [threading.Thread(target=work, args=(i,)) for i in range(len(cases))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    for (kind, w, in_dim, out_dim, x), outs in zip(cases, results):
        want = oracle.qmatvec(kind, w, in_dim, out_dim, x)
        scale = abs_dot_scale(kind, w, in_dim, out_dim, x)
        for y in outs:
            assert_close_scaled(y, want, scale, what="threaded")
        gpu.free_weight(w)


def test_reference_harness_against_this_library():
    """Run the reference's own gpu/test_matvec.cu (host C++, compiled from the
    reference tree into oracle/_ref/) with libaspidagpu.so as its
    ./libaspidagpu.so: all five K-quants vs its fp64 CPU dequant-dot (rel <
    1e-2) and batched == per-row (rel < 1e-4)."""
    exe = os.path.join(os.path.dirname(oracle.__file__), "_ref", "test_matvec")
    if not os.path.exists(exe):
        pytest.skip("oracle/_ref/test_matvec absent: it is built only where the reference tree is mounted, and "
                    "no reference build output travels to a GPU box")
    torch_cuda()
    r = subprocess.run([exe], cwd=os.path.dirname(aa.LIB_PATH), capture_output=True, text=True, timeout=600)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "PASS" in r.stdout


@pytest.mark.parametrize("kind", [aa.Q6_K, aa.Q8_0], ids=["Q6_K", "Q8_0"])
def test_multi_vector_sixteen_wave_column_walk(kind):
    """Three vectors (the multi-vector kernel's range) over more than 255
    tiles with rows of 32 super-blocks: 16-wave workgroups walking two columns
    per wave without prefetching (the prefetching walk does not fit Q6_K's and
    Q8_0's registers at 16 waves)."""
    gen = synth.rng(1616 + kind)
    batch, out_dim, in_dim = 3, 16448, 8192
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    X = synth.activations_np(batch * in_dim, gen).reshape(batch, in_dim)
    Y = _packed_matmul(kind, w, X, in_dim, out_dim)
    want = oracle.qmatmul(kind, w, in_dim, out_dim, X, nthreads=ncpu())
    assert_close_scaled(Y.ravel(), want.ravel(), _batched_scale(kind, w, in_dim, out_dim, X).ravel(),
                        what=f"{aa.KIND_NAMES[kind]} B={batch} {out_dim}x{in_dim}")
