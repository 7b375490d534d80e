"""GPU parity of the small-batch product (aspida_gpu_matmul and its device
form), the dense f32 matvec, concurrent callers, and the reference's own GPU
test harness (gpu/test_matvec.cu, built into oracle/_ref/) run against this
library as a drop-in."""
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
        pytest.skip("oracle/_ref/test_matvec not built (reference tree absent at build time)")
    torch_cuda()
    r = subprocess.run([exe], cwd=os.path.dirname(aa.LIB_PATH), capture_output=True, text=True, timeout=600)
    print(r.stdout[-3000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "PASS" in r.stdout
