"""GPU parity of the K-quant dequantizer and batch-1 matvec against the CPU oracle.

Dequantization is bit-exact.  Matvec outputs match the oracle's QMatVec within
MV_RTOL (2e-5) times sum_i |w_i x_i| per output, through the reference ABI
(aspida_gpu_matvec, host pointers, packed HBM mirror) and the device-pointer
entry points (packed layout, and the ggml-layout stream kernel under every
launch-shape override), over every kind, ragged row counts, one-super-block
rows, the benchmark shapes and scale fields holding +-0, subnormals, Inf and
NaN.  Packing round-trips byte for byte; packed launches are deterministic
and replay correctly from a HIP graph.
"""
import numpy as np
import pytest

import aspida_amd as aa
import oracle
from aspida_amd import synth
from gpu_helpers import (MFMA_RTOL, MV_RTOL, abs_dot_scale, assert_close_scaled, ncpu, stream, sync, to_dev,
                         torch_cuda)

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


# Row lengths of 1..56 super-blocks and ragged row counts: for the packed
# kernels every split of a tile's columns over waves and workgroups (one
# workgroup, LDS-only, cross-workgroup partial sums), for the ggml-layout
# stream kernel chunks of 16/8/4/2/1 super-blocks per wave, teams of 1..7
# waves, idle lanes.
SMALL_SHAPES = [(1, 256), (3, 512), (67, 768), (130, 4096), (257, 2304), (33, 3328), (70, 8192),
                (41, 14336), (16421, 1024)]
CONFIGS = [(1, 16), (2, 16), (4, 16), (2, 4), (4, 64)]


@pytest.mark.parametrize("kind", KINDS)
def test_matvec_small_shapes(kind, gpu):
    """Reference ABI (host pointers; packed HBM mirror)."""
    for i, (out_dim, in_dim) in enumerate(SMALL_SHAPES):
        _check_mv(gpu, kind, out_dim, in_dim, 1000 * kind + i, f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")


def _dev_mv(dev, kind, w, x, in_dim, out_dim, layout):
    """y from the device entry points: 'stream' = ggml layout with xsum,
    'packed' = pack then the packed matvec."""
    torch = torch_cuda()
    dw, dx = to_dev(w), to_dev(x)
    dy = torch.full((out_dim,), float("nan"), dtype=torch.float32, device="cuda")
    if layout == "stream":
        dq = torch.empty(in_dim // 16, dtype=torch.float32, device="cuda")
        dev.xsum(dx.data_ptr(), in_dim, 1, dq.data_ptr(), stream())
        dev.matvec(kind, dw.data_ptr(), in_dim, out_dim, dx.data_ptr(), dq.data_ptr(), dy.data_ptr(), stream())
    else:
        dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
        dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
        dev.matvec_packed(kind, dp.data_ptr(), in_dim, out_dim, dx.data_ptr(), dy.data_ptr(), stream())
    sync()
    return dy.cpu().numpy()


def _check_dev(dev, kind, out_dim, in_dim, seed, layout, what):
    gen = synth.rng(seed)
    w = synth.weight_np(kind, out_dim, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    y = _dev_mv(dev, kind, w, x, in_dim, out_dim, layout)
    want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
    return assert_close_scaled(y, want, abs_dot_scale(kind, w, in_dim, out_dim, x), what=what)


@pytest.mark.parametrize("kind", KINDS)
def test_packed_matvec_small_shapes(kind, dev):
    for i, (out_dim, in_dim) in enumerate(SMALL_SHAPES):
        _check_dev(dev, kind, out_dim, in_dim, 3000 * kind + i, "packed", f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")


@pytest.mark.parametrize("cfg", CONFIGS, ids=lambda c: f"R{c[0]}W{c[1]}")
@pytest.mark.parametrize("kind", KINDS)
def test_stream_matvec_small_shapes_all_configs(kind, cfg, dev):
    """The ggml-layout stream kernel under every launch-shape override."""
    assert dev.lib.aspida_kq_set_mv_config(*cfg) == 0
    try:
        for i, (out_dim, in_dim) in enumerate(SMALL_SHAPES):
            _check_dev(dev, kind, out_dim, in_dim, 1000 * kind + i, "stream",
                       f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")
    finally:
        dev.lib.aspida_kq_set_mv_config(0, 16)


@pytest.mark.parametrize("kind", KINDS)
def test_pack_unpack_round_trip(kind, dev):
    """Packing only moves bytes: unpack(pack(W)) == W byte for byte, the image
    has 64-row tiles, and the rows padding the last tile are zero."""
    torch = torch_cuda()
    for out_dim, in_dim in [(1, 256), (64, 512), (67, 768), (200, 4096)]:
        gen = synth.rng(50 + out_dim + kind)
        w = gen.integers(0, 256, aa.weight_bytes(kind, in_dim, out_dim), dtype=np.uint8)
        nb = dev.packed_bytes(kind, in_dim, out_dim)
        assert nb == -(-out_dim // 64) * 64 * (in_dim // 256) * aa.BLOCK_BYTES[kind]
        dw = to_dev(w)
        dp = torch.full((nb,), 0xA5, dtype=torch.uint8, device="cuda")
        dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
        back = torch.zeros_like(dw)
        dev.unpack(kind, dp.data_ptr(), in_dim, out_dim, back.data_ptr(), stream())
        sync()
        assert np.array_equal(back.cpu().numpy(), w)
        packed = dp.cpu().numpy()
        assert np.count_nonzero(packed) <= w.size            # padding rows hold zeros
        assert sorted(packed.tolist()) == sorted(np.concatenate(
            [w, np.zeros(nb - w.size, np.uint8)]).tolist())  # a permutation of W plus zeros


def test_packed_deterministic_and_graph_replay(dev):
    """Cross-workgroup partial sums are added in a fixed order, so repeated
    launches give identical bits; the launches capture into a HIP graph (the
    arrival counters re-arm themselves, no memset) and every replay, with
    eager work in between, reproduces the eager result."""
    torch = torch_cuda()
    gen = synth.rng(66)
    shapes = [(0, 4096, 14336), (1, 1024, 4096), (0, 5120, 4096)]
    bufs = []
    for kind, out_dim, in_dim in shapes:
        w = synth.weight_np(kind, out_dim, in_dim, gen)
        x = synth.activations_np(in_dim, gen)
        dw, dx = to_dev(w), to_dev(x)
        dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
        dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
        bufs.append((kind, out_dim, in_dim, dp, dx, torch.empty(out_dim, device="cuda"), w, x))
    s = torch.cuda.Stream()
    sync()

    def run(sp):
        for kind, out_dim, in_dim, dp, dx, dy, _, _ in bufs:
            dev.matvec_packed(kind, dp.data_ptr(), in_dim, out_dim, dx.data_ptr(), dy.data_ptr(), sp)

    with torch.cuda.stream(s):
        run(s.cuda_stream)
    s.synchronize()
    eager = [b[5].clone() for b in bufs]
    with torch.cuda.stream(s):
        run(s.cuda_stream)
    s.synchronize()
    for e, b in zip(eager, bufs):
        assert torch.equal(e, b[5])
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        run(s.cuda_stream)
    for rep in range(3):
        for b in bufs:
            b[5].fill_(float("nan"))
        sync()
        with torch.cuda.stream(s):
            g.replay()
        s.synchronize()
        for e, b in zip(eager, bufs):
            assert torch.equal(e, b[5]), f"replay {rep}"
    for (kind, out_dim, in_dim, _, _, _, w, x), e in zip(bufs, eager):
        want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
        assert_close_scaled(e.cpu().numpy(), want, abs_dot_scale(kind, w, in_dim, out_dim, x), what="graph")


def test_graph_replay_survives_workspace_growth(dev):
    """A graph captured on a stream keeps the workspace pointers of that
    moment; later, larger calls on the same stream grow the stream's
    workspace (partials, counters, small-batch buffer).  The library keeps
    the superseded buffers, so replaying the graph afterwards still gives the
    eager result, bit for bit."""
    torch = torch_cuda()
    gen = synth.rng(67)
    kind, out_a, in_a = aa.Q4_K, 1024, 4096          # split over workgroups: partials and counters
    wa, xa = synth.weight_np(kind, out_a, in_a, gen), synth.activations_np(in_a, gen)
    pa = torch.empty(dev.packed_bytes(kind, in_a, out_a), dtype=torch.uint8, device="cuda")
    dev.pack(kind, to_dev(wa).data_ptr(), in_a, out_a, pa.data_ptr(), stream())
    dxa, dya = to_dev(xa), torch.empty(out_a, device="cuda")
    out_b, in_b, batch = 8192, 14336, 48             # larger matvec and a small-batch product
    wb = synth.weight_np(kind, out_b, in_b, gen)
    pb = torch.empty(dev.packed_bytes(kind, in_b, out_b), dtype=torch.uint8, device="cuda")
    dev.pack(kind, to_dev(wb).data_ptr(), in_b, out_b, pb.data_ptr(), stream())
    dxb = to_dev(synth.activations_np(batch * in_b, gen))
    dyb = torch.empty(batch * out_b, device="cuda")
    s = torch.cuda.Stream()
    sync()
    with torch.cuda.stream(s):
        dev.matvec_packed(kind, pa.data_ptr(), in_a, out_a, dxa.data_ptr(), dya.data_ptr(), s.cuda_stream)
    s.synchronize()
    eager = dya.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=s):
        dev.matvec_packed(kind, pa.data_ptr(), in_a, out_a, dxa.data_ptr(), dya.data_ptr(), s.cuda_stream)
    with torch.cuda.stream(s):
        dev.matvec_packed(kind, pb.data_ptr(), in_b, out_b, dxb.data_ptr(), dyb.data_ptr(), s.cuda_stream)
        dev.matmul_packed(kind, pb.data_ptr(), in_b, out_b, batch, dxb.data_ptr(), dyb.data_ptr(), s.cuda_stream)
    s.synchronize()
    for rep in range(3):
        dya.fill_(float("nan"))
        sync()
        with torch.cuda.stream(s):
            g.replay()
            if rep == 1:   # eager work on the grown workspace between replays
                dev.matvec_packed(kind, pb.data_ptr(), in_b, out_b, dxb.data_ptr(), dyb.data_ptr(), s.cuda_stream)
        s.synchronize()
        assert torch.equal(eager, dya), f"replay {rep}"
    want = oracle.qmatvec(kind, wa, in_a, out_a, xa, nthreads=ncpu())
    assert_close_scaled(eager.cpu().numpy(), want, abs_dot_scale(kind, wa, in_a, out_a, xa), what="graph")


PAIR_CASES = [(aa.Q4_K, 5120, aa.Q6_K, 1024, 4096), (aa.Q5_K, 70, aa.Q6_K, 200, 2048), (aa.Q4_K, 64, aa.Q4_K, 3, 768),
              (aa.Q8_0, 130, aa.Q8_0, 64, 1024), (aa.Q6_K, 17, aa.Q6_K, 33, 14336), (aa.Q3_K, 40, aa.Q2_K, 50, 512)]


@pytest.mark.parametrize("case", PAIR_CASES, ids=lambda c: f"{aa.KIND_NAMES[c[0]]}{c[1]}_{aa.KIND_NAMES[c[2]]}{c[3]}_{c[4]}")
def test_packed_matvec_pair(case, dev):
    """Two matrices sharing x in one launch (last case: a pair without a fused
    kernel, served as two launches) equal the oracle for both outputs."""
    torch = torch_cuda()
    ka, oa, kb, ob, in_dim = case
    gen = synth.rng(4000 + oa + ob)
    wa, wb = synth.weight_np(ka, oa, in_dim, gen), synth.weight_np(kb, ob, in_dim, gen)
    x = synth.activations_np(in_dim, gen)
    pa = torch.empty(dev.packed_bytes(ka, in_dim, oa), dtype=torch.uint8, device="cuda")
    pb = torch.empty(dev.packed_bytes(kb, in_dim, ob), dtype=torch.uint8, device="cuda")
    dev.pack(ka, to_dev(wa).data_ptr(), in_dim, oa, pa.data_ptr(), stream())
    dev.pack(kb, to_dev(wb).data_ptr(), in_dim, ob, pb.data_ptr(), stream())
    dx = to_dev(x)
    ya = torch.full((oa,), float("nan"), device="cuda")
    yb = torch.full((ob,), float("nan"), device="cuda")
    dev.matvec2_packed(ka, pa.data_ptr(), oa, ya.data_ptr(), kb, pb.data_ptr(), ob, yb.data_ptr(), in_dim,
                       dx.data_ptr(), stream())
    sync()
    for k, w, o, y in ((ka, wa, oa, ya), (kb, wb, ob, yb)):
        want = oracle.qmatvec(k, w, in_dim, o, x, nthreads=ncpu())
        assert_close_scaled(y.cpu().numpy(), want, abs_dot_scale(k, w, in_dim, o, x), what=aa.KIND_NAMES[k])


def test_packed_rejects_bad_arguments(dev):
    torch = torch_cuda()
    x = torch.zeros(260, device="cuda")
    y = torch.zeros(64, device="cuda")
    p = torch.zeros(dev.packed_bytes(0, 256, 64), dtype=torch.uint8, device="cuda")
    lib = dev.lib
    assert lib.aspida_kq_matvec_packed_dev(0, p.data_ptr(), 256, 64, x.data_ptr() + 4, y.data_ptr(), None) < 0
    assert lib.aspida_kq_matvec_packed_dev(9, p.data_ptr(), 256, 64, x.data_ptr(), y.data_ptr(), None) < 0
    assert lib.aspida_kq_matvec_packed_dev(0, p.data_ptr(), 300, 64, x.data_ptr(), y.data_ptr(), None) < 0
    assert lib.aspida_kq_packed_bytes(0, 300, 64) == 0


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


@pytest.mark.parametrize("shape", BENCH_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
@pytest.mark.parametrize("kind", list(aa.KQUANTS))
def test_stream_matvec_benchmark_shapes(kind, shape, dev):
    out_dim, in_dim = shape
    _check_dev(dev, kind, out_dim, in_dim, 5 + kind, "stream", f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim}")


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


def _x_variants(in_dim, gen):
    """Activations that stress the MFMA kernel's per-column scaling: plain,
    outliers (x 1e4), tiny (1e-28), huge (1e30), one all-zero column, and mixed
    magnitudes inside a column."""
    base = synth.activations_np(in_dim, gen)
    out = {"plain": base}
    o = base.copy()
    o[gen.integers(0, in_dim, 7)] *= 1e4
    out["outliers"] = o
    out["tiny"] = (base * 1e-28).astype(np.float32)
    out["huge"] = (base * 1e30).astype(np.float32)
    z = base.copy()
    z[256:512] = 0.0
    out["zero_column"] = z
    m = base.copy()
    m[::3] *= 1e-6
    m[1::5] *= 1e3
    out["mixed"] = m
    return out


@pytest.mark.parametrize("engine", [0, 1], ids=["mfma", "valu"])
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K, aa.Q2_K, aa.Q5_K, aa.Q3_K],
                         ids=["Q4_K", "Q6_K", "Q2_K", "Q5_K", "Q3_K"])
def test_engines_activation_range(kind, engine, dev):
    """Both batch-1 engines for Q4_K and Q6_K against the oracle, over
    activations whose magnitudes span the f32 range, at shapes that take every
    split of the MFMA kernel (16-wave whole tiles, 4-wave groups over several
    workgroups, prefetching waves of several columns)."""
    torch = torch_cuda()
    gen = synth.rng(4040 + engine + 10 * kind)
    dev.set_mv_engine(engine)
    try:
        for out_dim, in_dim in [(130, 4096), (4096, 1024), (300, 14336), (28672, 512), (16448, 4096),
                                (16448, 2048)]:
            w = synth.weight_np(kind, out_dim, in_dim, gen)
            dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
            dw = to_dev(w)
            dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
            plan = dev.matvec_plan(kind, in_dim, out_dim)
            for name, x in _x_variants(in_dim, gen).items():
                print(f"engine {engine} {aa.KIND_NAMES[kind]} {out_dim}x{in_dim} plan {plan} x={name}", flush=True)
                dx = to_dev(x)
                dy = torch.full((out_dim,), float("nan"), dtype=torch.float32, device="cuda")
                dev.matvec_packed(kind, dp.data_ptr(), in_dim, out_dim, dx.data_ptr(), dy.data_ptr(), stream())
                sync()
                want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
                # Outliers: the matrix cores keep about 2^-18 of a sum's largest product, and an
                # outlier whose weight cancels against the min term leaves that behind.  Q2_K,
                # Q3_K and Q6_K take a column's dominant activations exactly (measured <= 2.6e-5
                # here); Q4_K and Q5_K keep them in the matrix-core sums (measured 7.3e-5 and
                # 7.9e-5 on the 512-column rows, where one column weighs most).
                rtol = MFMA_RTOL if engine == 0 and name in ("outliers", "mixed") else MV_RTOL
                r = assert_close_scaled(dy.cpu().numpy(), want, abs_dot_scale(kind, w, in_dim, out_dim, x),
                                        rtol=rtol, what=f"engine {engine} {out_dim}x{in_dim} {name}")
                print(f"  max err / sum|wx| = {r:.2e}", flush=True)
    finally:
        dev.set_mv_engine(0)


@pytest.mark.parametrize("kind", [aa.Q6_K, aa.Q2_K, aa.Q3_K], ids=["Q6_K", "Q2_K", "Q3_K"])
def test_dominant_activations_exact(kind, dev):
    """Columns whose activations are dominated by a few (at most 16 within 16x
    of the largest) take those activations out of the matrix-core sums: one
    1e6x element, 16 elements at 1e4x (the largest set taken out), 17 at 1e4x
    (left in: they carry most of sum |w x| themselves), and a column with
    only three nonzero entries, on both workgroup shapes.  Held to 3e-5 of
    sum |w x|, about ten times below what the matrix-core sums left behind
    for such columns."""
    torch = torch_cuda()
    gen = synth.rng(7100 + kind)
    in_dim = 1280
    x = synth.activations_np(in_dim, gen)
    x[17] *= np.float32(1e6)                              # column 0
    x[256 + gen.permutation(256)[:16]] *= np.float32(1e4)  # column 1: 16 dominant
    x[512 + gen.permutation(256)[:17]] *= np.float32(1e4)  # column 2: 17
    x[768:1024] = 0.0                                     # column 3: three nonzero
    x[768 + np.array([5, 77, 200])] = np.float32([3.0, -2.0, 1.5])
    try:
        for rows in (0, 1, 2):
            dev.set_mfma_rows(rows)
            for out_dim in (130, 4096):
                w = synth.weight_np(kind, out_dim, in_dim, gen)
                dp = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
                dw = to_dev(w)
                dev.pack(kind, dw.data_ptr(), in_dim, out_dim, dp.data_ptr(), stream())
                print(f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} rows mode {rows} "
                      f"plan {dev.matvec_plan(kind, in_dim, out_dim)}", flush=True)
                dx = to_dev(x)
                dy = torch.full((out_dim,), float("nan"), dtype=torch.float32, device="cuda")
                dev.matvec_packed(kind, dp.data_ptr(), in_dim, out_dim, dx.data_ptr(), dy.data_ptr(), stream())
                sync()
                want = oracle.qmatvec(kind, w, in_dim, out_dim, x, nthreads=ncpu())
                r = assert_close_scaled(dy.cpu().numpy(), want, abs_dot_scale(kind, w, in_dim, out_dim, x),
                                        rtol=3e-5, what=f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} rows {rows}")
                print(f"  max err / sum|wx| = {r:.2e}", flush=True)
    finally:
        dev.set_mfma_rows(0)


# Matrix-core matvec workgroup shapes forced (aspida_kq_set_mfma_rows: 64-row
# workgroups with partial sums across workgroups, 16-row workgroups over all
# columns) and column walks (one column, prefetching, one after another):
# ragged rows, a single 16-row block, long column runs, both pair kernels.
MFMA_SHAPE_CASES = [(64, 4096), (130, 4096), (1000, 2048), (4096, 4096), (300, 14336), (4096, 14336), (16448, 4096),
                    (37, 256)]


@pytest.mark.parametrize("pipe", [0, 1, 2], ids=["plan", "prefetch", "sequential"])
@pytest.mark.parametrize("rows", [1, 2], ids=["rows64", "rows16"])
@pytest.mark.parametrize("kind", [aa.Q4_K, aa.Q6_K, aa.Q2_K, aa.Q5_K, aa.Q3_K],
                         ids=["Q4_K", "Q6_K", "Q2_K", "Q5_K", "Q3_K"])
def test_mfma_workgroup_shapes(kind, rows, pipe, dev):
    dev.set_mfma_rows(rows)
    dev.lib.aspida_kq_set_mfma_pipeline(pipe)
    try:
        for i, (out_dim, in_dim) in enumerate(MFMA_SHAPE_CASES):
            plan = dev.matvec_plan(kind, in_dim, out_dim)
            assert plan[0] and plan[5] == (rows == 2), plan
            _check_dev(dev, kind, out_dim, in_dim, 5100 + 10 * i + kind, "packed",
                       f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} rows={rows} pipe={pipe} plan={plan}")
    finally:
        dev.set_mfma_rows(0)
        dev.lib.aspida_kq_set_mfma_pipeline(0)


@pytest.mark.parametrize("rows", [1, 2], ids=["rows64", "rows16"])
@pytest.mark.parametrize("case", PAIR_CASES[:5], ids=lambda c: f"{aa.KIND_NAMES[c[0]]}{c[1]}_{aa.KIND_NAMES[c[2]]}{c[3]}_{c[4]}")
def test_packed_matvec_pair_workgroup_shapes(case, rows, dev):
    dev.set_mfma_rows(rows)
    try:
        test_packed_matvec_pair(case, dev)
    finally:
        dev.set_mfma_rows(0)


@pytest.mark.parametrize("kind,out_dim,in_dim,spw", [(aa.Q6_K, 65600, 4096, 2), (aa.Q4_K, 16448, 8192, 4),
                                                     (aa.Q6_K, 8192, 28672, 14)],
                         ids=["q6k-head-class", "q4k-70b-ffn-class", "q6k-70b-down"])
def test_tall_plans_take_8_wave_16_row_groups(kind, out_dim, in_dim, spw, dev):
    """Matrices of more 16-row blocks than CUs take 16-row workgroups of 8
    waves walking `spw` columns each: a Q6_K matrix of more than 1024 64-row
    tiles (the output head's class), a Q4_K one of 257 tiles with 32-block rows
    (the 70B FFN's class) and the 70B down projection -- and match the oracle."""
    plan = dev.matvec_plan(kind, in_dim, out_dim)
    assert plan[0] and plan[5] and plan[1] == 8 and plan[3] == spw, plan
    _check_dev(dev, kind, out_dim, in_dim, 6161, "packed", f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} plan={plan}")


Q2Q3_PLAN_CASES = [
    # kind, out, in, (mfma, waves, groups per tile, columns per wave, one after another, 16-row)
    (aa.Q3_K, 6144, 4096, (True, 8, 1, 2, False, True)),
    (aa.Q2_K, 4096, 14336, (True, 14, 1, 4, False, True)),
    (aa.Q2_K, 16448, 8192, (True, 4, 1, 8, False, False)),
    (aa.Q3_K, 16448, 4096, (True, 4, 4, 1, False, False)),
    (aa.Q2_K, 8192, 20480, (True, 4, 4, 5, False, False)),
]


@pytest.mark.parametrize("kind,out_dim,in_dim,plan", Q2Q3_PLAN_CASES,
                         ids=["q3k-two-blocks-per-cu", "q2k-long-rows-block-per-cu", "q2k-tall",
                              "q3k-tall-split", "q2k-long-rows"])
def test_q2_q3_plans(kind, out_dim, in_dim, plan, dev):
    """The Q2_K / Q3_K splits of the MFMA matvec: 16-row workgroups of
    prefetching waves at 1.5-2 blocks per CU (or one, with long rows), 4
    prefetching waves per 64-row tile for tall Q2_K, a row split into 4-block
    groups for tall Q3_K, and 4 groups of 4 waves walking columns for long
    Q2_K rows -- each the chosen plan, and each matching the oracle."""
    got = dev.matvec_plan(kind, in_dim, out_dim)
    assert got == plan, got
    _check_dev(dev, kind, out_dim, in_dim, 6262 + kind, "packed", f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} plan={got}")


def test_q8_0_sixteen_wave_column_walk(dev):
    """Q8_0 on 16-wave workgroups walking several columns per wave (more than
    255 tiles, rows of 32 super-blocks) takes the walk without prefetching --
    the prefetching one does not fit Q8_0's registers at 16 waves -- and
    matches the oracle."""
    kind, out_dim, in_dim = aa.Q8_0, 16448, 8192
    plan = dev.matvec_plan(kind, in_dim, out_dim)
    assert not plan[0] and plan[1] == 16 and plan[3] == 2, plan
    _check_dev(dev, kind, out_dim, in_dim, 8080, "packed", f"Q8_0 {out_dim}x{in_dim} plan={plan}")


@pytest.mark.parametrize("kind,out_dim,in_dim", [(aa.Q4_K, 57344, 8192), (aa.Q6_K, 128256, 8192),
                                                 (aa.Q6_K, 128256, 4096), (aa.Q4_K, 28672, 4096)],
                         ids=["70b-gate_up", "70b-head", "8b-head", "8b-gate_up"])
def test_full_size_decode_launches_sampled_rows(kind, out_dim, in_dim, dev):
    """The decode launches at their full Llama-3 sizes -- 70B gate|up (Q4_K
    57344x8192, 264 MB) and head (Q6_K 128256x8192, 862 MB), and the 8B ones --
    weights generated on the device, packed and run by the packed matvec
    exactly as the benchmark runs them.  A sample of rows (the first and last
    64-row tiles, and 384 spread over the rest) is compared with the oracle's
    QMatVec over the same rows' bytes."""
    torch = torch_cuda()
    g = torch.Generator(device="cuda")
    g.manual_seed(7000 + out_dim + kind)
    raw = synth.blocks_torch(kind, out_dim * (in_dim // 256), generator=g)
    p = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
    dev.pack(kind, raw.data_ptr(), in_dim, out_dim, p.data_ptr(), stream())
    x = synth.activations_np(in_dim, synth.rng(out_dim + in_dim))
    dx = to_dev(x)
    y = torch.full((out_dim,), float("nan"), device="cuda")
    dev.matvec_packed(kind, p.data_ptr(), in_dim, out_dim, dx.data_ptr(), y.data_ptr(), stream())
    sync()
    gen = synth.rng(out_dim * 3 + kind)
    rows = np.unique(np.concatenate([np.arange(64), np.arange(out_dim - 64, out_dim),
                                     gen.choice(out_dim, 384, replace=False)]))
    bpr = (in_dim // 256) * aa.BLOCK_BYTES[kind]
    idx = torch.from_numpy(rows).cuda()
    w_rows = raw.view(out_dim, bpr).index_select(0, idx).cpu().numpy().reshape(-1)
    del raw, p
    got = y.cpu().numpy()[rows]
    want = oracle.qmatvec(kind, w_rows, in_dim, rows.size, x, nthreads=ncpu())
    assert_close_scaled(got, want, abs_dot_scale(kind, w_rows, in_dim, rows.size, x),
                        what=f"{aa.KIND_NAMES[kind]} {out_dim}x{in_dim} ({rows.size} sampled rows)")
