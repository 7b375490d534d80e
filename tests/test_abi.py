"""CPU-only checks of the C-ABI library: it loads, exports every symbol
include/aspidagpu.h declares (and the five the Ada host resolves), and its
argument validation rejects bad calls before any GPU work, the way the Ada
binding would see it: NaN-filled output plus a non-zero aspida_gpu_last_error.
"""
import ctypes
import subprocess

import numpy as np
import pytest

import aspida_amd as aa

# Symbols Aspida's Ada side resolves (src/llm/llm_gpu.adb:100-146,
# src/llm/llm_qwen_gpu.adb:257-266 and 340).
ADA_SYMBOLS = ["aspida_gpu_matvec", "aspida_gpu_matmul", "aspida_gpu_dense_matvec",
               "aspida_gpu_free_weight", "aspida_gpu_moe_experts", "aspida_gpu_last_error"]


@pytest.fixture(scope="module")
def lib():
    return aa.load()


def test_header_symbols_exported(lib):
    declared = aa.exported_symbols_declared()
    assert set(ADA_SYMBOLS) <= set(declared)
    out = subprocess.run(["nm", "-D", "--defined-only", aa.LIB_PATH], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    missing = [s for s in declared if s not in exported]
    assert not missing, missing
    for s in declared:
        assert getattr(lib, s) is not None


def test_dlopen_like_the_ada_host():
    """RTLD_NOW dlopen of the library file, then dlsym of each Ada symbol."""
    h = ctypes.CDLL(aa.LIB_PATH, mode=ctypes.RTLD_LOCAL | 2)
    for s in ADA_SYMBOLS:
        assert ctypes.cast(getattr(h, s), ctypes.c_void_p).value


def _nan_and_error(g, y):
    return bool(np.all(np.isnan(y))) and g.last_error() != 0 and g.last_error() == 0


def test_matvec_rejects_bad_arguments(lib):
    g = aa.LLMGpu()
    g.last_error()
    x = np.ones(256, np.float32)
    w = np.zeros(144, np.uint8)
    assert _nan_and_error(g, g.matvec(w, 0, 300, 1, np.ones(300, np.float32)))   # in % 256 /= 0
    assert _nan_and_error(g, g.matvec(w, 0, 256, 2, x))                          # wbytes too small
    assert _nan_and_error(g, g.matvec(w, 9, 256, 1, x))                          # unknown kind
    assert _nan_and_error(g, g.matvec(w, -1, 256, 1, x))
    assert _nan_and_error(g, g.matvec(w, 0, 0, 1, x))


def test_matmul_batch_zero_is_a_noop(lib):
    y = np.full(4, 7.0, np.float32)
    w = np.zeros(144, np.uint8)
    x = np.ones(256, np.float32)
    lib.aspida_gpu_matmul(w.ctypes.data, w.nbytes, 0, 256, 1, 0, x.ctypes.data, y.ctypes.data)
    assert np.all(y == 7.0) and lib.aspida_gpu_last_error() == 0


def test_dense_rejects_short_buffer(lib):
    g = aa.LLMGpu()
    w = np.zeros((2, 8), np.float32)
    y = np.empty(3, np.float32)
    x = np.ones(8, np.float32)
    lib.aspida_gpu_dense_matvec(w.ctypes.data, w.nbytes, 8, 3, x.ctypes.data, y.ctypes.data)
    assert np.all(np.isnan(y)) and g.last_error() != 0


def test_moe_rejects_bad_routing(lib):
    g = aa.LLMGpu()
    dim, inter, n_exp = 256, 256, 2
    gw = np.zeros(n_exp * inter * 144, np.uint8)
    dw = np.zeros(n_exp * dim * 210, np.uint8)
    sg, sd = np.zeros(inter * 144, np.uint8), np.zeros(dim * 210, np.uint8)
    x = np.ones(dim, np.float32)
    args = ((gw, 0), (gw, 0), (dw, 1), (sg, 0), (sg, 0), (sd, 1))
    y = g.moe_experts(x, dim, 2, inter, n_exp, [0, 5], [0.5, 0.5], *args)     # expert id out of range
    assert np.all(np.isnan(y)) and g.last_error() != 0
    y = g.moe_experts(x, dim, 3, inter, n_exp, [0, 1, 0], [0.3, 0.3, 0.4], *args)   # top_k > n_exp
    assert np.all(np.isnan(y)) and g.last_error() != 0
    y = g.moe_experts(x, 200, 1, inter, n_exp, [0], [1.0], *args)              # dim % 256 /= 0
    assert np.all(np.isnan(y)) and g.last_error() != 0


def test_device_entry_points_reject_bad_arguments(lib):
    assert lib.aspida_kq_matvec_dev(0, None, 256, 1, None, None, None, None) < 0
    assert lib.aspida_kq_matvec_dev(7, 1, 256, 1, 1, 1, 1, None) < 0
    assert lib.aspida_kq_matmul_dev(0, 1, 300, 1, 2, 1, 1, 1, None) < 0
    assert lib.aspida_kq_dequant_dev(0, 1, 256, 0, 1, None) < 0
    assert lib.aspida_moe_route_dev(None, 128, 2048, 1, 8, None, None, None, None, None) < 0
    assert lib.aspida_kq_set_mv_config(3, 16) < 0
    assert lib.aspida_kq_set_mv_config(2, 0) < 0
    assert lib.aspida_kq_set_mv_config(0, 16) == 0
    assert lib.aspida_moe_work_floats(1, 2048, 8, 768) > 9 * 768 * 3


def test_grouped_moe_rejects_bad_arguments(lib):
    """aspida_moe_experts_packed_dev validates before any launch (the fake
    pointers are never dereferenced)."""
    assert lib.aspida_moe_packed_work_bytes(0, 2048, 768, 8) < 0
    assert lib.aspida_moe_packed_work_bytes(1, 2048, 768, 33) < 0
    # one token: h 9 x 768, yk 9 x 2048 floats, gsh, 128 counters (16-row blocks of dim) of 256 B, the
    # published schedule (1024 + 2 job offsets and 9 jobs, rounded to 256 B) and the chunk table (a count
    # and at most ceil(9 / 2) + 8 + 1 chunks of 16 B)
    sched = ((1024 + 2 + 9) * 4 + 255) // 256 * 256
    table = (1 + (9 + 1) // 2 + 8 + 1) * 16
    assert lib.aspida_moe_packed_work_bytes(1, 2048, 768, 8) == 4 * 9 * (768 + 2048) + 256 + 128 * 256 + sched + table
    # From 96 tokens the Q4_K / Q6_K experts may take the prefill products, in sequences of at
    # most 1024 tokens: the size grows with T up to 1024 tokens and no further
    ws = [lib.aspida_moe_packed_work_bytes(T, 2048, 768, 8) for T in (32, 96, 512, 1024, 1025, 5000)]
    assert ws[0] < ws[1] < ws[2] < ws[3] == ws[4] == ws[5]
    # below 96 tokens, T * top_k above the per-launch job bound: sized for one chunk of 1024 jobs' tokens
    assert lib.aspida_moe_packed_work_bytes(95, 512, 256, 32) == lib.aspida_moe_packed_work_bytes(32, 512, 256, 32)
    one = 256
    args = dict(x=one, T=1, dim=2048, top_k=8, intermed=768, n_exp=128, idx=one, tw=one, g=one, u=one, gk=0, d=one,
                dk=1, sg=one, su=one, sd=one, sgi=None, work=one, y=one)

    def call(**kw):
        a = {**args, **kw}
        return lib.aspida_moe_experts_packed_dev(a["x"], a["T"], a["dim"], a["top_k"], a["intermed"], a["n_exp"],
                                                 a["idx"], a["tw"], a["g"], a["u"], a["gk"], a["d"], a["dk"],
                                                 a["sg"], a["su"], a["sd"], a["sgi"], a["work"], a["y"], None)
    assert call(dim=2000) < 0
    assert call(intermed=700) < 0
    assert call(top_k=129) < 0
    assert call(top_k=0) < 0
    assert call(T=0) < 0
    assert call(x=None) < 0
    assert call(gk=9) < 0
    assert call(dk=-1) < 0
    assert call(x=one + 4) < 0          # x must be 16-byte aligned
    assert call(work=one + 16) < 0      # work must be 256-byte aligned
    assert lib.aspida_moe_pack_experts_dev(0, one, 10, 256, 64, 2, one, None) < 0   # stride below one matrix
    assert lib.aspida_moe_pack_experts_dev(0, one, 64 * 144, 300, 64, 2, one, None) < 0


def test_chain_rejects_bad_steps(lib):
    """aspida_kq_chain_create validates before allocating: a step that writes
    what an earlier step reads, an input straddling a producer's output, an
    unaligned x, a bad kind."""
    def mk(steps):
        arr = (aa.KqStep * len(steps))(*[aa.KqStep(k, i, o, 0, p, x, y) for k, p, i, o, x, y in steps])
        return lib.aspida_kq_chain_create(arr, len(steps))
    B = 1 << 20                         # fake device addresses, never dereferenced
    ok0 = (0, 4096, 256, 64, B, B + 4096)
    assert not mk([(0, 4096, 256, 64, B, B + 512)])                       # x overlaps its own y
    assert not mk([ok0, (0, 4096, 256, 64, B + 8192, B)])                 # writes x of step 0
    assert not mk([ok0, (0, 4096, 256, 64, B + 4096 + 128, B + 8192)])   # x straddles step 0's y
    assert not mk([(0, 4096, 256, 64, B + 4, B + 4096)])                  # x not 16-byte aligned
    assert not mk([(9, 4096, 256, 64, B, B + 4096)])                      # bad kind
    assert not mk([(0, 4096, 300, 64, B, B + 4096)])                      # in_dim % 256
    assert lib.aspida_gpu_last_error() != 0
    assert lib.aspida_kq_chain_run(None, None) < 0
    assert lib.aspida_kq_chain_check(None) < 0
    lib.aspida_kq_chain_destroy(None)


def _matmul_ws(lib, kind, in_dim, out_dim, batch):
    alloc, need = ctypes.c_longlong(), ctypes.c_longlong()
    assert lib.aspida_kq_matmul_workspace(kind, in_dim, out_dim, batch, ctypes.byref(alloc), ctypes.byref(need)) == 0
    return alloc.value, need.value


def test_matmul_workspace_covers_every_launch(lib):
    """The small-batch workspace the library allocates for a product holds
    what each of its launches writes, for every kind, over shapes of the
    Qwen2 and Llama families and every batch up to 130 (launch paddings of
    16, 32 and 64 vectors and the Q6_K step of 32 give different column
    splits).  Host-only query: no GPU work."""
    shapes = [(8960, 1536), (1536, 8960), (3584, 3584), (3584, 18944), (18944, 3584), (4096, 4096),
              (4096, 14336), (14336, 4096), (2048, 768), (768, 2048), (256, 64), (8192, 28672), (28672, 8192)]
    for kind in aa.KINDS:
        for in_dim, out_dim in shapes:
            for batch in list(range(2, 70)) + [96, 97, 127, 128, 130]:
                alloc, need = _matmul_ws(lib, kind, in_dim, out_dim, batch)
                assert alloc >= need, (aa.KIND_NAMES[kind], in_dim, out_dim, batch, alloc, need)


def test_matmul_workspace_advisor_shapes(lib):
    """The shapes where a 64-row padding undersized the buffer: Q6_K
    8960->1536 at B=48 and Q4_K/Q6_K 3584x3584 at B=48 and 65 -- on the
    64-vector kernel (engine 2), whose launches need the workspace, and on the
    built-in pick (Q6_K there runs the one-pass kernel, which needs none)."""
    cases = [(aa.Q6_K, 8960, 1536, 48), (aa.Q4_K, 3584, 3584, 48), (aa.Q6_K, 3584, 3584, 48),
             (aa.Q4_K, 3584, 3584, 65), (aa.Q6_K, 3584, 3584, 65)]
    assert lib.aspida_kq_set_mm_engine(2) == 0
    try:
        for kind, in_dim, out_dim, batch in cases:
            alloc, need = _matmul_ws(lib, kind, in_dim, out_dim, batch)
            assert need > 0 and alloc >= need, (kind, in_dim, out_dim, batch, alloc, need)
    finally:
        assert lib.aspida_kq_set_mm_engine(0) == 0
    for kind, in_dim, out_dim, batch in cases:
        alloc, need = _matmul_ws(lib, kind, in_dim, out_dim, batch)
        assert alloc >= need, (kind, in_dim, out_dim, batch, alloc, need)


def test_chain_abi_rejects_without_a_model(lib):
    """The reference chain ABI (aspida_gpu_chain_*) with nothing registered: not ready,
    a forward reports an error and launches nothing, bad layer arguments are refused
    before any device work, and reset clears the failure."""
    lib.aspida_gpu_chain_reset()
    lib.aspida_gpu_last_error()
    assert lib.aspida_gpu_chain_ready() == 0
    y = np.full(4, 7.0, np.float32)
    lib.aspida_gpu_chain_forward(0, 0, None, y.ctypes.data)
    assert lib.aspida_gpu_last_error() != 0
    lib.aspida_gpu_chain_forward_batch(0, None, None, None, y.ctypes.data)      # B < 1: a no-op
    assert lib.aspida_gpu_last_error() == 0 and np.all(y == 7.0)
    n = np.ones(300, np.float32)
    assert lib.aspida_kq_chain_layer(n.ctypes.data, n.nbytes, n.ctypes.data, n.nbytes, None, 0, 0) < 0  # dim % 256
    m = np.ones(256, np.float32)
    assert lib.aspida_kq_chain_layer(m.ctypes.data, m.nbytes, n.ctypes.data, n.nbytes, None, 0, 0) < 0  # norms differ
    assert lib.aspida_kq_chain_layer(m.ctypes.data, m.nbytes, m.ctypes.data, m.nbytes, m.ctypes.data, 0, 9) < 0
    assert lib.aspida_gpu_last_error() != 0
    # chain_moe with no layer is a no-op (gpu_matvec.cu:2152), chain_model with a bad kind fails
    lib.aspida_gpu_chain_reset()
    lib.aspida_gpu_chain_moe(*([None, 0, 0] * 7), None, 0, 0, 8, 2, 256)
    assert lib.aspida_gpu_last_error() == 0
    lib.aspida_gpu_chain_model(m.ctypes.data, m.nbytes, m.ctypes.data, m.nbytes, m.ctypes.data, m.nbytes, 9, 256, 1)
    assert lib.aspida_gpu_last_error() != 0 and lib.aspida_gpu_chain_ready() == 0
    lib.aspida_gpu_chain_reset()
    assert lib.aspida_kq_chain_forward_layers(1, None, 0, None) < 0
    assert lib.aspida_kq_chain_graphs() == 0
