"""CPU oracle for the K-quant hot path -- TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``liboracle.so`` (built from ``kq_oracle.c``), the C
restatement of Aspida's CPU path (src/llm/llm_dequant.adb, llm_pool.adb,
llm_moe.adb).  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker or the reported CPU baseline -- never as the thing measured or shipped.

``ref_deq_block`` exposes the CPU dequantizer of the reference's own GPU test
harness (gpu/test_matvec.cu:17-70), compiled from the reference tree into
``oracle/_ref/`` when that tree is mounted; it is ``None`` otherwise.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
REF_DIR = os.path.join(_HERE, "_ref")

KIND_Q4_K, KIND_Q6_K, KIND_Q5_K, KIND_Q3_K, KIND_Q2_K, KIND_Q8_0, KIND_DENSE = 0, 1, 2, 3, 4, 5, -1
KQUANTS = (KIND_Q4_K, KIND_Q6_K, KIND_Q5_K, KIND_Q3_K, KIND_Q2_K)
KIND_NAMES = {0: "Q4_K", 1: "Q6_K", 2: "Q5_K", 3: "Q3_K", 4: "Q2_K", 5: "Q8_0", -1: "F32"}
BLOCK_BYTES = {0: 144, 1: 210, 2: 176, 3: 110, 4: 84, 5: 272}

_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run `make -C oracle`)")
        L = ctypes.CDLL(LIB_PATH)
        P, I, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
        L.kqo_f16_to_f32.argtypes = [ctypes.c_uint8, ctypes.c_uint8]
        L.kqo_f16_to_f32.restype = F
        L.kqo_decode_block.argtypes = [I, P, P]
        L.kqo_dequant_rows.argtypes = [I, P, I, I, P]
        L.kqo_qmatvec.argtypes = [I, P, I, I, P, P, I, I]
        L.kqo_qmatmul.argtypes = [I, P, I, I, I, P, P, I]
        L.kqo_dense_matvec.argtypes = [P, I, I, P, P]
        L.kqo_dense_matvec.restype = None
        L.kqo_pool_chunks.argtypes = [I, I, I, I, P, P]
        L.kqo_route.argtypes = [P, I, I, P, P]
        L.kqo_route.restype = None
        L.kqo_moe_experts.argtypes = [P, I, I, I, I, P, P] + [P, I] * 6 + [P, I, P, I]
        L.kqo_moe_forward.argtypes = [P, I, I, I, I, P] + [P, I] * 6 + [P, I, P, P, P, I]
        L.kqo_rmsnorm.argtypes = [P, P, I, F, P]
        L.kqo_rmsnorm.restype = None
        _lib = L
    return _lib


def use_library(path):
    """Bind a different build of the same oracle source (e.g. one compiled
    -march=native for the host at run time); later calls use it."""
    global LIB_PATH, _lib
    LIB_PATH = path
    _lib = None


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def f16_to_f32(lo, hi):
    return lib().kqo_f16_to_f32(lo, hi)


def f16_table():
    """All 65536 half patterns decoded with Aspida's rule, as float32[65536]."""
    out = np.empty(65536, np.float32)
    L = lib()
    for h in range(65536):
        out[h] = L.kqo_f16_to_f32(h & 0xFF, h >> 8)
    return out


def dequant(kind, w, in_dim, out_dim):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    need = out_dim * (in_dim // 256) * BLOCK_BYTES[kind]
    if w.size < need:
        raise ValueError("weight buffer too small")
    dst = np.empty((out_dim, in_dim), np.float32)
    rc = lib().kqo_dequant_rows(kind, _ptr(w), in_dim, out_dim, _ptr(dst))
    if rc:
        raise ValueError(f"kqo_dequant_rows rc={rc}")
    return dst


def qmatvec(kind, w, in_dim, out_dim, x, nthreads=1, min_grain=2048):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    if x.size != in_dim:
        raise ValueError("QMatVec: input length does not match in_dim")
    y = np.empty(out_dim, np.float32)
    rc = lib().kqo_qmatvec(kind, _ptr(w), in_dim, out_dim, _ptr(x), _ptr(y), nthreads, min_grain)
    if rc:
        raise ValueError(f"kqo_qmatvec rc={rc}")
    return y


def qmatmul(kind, w, in_dim, out_dim, x, nthreads=1):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, in_dim)
    y = np.empty((x.shape[0], out_dim), np.float32)
    rc = lib().kqo_qmatmul(kind, _ptr(w), in_dim, out_dim, x.shape[0], _ptr(x), _ptr(y), nthreads)
    if rc:
        raise ValueError(f"kqo_qmatmul rc={rc}")
    return y


def dense_matvec(w, x):
    w = np.ascontiguousarray(w, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(w.shape[0], np.float32)
    lib().kqo_dense_matvec(_ptr(w), w.shape[1], w.shape[0], _ptr(x), _ptr(y))
    return y


def pool_chunks(first, last, min_grain, ncpu):
    lo = np.zeros(max(ncpu, 1), np.int32)
    hi = np.zeros(max(ncpu, 1), np.int32)
    n = lib().kqo_pool_chunks(first, last, min_grain, ncpu, _ptr(lo), _ptr(hi))
    return list(zip(lo[:n].tolist(), hi[:n].tolist()))


def route(logits, top_k):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    idx = np.zeros(top_k, np.int32)
    w = np.zeros(top_k, np.float32)
    lib().kqo_route(_ptr(logits), logits.size, top_k, _ptr(idx), _ptr(w))
    return idx, w


def _wk(w):
    """(array, kind) -> (pointer, kind) keeping dense f32 and quantized bytes apart."""
    arr, kind = w
    arr = np.ascontiguousarray(arr, dtype=np.float32 if kind < 0 else np.uint8)
    return arr, kind


def moe_experts(x, dim, top_k, intermed, n_exp, top_idx, top_w, gate, up, down,
                shg, shu, shd, shared_gate_inp=None, nthreads=1):
    """gate/up/down/shg/shu/shd are (array, kind) pairs."""
    ws = [_wk(t) for t in (gate, up, down, shg, shu, shd)]
    x = np.ascontiguousarray(x, dtype=np.float32)
    idx = np.ascontiguousarray(top_idx, dtype=np.int32)
    tw = np.ascontiguousarray(top_w, dtype=np.float32)
    sgi = None if shared_gate_inp is None else np.ascontiguousarray(shared_gate_inp, dtype=np.float32)
    y = np.empty(dim, np.float32)
    args = []
    for a, k in ws:
        args += [_ptr(a), k]
    rc = lib().kqo_moe_experts(_ptr(x), dim, top_k, intermed, n_exp, _ptr(idx), _ptr(tw), *args,
                               _ptr(sgi), 0 if sgi is None else sgi.size, _ptr(y), nthreads)
    if rc:
        raise ValueError(f"kqo_moe_experts rc={rc}")
    return y


def moe_forward(x, dim, intermed, n_exp, top_k, router_w, gate, up, down, shg, shu, shd,
                shared_gate_inp=None, nthreads=1):
    ws = [_wk(t) for t in (gate, up, down, shg, shu, shd)]
    x = np.ascontiguousarray(x, dtype=np.float32)
    rw = np.ascontiguousarray(router_w, dtype=np.float32)
    sgi = None if shared_gate_inp is None else np.ascontiguousarray(shared_gate_inp, dtype=np.float32)
    k = min(top_k, n_exp)
    y = np.empty(dim, np.float32)
    idx = np.zeros(k, np.int32)
    tw = np.zeros(k, np.float32)
    args = []
    for a, kk in ws:
        args += [_ptr(a), kk]
    rc = lib().kqo_moe_forward(_ptr(x), dim, intermed, n_exp, top_k, _ptr(rw), *args,
                               _ptr(sgi), 0 if sgi is None else sgi.size,
                               _ptr(y), _ptr(idx), _ptr(tw), nthreads)
    if rc:
        raise ValueError(f"kqo_moe_forward rc={rc}")
    return y, idx, tw


_ref = None


def ref_lib():
    """The reference harness's dequantizer (oracle/_ref/libref_deq.so) or None."""
    global _ref
    if _ref is None:
        p = os.path.join(REF_DIR, "libref_deq.so")
        if not os.path.exists(p):
            return None
        L = ctypes.CDLL(p)
        L.ref_deq_block.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
        L.ref_deq_block.restype = None
        _ref = L
    return _ref


def ref_deq_block(kind, blk):
    L = ref_lib()
    if L is None:
        return None
    blk = np.ascontiguousarray(blk, dtype=np.uint8)
    out = np.empty(256, np.float32)
    L.ref_deq_block(kind, _ptr(blk), _ptr(out))
    return out


def rmsnorm(x, w, eps=1e-6):
    """LLM_RMSNorm.Forward (src/llm/llm_rmsnorm.adb:10-41)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    y = np.empty(x.size, np.float32)
    lib().kqo_rmsnorm(_ptr(x), _ptr(w), x.size, eps, _ptr(y))
    return y


def matvec_any(w, in_dim, out_dim, x):
    """(array, kind) matrix times x: QMatVec for a quantised kind, the dense
    ascending-sum matvec for kind -1 (f32 [out][in])."""
    arr, kind = w
    if kind == -1:
        return dense_matvec(np.reshape(arr, (out_dim, in_dim)), x)
    return qmatvec(kind, arr, in_dim, out_dim, x)


def router_f32(router, dim, n_exp):
    """The f32 [n_exp][dim] router of a MoE block: as given, or decoded from a
    quantised kind by the Ada decoders (llm_dequant.adb:122-630)."""
    arr, kind = router
    if kind == -1:
        return np.ascontiguousarray(arr, np.float32).reshape(n_exp, dim)
    return dequant(kind, arr, dim, n_exp)


def chain_forward(model, row, n_layers=None, logits=True):
    """One token through the resident model chain.  Per layer, LLM_Qwen_Blk.Step
    (src/llm/llm_qwen_blk.adb:125-170): nx = RMSNorm(H, attn_norm), H += Mix nx
    (the mixer a matvec, the chain's stand-in for attention / delta-net), then
    nr = RMSNorm(H, post_norm), H += LLM_MoE.Forward(nr) (llm_moe.adb:136-299);
    at the end logits = LM RMSNorm(H, final_norm) (llm_qwen.adb:1199-1203).

    model: {"embed": f32 [rows][dim], "fnorm": f32 [dim], "lm": (array, kind),
    "vocab": int, "layers": [{"attn_norm", "post_norm", "mix": (array, kind) or
    None, "moe": None or {"router": (array, kind), "gate", "up", "down", "shg",
    "shu", "shd": (array, kind), "sgi": f32 [dim] or None, "n_exp", "top_k",
    "intermed"}}]}.  Returns (H after n_layers layers, logits or None, the
    routed experts of each MoE layer as (top_idx, top_w, router logits)).
    """
    layers = model["layers"] if n_layers is None else model["layers"][:n_layers]
    E = np.asarray(model["embed"], np.float32)
    dim = E.shape[1]
    H = E[row].copy()
    routes = []
    for L in layers:
        if L.get("mix") is not None:
            nx = rmsnorm(H, L["attn_norm"])
            H = (H + matvec_any(L["mix"], dim, dim, nx)).astype(np.float32)
        M = L.get("moe")
        if M is not None:
            nr = rmsnorm(H, L["post_norm"])
            rw = router_f32(M["router"], dim, M["n_exp"])
            y, idx, tw = moe_forward(nr, dim, M["intermed"], M["n_exp"], M["top_k"], rw, M["gate"], M["up"],
                                     M["down"], M["shg"], M["shu"], M["shd"], shared_gate_inp=M.get("sgi"))
            routes.append((idx, tw, dense_matvec(rw, nr)))
            H = (H + y).astype(np.float32)
    out = None
    if logits:
        out = matvec_any(model["lm"], dim, model["vocab"], rmsnorm(H, model["fnorm"]))
    return H, out, routes
