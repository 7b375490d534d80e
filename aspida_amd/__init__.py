"""aspida_amd -- MI355X (gfx950) implementation of Aspida's quantized-weight GPU path.

The product is the C-ABI library ``libaspidagpu.so`` (HIP kernels + the
reference shim's symbol surface, declared in ``include/aspidagpu.h``).  This
module is its host-side Python binding:

* ``LLMGpu`` mirrors the Ada binding ``LLM_GPU`` (src/llm/llm_gpu.ads,
  llm_gpu.adb:80-185): ``available``, ``matvec``, ``matmul``,
  ``dense_matvec``, ``free_weight`` over the host-pointer ABI, and
  ``moe_experts`` mirrors ``LLM_Qwen_GPU.MoE_Experts`` (llm_qwen_gpu.adb).
* ``dev`` exposes the device-pointer entry points (integers for device
  addresses and the HIP stream), used with activations already in HBM.

There is no CPU fallback here: if the library is missing or fails to load,
``load()`` raises.  The Ada host keeps its own CPU fallback, as before.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaspidagpu.so")
HEADER = os.path.join(HERE, "..", "include", "aspidagpu.h")

# LLM_Weight.Kind_Code (src/llm/llm_weight.adb:277-292)
Q4_K, Q6_K, Q5_K, Q3_K, Q2_K, Q8_0 = 0, 1, 2, 3, 4, 5
KQUANTS = (Q4_K, Q6_K, Q5_K, Q3_K, Q2_K)
KINDS = KQUANTS + (Q8_0,)
KIND_NAMES = {Q4_K: "Q4_K", Q6_K: "Q6_K", Q5_K: "Q5_K", Q3_K: "Q3_K", Q2_K: "Q2_K", Q8_0: "Q8_0"}
BLOCK_BYTES = {Q4_K: 144, Q6_K: 210, Q5_K: 176, Q3_K: 110, Q2_K: 84, Q8_0: 272}

_lib = None


def weight_bytes(kind, in_dim, out_dim):
    return out_dim * (in_dim // 256) * BLOCK_BYTES[kind]


def load(path=None):
    """dlopen libaspidagpu.so (RTLD_NOW, as llm_gpu.adb:90) and bind its symbols."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or os.environ.get("ASPIDA_GPU_LIB") or LIB_PATH
    if not os.path.exists(p):
        raise RuntimeError(f"libaspidagpu.so not found at {p}: build it with `python -m aspida_amd.build`")
    L = ctypes.CDLL(p, mode=ctypes.RTLD_GLOBAL)
    P, I, LG, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_float
    sig = {
        "aspida_gpu_matvec": (None, [P, LG, I, I, I, P, P]),
        "aspida_gpu_matmul": (None, [P, LG, I, I, I, I, P, P]),
        "aspida_gpu_dense_matvec": (None, [P, LG, I, I, P, P]),
        "aspida_gpu_free_weight": (None, [P]),
        "aspida_gpu_moe_experts": (None, [P, I, I, I, I, P, P] + [P, LG, I] * 6 + [P, I, P]),
        "aspida_gpu_last_error": (I, []),
        "aspida_kq_xsum_dev": (I, [P, I, I, P, P]),
        "aspida_kq_matvec_dev": (I, [I, P, I, I, P, P, P, P]),
        "aspida_kq_matmul_dev": (I, [I, P, I, I, I, P, P, P, P]),
        "aspida_kq_packed_bytes": (ctypes.c_longlong, [I, I, I]),
        "aspida_kq_pack_dev": (I, [I, P, I, I, P, P]),
        "aspida_kq_packed_plan": (I, [I, I, P, P, P]),
        "aspida_kq_matvec_plan": (I, [I, I, I, P, P, P]),
        "aspida_kq_unpack_dev": (I, [I, P, I, I, P, P]),
        "aspida_kq_matvec_packed_dev": (I, [I, P, I, I, P, P, P]),
        "aspida_kq_matvec_packed_noalloc_dev": (I, [I, P, I, I, P, P, P]),
        "aspida_kq_matmul_packed_dev": (I, [I, P, I, I, I, P, P, P]),
        "aspida_kq_matvec2_packed_dev": (I, [I, P, I, P, I, P, I, P, I, P, P]),
        "aspida_kq_matmul_valu_dev": (I, [I, P, I, I, I, P, P, P, P]),
        "aspida_kq_dequant_dev": (I, [I, P, I, I, P, P]),
        "aspida_dense_matvec_dev": (I, [P, I, I, P, P, P]),
        "aspida_moe_route_dev": (I, [P, I, I, I, I, P, P, P, P, P]),
        "aspida_moe_work_floats": (LG, [I, I, I, I]),
        "aspida_moe_experts_dev": (I, [P, I, I, I, I, I, P, P] + [P, LG, I] * 3 + [P, I] * 3 + [P, P, P, P]),
        "aspida_moe_packed_work_bytes": (LG, [I, I, I, I]),
        "aspida_moe_pack_experts_dev": (I, [I, P, LG, I, I, I, P, P]),
        "aspida_moe_experts_packed_dev": (I, [P, I, I, I, I, I, P, P, P, P, I, P, I, P, P, P, P, P, P, P]),
        "aspida_kq_chain_create": (P, [P, I]),
        "aspida_kq_chain_run": (I, [P, P]),
        "aspida_kq_chain_check": (I, [P]),
        "aspida_kq_chain_workgroups": (I, [P]),
        "aspida_kq_chain_destroy": (None, [P]),
        "aspida_gpu_chain_reset": (None, []),
        "aspida_gpu_chain_moe": (None, [P, LG, I] * 7 + [P, LG, I, I, I, I]),
        "aspida_gpu_chain_model": (None, [P, LG, P, LG, P, LG, I, I, I]),
        "aspida_gpu_chain_ready": (I, []),
        "aspida_gpu_chain_begin": (None, [P]),
        "aspida_gpu_chain_end": (None, []),
        "aspida_gpu_chain_forward": (None, [I, I, P, P]),
        "aspida_gpu_chain_forward_batch": (None, [I, P, P, P, P]),
        "aspida_kq_chain_layer": (I, [P, LG, P, LG, P, LG, I]),
        "aspida_kq_chain_forward_layers": (I, [I, P, I, P]),
        "aspida_kq_chain_set_graphs": (I, [I]),
        "aspida_kq_chain_graphs": (I, []),
        "aspida_kq_matmul_workspace": (I, [I, I, I, I, P, P]),
        "aspida_kq_set_packed_plan": (I, [I, I]),
        "aspida_kq_set_mv_engine": (I, [I]),
        "aspida_kq_set_mfma_rows": (I, [I]),
        "aspida_kq_set_mm_engine": (I, [I]),
        "aspida_kq_set_mfma_pipeline": (I, [I]),
        "aspida_kq_set_mv_config": (I, [I, I]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = L
    return L


def exported_symbols_declared():
    """Function names declared in include/aspidagpu.h."""
    import re
    txt = open(HEADER).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?!typedef\b)(?:const\s+)?[A-Za-z_]\w*(?:\s+\w+)*[\s\*]+(aspida_\w+)\s*\(",
                                 txt, re.M)))


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


class LLMGpu:
    """Python mirror of the Ada package LLM_GPU over the host-pointer ABI.

    Weights are numpy uint8 buffers (f32 for dense); the library mirrors each
    into HBM keyed by its address, so keep the array alive and unchanged until
    ``free_weight``.
    """

    def __init__(self, path=None):
        self.lib = load(path)

    def available(self):
        return True

    def last_error(self):
        return self.lib.aspida_gpu_last_error()

    def matvec(self, w, kind, in_dim, out_dim, x, wbytes=None):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(out_dim, np.float32)
        wb = w.nbytes if wbytes is None else wbytes
        self.lib.aspida_gpu_matvec(_p(w), wb, kind, in_dim, out_dim, _p(x), _p(y))
        return y

    def matmul(self, w, kind, in_dim, out_dim, x, wbytes=None):
        x = np.ascontiguousarray(x, np.float32).reshape(-1, in_dim)
        y = np.empty((x.shape[0], out_dim), np.float32)
        wb = w.nbytes if wbytes is None else wbytes
        self.lib.aspida_gpu_matmul(_p(w), wb, kind, in_dim, out_dim, x.shape[0], _p(x), _p(y))
        return y

    def dense_matvec(self, w, x):
        w = np.ascontiguousarray(w, np.float32)
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty(w.shape[0], np.float32)
        self.lib.aspida_gpu_dense_matvec(_p(w), w.nbytes, w.shape[1], w.shape[0], _p(x), _p(y))
        return y

    def free_weight(self, w):
        self.lib.aspida_gpu_free_weight(_p(w))

    def moe_experts(self, x, dim, top_k, intermed, n_exp, top_idx, top_w, gate, up, down, shg, shu, shd,
                    shared_gate_inp=None):
        """gate/up/down/shg/shu/shd: (uint8 array, kind) pairs; experts are
        [n_exp][rows][cols] slabs of bytes / n_exp each."""
        x = np.ascontiguousarray(x, np.float32)
        idx = np.ascontiguousarray(top_idx, np.int32)
        tw = np.ascontiguousarray(top_w, np.float32)
        y = np.empty(dim, np.float32)
        args = []
        for arr, kind in (gate, up, down, shg, shu, shd):
            args += [_p(arr), arr.nbytes, kind]
        sgi = None if shared_gate_inp is None else np.ascontiguousarray(shared_gate_inp, np.float32)
        self.lib.aspida_gpu_moe_experts(_p(x), dim, top_k, intermed, n_exp, _p(idx), _p(tw), *args,
                                        _p(sgi), 0 if sgi is None else sgi.size, _p(y))
        return y


class ResidentChain:
    """Python mirror of the Ada chain procedures of LLM_Qwen_GPU
    (src/llm/llm_qwen_gpu.adb: Chain_Reset, Chain_MoE, Chain_Model,
    Chain_Ready, Chain_Forward, Chain_Forward_Batch) over the reference's
    chain ABI, with ``layer`` (aspida_kq_chain_layer) in place of
    Chain_Dnet / Chain_Fattn.  Weights are copied into HBM at registration,
    so the arrays may be dropped afterwards.  Matrices are (array, kind)
    pairs: uint8 GGML bytes, or f32 [out][in] for kind -1.
    """

    def __init__(self, path=None):
        self.lib = load(path)
        self.dim = self.vocab = 0

    def last_error(self):
        return self.lib.aspida_gpu_last_error()

    def reset(self):
        self.lib.aspida_gpu_chain_reset()
        self.dim = self.vocab = 0

    def layer(self, attn_norm, post_norm, mix=None):
        an = np.ascontiguousarray(attn_norm, np.float32)
        pn = np.ascontiguousarray(post_norm, np.float32)
        w, k = (None, 0) if mix is None else mix
        return self.lib.aspida_kq_chain_layer(_p(an), an.nbytes, _p(pn), pn.nbytes, _p(w),
                                              0 if w is None else w.nbytes, k)

    def moe(self, router, gate, up, down, shg, shu, shd, n_exp, top_k, intermed, sgi=None):
        args = []
        for arr, kind in (router, gate, up, down, shg, shu, shd):
            args += [_p(arr), arr.nbytes, kind]
        g = None if sgi is None else np.ascontiguousarray(sgi, np.float32)
        self.lib.aspida_gpu_chain_moe(*args, _p(g), 0 if g is None else g.nbytes, 0 if g is None else g.size,
                                      n_exp, top_k, intermed)

    def model(self, embed, fnorm, lm, dim, vocab):
        e = np.ascontiguousarray(embed, np.float32)
        f = np.ascontiguousarray(fnorm, np.float32)
        w, k = lm
        self.lib.aspida_gpu_chain_model(_p(e), e.nbytes, _p(f), f.nbytes, _p(w), w.nbytes, k, dim, vocab)
        self.dim, self.vocab = dim, vocab

    def ready(self):
        return self.lib.aspida_gpu_chain_ready() == 1

    def begin(self):
        self.lib.aspida_gpu_chain_begin(None)

    def end(self):
        self.lib.aspida_gpu_chain_end()

    def forward(self, row, pos=0):
        y = np.empty(self.vocab, np.float32)
        self.lib.aspida_gpu_chain_forward(int(row), int(pos), None, _p(y))
        return y

    def forward_batch(self, rows, pos=None):
        r = np.ascontiguousarray(rows, np.int32)
        ps = np.zeros(r.size, np.int32) if pos is None else np.ascontiguousarray(pos, np.int32)
        y = np.empty((r.size, self.vocab), np.float32)
        self.lib.aspida_gpu_chain_forward_batch(r.size, _p(r), _p(ps), None, _p(y))
        return y

    def hidden(self, rows, n_layers):
        """Residual stream [len(rows)][dim] after the first n_layers layers."""
        r = np.ascontiguousarray(np.atleast_1d(rows), np.int32)
        h = np.empty((r.size, self.dim), np.float32)
        rc = self.lib.aspida_kq_chain_forward_layers(r.size, _p(r), n_layers, _p(h))
        if rc:
            raise RuntimeError(f"aspida_kq_chain_forward_layers rc={rc}")
        return h

    def set_graphs(self, on):
        return self.lib.aspida_kq_chain_set_graphs(1 if on else 0)

    def graphs(self):
        return self.lib.aspida_kq_chain_graphs()


class DeviceOps:
    """Device-pointer entry points; pointers and the stream are plain ints."""

    def __init__(self, path=None):
        self.lib = load(path)

    def _ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with code {rc}")

    def xsum(self, x, in_dim, rows, xq, stream=0):
        self._ok(self.lib.aspida_kq_xsum_dev(x, in_dim, rows, xq, stream), "aspida_kq_xsum_dev")

    def matvec(self, kind, w, in_dim, out_dim, x, xq, y, stream=0):
        self._ok(self.lib.aspida_kq_matvec_dev(kind, w, in_dim, out_dim, x, xq, y, stream), "aspida_kq_matvec_dev")

    def packed_bytes(self, kind, in_dim, out_dim):
        return int(self.lib.aspida_kq_packed_bytes(kind, in_dim, out_dim))

    def packed_plan(self, in_dim, out_dim):
        """(waves per workgroup, workgroups per tile, columns per wave)."""
        v = [ctypes.c_int(0) for _ in range(3)]
        self._ok(self.lib.aspida_kq_packed_plan(in_dim, out_dim, *[ctypes.byref(a) for a in v]),
                 "aspida_kq_packed_plan")
        return tuple(a.value for a in v)

    def matvec_plan(self, kind, in_dim, out_dim):
        """(uses the MFMA kernel, waves per workgroup, workgroups per tile,
        columns per wave, columns taken one after another, 16-row
        workgroups) of
        aspida_kq_matvec_packed_dev for this kind."""
        v = [ctypes.c_int(0) for _ in range(3)]
        rc = self.lib.aspida_kq_matvec_plan(kind, in_dim, out_dim, *[ctypes.byref(a) for a in v])
        if rc < 0:
            raise RuntimeError(f"aspida_kq_matvec_plan failed with code {rc}")
        return (rc >= 1,) + tuple(a.value for a in v) + (rc in (2, 4), rc >= 3)

    def pack(self, kind, w, in_dim, out_dim, packed, stream=0):
        self._ok(self.lib.aspida_kq_pack_dev(kind, w, in_dim, out_dim, packed, stream), "aspida_kq_pack_dev")

    def unpack(self, kind, packed, in_dim, out_dim, w, stream=0):
        self._ok(self.lib.aspida_kq_unpack_dev(kind, packed, in_dim, out_dim, w, stream), "aspida_kq_unpack_dev")

    def matvec_packed(self, kind, packed, in_dim, out_dim, x, y, stream=0):
        self._ok(self.lib.aspida_kq_matvec_packed_dev(kind, packed, in_dim, out_dim, x, y, stream),
                 "aspida_kq_matvec_packed_dev")

    def matvec2_packed(self, kind_a, packed_a, out_a, y_a, kind_b, packed_b, out_b, y_b, in_dim, x, stream=0):
        self._ok(self.lib.aspida_kq_matvec2_packed_dev(kind_a, packed_a, out_a, y_a, kind_b, packed_b, out_b, y_b,
                                                       in_dim, x, stream), "aspida_kq_matvec2_packed_dev")

    def matmul_packed(self, kind, packed, in_dim, out_dim, batch, x, y, stream=0):
        self._ok(self.lib.aspida_kq_matmul_packed_dev(kind, packed, in_dim, out_dim, batch, x, y, stream),
                 "aspida_kq_matmul_packed_dev")

    def matmul(self, kind, w, in_dim, out_dim, batch, x, xq, y, stream=0, valu=False):
        fn = self.lib.aspida_kq_matmul_valu_dev if valu else self.lib.aspida_kq_matmul_dev
        self._ok(fn(kind, w, in_dim, out_dim, batch, x, xq, y, stream), "aspida_kq_matmul_dev")

    def dequant(self, kind, w, in_dim, out_dim, dst, stream=0):
        self._ok(self.lib.aspida_kq_dequant_dev(kind, w, in_dim, out_dim, dst, stream), "aspida_kq_dequant_dev")

    def dense(self, w, in_dim, out_dim, x, y, stream=0):
        self._ok(self.lib.aspida_dense_matvec_dev(w, in_dim, out_dim, x, y, stream), "aspida_dense_matvec_dev")

    def route(self, router_w, n_exp, dim, T, top_k, x, logits, top_idx, top_w, stream=0):
        self._ok(self.lib.aspida_moe_route_dev(router_w, n_exp, dim, T, top_k, x, logits, top_idx, top_w, stream),
                 "aspida_moe_route_dev")

    def moe_work_floats(self, T, dim, top_k, intermed):
        return int(self.lib.aspida_moe_work_floats(T, dim, top_k, intermed))

    def moe_experts(self, x, T, dim, top_k, intermed, n_exp, top_idx, top_w, gate, up, down, shg, shu, shd,
                    shared_gate_inp, work, y, stream=0):
        """gate/up/down: (ptr, stride_bytes, kind); shg/shu/shd: (ptr, kind)."""
        args = [*gate, *up, *down, *shg, *shu, *shd]
        self._ok(self.lib.aspida_moe_experts_dev(x, T, dim, top_k, intermed, n_exp, top_idx, top_w, *args,
                                                 shared_gate_inp or 0, work, y, stream),
                 "aspida_moe_experts_dev")

    def moe_packed_work_bytes(self, T, dim, intermed, top_k):
        n = int(self.lib.aspida_moe_packed_work_bytes(T, dim, intermed, top_k))
        if n < 0:
            raise ValueError(f"aspida_moe_packed_work_bytes: bad arguments ({T}, {dim}, {intermed}, {top_k})")
        return n

    def pack_experts(self, kind, src, src_stride, in_dim, out_dim, n, dst, stream=0):
        """Pack n ggml matrices src_stride bytes apart into dst, packed_bytes apart."""
        self._ok(self.lib.aspida_moe_pack_experts_dev(kind, src, src_stride, in_dim, out_dim, n, dst, stream),
                 "aspida_moe_pack_experts_dev")

    def moe_experts_packed(self, x, T, dim, top_k, intermed, n_exp, top_idx, top_w, gate, up, gu_kind, down,
                           down_kind, shg, shu, shd, shared_gate_inp, work, y, stream=0):
        """Grouped MoE experts over packed expert tensors (device pointers)."""
        self._ok(self.lib.aspida_moe_experts_packed_dev(x, T, dim, top_k, intermed, n_exp, top_idx, top_w, gate, up,
                                                        gu_kind, down, down_kind, shg, shu, shd,
                                                        shared_gate_inp or 0, work, y, stream),
                 "aspida_moe_experts_packed_dev")

    def chain(self, steps):
        """A resident decode chain over steps [(kind, packed_ptr, in_dim, out_dim, x_ptr, y_ptr), ...]."""
        return Chain(self.lib, steps)

    def set_mv_config(self, rows_per_wave=0, waves_per_cu=16):
        self._ok(self.lib.aspida_kq_set_mv_config(rows_per_wave, waves_per_cu), "aspida_kq_set_mv_config")

    def set_mv_engine(self, engine):
        """0: MFMA for Q4_K and Q6_K (default), 1: the VALU kernel for every kind."""
        self._ok(self.lib.aspida_kq_set_mv_engine(engine), "aspida_kq_set_mv_engine")

    def set_mfma_rows(self, mode):
        """Matrix-core matvec workgroups: 0 built-in choice, 1 64-row, 2 16-row."""
        self._ok(self.lib.aspida_kq_set_mfma_rows(mode), "aspida_kq_set_mfma_rows")

    def set_mm_engine(self, engine):
        """Batches > 1: 0 built-in choice, 1 VALU, 2 64-vector MFMA, 3 16-vector MFMA,
        4 one-pass MFMA, 5 batch-1 MFMA on up to 4 vectors, 6 wave-per-column MFMA."""
        self._ok(self.lib.aspida_kq_set_mm_engine(engine), "aspida_kq_set_mm_engine")


class KqStep(ctypes.Structure):
    """aspida_kq_step (include/aspidagpu.h)."""
    _fields_ = [("kind", ctypes.c_int), ("in_dim", ctypes.c_int), ("out_dim", ctypes.c_int),
                ("reserved", ctypes.c_int), ("packed", ctypes.c_void_p), ("x", ctypes.c_void_p),
                ("y", ctypes.c_void_p)]


class Chain:
    """aspida_kq_chain_*: create on construction, run(stream), check(), close()."""

    def __init__(self, lib, steps):
        self.lib = lib
        arr = (KqStep * len(steps))(*[KqStep(k, i, o, 0, p, x, y) for k, p, i, o, x, y in steps])
        self.h = lib.aspida_kq_chain_create(arr, len(steps))
        if not self.h:
            raise RuntimeError(f"aspida_kq_chain_create failed (error {lib.aspida_gpu_last_error()})")

    def run(self, stream=0):
        rc = self.lib.aspida_kq_chain_run(self.h, stream)
        if rc:
            raise RuntimeError(f"aspida_kq_chain_run: error {rc}")

    def check(self):
        """True when every dependency wait since the last check completed."""
        rc = self.lib.aspida_kq_chain_check(self.h)
        if rc < 0:
            raise RuntimeError(f"aspida_kq_chain_check: error {rc}")
        return rc == 0

    def workgroups(self):
        return int(self.lib.aspida_kq_chain_workgroups(self.h))

    def close(self):
        if self.h:
            self.lib.aspida_kq_chain_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

