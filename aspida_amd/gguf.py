"""GGUF model files: tensor layout through libaspidagpu's reader (aspida_gguf_*).

The reader applies the reference loader's rules (src/llm/llm_gguf.adb:317-560);
this module wraps it, maps a tensor's bytes from the file, and hands K-quant
weights to the packed device path.  dims[0] is ne0 (a weight's in_dim), dims[1]
ne1 (its out_dim), as LLM_Weight reads them (src/llm/llm_weight.adb:115-131).
"""
import ctypes

import numpy as np

from . import load, KIND_NAMES


class TensorInfo(ctypes.Structure):
    """aspida_gguf_tensor_info (include/aspidagpu.h)."""
    _fields_ = [("name", ctypes.c_char_p), ("ggml_type", ctypes.c_int), ("kind", ctypes.c_int),
                ("n_dims", ctypes.c_int), ("dims", ctypes.c_longlong * 4), ("file_offset", ctypes.c_longlong),
                ("bytes", ctypes.c_longlong)]


def _bind(lib):
    P, I, LL, S = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong, ctypes.c_char_p
    for name, res, args in (("aspida_gguf_open", P, [S]), ("aspida_gguf_error", S, []),
                            ("aspida_gguf_close", None, [P]), ("aspida_gguf_version", I, [P]),
                            ("aspida_gguf_alignment", LL, [P]), ("aspida_gguf_data_start", LL, [P]),
                            ("aspida_gguf_tensor_count", LL, [P]), ("aspida_gguf_meta_count", LL, [P]),
                            ("aspida_gguf_meta", S, [P, S]), ("aspida_gguf_find", LL, [P, S]),
                            ("aspida_gguf_tensor", I, [P, LL, ctypes.POINTER(TensorInfo)]),
                            ("aspida_gguf_read", LL, [P, LL, P, LL])):
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


# The Q4_K_M mix: Q6_K for the output head and every attn_v and ffn_down
# projection, Q4_K elsewhere (tools/probes/requantize.adb:103-113).
def q4_k_m_kind(name):
    if name == "output.weight" or name.endswith("attn_v.weight") or name.endswith("ffn_down.weight"):
        return 1   # Q6_K
    return 0       # Q4_K


class GGUFFile:
    """A parsed GGUF file.  Raises ValueError on a malformed one."""

    def __init__(self, path, lib=None):
        self.lib = _bind(lib or load())
        self.path = str(path)
        self.h = self.lib.aspida_gguf_open(self.path.encode())
        if not self.h:
            raise ValueError(f"{self.path}: {self.lib.aspida_gguf_error().decode()}")
        self.version = self.lib.aspida_gguf_version(self.h)
        self.alignment = self.lib.aspida_gguf_alignment(self.h)
        self.data_start = self.lib.aspida_gguf_data_start(self.h)
        self.tensors = []
        for i in range(self.lib.aspida_gguf_tensor_count(self.h)):
            t = TensorInfo()
            if self.lib.aspida_gguf_tensor(self.h, i, ctypes.byref(t)):
                raise ValueError(f"{self.path}: tensor {i} unreadable")
            self.tensors.append({"name": t.name.decode(), "ggml_type": t.ggml_type, "kind": t.kind,
                                 "dims": [t.dims[d] for d in range(t.n_dims)], "offset": t.file_offset,
                                 "bytes": t.bytes})
        self.by_name = {t["name"]: t for t in self.tensors}

    def meta(self, key):
        v = self.lib.aspida_gguf_meta(self.h, key.encode())
        return None if v is None else v.decode(errors="replace")

    def data(self, name):
        """The tensor's bytes, memory-mapped read-only from the file."""
        t = self.by_name[name]
        return np.memmap(self.path, dtype=np.uint8, mode="r", offset=t["offset"], shape=(t["bytes"],))

    def weight(self, name):
        """(bytes, kind, in_dim, out_dim) of a K-quant or Q8_0 weight matrix."""
        t = self.by_name[name]
        if t["kind"] < 0:
            raise ValueError(f"{name}: GGML type {t['ggml_type']} is not a kind this library runs")
        dims = t["dims"] + [1] * (2 - len(t["dims"]))
        if len(t["dims"]) > 2 and any(d != 1 for d in t["dims"][2:]):
            raise ValueError(f"{name}: {len(t['dims'])}-d tensor (expert stacks: use expert slices)")
        in_dim, out_dim = int(dims[0]), int(dims[1])
        if in_dim % 256:
            raise ValueError(f"{name}: ne0 = {in_dim} is not a multiple of 256")
        return self.data(name), t["kind"], in_dim, out_dim

    def check_q4_k_m(self):
        """Names of the 2-d weights whose kind differs from the Q4_K_M mix's."""
        return [t["name"] for t in self.tensors
                if t["name"].endswith(".weight") and len(t["dims"]) == 2 and t["kind"] >= 0
                and t["kind"] != q4_k_m_kind(t["name"])]

    def to_device_packed(self, dev, name, stream=None):
        """Upload and pack a weight for the packed kernels on `stream` (torch's
        current stream by default); returns (packed tensor, kind, in_dim, out_dim)."""
        import torch
        raw, kind, in_dim, out_dim = self.weight(name)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        src = torch.from_numpy(np.array(raw)).cuda()
        dst = torch.empty(dev.packed_bytes(kind, in_dim, out_dim), dtype=torch.uint8, device="cuda")
        dev.pack(kind, src.data_ptr(), in_dim, out_dim, dst.data_ptr(), stream)
        torch.cuda.synchronize()
        return dst, kind, in_dim, out_dim

    def close(self):
        if self.h:
            self.lib.aspida_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def summary(self):
        return [(t["name"], KIND_NAMES.get(t["kind"], f"ggml{t['ggml_type']}"), t["dims"], t["bytes"])
                for t in self.tensors]
