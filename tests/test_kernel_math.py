"""The kernels' per-format block arithmetic (aspida_amd/csrc/kq_blocks.h),
compiled for the host CPU by tests/emul, against the oracle: every quarter
dot of every format within 1e-6 of sum |w_i x_i|, and the dword-aligned load
helpers at both alignments the formats produce.  No GPU needed."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from aspida_amd import synth

LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "emul", "libkq_emul.so")


@pytest.fixture(scope="module")
def emul():
    if not os.path.exists(LIB):
        pytest.skip("tests/emul/libkq_emul.so not built (run build())")
    L = ctypes.CDLL(LIB)
    L.kq_emul_quarter.restype = ctypes.c_float
    L.kq_emul_quarter.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    L.kq_emul_ld16e.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    L.kq_emul_ld12e.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return L


@pytest.mark.parametrize("kind", list(oracle.KQUANTS) + [oracle.KIND_Q8_0])
@pytest.mark.parametrize("offset", [0, 2])
def test_quarter_dots_match_oracle(emul, kind, offset):
    gen = synth.rng(31 * kind + offset)
    bb = oracle.BLOCK_BYTES[kind]
    buf = np.zeros(bb + 64, np.uint8)
    base = (16 - buf.ctypes.data % 16) % 16 + offset   # super-block at 16k + offset
    worst = 0.0
    for t in range(60):
        blk = synth.blocks_np(kind, 1, gen) if t % 3 else gen.integers(0, 256, bb, dtype=np.uint8)
        buf[base:base + bb] = blk
        x = synth.activations_np(256, gen)
        xq = x.reshape(16, 16).sum(1, dtype=np.float32)
        got = sum(emul.kq_emul_quarter(kind, buf.ctypes.data + base, c, x.ctypes.data, xq.ctypes.data)
                  for c in range(4))
        w = oracle.dequant(kind, blk, 256, 1)[0].astype(np.float64)
        scale = np.abs(w) @ np.abs(x.astype(np.float64))
        err = abs(got - w @ x) / max(scale, 1e-30)
        worst = max(worst, err)
    assert worst < 1e-6, worst


@pytest.mark.parametrize("offset", [0, 2, 4, 6])
def test_aligned_loads(emul, offset):
    buf = np.arange(96, dtype=np.uint8)
    base = (16 - buf.ctypes.data % 16) % 16 + offset
    out = np.zeros(16, np.uint8)
    emul.kq_emul_ld16e(buf.ctypes.data + base, out.ctypes.data)
    assert out.tolist() == buf[base:base + 16].tolist()
    out[:] = 0
    emul.kq_emul_ld12e(buf.ctypes.data + base, out.ctypes.data)
    assert out[:12].tolist() == buf[base:base + 12].tolist()
