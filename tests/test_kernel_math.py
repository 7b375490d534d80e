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


def _emul_packed(emul):
    emul.kq_emul_packed_offset.restype = ctypes.c_int
    emul.kq_emul_packed_offset.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    emul.kq_emul_packed_row.restype = ctypes.c_float
    emul.kq_emul_packed_row.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    return emul


def packed_offsets(emul, kind):
    bb = oracle.BLOCK_BYTES[kind]
    return np.array([[emul.kq_emul_packed_offset(kind, r, b) for b in range(bb)] for r in range(64)], np.int64)


@pytest.mark.parametrize("kind", list(oracle.KQUANTS) + [oracle.KIND_Q8_0])
def test_packed_layout_is_a_permutation(emul, kind):
    """Every byte of the 64 super-blocks of a (tile, column) group has its own
    slot, and the slots fill exactly 64 * block bytes."""
    off = packed_offsets(_emul_packed(emul), kind)
    assert sorted(off.ravel().tolist()) == list(range(64 * oracle.BLOCK_BYTES[kind]))


@pytest.mark.parametrize("kind", list(oracle.KQUANTS) + [oracle.KIND_Q8_0])
def test_packed_rows_match_oracle(emul, kind):
    """Each lane's registers (Packed<K>::load) and quarter views
    (Packed<K>::quarter) over a packed group reproduce the row's dot product:
    the chunk indices agree with the ggml field offsets of every format."""
    emul = _emul_packed(emul)
    bb = oracle.BLOCK_BYTES[kind]
    off = packed_offsets(emul, kind)
    gen = synth.rng(700 + kind)
    rows = synth.blocks_np(kind, 64, gen).reshape(64, bb)
    rows[::7] = gen.integers(0, 256, (len(rows[::7]), bb), dtype=np.uint8)   # raw bytes too
    buf = np.zeros(64 * bb + 32, np.uint8)
    base = (16 - buf.ctypes.data % 16) % 16
    grp = buf[base:base + 64 * bb]
    grp[off.ravel()] = rows.ravel()
    x = synth.activations_np(256, gen)
    s16 = x.reshape(16, 16).sum(1, dtype=np.float32)
    w = oracle.dequant(kind, rows.ravel(), 256, 64).astype(np.float64)
    ref = w @ x.astype(np.float64)
    scale = np.abs(w) @ np.abs(x.astype(np.float64))
    got = np.array([emul.kq_emul_packed_row(kind, grp.ctypes.data, r, x.ctypes.data, s16.ctypes.data)
                    for r in range(64)])
    err = np.abs(got - ref) / np.maximum(scale, 1e-30)
    assert err.max() < 1e-6, err.max()


def test_mv16_block_order_is_a_permutation_keeping_tiles_on_one_xcd(emul):
    """The 16-row kernels' block order (mv16_block, kq_packed.h): for every
    grid size it is a permutation of the blocks, so each block is computed
    exactly once; within whole rounds of 32 workgroups the four blocks of a
    64-row tile go to workgroups of one XCD (workgroup p on XCD p % 8) and of
    one round, and the rows of a partial last round keep their order."""
    f = emul.kq_emul_mv16_block
    f.restype = ctypes.c_int
    f.argtypes = [ctypes.c_int, ctypes.c_int]
    for n in list(range(1, 300)) + [1000, 1024, 4096, 8017, 32064]:
        blocks = [f(p, n) for p in range(n)]
        assert sorted(blocks) == list(range(n)), n
        full = n - n % 32
        where = {b: p for p, b in enumerate(blocks)}
        for t in range(full // 4):
            ps = [where[4 * t + r] for r in range(4)]
            assert len({p % 8 for p in ps}) == 1, (n, t, ps)
            assert len({p // 32 for p in ps}) == 1, (n, t, ps)
        assert blocks[full:] == list(range(full, n)), n
