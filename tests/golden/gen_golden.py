"""Generate the golden fixtures under tests/golden/ (run from the repo root):

    python tests/golden/gen_golden.py

Nothing here calls the oracle or the GPU library.  Expected values come from
an independent restatement of the ggml K-quant layouts (element -> bit fields
-> scale index, written out below from the block descriptions) evaluated
with exact arithmetic: every product d*sc*q and dmin*m is exact in binary64,
and so is their difference, so a single numpy float32() rounding gives the
correctly rounded f32 -- the value the CPU decoders produce with one rounding
(src/llm/llm_dequant.adb:122-554).  Each value is cross-checked against
fractions.Fraction.

Fixtures:
  kq_kat.npz     known-answer blocks.  Q2_K/Q3_K are the hand-built blocks of
                 the reference test tests/test_kquant_synth.adb:110-179 (same
                 scale/min/code patterns, same inverse packing, d=0.5,
                 dmin=0.25), with its x pattern 0.01*((i mod 11)-5) for the
                 fused-dot check; Q4_K/Q5_K/Q6_K/Q8_0 are analogous blocks
                 built by packing chosen codes and scales.
  kq_random.npz  seeded random blocks per kind (scales ~ |N(0, 2e-3)| in f16,
                 some replaced by +-0, subnormals, max normal, +-Inf and NaN)
                 and their exact dequantized values.
  kq_matvec.npz  small random matrices + activations with exact dot products
                 (binary64 of the exact rational sum) and sum |w_i x_i|.
  moe_kat.npz    tests/test_moe.adb's tiny dense MoE (2 experts, dim 2,
                 intermed 2, x = (0.7, -0.2)) with fp64 expected outputs for
                 top-k 2 and 1.
"""
import math
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
BLOCK_BYTES = {0: 144, 1: 210, 2: 176, 3: 110, 4: 84, 5: 272}
NAMES = {0: "q4k", 1: "q6k", 2: "q5k", 3: "q3k", 4: "q2k", 5: "q80"}


# ---- f16 ---------------------------------------------------------------------

def f16_val(lo, hi):
    """Half from two LE bytes, exponent 31 read as +0.0 (llm_dequant.adb:46-48)."""
    h = int(lo) | (int(hi) << 8)
    if (h >> 10) & 0x1F == 31:
        return 0.0
    return float(np.array([h], np.uint16).view(np.float16)[0])


def f16_bytes(v):
    h = int(np.array([v], np.float16).view(np.uint16)[0])
    return h & 0xFF, h >> 8


# ---- element -> fields maps (one per format) ----------------------------------

def scale_min_k4(sc, j):
    """(scale, min) j of the 12 packed bytes shared by Q4_K/Q5_K."""
    if j < 4:
        return sc[j] & 63, sc[j + 4] & 63
    return (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4), (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4)


def q3_scale(sc12, i):
    """Signed 6-bit scale i of Q3_K: low nibble from byte i%8 (high nibble when
    i >= 8), top two bits from byte 8 + i%4 at bit 2*(i//4)."""
    lo = (sc12[i % 8] >> (4 * (i // 8))) & 0xF
    hi = (sc12[8 + i % 4] >> (2 * (i // 4))) & 3
    return (lo | (hi << 4)) - 32


def terms(kind, b, p):
    """(scale_coeff, code, min_coeff) such that w = scale_coeff*code - min_coeff
    exactly, for element p of block bytes b (python ints / floats)."""
    b = [int(v) for v in b]
    if kind == 0:    # Q4_K: d, dmin, sc[12], qs[128]
        g, hi, l = p // 64, (p % 64) // 32, p % 32
        s, m = scale_min_k4(b[4:16], 2 * g + hi)
        q = b[16 + 32 * g + l]
        code = (q >> 4) if hi else (q & 0xF)
        return f16_val(b[0], b[1]) * s, code, f16_val(b[2], b[3]) * m
    if kind == 2:    # Q5_K: d, dmin, sc[12], qh[32], qs[128]
        g, hi, l = p // 64, (p % 64) // 32, p % 32
        s, m = scale_min_k4(b[4:16], 2 * g + hi)
        q = b[48 + 32 * g + l]
        code = ((q >> 4) if hi else (q & 0xF)) + (((b[16 + l] >> (2 * g + hi)) & 1) << 4)
        return f16_val(b[0], b[1]) * s, code, f16_val(b[2], b[3]) * m
    if kind == 1:    # Q6_K: ql[128], qh[64], int8 sc[16], d
        h, k, l = p // 128, (p % 128) // 32, p % 32
        ql = b[64 * h + l + 32 * (k & 1)]
        nib = (ql >> 4) if (k & 2) else (ql & 0xF)
        code = (nib | (((b[128 + 32 * h + l] >> (2 * k)) & 3) << 4)) - 32
        sc = b[192 + 8 * h + l // 16 + 2 * k]
        sc = sc - 256 if sc >= 128 else sc
        return f16_val(b[208], b[209]) * sc, code, 0.0
    nh, j, g, l = p // 128, (p % 128) // 32, (p % 32) // 16, p % 16
    if kind == 3:    # Q3_K: hmask[32], qs[64], sc[12], d
        low2 = (b[32 + 32 * nh + 16 * g + l] >> (2 * j)) & 3
        hbit = (b[16 * g + l] >> (4 * nh + j)) & 1
        return f16_val(b[108], b[109]) * q3_scale(b[96:108], 8 * nh + 2 * j + g), low2 + 4 * hbit - 4, 0.0
    if kind == 4:    # Q2_K: sc[16], qs[64], d, dmin
        s = b[8 * nh + 2 * j + g]
        q = (b[16 + 32 * nh + 16 * g + l] >> (2 * j)) & 3
        return f16_val(b[80], b[81]) * (s & 0xF), q, f16_val(b[82], b[83]) * (s >> 4)
    if kind == 5:    # Q8_0: 8 x (d, int8[32])
        blk, e = p // 32, p % 32
        q = b[34 * blk + 2 + e]
        return f16_val(b[34 * blk], b[34 * blk + 1]), q - 256 if q >= 128 else q, 0.0
    raise ValueError(kind)


def exact_f32(a, code, m):
    """float32 of a*code - m with one rounding; asserts binary64 was exact."""
    v = a * code - m
    fr = Fraction(a) * code - Fraction(m)
    assert Fraction(v) == fr, (a, code, m)
    return np.float32(v)


def dequant_block(kind, blk):
    return np.array([exact_f32(*terms(kind, blk, p)) for p in range(256)], np.float32)


# ---- known-answer blocks ------------------------------------------------------

def kq_split(p):
    return p // 128, (p % 128) // 32, (p % 32) // 16, p % 16


def kat_q2k():
    """tests/test_kquant_synth.adb:110-137."""
    blk = np.zeros(84, np.int64)
    sc4 = [(s % 7) + 1 for s in range(16)]
    mn4 = [s % 5 for s in range(16)]
    for s in range(16):
        blk[s] = sc4[s] + 16 * mn4[s]
    exp = np.zeros(256, np.float32)
    for p in range(256):
        nh, j, g, l = kq_split(p)
        q = p % 4
        blk[16 + nh * 32 + g * 16 + l] += q * (1 << (2 * j))
        iss = nh * 8 + j * 2 + g
        exp[p] = np.float32(0.5 * sc4[iss] * q - 0.25 * mn4[iss])
    blk[80], blk[81] = f16_bytes(0.5)
    blk[82], blk[83] = f16_bytes(0.25)
    return blk.astype(np.uint8), exp


def kat_q3k():
    """tests/test_kquant_synth.adb:143-179."""
    blk = np.zeros(110, np.int64)
    sc6 = [(s * 4) % 64 for s in range(16)]
    for k in range(4):
        blk[96 + k] = (sc6[k] % 16) + (sc6[8 + k] % 16) * 16
        blk[100 + k] = (sc6[4 + k] % 16) + (sc6[12 + k] % 16) * 16
        blk[104 + k] = sc6[k] // 16 + (sc6[4 + k] // 16) * 4 + (sc6[8 + k] // 16) * 16 + (sc6[12 + k] // 16) * 64
    exp = np.zeros(256, np.float32)
    for p in range(256):
        nh, j, g, l = kq_split(p)
        q3 = p % 8
        blk[32 + nh * 32 + g * 16 + l] += (q3 % 4) * (1 << (2 * j))
        blk[g * 16 + l] += (q3 // 4) * (1 << (nh * 4 + j))
        exp[p] = np.float32(0.5 * (sc6[nh * 8 + 2 * j + g] - 32) * (q3 - 4))
    blk[108], blk[109] = f16_bytes(0.5)
    return blk.astype(np.uint8), exp


def pack_k4_scales(sc, mn):
    """Inverse of get_scale_min_k4 for eight 6-bit (scale, min) pairs."""
    out = [0] * 12
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return out


def kat_q4k():
    sc = [(7 * j + 5) % 64 for j in range(8)]
    mn = [(11 * j + 3) % 64 for j in range(8)]
    blk = np.zeros(144, np.int64)
    blk[0], blk[1] = f16_bytes(0.5)
    blk[2], blk[3] = f16_bytes(0.25)
    blk[4:16] = pack_k4_scales(sc, mn)
    exp = np.zeros(256, np.float32)
    for p in range(256):
        g, hi, l = p // 64, (p % 64) // 32, p % 32
        q = (p * 7 + 3) % 16
        blk[16 + 32 * g + l] += q << (4 * hi)
        exp[p] = np.float32(0.5 * sc[2 * g + hi] * q - 0.25 * mn[2 * g + hi])
    return blk.astype(np.uint8), exp


def kat_q5k():
    sc = [(13 * j + 2) % 64 for j in range(8)]
    mn = [(5 * j + 9) % 64 for j in range(8)]
    blk = np.zeros(176, np.int64)
    blk[0], blk[1] = f16_bytes(0.5)
    blk[2], blk[3] = f16_bytes(0.25)
    blk[4:16] = pack_k4_scales(sc, mn)
    exp = np.zeros(256, np.float32)
    for p in range(256):
        g, hi, l = p // 64, (p % 64) // 32, p % 32
        q = (p * 11 + 1) % 32
        blk[48 + 32 * g + l] += (q & 15) << (4 * hi)
        blk[16 + l] += (q >> 4) << (2 * g + hi)
        exp[p] = np.float32(0.5 * sc[2 * g + hi] * q - 0.25 * mn[2 * g + hi])
    return blk.astype(np.uint8), exp


def kat_q6k():
    sc = [((9 * i + 4) % 256) - 128 for i in range(16)]
    blk = np.zeros(210, np.int64)
    for i in range(16):
        blk[192 + i] = sc[i] & 0xFF
    blk[208], blk[209] = f16_bytes(0.5)
    exp = np.zeros(256, np.float32)
    for p in range(256):
        h, k, l = p // 128, (p % 128) // 32, p % 32
        q = (p * 5 + 7) % 64
        blk[64 * h + l + 32 * (k & 1)] += (q & 15) << (4 * (k >> 1))
        blk[128 + 32 * h + l] += (q >> 4) << (2 * k)
        exp[p] = np.float32(0.5 * sc[8 * h + l // 16 + 2 * k] * (q - 32))
    return blk.astype(np.uint8), exp


def kat_q80():
    blk = np.zeros(272, np.int64)
    exp = np.zeros(256, np.float32)
    ds = [0.5, 0.25, 2.0, 1.0, 0.125, 4.0, 0.75, 1.5]
    for k in range(8):
        blk[34 * k], blk[34 * k + 1] = f16_bytes(ds[k])
        for e in range(32):
            q = ((k * 32 + e) * 37) % 256 - 128
            blk[34 * k + 2 + e] = q & 0xFF
            exp[32 * k + e] = np.float32(ds[k] * q)
    return blk.astype(np.uint8), exp


# ---- random blocks --------------------------------------------------------------

SPECIAL_F16 = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x7BFF, 0xFBFF, 0x7C00, 0xFC00, 0x7E00, 0xFE01,
               0x3C00, 0xBC00, 0x7C01]


def f16_scale(rng, n):
    return np.abs(rng.normal(0.0, 2e-3, n)).astype(np.float16).view(np.uint16)


def random_blocks(kind, rng, nblk, special=True):
    """Random bytes, with the f16 scale fields drawn from |N(0, 2e-3)| (some
    replaced by special values when `special`)."""
    bb = BLOCK_BYTES[kind]
    b = rng.integers(0, 256, (nblk, bb), dtype=np.uint8)
    if kind in (0, 2):
        offs = [0, 2]
    elif kind == 1:
        offs = [208]
    elif kind == 3:
        offs = [108]
    elif kind == 4:
        offs = [80, 82]
    else:
        offs = [34 * k for k in range(8)]
    for o in offs:
        v = f16_scale(rng, nblk)
        if special:
            for i in range(0, nblk, 4):
                v[i] = SPECIAL_F16[(i // 4 + o) % len(SPECIAL_F16)]
        b[:, o] = v & 0xFF
        b[:, o + 1] = v >> 8
    return b


# ---- MoE known-answer case (tests/test_moe.adb) --------------------------------

def moe_kat():
    n_exp, dim, ff = 2, 2, 2

    def mk(rows, cols, seed):
        return np.array([[np.float32(0.1) * np.float32(((r * 7 + c * 3 + seed) % 11) - 5) for c in range(1, cols + 1)]
                         for r in range(1, rows + 1)], np.float32)

    def mk3(d1, d2, d3, seed):
        return np.array([[[np.float32(0.1) * np.float32(((a * 13 + b * 7 + c * 3 + seed) % 11) - 5)
                           for c in range(1, d3 + 1)]
                          for b in range(1, d2 + 1)] for a in range(1, d1 + 1)], np.float32)

    w = dict(gate_inp=mk(n_exp, dim, 1), gate_exp=mk3(n_exp, ff, dim, 2), up_exp=mk3(n_exp, ff, dim, 3),
             down_exp=mk3(n_exp, dim, ff, 4), sh_gate=mk(ff, dim, 5), sh_up=mk(ff, dim, 6), sh_down=mk(dim, ff, 7))
    x = np.array([0.7, -0.2], np.float32)
    f = {k: v.astype(np.float64) for k, v in w.items()}
    xd = x.astype(np.float64)

    def silu(v):
        return v / (1.0 + math.exp(-v))

    def swiglu(g, u, d):
        h = np.array([silu(a) * b for a, b in zip(g @ xd, u @ xd)])
        return d @ h

    logits = f["gate_inp"] @ xd
    p = np.exp(logits - logits.max())
    p /= p.sum()
    out = {}
    for top_k in (2, 1):
        order = sorted(range(n_exp), key=lambda e: (-p[e], e))[:top_k]
        wsum = sum(p[e] for e in order)
        y = np.zeros(dim)
        for e in order:
            y += (p[e] / wsum) * swiglu(f["gate_exp"][e], f["up_exp"][e], f["down_exp"][e])
        y += swiglu(f["sh_gate"], f["sh_up"], f["sh_down"])
        out[f"expected_top{top_k}"] = y
        out[f"idx_top{top_k}"] = np.array(order, np.int32)
    return dict(x=x, **w, **out)


def main():
    rng = np.random.Generator(np.random.PCG64(20261201))
    kat = {}
    # Ada: 0.01 * Float(k) in single precision
    xpat = np.array([np.float32(0.01) * np.float32((i % 11) - 5) for i in range(1, 257)], np.float32)
    kat["x_pattern"] = xpat
    for name, fn in (("q2k", kat_q2k), ("q3k", kat_q3k), ("q4k", kat_q4k), ("q5k", kat_q5k), ("q6k", kat_q6k),
                     ("q80", kat_q80)):
        blk, exp = fn()
        kind = {v: k for k, v in NAMES.items()}[name]
        # the packing must agree with the independent field map
        assert np.array_equal(dequant_block(kind, blk).view(np.uint32), exp.view(np.uint32)), name
        kat[f"{name}_block"] = blk
        kat[f"{name}_expected"] = exp
        dot = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(exp, xpat))
        kat[f"{name}_dot"] = np.float64(float(dot))
    np.savez_compressed(os.path.join(HERE, "kq_kat.npz"), **kat)

    rnd = {}
    for kind, name in NAMES.items():
        blocks = random_blocks(kind, rng, 48)
        rnd[f"{name}_blocks"] = blocks
        rnd[f"{name}_expected"] = np.stack([dequant_block(kind, b) for b in blocks])
    np.savez_compressed(os.path.join(HERE, "kq_random.npz"), **rnd)

    mv = {}
    for kind, name in NAMES.items():
        out_dim, in_dim = 6, 512
        blocks = random_blocks(kind, rng, out_dim * in_dim // 256, special=False)
        x = rng.standard_normal(in_dim).astype(np.float32)
        wrows = np.stack([dequant_block(kind, b) for b in blocks]).reshape(out_dim, in_dim)
        dots, mags = [], []
        for o in range(out_dim):
            dots.append(float(sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(wrows[o], x))))
            mags.append(float(np.sum(np.abs(wrows[o].astype(np.float64) * x.astype(np.float64)))))
        mv[f"{name}_w"] = blocks.reshape(-1)
        mv[f"{name}_x"] = x
        mv[f"{name}_dot"] = np.array(dots)
        mv[f"{name}_mag"] = np.array(mags)
        mv[f"{name}_shape"] = np.array([out_dim, in_dim], np.int32)
    np.savez_compressed(os.path.join(HERE, "kq_matvec.npz"), **mv)

    np.savez_compressed(os.path.join(HERE, "moe_kat.npz"), **moe_kat())
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))


if __name__ == "__main__":
    main()
