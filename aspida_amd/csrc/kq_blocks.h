// kq_blocks.h -- per-format partial dot products over one quarter of a
// super-block (64 of its 256 elements).
//
// For each format, Block<KIND> splits the work of one quarter c (0..3) into
//   load_w(sb, c)        the raw bytes of the super-block at `sb` that quarter
//                        c needs (codes, scales, d/dmin), as dwords;
//   load_x(xs, xq, c, X) the 64 activations quarter c multiplies, from the
//                        super-block's 256 activations xs, and the sums of
//                        its scale sub-blocks' activations from xq, the
//                        per-16 group sums (xsum16 in kq_matvec.hip);
//   dot(W, c, X)         sum_i w_i * x_i over the quarter, where w_i is the
//                        element's dequantized value (the decoders of
//                        src/llm/llm_dequant.adb:122-554).
// quarter(sb, c, xs, xq) chains the three.  Every quarter owns whole scale
// sub-blocks, so it reads each scale once.  Kernels that keep a quarter's
// activations in registers across many rows call load_x once.
//
// Arithmetic.  Instead of forming w_i = d*sc*q_i - dmin*m per element, each
// sub-block s is reduced as (d*sc_s) * sum(q_i x_i) - (dmin*m_s) * sum(x_i),
// with q_i exact small integers fed to v_fma_mix_f32 as f16 subnormals (see
// kq_common.h) and f32 activations and accumulators throughout.  This is a
// different rounding order from the CPU's, not a lower precision: the
// products q_i*x_i are exact and every sum is an f32 sum.  Activations whose
// products fall below 2^-126 (|x| < ~1e-31) lose relative precision.
//
// Alignment.  Q6_K (210 B), Q3_K (110 B) and Q8_0 (34 B blocks) leave fields
// at 2 mod 4; those are read with dword-aligned loads and funnel shifts
// (ld16e / ld12e), which may read up to 2 bytes past the field -- for every
// field below that stays inside its super-block.
#pragma once
#include "kq_common.h"

namespace kq {

// 16 bytes at an even address p, using only dword-aligned loads.  When p % 4
// == 2 this also reads bytes p+16 and p+17.
// The aligned base is formed by pointer arithmetic on p (not through an
// integer), so the compiler keeps the global address space and emits global
// (not flat) loads whose completion it can count precisely.
__device__ __forceinline__ uint4 ld16e(const uint8_t* p) {
  const uint32_t mis = (uint32_t)((uintptr_t)p & 3);
  const uint8_t* q = p - mis;
  const uint32_t sh = mis * 8;
  uint4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(q, 4), 16);
  uint32_t e;
  __builtin_memcpy(&e, __builtin_assume_aligned(q + (sh ? 16 : 12), 4), 4);
  uint4 r;
  r.x = __builtin_amdgcn_alignbit(v.y, v.x, sh);
  r.y = __builtin_amdgcn_alignbit(v.z, v.y, sh);
  r.z = __builtin_amdgcn_alignbit(v.w, v.z, sh);
  r.w = __builtin_amdgcn_alignbit(e, v.w, sh);
  return r;
}

// 12 bytes at an even address p (returned in x, y, z), reading only the
// dwords that overlap [p, p+12).
__device__ __forceinline__ uint4 ld12e(const uint8_t* p) {
  const uint32_t mis = (uint32_t)((uintptr_t)p & 3);
  const uint8_t* q = p - mis;
  const uint32_t sh = mis * 8;
  uint32_t v0, v1, v2, v3;
  __builtin_memcpy(&v0, __builtin_assume_aligned(q, 4), 4);
  __builtin_memcpy(&v1, __builtin_assume_aligned(q + 4, 4), 4);
  __builtin_memcpy(&v2, __builtin_assume_aligned(q + 8, 4), 4);
  __builtin_memcpy(&v3, __builtin_assume_aligned(q + (sh ? 12 : 8), 4), 4);
  uint4 r;
  r.x = __builtin_amdgcn_alignbit(v1, v0, sh);
  r.y = __builtin_amdgcn_alignbit(v2, v1, sh);
  r.z = __builtin_amdgcn_alignbit(v3, v2, sh);
  r.w = 0;
  return r;
}

// Accumulate 4 bytes' worth of codes: `pa` holds the codes of bytes 0 and 2
// of a dword in its two f16 mantissas, `pb` those of bytes 1 and 3; x4 are the
// activations of those four consecutive elements.
__device__ __forceinline__ float fma_quad(uint32_t pa, uint32_t pb, const float* x4, float acc) {
  acc = fma_pair(pa, x4[0], x4[2], acc);
  return fma_pair(pb, x4[1], x4[3], acc);
}

template <int N>
__device__ __forceinline__ void copy_x(float* dst, const float* src) {
#pragma unroll
  for (int i = 0; i < N; ++i) dst[i] = src[i];
}

// Q4_K/Q5_K (scale, min) pair j of the 12 packed bytes (get_scale_min_k4;
// llm_dequant.adb:514-525).  h1/h2/h3 are the scale bytes 0-3, 4-7, 8-11.
// Branch-free: for j < 4 the pair is bytes j and j+4 masked to 6 bits, which
// is the same "low nibble | two bits above it" split with the nibble taken
// from h1/h2 and the two bits from bits 4-5 of the same bytes.
__device__ __forceinline__ void scale_min_k4(uint32_t h1, uint32_t h2, uint32_t h3, int j,
                                             uint32_t& sc, uint32_t& m) {
  const uint32_t b = (uint32_t)(j & 3) * 8;
  const bool hi = j >= 4;
  const uint32_t top = b + (hi ? 6u : 4u);
  sc = bfe(hi ? h3 : h1, b, 4) | (bfe(h1, top, 2) << 4);
  m = bfe(hi ? h3 : h2, b + (hi ? 4u : 0u), 4) | (bfe(h2, top, 2) << 4);
}

// Activations of one quarter: 64 values in the order dot() consumes them, and
// up to four sub-block sums.
struct XQuarter {
  float v[64];
  float s[4];
};

template <int KIND> struct Block;

// ---- Q4_K (144 B): quarter g owns qs[32g..32g+31]: low nibbles are elements
// 64g+l (sub-block 2g), high nibbles 64g+32+l (sub-block 2g+1)
// (Decode_Q4K_Block, llm_dequant.adb:536-553).  X: v[0..31] = x[64g+l],
// v[32..63] = x[64g+32+l]; s[0], s[1] = their sums.
template <> struct Block<Q4_K> {
  static constexpr int BYTES = 144;
  struct W { uint4 h, qa, qb; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int g) {
    return W{ld16(sb), ld16(sb + 16 + 32 * g), ld16(sb + 32 + 32 * g)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int g, XQuarter& x) {
    copy_x<64>(x.v, xs + 64 * g);
    x.s[0] = xq[4 * g] + xq[4 * g + 1];
    x.s[1] = xq[4 * g + 2] + xq[4 * g + 3];
  }
  __device__ static __forceinline__ float dot(const W& wb, int g, const XQuarter& x) {
    const uint32_t w[8] = {wb.qa.x, wb.qa.y, wb.qa.z, wb.qa.w, wb.qb.x, wb.qb.y, wb.qb.z, wb.qb.w};
    float al = 0.f, ah = 0.f;  // units 2^-24 and 2^-20
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t s = w[k] >> 8;
      al = fma_quad(w[k] & 0x000F000Fu, s & 0x000F000Fu, x.v + 4 * k, al);
      ah = fma_quad(w[k] & 0x00F000F0u, s & 0x00F000F0u, x.v + 32 + 4 * k, ah);
    }
    uint32_t s0, m0, s1, m1;
    scale_min_k4(wb.h.y, wb.h.z, wb.h.w, 2 * g, s0, m0);
    scale_min_k4(wb.h.y, wb.h.z, wb.h.w, 2 * g + 1, s1, m1);
    const float d = f16_ada(wb.h.x & 0xFFFFu), dmin = f16_ada(wb.h.x >> 16);
    float r = -(dmin * (float)m0) * x.s[0];
    r = __builtin_fmaf(-(dmin * (float)m1), x.s[1], r);
    r = __builtin_fmaf(d * (float)s0 * 16777216.f, al, r);
    return __builtin_fmaf(d * (float)s1 * 1048576.f, ah, r);
  }
};

// ---- Q5_K (176 B): as Q4_K, with the 5th bit of element 64g+l (resp.
// 64g+32+l) in bit 2g (resp. 2g+1) of qh[l] (Decode_Q5K_Block, 473-497).
template <> struct Block<Q5_K> {
  static constexpr int BYTES = 176;
  struct W { uint4 h, ha, hb, qa, qb; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int g) {
    return W{ld16(sb), ld16(sb + 16), ld16(sb + 32), ld16(sb + 48 + 32 * g), ld16(sb + 64 + 32 * g)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int g, XQuarter& x) {
    Block<Q4_K>::load_x(xs, xq, g, x);
  }
  __device__ static __forceinline__ float dot(const W& wb, int g, const XQuarter& x) {
    const uint32_t w[8] = {wb.qa.x, wb.qa.y, wb.qa.z, wb.qa.w, wb.qb.x, wb.qb.y, wb.qb.z, wb.qb.w};
    const uint32_t hq[8] = {wb.ha.x, wb.ha.y, wb.ha.z, wb.ha.w, wb.hb.x, wb.hb.y, wb.hb.z, wb.hb.w};
    // Rotations that bring bit 2g (resp. 2g+1) of every byte to bit 4.
    const uint32_t rl = (uint32_t)(2 * g + 28) & 31u, rh = (uint32_t)(2 * g + 29) & 31u;
    float al = 0.f, ah = 0.f;  // both in units 2^-24
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t zl = (w[k] & 0x0F0F0F0Fu) | (rotr(hq[k], rl) & 0x10101010u);
      const uint32_t zh = ((w[k] >> 4) & 0x0F0F0F0Fu) | (rotr(hq[k], rh) & 0x10101010u);
      al = fma_quad(zl & 0x001F001Fu, (zl >> 8) & 0x001F001Fu, x.v + 4 * k, al);
      ah = fma_quad(zh & 0x001F001Fu, (zh >> 8) & 0x001F001Fu, x.v + 32 + 4 * k, ah);
    }
    uint32_t s0, m0, s1, m1;
    scale_min_k4(wb.h.y, wb.h.z, wb.h.w, 2 * g, s0, m0);
    scale_min_k4(wb.h.y, wb.h.z, wb.h.w, 2 * g + 1, s1, m1);
    const float d = f16_ada(wb.h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(wb.h.x >> 16);
    float r = -(dmin * (float)m0) * x.s[0];
    r = __builtin_fmaf(-(dmin * (float)m1), x.s[1], r);
    r = __builtin_fmaf(d * (float)s0, al, r);
    return __builtin_fmaf(d * (float)s1, ah, r);
  }
};

// ---- Q6_K (210 B): quarter c = 2h + t owns l = 16t..16t+15 of half h, i.e.
// the four 16-element sub-blocks 8h + t + 2k, k = 0..3, whose 6-bit codes are
// ql[64h+l] (low nibble: k=0, high: k=2), ql[64h+32+l] (k=1, k=3) plus two
// bits of qh[32h+l] (Decode_Q6K_Block, llm_dequant.adb:140-181).
// X: v[16k + i] = x[128h + 16t + 32k + i]; s[k] = its sub-block sum.
template <> struct Block<Q6_K> {
  static constexpr int BYTES = 210;
  struct W { uint4 a, b, q, s; uint32_t d; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int c) {
    const int hh = c >> 1, t = c & 1;
    return W{ld16e(sb + 64 * hh + 16 * t), ld16e(sb + 64 * hh + 32 + 16 * t),
             ld16e(sb + 128 + 32 * hh + 16 * t), ld16e(sb + 192), ld2(sb + 208)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int c, XQuarter& x) {
    const int hh = c >> 1, t = c & 1;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      copy_x<16>(x.v + 16 * k, xs + 128 * hh + 16 * t + 32 * k);
      x.s[k] = xq[8 * hh + t + 2 * k];
    }
  }
  __device__ static __forceinline__ float dot(const W& wb, int c, const XQuarter& x) {
    const int hh = c >> 1, t = c & 1;
    const float d = f16_ada(wb.d) * 16777216.f;
    const uint32_t a[4] = {wb.a.x, wb.a.y, wb.a.z, wb.a.w}, b[4] = {wb.b.x, wb.b.y, wb.b.z, wb.b.w};
    const uint32_t q[4] = {wb.q.x, wb.q.y, wb.q.z, wb.q.w};
    float a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f;  // units 2^-24
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t z1 = (a[k] & 0x0F0F0F0Fu) | ((q[k] << 4) & 0x30303030u);
      const uint32_t z2 = (b[k] & 0x0F0F0F0Fu) | ((q[k] << 2) & 0x30303030u);
      const uint32_t z3 = ((a[k] >> 4) & 0x0F0F0F0Fu) | (q[k] & 0x30303030u);
      const uint32_t z4 = ((b[k] >> 4) & 0x0F0F0F0Fu) | ((q[k] >> 2) & 0x30303030u);
      a1 = fma_quad(z1 & 0x003F003Fu, (z1 >> 8) & 0x003F003Fu, x.v + 4 * k, a1);
      a2 = fma_quad(z2 & 0x003F003Fu, (z2 >> 8) & 0x003F003Fu, x.v + 16 + 4 * k, a2);
      a3 = fma_quad(z3 & 0x003F003Fu, (z3 >> 8) & 0x003F003Fu, x.v + 32 + 4 * k, a3);
      a4 = fma_quad(z4 & 0x003F003Fu, (z4 >> 8) & 0x003F003Fu, x.v + 48 + 4 * k, a4);
    }
    // int8 scales sc[8h + t + 2k]: dword 2h holds k = 0, 1; dword 2h+1 holds k = 2, 3.
    const uint32_t sw0 = hh ? wb.s.z : wb.s.x, sw1 = hh ? wb.s.w : wb.s.y;
    // v_bfe_i32 sign-extends, but the builtin's result type is unsigned:
    // convert from int32_t.
    const float c1 = (float)(int32_t)__builtin_amdgcn_sbfe(sw0, 8 * t, 8);
    const float c2 = (float)(int32_t)__builtin_amdgcn_sbfe(sw0, 8 * t + 16, 8);
    const float c3 = (float)(int32_t)__builtin_amdgcn_sbfe(sw1, 8 * t, 8);
    const float c4 = (float)(int32_t)__builtin_amdgcn_sbfe(sw1, 8 * t + 16, 8);
    // The codes are stored offset by 32: sum (q-32) x = sum q x - 32 sum x.
    const float k32 = 32.f / 16777216.f;
    float r = (d * c1) * (a1 - k32 * x.s[0]);
    r = __builtin_fmaf(d * c2, a2 - k32 * x.s[1], r);
    r = __builtin_fmaf(d * c3, a3 - k32 * x.s[2], r);
    return __builtin_fmaf(d * c4, a4 - k32 * x.s[3], r);
  }
};

// X layout shared by Q3_K and Q2_K: v[16j + l] = x[128nh + 32j + 16g + l],
// s[j] = the sum of that 16-element sub-block.
__device__ __forceinline__ void load_x_nhg(const float* xs, const float* xq, int c, XQuarter& x) {
  const int nh = c >> 1, g = c & 1;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    copy_x<16>(x.v + 16 * j, xs + 128 * nh + 16 * g + 32 * j);
    x.s[j] = xq[8 * nh + g + 2 * j];
  }
}

// ---- Q3_K (110 B): element P = 128nh + 32j + 16g + l has its low two bits
// in field j of qs[32nh+16g+l], its high bit in bit 4nh+j of hmask[16g+l],
// scale index 8nh+2j+g (Decode_Q3K_Block, llm_dequant.adb:247-266).  Quarter
// c = 2nh + g owns the 16-element sub-blocks j = 0..3 of that (nh, g).
template <> struct Block<Q3_K> {
  static constexpr int BYTES = 110;
  struct W { uint4 q, m, s; uint32_t d; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int c) {
    const int nh = c >> 1, g = c & 1;
    return W{ld16e(sb + 32 + 32 * nh + 16 * g), ld16e(sb + 16 * g), ld12e(sb + 96), ld2(sb + 108)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int c, XQuarter& x) {
    load_x_nhg(xs, xq, c, x);
  }
  __device__ static __forceinline__ float dot(const W& wb, int c, const XQuarter& x) {
    const int nh = c >> 1, g = c & 1;
    const float d = f16_ada(wb.d);
    const uint32_t w[4] = {wb.q.x, wb.q.y, wb.q.z, wb.q.w}, hm[4] = {wb.m.x, wb.m.y, wb.m.z, wb.m.w};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // Place the 3-bit code (low2 | hbit << 2) at bit f of each byte: f = 2j
      // for j < 3; field 3 is first shifted down to bit 4 so the high bit stays
      // inside its byte.  Units are 2^(f-24).
      const int f = j < 3 ? 2 * j : 4;
      const uint32_t rot = (uint32_t)(4 * nh + j - (f + 2)) & 31u;
      const uint32_t ins = 0x04040404u << f, pm = 0x00070007u << f;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t lw = j < 3 ? w[k] : (w[k] >> 2);
        const uint32_t v = (rotr(hm[k], rot) & ins) | (lw & ~ins);
        acc[j] = fma_quad(v & pm, (v >> 8) & pm, x.v + 16 * j + 4 * k, acc[j]);
      }
    }
    // 16 signed 6-bit scales (llm_dequant.adb:219-245): scale index 8nh+2j+g is
    // byte (g + 2(j&1)) of S_(2nh + (j>>1)).
    const uint32_t a[2] = {wb.s.x, wb.s.y}, tmp = wb.s.z;
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int jj = j >> 1;
      const uint32_t bt = 8u * (uint32_t)(g + 2 * (j & 1));
      const uint32_t sc6 = bfe(a[jj], bt + 4u * nh, 4) | (bfe(tmp, bt + 4u * nh + 2u * jj, 2) << 4);
      const float ds = d * (float)((int)sc6 - 32);
      const float unit = j < 3 ? (float)(1 << (24 - 2 * j)) : 1048576.f;
      // codes are stored offset by 4: sum (v-4) x = sum v x - 4 sum x.
      r = __builtin_fmaf(ds, __builtin_fmaf(acc[j], unit, -4.f * x.s[j]), r);
    }
    return r;
  }
};

// ---- Q2_K (84 B): element P = 128nh + 32j + 16g + l is field j of
// qs[32nh+16g+l] with scale/min byte 8nh+2j+g (Decode_Q2K_Block,
// llm_dequant.adb:304-320).  Quarter c = 2nh + g owns sub-blocks j = 0..3.
// 84-byte blocks keep every field dword-aligned.
template <> struct Block<Q2_K> {
  static constexpr int BYTES = 84;
  struct W { uint4 q; uint2 s; uint32_t d; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int c) {
    const int nh = c >> 1, g = c & 1;
    return W{ld16(sb + 16 + 32 * nh + 16 * g), ld8(sb + 8 * nh), ld4(sb + 80)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int c, XQuarter& x) {
    load_x_nhg(xs, xq, c, x);
  }
  __device__ static __forceinline__ float dot(const W& wb, int c, const XQuarter& x) {
    const int g = c & 1;
    const float d = f16_ada(wb.d & 0xFFFFu), dmin = f16_ada(wb.d >> 16);
    const uint32_t w[4] = {wb.q.x, wb.q.y, wb.q.z, wb.q.w};
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // units 2^(2j-24)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t s = w[k] >> 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t pm = 0x00030003u << (2 * j);
        acc[j] = fma_quad(w[k] & pm, s & pm, x.v + 16 * j + 4 * k, acc[j]);
      }
    }
    const uint32_t sw[2] = {wb.s.x, wb.s.y};
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t bt = 8u * (uint32_t)(g + 2 * (j & 1));
      const uint32_t scb = sw[j >> 1];
      const float dl = d * (float)bfe(scb, bt, 4) * (float)(1 << (24 - 2 * j));
      const float ml = dmin * (float)bfe(scb, bt + 4, 4);
      r = __builtin_fmaf(dl, acc[j], __builtin_fmaf(-ml, x.s[j], r));
    }
    return r;
  }
};

// ---- Q8_0 (8 x 34 B per 256 elements): quarter c owns 32-element blocks 2c
// and 2c+1; w = d * int8 (Dequant_Q8_0, llm_dequant.adb:606-630).  Codes are
// biased by +128 (x ^ 0x80) so they are unsigned f16 subnormals.
template <> struct Block<Q8_0> {
  static constexpr int BYTES = 272;
  struct W { uint4 a0, b0, a1, b1; uint32_t d0, d1; };
  __device__ static __forceinline__ W load_w(const uint8_t* sb, int c) {
    const uint8_t* b = sb + 68 * c;
    return W{ld16e(b + 2), ld16e(b + 18), ld16e(b + 36), ld16e(b + 52), ld2(b), ld2(b + 34)};
  }
  __device__ static __forceinline__ void load_x(const float* xs, const float* xq, int c, XQuarter& x) {
    Block<Q4_K>::load_x(xs, xq, c, x);
  }
  __device__ static __forceinline__ float half_dot(uint4 A, uint4 B, uint32_t dbits, const float* x, float xs) {
    const uint32_t w[8] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w};
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t u = w[k] ^ 0x80808080u;
      acc = fma_quad(u & 0x00FF00FFu, (u >> 8) & 0x00FF00FFu, x + 4 * k, acc);
    }
    return f16_ada(dbits) * 16777216.f * __builtin_fmaf(-128.f / 16777216.f, xs, acc);
  }
  __device__ static __forceinline__ float dot(const W& wb, int c, const XQuarter& x) {
    (void)c;
    return half_dot(wb.a0, wb.b0, wb.d0, x.v, x.s[0]) + half_dot(wb.a1, wb.b1, wb.d1, x.v + 32, x.s[1]);
  }
};

template <int KIND>
__device__ __forceinline__ float quarter(const uint8_t* sb, int c, const float* xs, const float* xq) {
  XQuarter x;
  Block<KIND>::load_x(xs, xq, c, x);
  return Block<KIND>::dot(Block<KIND>::load_w(sb, c), c, x);
}

}  // namespace kq
