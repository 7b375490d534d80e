// kq_blocks.h -- per-format partial dot products over one quarter of a
// super-block (64 of its 256 elements).
//
// quarter<KIND>(sb, c, xs, xq) returns sum_i w_i * x_i over the 64 elements
// that quarter c (0..3) of the super-block at `sb` owns, where w_i is the
// element's dequantized value (the decoders of src/llm/llm_dequant.adb:
// 122-554), xs points at the 256 activations of that super-block and xq at
// their 16 sums over consecutive groups of 16 (xsum16 in kq_matvec.hip).
// Every quarter owns whole scale sub-blocks, so it reads each scale once.
//
// Arithmetic.  Instead of forming w_i = d*sc*q_i - dmin*m per element, each
// sub-block s is reduced as (d*sc_s) * sum(q_i x_i) - (dmin*m_s) * sum(x_i),
// with q_i exact small integers fed to v_fma_mix_f32 as f16 subnormals (see
// kq_common.h) and f32 activations and accumulators throughout.  This is a
// different rounding order from the CPU's, not a lower precision: the
// products q_i*x_i are exact and every sum is an f32 sum.  Activations whose
// products fall below 2^-126 (|x| < ~1e-31) lose relative precision.
//
// The element -> (byte, bit field, scale) maps below are the ones of the CPU
// decoders; the comments name the lines each restates.
#pragma once
#include "kq_common.h"

namespace kq {

// Accumulate 4 bytes' worth of codes: `pa` holds the codes of bytes 0 and 2
// of a dword in its two f16 mantissas, `pb` those of bytes 1 and 3; x4 are the
// activations of those four consecutive elements.
__device__ __forceinline__ float fma_quad(uint32_t pa, uint32_t pb, const float* x4, float acc) {
  acc = fma_pair(pa, x4[0], x4[2], acc);
  return fma_pair(pb, x4[1], x4[3], acc);
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

template <int KIND> struct Block;

// ---- Q4_K (144 B): quarter g owns qs[32g..32g+31]: low nibbles are elements
// 64g+l (sub-block 2g), high nibbles 64g+32+l (sub-block 2g+1)
// (Decode_Q4K_Block, llm_dequant.adb:536-553).
template <> struct Block<Q4_K> {
  static constexpr int BYTES = 144;
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int g, const float* xs, const float* xq) {
    const uint4 h = ld16(sb);
    const uint4 qa = ld16(sb + 16 + 32 * g), qb = ld16(sb + 32 + 32 * g);
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const float* xl = xs + 64 * g;
    const float* xh = xl + 32;
    float al = 0.f, ah = 0.f;  // units 2^-24 and 2^-20
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t s = w[k] >> 8;
      al = fma_quad(w[k] & 0x000F000Fu, s & 0x000F000Fu, xl + 4 * k, al);
      ah = fma_quad(w[k] & 0x00F000F0u, s & 0x00F000F0u, xh + 4 * k, ah);
    }
    uint32_t s0, m0, s1, m1;
    scale_min_k4(h.y, h.z, h.w, 2 * g, s0, m0);
    scale_min_k4(h.y, h.z, h.w, 2 * g + 1, s1, m1);
    const float d = f16_ada(h.x & 0xFFFFu), dmin = f16_ada(h.x >> 16);
    const float sl = xq[4 * g] + xq[4 * g + 1], sh = xq[4 * g + 2] + xq[4 * g + 3];
    float r = -(dmin * (float)m0) * sl;
    r = __builtin_fmaf(-(dmin * (float)m1), sh, r);
    r = __builtin_fmaf(d * (float)s0 * 16777216.f, al, r);
    return __builtin_fmaf(d * (float)s1 * 1048576.f, ah, r);
  }
};

// ---- Q5_K (176 B): as Q4_K, with the 5th bit of element 64g+l (resp.
// 64g+32+l) in bit 2g (resp. 2g+1) of qh[l] (Decode_Q5K_Block, 473-497).
template <> struct Block<Q5_K> {
  static constexpr int BYTES = 176;
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int g, const float* xs, const float* xq) {
    const uint4 h = ld16(sb);
    const uint4 ha = ld16(sb + 16), hb = ld16(sb + 32);
    const uint4 qa = ld16(sb + 48 + 32 * g), qb = ld16(sb + 64 + 32 * g);
    const uint32_t w[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    const uint32_t hq[8] = {ha.x, ha.y, ha.z, ha.w, hb.x, hb.y, hb.z, hb.w};
    const float* xl = xs + 64 * g;
    const float* xh = xl + 32;
    // Rotations that bring bit 2g (resp. 2g+1) of every byte to bit 4.
    const uint32_t rl = (uint32_t)(2 * g + 28) & 31u, rh = (uint32_t)(2 * g + 29) & 31u;
    float al = 0.f, ah = 0.f;  // both in units 2^-24
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t zl = (w[k] & 0x0F0F0F0Fu) | (rotr(hq[k], rl) & 0x10101010u);
      const uint32_t zh = ((w[k] >> 4) & 0x0F0F0F0Fu) | (rotr(hq[k], rh) & 0x10101010u);
      al = fma_quad(zl & 0x001F001Fu, (zl >> 8) & 0x001F001Fu, xl + 4 * k, al);
      ah = fma_quad(zh & 0x001F001Fu, (zh >> 8) & 0x001F001Fu, xh + 4 * k, ah);
    }
    uint32_t s0, m0, s1, m1;
    scale_min_k4(h.y, h.z, h.w, 2 * g, s0, m0);
    scale_min_k4(h.y, h.z, h.w, 2 * g + 1, s1, m1);
    const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(h.x >> 16);
    const float sl = xq[4 * g] + xq[4 * g + 1], sh = xq[4 * g + 2] + xq[4 * g + 3];
    float r = -(dmin * (float)m0) * sl;
    r = __builtin_fmaf(-(dmin * (float)m1), sh, r);
    r = __builtin_fmaf(d * (float)s0, al, r);
    return __builtin_fmaf(d * (float)s1, ah, r);
  }
};

// ---- Q6_K (210 B): quarter c = 2h + t owns l = 16t..16t+15 of half h, i.e.
// the four 16-element sub-blocks 8h + t + 2k, k = 0..3, whose 6-bit codes are
// ql[64h+l] (low nibble: k=0, high: k=2), ql[64h+32+l] (k=1, k=3) plus two
// bits of qh[32h+l] (Decode_Q6K_Block, llm_dequant.adb:140-181).
template <> struct Block<Q6_K> {
  static constexpr int BYTES = 210;
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int c, const float* xs, const float* xq) {
    const int hh = c >> 1, t = c & 1;
    const uint4 A = ld16(sb + 64 * hh + 16 * t);
    const uint4 B = ld16(sb + 64 * hh + 32 + 16 * t);
    const uint4 H = ld16(sb + 128 + 32 * hh + 16 * t);
    const uint4 S = ld16(sb + 192);
    const float d = f16_ada(ld2(sb + 208)) * 16777216.f;
    const uint32_t a[4] = {A.x, A.y, A.z, A.w}, b[4] = {B.x, B.y, B.z, B.w}, q[4] = {H.x, H.y, H.z, H.w};
    const float* x1 = xs + 128 * hh + 16 * t;
    float a1 = 0.f, a2 = 0.f, a3 = 0.f, a4 = 0.f;  // units 2^-24
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t z1 = (a[k] & 0x0F0F0F0Fu) | ((q[k] << 4) & 0x30303030u);
      const uint32_t z2 = (b[k] & 0x0F0F0F0Fu) | ((q[k] << 2) & 0x30303030u);
      const uint32_t z3 = ((a[k] >> 4) & 0x0F0F0F0Fu) | (q[k] & 0x30303030u);
      const uint32_t z4 = ((b[k] >> 4) & 0x0F0F0F0Fu) | ((q[k] >> 2) & 0x30303030u);
      a1 = fma_quad(z1 & 0x003F003Fu, (z1 >> 8) & 0x003F003Fu, x1 + 4 * k, a1);
      a2 = fma_quad(z2 & 0x003F003Fu, (z2 >> 8) & 0x003F003Fu, x1 + 32 + 4 * k, a2);
      a3 = fma_quad(z3 & 0x003F003Fu, (z3 >> 8) & 0x003F003Fu, x1 + 64 + 4 * k, a3);
      a4 = fma_quad(z4 & 0x003F003Fu, (z4 >> 8) & 0x003F003Fu, x1 + 96 + 4 * k, a4);
    }
    // int8 scales sc[8h + t + 2k]: dword 2h holds k = 0, 1; dword 2h+1 holds k = 2, 3.
    const uint32_t sw0 = hh ? S.z : S.x, sw1 = hh ? S.w : S.y;
    const float c1 = (float)__builtin_amdgcn_sbfe(sw0, 8 * t, 8);
    const float c2 = (float)__builtin_amdgcn_sbfe(sw0, 8 * t + 16, 8);
    const float c3 = (float)__builtin_amdgcn_sbfe(sw1, 8 * t, 8);
    const float c4 = (float)__builtin_amdgcn_sbfe(sw1, 8 * t + 16, 8);
    // The codes are stored offset by 32: sum (q-32) x = sum q x - 32 sum x.
    const float k32 = 32.f / 16777216.f;
    const float* q1 = xq + 8 * hh + t;
    float r = (d * c1) * (a1 - k32 * q1[0]);
    r = __builtin_fmaf(d * c2, a2 - k32 * q1[2], r);
    r = __builtin_fmaf(d * c3, a3 - k32 * q1[4], r);
    return __builtin_fmaf(d * c4, a4 - k32 * q1[6], r);
  }
};

// ---- Q3_K (110 B): element P = 128nh + 32j + 16g + l has its low two bits
// in field j of qs[32nh+16g+l], its high bit in bit 4nh+j of hmask[16g+l],
// scale index 8nh+2j+g (Decode_Q3K_Block, llm_dequant.adb:247-266).  Quarter
// c = 2nh + g owns the 16-element sub-blocks j = 0..3 of that (nh, g).
template <> struct Block<Q3_K> {
  static constexpr int BYTES = 110;
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int c, const float* xs, const float* xq) {
    const int nh = c >> 1, g = c & 1;
    const uint4 Q = ld16(sb + 32 + 32 * nh + 16 * g);
    const uint4 M = ld16(sb + 16 * g);
    const uint2 A = ld8(sb + 96);
    const uint32_t tmp = ld4(sb + 104);
    const float d = f16_ada(ld2(sb + 108));
    const uint32_t w[4] = {Q.x, Q.y, Q.z, Q.w}, hm[4] = {M.x, M.y, M.z, M.w};
    const float* x0 = xs + 128 * nh + 16 * g;
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
        acc[j] = fma_quad(v & pm, (v >> 8) & pm, x0 + 32 * j + 4 * k, acc[j]);
      }
    }
    // 16 signed 6-bit scales (llm_dequant.adb:219-245): scale index 8nh+2j+g is
    // byte (g + 2(j&1)) of S_(2nh + (j>>1)).
    const uint32_t a[2] = {A.x, A.y};
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int jj = j >> 1;
      const uint32_t bt = 8u * (uint32_t)(g + 2 * (j & 1));
      const uint32_t sc6 = bfe(a[jj], bt + 4u * nh, 4) | (bfe(tmp, bt + 4u * nh + 2u * jj, 2) << 4);
      const float ds = d * (float)((int)sc6 - 32);
      const float unit = j < 3 ? (float)(1 << (24 - 2 * j)) : 1048576.f;
      // codes are stored offset by 4: sum (v-4) x = sum v x - 4 sum x.
      r = __builtin_fmaf(ds, __builtin_fmaf(acc[j], unit, -4.f * xq[8 * nh + g + 2 * j]), r);
    }
    return r;
  }
};

// ---- Q2_K (84 B): element P = 128nh + 32j + 16g + l is field j of
// qs[32nh+16g+l] with scale/min byte 8nh+2j+g (Decode_Q2K_Block,
// llm_dequant.adb:304-320).  Quarter c = 2nh + g owns sub-blocks j = 0..3.
template <> struct Block<Q2_K> {
  static constexpr int BYTES = 84;
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int c, const float* xs, const float* xq) {
    const int nh = c >> 1, g = c & 1;
    const uint4 Q = ld16(sb + 16 + 32 * nh + 16 * g);
    const uint2 S = ld8(sb + 8 * nh);
    const uint32_t dd = ld4(sb + 80);
    const float d = f16_ada(dd & 0xFFFFu), dmin = f16_ada(dd >> 16);
    const uint32_t w[4] = {Q.x, Q.y, Q.z, Q.w};
    const float* x0 = xs + 128 * nh + 16 * g;
    float acc[4] = {0.f, 0.f, 0.f, 0.f};  // units 2^(2j-24)
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t s = w[k] >> 8;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const uint32_t pm = 0x00030003u << (2 * j);
        acc[j] = fma_quad(w[k] & pm, s & pm, x0 + 32 * j + 4 * k, acc[j]);
      }
    }
    const uint32_t sw[2] = {S.x, S.y};
    float r = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t bt = 8u * (uint32_t)(g + 2 * (j & 1));
      const uint32_t scb = sw[j >> 1];
      const float dl = d * (float)bfe(scb, bt, 4) * (float)(1 << (24 - 2 * j));
      const float ml = dmin * (float)bfe(scb, bt + 4, 4);
      r = __builtin_fmaf(dl, acc[j], __builtin_fmaf(-ml, xq[8 * nh + g + 2 * j], r));
    }
    return r;
  }
};

// ---- Q8_0 (8 x 34 B per 256 elements): quarter c owns 32-element blocks 2c
// and 2c+1; w = d * int8 (Dequant_Q8_0, llm_dequant.adb:606-630).  Codes are
// biased by +128 (x ^ 0x80) so they are unsigned f16 subnormals.
template <> struct Block<Q8_0> {
  static constexpr int BYTES = 272;
  __device__ static __forceinline__ float half_block(const uint8_t* b, const float* x, const float* q) {
    const float d = f16_ada(ld2(b)) * 16777216.f;
    const uint4 A = ld16(b + 2), B = ld16(b + 18);
    const uint32_t w[8] = {A.x, A.y, A.z, A.w, B.x, B.y, B.z, B.w};
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const uint32_t u = w[k] ^ 0x80808080u;
      acc = fma_quad(u & 0x00FF00FFu, (u >> 8) & 0x00FF00FFu, x + 4 * k, acc);
    }
    return d * __builtin_fmaf(-128.f / 16777216.f, q[0] + q[1], acc);
  }
  __device__ static __forceinline__ float quarter(const uint8_t* sb, int c, const float* xs, const float* xq) {
    return half_block(sb + 68 * c, xs + 64 * c, xq + 4 * c) +
           half_block(sb + 68 * c + 34, xs + 64 * c + 32, xq + 4 * c + 2);
  }
};

}  // namespace kq
