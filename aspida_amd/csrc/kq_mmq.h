// kq_mmq.h -- the matrix-core arithmetic of the small-batch K-quant products
// (kq_mmq.hip), shared with the grouped MoE prefill products
// (kq_moe_prefill.hip): the activation split, the activation tiles staged in
// LDS, and one super-block column of Q4_K or Q6_K weights multiplied against
// such a tile.  Numerics and MFMA lane layouts: the notes at the top of
// kq_mmq.hip.
#pragma once
#include "kq_packed.h"

namespace kq {

typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

// ---- activation split ------------------------------------------------------
//
// One workgroup per activation row b < Bpad (rows >= B are zero), one quad of
// consecutive elements per thread:
//   xh/xl[b][k]      f16 hi/lo of x[b][k] * s_b, quads stored as (0, 2, 1, 3);
//   sh/sl[b][u][16]  f16 hi/lo of XSUM_UNIT times the SUB-element sums of
//                    super-block u (16 sums for SUB = 16; 8 sums then 8 zeros
//                    for SUB = 32), each sum over x[b][k] * s_b in f32 (quad
//                    sums ((x0 + x1) + (x2 + x3)), then a lane tree);
//   inv[b]           1 / s_b.
// Sub-block sums are stored times XSUM_UNIT (sums of up to 32 values below
// 2^14 would overflow f16); the kernels multiply the min / offset terms back.
constexpr float XSUM_UNIT = 1.f / 64.f;

__device__ __forceinline__ uint32_t pack_h(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// The split of B rows of in_dim activations, one workgroup per row
// (kq_mmq.hip); rows b with B <= b < grid rows are written as zeros.
hipError_t launch_xsplit(int sub, const float* X, int B, int grid_rows, int in_dim, _Float16* xh, _Float16* xl,
                         _Float16* sh, _Float16* sl, float* inv, hipStream_t s);

// ---- shared pieces ---------------------------------------------------------

__device__ __forceinline__ h8 as_h8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
  return __builtin_bit_cast(h8, make_uint4(a, b, c, d));
}
__device__ __forceinline__ h4 as_h4(uint32_t a, uint32_t b) { return __builtin_bit_cast(h4, make_uint2(a, b)); }
__device__ __forceinline__ h8 ldh8(const _Float16* p) {
  uint4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 16), 16);
  return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ h4 ldh4(const _Float16* p) {
  uint2 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 8), 8);
  return __builtin_bit_cast(h4, v);
}
__device__ __forceinline__ f4 mfma32(h8 a, h8 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ f4 mfma16(h4 a, h4 b, f4 c) { return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0); }
__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
  const _Float16 x = (_Float16)a, y = (_Float16)b;
  return (uint32_t)__builtin_bit_cast(uint16_t, x) | ((uint32_t)__builtin_bit_cast(uint16_t, y) << 16);
}

// ---- activation tiles in LDS --------------------------------------------------
//
// The four waves of a workgroup multiply the same activations, so each super-
// block column's activation tile -- BP rows of hi[256] | lo[256] halves plus
// the 16 hi and 16 lo sub-block sums -- is staged once in LDS, double-
// buffered: the tile of column c + 1 is loaded into registers while column c
// is computed, and written to the other buffer afterwards.
constexpr int XROW = 512 + 8;   // halves per activation row (hi, lo, pad)
constexpr int SROW = 32 + 8;    // halves per row of sums (hi 16, lo 16, pad)

template <int MB>
struct XTile {
  static constexpr int BP = 16 * MB;
  static constexpr int NX = BP * 64 / 256;  // uint4 of x per thread
};

// Thread t's share of a column's activation tile: x chunks t + 256 u (row
// i / 64, chunk i % 64: hi 0..31, lo 32..63) and, for t < 4 BP, one chunk of
// sums (row t / 4: hi 0, 1, lo 2, 3).
// Register copies of the tile are native vectors: an array of the HIP
// uint4 class, copied with memcpy, stays in memory (then promoted to LDS,
// whose per-thread indexing reads the workgroup size from the dispatch
// packet at every launch).
typedef uint32_t xu4 __attribute__((ext_vector_type(4)));


template <int MB>
__device__ __forceinline__ void xtile_store(_Float16* xb, _Float16* sb, const xu4 (&v)[XTile<MB>::NX],
                                            const xu4& sv) {
  const int t = threadIdx.x;
#pragma unroll
  for (int u = 0; u < XTile<MB>::NX; ++u) {
    const int i = t + 256 * u, b = i >> 6, part = i & 63;
    *reinterpret_cast<xu4*>(xb + b * XROW + (part < 32 ? 0 : 256) + 8 * (part & 31)) = v[u];
  }
  if (t < XTile<MB>::BP * 4) {
    const int b = t >> 2, part = t & 3;
    *reinterpret_cast<xu4*>(sb + b * SROW + (part < 2 ? 0 : 16) + 8 * (part & 1)) = sv;
  }
}

__device__ __forceinline__ h8 lds_h8(const _Float16* p) {
  uint4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 16), 16);
  return __builtin_bit_cast(h8, v);
}
__device__ __forceinline__ h4 lds_h4(const _Float16* p) {
  uint2 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 8), 8);
  return __builtin_bit_cast(h4, v);
}

// ---- Q4_K: 32-element sub-blocks, v_mfma_f32_16x16x32_f16 ---------------------
struct Q4Regs {
  uint4 h;
  uint2 wc[4];
};

// Lane (j, q) of a wave's 16-row block: weight row `row` (= 16 block + j) of
// the 64-row tile whose super-block column starts at g.
__device__ __forceinline__ void q4k_load(const uint8_t* g, int row, int q, bool nt, Q4Regs& r) {
  r.h = nt ? ld16nt(g + 16 * row) : ld16(g + 16 * row);
#pragma unroll
  for (int gq = 0; gq < 4; ++gq) {
    const uint8_t* src = g + (1 + 2 * gq + (q >> 1)) * 1024 + 16 * row + 8 * (q & 1);
    r.wc[gq] = nt ? ld8nt(src) : ld8(src);
  }
}

// One Q4_K super-block column of RB 16-row blocks against the MB 16-row
// activation blocks staged at xbuf / sbuf: acc[rb][mb] += the column's dots.
template <int MB, int RB>
__device__ __forceinline__ void q4k_column(const Q4Regs (&cur)[RB], const _Float16* xbuf, const _Float16* sbuf, int j,
                                           int q, f4 (&acc)[RB][MB]) {
  // The sub-block scales go into the weight operand: sc_t q (low nibbles)
  // and (sc_t / 16)(16 q) (high nibbles, which the mask leaves times 16) are
  // integers up to 945, exact as f16 subnormals times 2^-24, so the column's
  // eight sub-blocks share one MFMA chain per activation block and d scales
  // the column once.  The eight mins form an f16 B operand (lane group q:
  // mins 4q .. 4q+3; groups 2, 3 zero) for the min term.
  float d[RB], dmin[RB];
  h8 bw[RB][8];  // [rb][2 gq + nibble]
  h4 mins[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 h = cur[rb].h;
    d[rb] = f16_ada(h.x & 0xFFFFu) * 16777216.f;
    dmin[rb] = f16_ada(h.x >> 16) * (1.f / XSUM_UNIT);
    float mv[8];
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      uint32_t sc0, m0, sc1, m1;
      scale_min_k4(h.y, h.z, h.w, 2 * gq, sc0, m0);
      scale_min_k4(h.y, h.z, h.w, 2 * gq + 1, sc1, m1);
      mv[2 * gq] = (float)m0;
      mv[2 * gq + 1] = (float)m1;
      const _Float16 s0 = (_Float16)(float)sc0, s1 = (_Float16)((float)sc1 * 0.0625f);
      // Codes: bytes 8q .. 8q+7 of the 32-byte group gq, both nibbles.
      const uint32_t x0 = cur[rb].wc[gq].x, x1 = cur[rb].wc[gq].y, y0 = x0 >> 8, y1 = x1 >> 8;
      bw[rb][2 * gq] = as_h8(x0 & 0x000F000Fu, y0 & 0x000F000Fu, x1 & 0x000F000Fu, y1 & 0x000F000Fu) * s0;
      bw[rb][2 * gq + 1] = as_h8(x0 & 0x00F000F0u, y0 & 0x00F000F0u, x1 & 0x00F000F0u, y1 & 0x00F000F0u) * s1;
    }
    mins[rb] = as_h4(q == 0 ? pack_h2(mv[0], mv[1]) : q == 1 ? pack_h2(mv[4], mv[5]) : 0u,
                     q == 0 ? pack_h2(mv[2], mv[3]) : q == 1 ? pack_h2(mv[6], mv[7]) : 0u);
  }
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const _Float16* xr = xbuf + (16 * mb + j) * XROW + 8 * q;
    const _Float16* sr = sbuf + (16 * mb + j) * SROW + 4 * q;
    f4 D[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) D[rb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      const h8 a0 = lds_h8(xr + 64 * gq), a1 = lds_h8(xr + 64 * gq + 32);
      const h8 a2 = lds_h8(xr + 256 + 64 * gq), a3 = lds_h8(xr + 256 + 64 * gq + 32);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        D[rb] = mfma32(a0, bw[rb][2 * gq], D[rb]);
        D[rb] = mfma32(a1, bw[rb][2 * gq + 1], D[rb]);
        D[rb] = mfma32(a2, bw[rb][2 * gq], D[rb]);
        D[rb] = mfma32(a3, bw[rb][2 * gq + 1], D[rb]);
      }
    }
    // Min terms: acc -= dmin * sum_t m_t * xsum_t.
    const h4 s0 = lds_h4(sr), s1 = lds_h4(sr + 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      f4 Dm = mfma16(s0, mins[rb], f4{0.f, 0.f, 0.f, 0.f});
      Dm = mfma16(s1, mins[rb], Dm);
      acc[rb][mb] += d[rb] * D[rb];
      acc[rb][mb] -= dmin[rb] * Dm;
    }
  }
}

// ---- Q6_K: 16-element sub-blocks, v_mfma_f32_16x16x16f16 ---------------------
// Sub-block 8h + 2k + t holds elements 128h + 32k + 16t + i; lane group q
// supplies i = 4q .. 4q+3: ql bytes 64h + 16t + 4q (k = 0, 2) and
// 64h + 32 + 16t + 4q (k = 1, 3), qh bytes 32h + 16t + 4q.
struct Q6Regs {
  uint32_t d;
  uint4 sc;
  uint32_t wa[4], wb[4], wq[4];  // [hh * 2 + t]
};

__device__ __forceinline__ void q6k_load(const uint8_t* g, int row, int q, Q6Regs& r) {
  r.d = ld2(g + 13 * 1024 + 2 * row);
  r.sc = ld16(g + 12 * 1024 + 16 * row);
#pragma unroll
  for (int ht = 0; ht < 4; ++ht) {
    const int hh = ht >> 1, t = ht & 1, ro = 16 * row + 4 * q;
    r.wa[ht] = ld4(g + (4 * hh + t) * 1024 + ro);
    r.wb[ht] = ld4(g + (4 * hh + 2 + t) * 1024 + ro);
    r.wq[ht] = ld4(g + (8 + 2 * hh + t) * 1024 + ro);
  }
}

// One Q6_K super-block column of a 16-row block against the MB activation
// blocks staged at xbuf / sbuf.
template <int MB>
__device__ __forceinline__ void q6k_column(const Q6Regs& cur, const _Float16* xbuf, const _Float16* sbuf, int j, int q,
                                           f4 (&acc)[MB]) {
  const float d = f16_ada(cur.d);
  const uint4 scw = cur.sc;
  // lane group q: int8 scales 4q .. 4q+3 as f16 (exact), for the offset MFMA.
  const uint32_t w4 = q == 0 ? scw.x : q == 1 ? scw.y : q == 2 ? scw.z : scw.w;
  const h4 scb = as_h4(pack_h2((float)(int8_t)(w4 & 0xFF), (float)(int8_t)((w4 >> 8) & 0xFF)),
                       pack_h2((float)(int8_t)((w4 >> 16) & 0xFF), (float)(int8_t)(w4 >> 24)));
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const _Float16* xr = xbuf + (16 * mb + j) * XROW + 4 * q;
    const _Float16* sr = sbuf + (16 * mb + j) * SROW + 4 * q;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      const int hh = ht >> 1, t = ht & 1;
      const uint32_t A = cur.wa[ht], Bw = cur.wb[ht], Qw = cur.wq[ht];
      const uint32_t z[4] = {(A & 0x0F0F0F0Fu) | ((Qw << 4) & 0x30303030u),
                             (Bw & 0x0F0F0F0Fu) | ((Qw << 2) & 0x30303030u),
                             ((A >> 4) & 0x0F0F0F0Fu) | (Qw & 0x30303030u),
                             ((Bw >> 4) & 0x0F0F0F0Fu) | ((Qw >> 2) & 0x30303030u)};
      const uint32_t sw0 = hh ? scw.z : scw.x, sw1 = hh ? scw.w : scw.y;
      const int xo = 128 * hh + 16 * t;
      f4 D[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const h4 bq = as_h4(z[k] & 0x003F003Fu, (z[k] >> 8) & 0x003F003Fu);
        D[k] = mfma16(lds_h4(xr + xo + 32 * k), bq, f4{0.f, 0.f, 0.f, 0.f});
        D[k] = mfma16(lds_h4(xr + 256 + xo + 32 * k), bq, D[k]);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        // sub-block 8hh + 2k + t: int8 scale byte (2k + t) of the dword pair (sw0, sw1)
        const uint32_t sw = k < 2 ? sw0 : sw1;
        const float sc = (float)(int32_t)__builtin_amdgcn_sbfe(sw, 8 * t + 16 * (k & 1), 8);
        acc[mb] += (d * sc * 16777216.f) * D[k];
      }
    }
    // Code offset: acc -= 32 d sum_s sc_s xsum_s.
    f4 D = mfma16(lds_h4(sr), scb, f4{0.f, 0.f, 0.f, 0.f});
    D = mfma16(lds_h4(sr + 16), scb, D);
    acc[mb] -= (32.f * d * (1.f / XSUM_UNIT)) * D;
  }
}

}  // namespace kq
