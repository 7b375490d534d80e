// kq_mv_mfma.h -- the column arithmetic of the matrix-core matvec
// (kq_mv_mfma.hip), shared with the matrix-core MoE experts (kq_moe_mfma.hip):
// the per-column activation image, the packed column loads of 16-row blocks,
// and one column's MFMA dot with its scales.  The layout and accuracy notes
// are at the top of kq_mv_mfma.hip.
#pragma once
#include <algorithm>

#include "kq_elem.h"
#include "kq_packed.h"

namespace kq {

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_f16x2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ mf4 mfma_f16(uint4 a, uint4 b, mf4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8, a), __builtin_bit_cast(mh8, b), c, 0, 0, 0);
}

// Per-lane constants of one wave.
struct MvLane {
  uint32_t* wr_hi;  // this lane's image writes (plane hi; plane lo is the next lane's slot)
  float odd;        // activation factor of this lane's elements (Q4_K high nibbles: 1/16)
  bool xs_writer;   // this lane stores a sub-block sum ...
  int xs_pos;       // ... at this index of the wave's sum array
  // Q4_K scale extraction for sub-blocks 2g, 2g+1 (get_scale_min_k4,
  // llm_dequant.adb:514-525): both pairs sit in bytes b0, b0 + 1 of the scale
  // dwords; g >= 2 takes the low/high nibbles of the third dword plus two bits
  // from the first/second.
  bool upper;
  uint32_t b0, m1, m2, mshift;
};

// Image slot of A row m = 4 grp + r in lane group grp (the MFMA's lane
// 16 grp + m = 20 grp + r): the full 64-lane image, or the compact one that
// keeps only these 16 data lanes (4 grp + r) plus slot 16, always zero, which
// every other lane reads.
template <int IL>
__device__ __forceinline__ constexpr int img_slot(int grp, int r) {
  return IL == 64 ? 20 * grp + r : 4 * grp + r;
}

template <int KIND, int IL>
__device__ __forceinline__ MvLane mv_lane(uint4 (&img)[8][IL], int lane) {
  MvLane L;
  const int g = lane >> 4;
  L.upper = g >= 2;
  L.b0 = 16u * (uint32_t)(g & 1);
  L.m1 = L.upper ? 0x0F0Fu : 0x3F3Fu;
  L.m2 = L.upper ? 0x3030u : 0u;
  L.mshift = L.b0 + (L.upper ? 4u : 0u);
  if (KIND == Q4_K || KIND == Q5_K) {
    // Elements 4 lane .. +3 = elements 4 bj .. of sub-block bs: MFMA bj, rows
    // m = 2 bs (+1) of k-group bs / 2, dwords 2 (bs % 2) + {0, 1}.
    const int bs = lane >> 3, bj = lane & 7;
    L.wr_hi = reinterpret_cast<uint32_t*>(&img[bj][img_slot<IL>(bs >> 1, 2 * (bs & 1))]) + 2 * (bs & 1);
    L.odd = (bs & 1) ? 0.0625f : 1.f;
    L.xs_writer = bj == 4;  // after the quad sums and row_shr:4
    L.xs_pos = bs;
  } else {
    // Element E = 4 lane = 128 h + 32 k + 16 t + 4 j: quarter c = 2h + t,
    // MFMA (T = k / 2, j) = image slot 4T + j, rows m = 4c + 2 (k % 2) (+1),
    // dwords 2 (k % 2) + {0, 1}.  Sub-block E / 16 = 8h + 2k + t, stored at
    // 4c + k so that lane group c reads its four sums as one float4.
    const int E = 4 * lane, h = E >> 7, k = (E >> 5) & 3, t = (E >> 4) & 1, j = (E >> 2) & 3;
    const int c = 2 * h + t;
    L.wr_hi = reinterpret_cast<uint32_t*>(&img[4 * (k >> 1) + j][img_slot<IL>(c, 2 * (k & 1))]) + 2 * (k & 1);
    L.odd = 1.f;
    L.xs_writer = (lane & 3) == 0;  // after the quad sums
    L.xs_pos = 4 * c + k;
  }
  return L;
}

// Builds the column's A image and sub-block sums of x S from the lane's
// float4 of x; returns 1/S.  S = 2^se puts the column's largest |x| just below
// 2^14: se = 14 - e for max |x| = f 2^e, f in [0.5, 1), i.e. 140 minus its
// biased exponent, at most 120 (0 for an all-zero column or a non-finite
// maximum).  The exponent arithmetic is wave-uniform (scalar instructions).
template <int KIND>
__device__ __forceinline__ float build_image(float4 xv, const MvLane& L, float* xsum,
                                             uint32_t mx /* wave_max_abs_bits(xv) */) {
  const int se = (mx == 0u || mx >= 0x7F800000u) ? 0 : std::min(140 - (int)(mx >> 23), 120);
  const float S = __builtin_bit_cast(float, (uint32_t)(se + 127) << 23);
  const float sl = S * L.odd;
  const float v0 = xv.x * sl, v1 = xv.y * sl, v2 = xv.z * sl, v3 = xv.w * sl;
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1, h2 = (_Float16)v2, h3 = (_Float16)v3;
  // lo is stored times 2^11 (exact: a power of two), so that its products
  // stay as large as hi's inside the matrix cores' sums.  (Written with the
  // scalar conversions: the same arithmetic through gfx950's packed
  // v_cvt_pk_f16_f32 gave NaN outputs in the grouped MoE kernels on MI355X,
  // cause not identified.)
  const _Float16 l0 = (_Float16)((v0 - (float)h0) * 2048.f), l1 = (_Float16)((v1 - (float)h1) * 2048.f);
  const _Float16 l2 = (_Float16)((v2 - (float)h2) * 2048.f), l3 = (_Float16)((v3 - (float)h3) * 2048.f);
  float su = (xv.x + xv.y) + (xv.z + xv.w);
  su += dpp_from<0xB1>(su, 0.f);
  su += dpp_from<0x4E>(su, 0.f);
  if (KIND == Q4_K || KIND == Q5_K) su += dpp_from<0x114>(su, 0.f);  // 32-element sub-blocks: two quads
  *reinterpret_cast<uint2*>(L.wr_hi) = make_uint2(pack_f16x2(h0, h2), pack_f16x2(h1, h3));
  *reinterpret_cast<uint2*>(L.wr_hi + 4) = make_uint2(pack_f16x2(l0, l2), pack_f16x2(l1, l3));
  if (L.xs_writer) xsum[L.xs_pos] = su * S;
  return __builtin_bit_cast(float, (uint32_t)(127 - se) << 23);
}

// One super-block column of RB 16-row blocks (RB = 4: the whole 64-row tile;
// RB = 1: block rb0 of it) as lane (n, g) loads it.
template <int KIND, int RB> struct MvCol;

// Q4_K: the header (d, dmin, scales) -- with RB = 4 of row `lane`, one
// coalesced 1 KB load shared through LDS; with RB = 1 of the lane's own row
// 16 rb0 + n -- and the qs chunks 1 + 2g, 2 + 2g of rows 16 rb + n.
template <int RB> struct MvCol<Q4_K, RB> {
  uint4 h, a[RB], b[RB];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, g = lane >> 4;
    h = ld16nt(grp + (RB == 4 ? lane : 16 * rb0 + n) * 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      a[rb] = ld16nt(r + (1 + 2 * g) * 1024);
      b[rb] = ld16nt(r + (2 + 2 * g) * 1024);
    }
  }
};

// Q6_K (g = 2h + t): ql chunks 4h + t (codes k = 0, 2), 4h + 2 + t (k = 1, 3)
// and qh chunk 8 + 2h + t of rows 16 rb + n; the scale chunk 12 and d of row
// `lane` (RB = 4) or of the lane's own row (RB = 1).
template <int RB> struct MvCol<Q6_K, RB> {
  uint4 a[RB], b[RB], q[RB], sc;
  uint32_t d;
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, g = lane >> 4, h = g >> 1, t = g & 1;
    const int hr = RB == 4 ? lane : 16 * rb0 + n;
    sc = ld16nt(grp + 12 * 1024 + hr * 16);
    d = ld2(grp + 13 * 1024 + hr * 2);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      a[rb] = ld16nt(r + (4 * h + t) * 1024);
      b[rb] = ld16nt(r + (4 * h + 2 + t) * 1024);
      q[rb] = ld16nt(r + (8 + 2 * h + t) * 1024);
    }
  }
};

// Q5_K: as Q4_K (header chunk 0; quarter g's qs chunks 3 + 2g, 4 + 2g), plus
// the qh chunks 1 and 2 of rows 16 rb + n (the fifth bits of elements
// l = 0..15 and 16..31 of every quarter; bit 2g for sub-block 2g, 2g + 1 for
// 2g + 1).
template <int RB> struct MvCol<Q5_K, RB> {
  uint4 h, a[RB], b[RB], ha[RB], hb[RB];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, g = lane >> 4;
    h = ld16nt(grp + (RB == 4 ? lane : 16 * rb0 + n) * 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      a[rb] = ld16nt(r + (3 + 2 * g) * 1024);
      b[rb] = ld16nt(r + (4 + 2 * g) * 1024);
      ha[rb] = ld16nt(r + 1 * 1024);
      hb[rb] = ld16nt(r + 2 * 1024);
    }
  }
};

// Q3_K (quarter c = 2 nh + g): qs chunk 2 + c (low-bit fields k = 0..3 of
// elements l = 0..15) and hmask chunk g (their high bits 4 nh + k) of rows
// 16 rb + n; the 12 scale bytes and d of row `lane` (RB = 4) or of the lane's
// own row (RB = 1).
template <int RB> struct MvCol<Q3_K, RB> {
  uint4 q[RB], m[RB], sc;
  uint32_t d;
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, c = lane >> 4;
    const int hr = RB == 4 ? lane : 16 * rb0 + n;
    const uint8_t* sp = grp + 6 * 1024 + 12 * hr;
    sc = make_uint4(ld4(sp), ld4(sp + 4), ld4(sp + 8), 0u);
    d = ld2(grp + 6 * 1024 + 768 + 2 * hr);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      q[rb] = ld16nt(r + (2 + c) * 1024);
      m[rb] = ld16nt(r + (c & 1) * 1024);
    }
  }
};

// Q2_K (quarter c = 2 nh + g): qs chunk 1 + c (fields k = 0..3 of elements
// l = 0..15) of rows 16 rb + n; the scale chunk 0 and d | dmin << 16 of row
// `lane` (RB = 4) or of the lane's own row (RB = 1).
template <int RB> struct MvCol<Q2_K, RB> {
  uint4 q[RB], sc;
  uint32_t d;
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, c = lane >> 4;
    const int hr = RB == 4 ? lane : 16 * rb0 + n;
    sc = ld16nt(grp + hr * 16);
    d = ld4(grp + 5 * 1024 + hr * 4);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) q[rb] = ld16nt(grp + (1 + c) * 1024 + (16 * (rb0 + rb) + n) * 16);
  }
};

// Bytes 0 and 2 of z as two f16 halves, and bytes 1 and 3.
__device__ __forceinline__ uint32_t bytes02(uint32_t z) { return __builtin_amdgcn_perm(z, z, 0x0C020C00u); }
__device__ __forceinline__ uint32_t bytes13(uint32_t z) { return __builtin_amdgcn_perm(z, z, 0x0C030C01u); }

// The per-row header words of a column, shared through LDS.
template <int KIND> struct MvHdr;
template <> struct MvHdr<Q4_K> {
  uint4 h[64];
};
template <> struct MvHdr<Q5_K> {
  uint4 h[64];
};
template <> struct MvHdr<Q6_K> {
  uint4 sc[64];
  uint32_t d[64];
};
template <> struct MvHdr<Q2_K> {
  uint4 sc[64];
  uint32_t d[64];
};
template <> struct MvHdr<Q3_K> {
  uint4 sc[64];
  uint32_t d[64];
};

// Lane `lane`'s A fragment of MFMA j: from the full image, or from the
// compact one (the 16 data lanes 20 grp + r, r < 4, read their slot, the
// others the zero slot).
template <int IL>
__device__ __forceinline__ uint4 img_frag(const uint4 (&img)[8][IL], int j, int lane) {
  if (IL == 64) return img[j][lane];
  const int grp = lane >> 4, m = lane & 15;
  return img[j][(m >> 2) == grp ? 4 * grp + (m & 3) : 16];
}

__device__ __forceinline__ uint32_t dword_of(const uint4& v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// One super-block column of RB row blocks: the A image, the row blocks' MFMA
// chains interleaved (consecutive MFMAs independent), then the scales.
template <int RB, int IL>
__device__ __forceinline__ void mv_dot(const MvCol<Q4_K, RB>& c, const uint4 (&img)[8][IL], const float* xsum,
                                       float invS, const MvLane& L, MvHdr<Q4_K>* hdr, int lane,
                                       float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  if (RB == 4) hdr->h[lane] = c.h;
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float2 X = *reinterpret_cast<const float2*>(&xsum[2 * g]);
  uint4 H[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) H[rb] = RB == 4 ? hdr->h[16 * rb + n] : c.h;
  __builtin_amdgcn_wave_barrier();
  mf4 D[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t q = dword_of(j < 4 ? c.a[rb] : c.b[rb], j & 3);
      const uint32_t t = q >> 8;
      D[rb] = mfma_f16(A[j], make_uint4(q & 0x000F000Fu, t & 0x000F000Fu, q & 0x00F000F0u, t & 0x00F000F0u), D[rb]);
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 h = H[rb];
    const float sa = __builtin_fmaf(D[rb][1], 1.f / 2048.f, D[rb][0]);
    const float sb = __builtin_fmaf(D[rb][3], 1.f / 2048.f, D[rb][2]);
    const uint32_t psc = L.upper ? h.w : h.y, pm = L.upper ? h.w : h.z;
    const uint32_t scp = ((psc >> L.b0) & L.m1) | ((h.y >> (L.b0 + 2u)) & L.m2);
    const uint32_t mp = ((pm >> L.mshift) & L.m1) | ((h.z >> (L.b0 + 2u)) & L.m2);
    const float sca = (float)(scp & 0xFFu), scb = (float)((scp >> 8) & 0xFFu);
    const float ma = (float)(mp & 0xFFu), mb = (float)((mp >> 8) & 0xFFu);
    const float T = __builtin_fmaf(scb, sb, sca * sa);
    const float M = __builtin_fmaf(mb, X.y, ma * X.x);
    const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(h.x >> 16);
    acc[rb] = __builtin_fmaf(__builtin_fmaf(d, T, -(dmin * M)), invS, acc[rb]);
  }
}


template <int RB, int IL>
__device__ __forceinline__ void mv_dot(const MvCol<Q6_K, RB>& c, const uint4 (&img)[8][IL], const float* xsum,
                                       float invS, const MvLane& L, MvHdr<Q6_K>* hdr, int lane,
                                       float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  if (RB == 4) {
    hdr->sc[lane] = c.sc;
    hdr->d[lane] = c.d;
  }
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float4 X = *reinterpret_cast<const float4*>(&xsum[4 * g]);  // sub-blocks k = 0..3 of quarter g
  uint2 SC[RB];
  uint32_t DD[RB];
  const bool half1 = g >= 2;  // the scales of half 1 are dwords 2, 3 of the scale chunk
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 s4 = RB == 4 ? hdr->sc[16 * rb + n] : c.sc;
    SC[rb] = half1 ? make_uint2(s4.z, s4.w) : make_uint2(s4.x, s4.y);
    DD[rb] = RB == 4 ? hdr->d[16 * rb + n] : c.d;
  }
  __builtin_amdgcn_wave_barrier();
  mf4 D0[RB], D1[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D0[rb] = D1[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t a = dword_of(c.a[rb], j), b = dword_of(c.b[rb], j), q = dword_of(c.q[rb], j);
      // 6-bit codes of sub-blocks k = 0..3 as bytes (as Block<Q6_K>::dot).
      const uint32_t z0 = (a & 0x0F0F0F0Fu) | ((q << 4) & 0x30303030u);
      const uint32_t z1 = (b & 0x0F0F0F0Fu) | ((q << 2) & 0x30303030u);
      const uint32_t z2 = ((a >> 4) & 0x0F0F0F0Fu) | (q & 0x30303030u);
      const uint32_t z3 = ((b >> 4) & 0x0F0F0F0Fu) | ((q >> 2) & 0x30303030u);
      D0[rb] = mfma_f16(A[j], make_uint4(bytes02(z0), bytes13(z0), bytes02(z1), bytes13(z1)), D0[rb]);
      D1[rb] = mfma_f16(A[4 + j], make_uint4(bytes02(z2), bytes13(z2), bytes02(z3), bytes13(z3)), D1[rb]);
    }
  }
  const int tb = 8 * (g & 1);  // byte t of each scale dword
  constexpr float K32 = 32.f / 16777216.f;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float s0 = __builtin_fmaf(D0[rb][1], 1.f / 2048.f, D0[rb][0]);
    const float s1 = __builtin_fmaf(D0[rb][3], 1.f / 2048.f, D0[rb][2]);
    const float s2 = __builtin_fmaf(D1[rb][1], 1.f / 2048.f, D1[rb][0]);
    const float s3 = __builtin_fmaf(D1[rb][3], 1.f / 2048.f, D1[rb][2]);
    // int8 scales sc[8h + t + 2k]: dword 2h holds k = 0, 1; dword 2h + 1 holds k = 2, 3.
    const float c0 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].x, tb, 8);
    const float c1 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].x, tb + 16, 8);
    const float c2 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].y, tb, 8);
    const float c3 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].y, tb + 16, 8);
    // The codes are stored offset by 32: sum (q - 32) x = sum q x - 32 sum x.
    float T = c0 * __builtin_fmaf(-K32, X.x, s0);
    T = __builtin_fmaf(c1, __builtin_fmaf(-K32, X.y, s1), T);
    T = __builtin_fmaf(c2, __builtin_fmaf(-K32, X.z, s2), T);
    T = __builtin_fmaf(c3, __builtin_fmaf(-K32, X.w, s3), T);
    const float d = f16_ada(DD[rb]) * 16777216.f;
    acc[rb] = __builtin_fmaf(d * T, invS, acc[rb]);
  }
}


// Q5_K (Decode_Q5K_Block, llm_dequant.adb:426-498): Q4_K's columns with a
// fifth code bit, code = nibble + 16 hbit.  The nibbles take Q4_K's MFMAs; the
// fifth bits take one more MFMA each, against the same activation fragments,
// with qh dword j's bit 2g (sub-block 2g) and 2g + 1 (sub-block 2g + 1) left
// in place as the subnormals 2^(2g-24) and 2^(2g+1-24).  Their sums are
// scaled back per lane: 16 2^-2g for sub-block 2g, and 16 2^-(2g+1) 16 for
// 2g + 1, whose activations the image holds divided by 16.
template <int RB, int IL>
__device__ __forceinline__ void mv_dot(const MvCol<Q5_K, RB>& c, const uint4 (&img)[8][IL], const float* xsum,
                                       float invS, const MvLane& L, MvHdr<Q5_K>* hdr, int lane,
                                       float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  if (RB == 4) hdr->h[lane] = c.h;
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float2 X = *reinterpret_cast<const float2*>(&xsum[2 * g]);
  uint4 H[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) H[rb] = RB == 4 ? hdr->h[16 * rb + n] : c.h;
  __builtin_amdgcn_wave_barrier();
  const uint32_t m0 = 0x00010001u << (2 * g), m1 = 0x00020002u << (2 * g);
  mf4 D[RB], E[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D[rb] = E[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t q = dword_of(j < 4 ? c.a[rb] : c.b[rb], j & 3), t = q >> 8;
      const uint32_t hq = dword_of(j < 4 ? c.ha[rb] : c.hb[rb], j & 3), ht = hq >> 8;
      D[rb] = mfma_f16(A[j], make_uint4(q & 0x000F000Fu, t & 0x000F000Fu, q & 0x00F000F0u, t & 0x00F000F0u), D[rb]);
      E[rb] = mfma_f16(A[j], make_uint4(hq & m0, ht & m0, hq & m1, ht & m1), E[rb]);
    }
  }
  const float fa = 16.f * __builtin_ldexpf(1.f, -2 * g), fb = 128.f * __builtin_ldexpf(1.f, -2 * g);
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 h = H[rb];
    const float ea = __builtin_fmaf(E[rb][1], 1.f / 2048.f, E[rb][0]);
    const float eb = __builtin_fmaf(E[rb][3], 1.f / 2048.f, E[rb][2]);
    const float sa = __builtin_fmaf(fa, ea, __builtin_fmaf(D[rb][1], 1.f / 2048.f, D[rb][0]));
    const float sb = __builtin_fmaf(fb, eb, __builtin_fmaf(D[rb][3], 1.f / 2048.f, D[rb][2]));
    const uint32_t psc = L.upper ? h.w : h.y, pm = L.upper ? h.w : h.z;
    const uint32_t scp = ((psc >> L.b0) & L.m1) | ((h.y >> (L.b0 + 2u)) & L.m2);
    const uint32_t mp = ((pm >> L.mshift) & L.m1) | ((h.z >> (L.b0 + 2u)) & L.m2);
    const float sca = (float)(scp & 0xFFu), scb = (float)((scp >> 8) & 0xFFu);
    const float ma = (float)(mp & 0xFFu), mb = (float)((mp >> 8) & 0xFFu);
    const float T = __builtin_fmaf(scb, sb, sca * sa);
    const float M = __builtin_fmaf(mb, X.y, ma * X.x);
    const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(h.x >> 16);
    acc[rb] = __builtin_fmaf(__builtin_fmaf(d, T, -(dmin * M)), invS, acc[rb]);
  }
}


// Q2_K: element 128 nh + 32 k + 16 g + l is field k of qs byte
// 32 nh + 16 g + l with scale/min byte 8 nh + 2 k + g (Decode_Q2K_Block,
// llm_dequant.adb:304-320) -- the element and sub-block layout of Q6_K's
// quarters, so the A image is Q6_K's.  MFMA (T, j) takes fields 2T, 2T + 1 of
// qs dword j left in place: code q of field k is the subnormal q 2^(2k-24),
// whose factor 4^k the scales absorb.
template <int RB, int IL>
__device__ __forceinline__ void mv_dot(const MvCol<Q2_K, RB>& c, const uint4 (&img)[8][IL], const float* xsum,
                                       float invS, const MvLane& L, MvHdr<Q2_K>* hdr, int lane,
                                       float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  if (RB == 4) {
    hdr->sc[lane] = c.sc;
    hdr->d[lane] = c.d;
  }
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float4 X = *reinterpret_cast<const float4*>(&xsum[4 * g]);  // sub-blocks k = 0..3 of quarter g
  uint2 SC[RB];
  uint32_t DD[RB];
  const bool nh1 = g >= 2;  // scale bytes 8 nh + 2k + g: dwords 2 nh (k < 2) and 2 nh + 1
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 s4 = RB == 4 ? hdr->sc[16 * rb + n] : c.sc;
    SC[rb] = nh1 ? make_uint2(s4.z, s4.w) : make_uint2(s4.x, s4.y);
    DD[rb] = RB == 4 ? hdr->d[16 * rb + n] : c.d;
  }
  __builtin_amdgcn_wave_barrier();
  mf4 D0[RB], D1[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D0[rb] = D1[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t w = dword_of(c.q[rb], j), t = w >> 8;
      D0[rb] = mfma_f16(A[j], make_uint4(w & 0x00030003u, t & 0x00030003u, w & 0x000C000Cu, t & 0x000C000Cu), D0[rb]);
      D1[rb] = mfma_f16(A[4 + j], make_uint4(w & 0x00300030u, t & 0x00300030u, w & 0x00C000C0u, t & 0x00C000C0u),
                        D1[rb]);
    }
  }
  const uint32_t tb = 8u * (uint32_t)(g & 1);  // byte 2 (k % 2) + g of each scale dword
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float s0 = __builtin_fmaf(D0[rb][1], 1.f / 2048.f, D0[rb][0]);
    const float s1 = __builtin_fmaf(D0[rb][3], 1.f / 2048.f, D0[rb][2]);
    const float s2 = __builtin_fmaf(D1[rb][1], 1.f / 2048.f, D1[rb][0]);
    const float s3 = __builtin_fmaf(D1[rb][3], 1.f / 2048.f, D1[rb][2]);
    const uint32_t b0 = bfe(SC[rb].x, tb, 8), b1 = bfe(SC[rb].x, tb + 16, 8);
    const uint32_t b2 = bfe(SC[rb].y, tb, 8), b3 = bfe(SC[rb].y, tb + 16, 8);
    // scale = low nibble, min = high nibble (llm_dequant.adb:304-320).
    float T = (float)(b0 & 15u) * s0;
    T = __builtin_fmaf((float)(b1 & 15u) * 0.25f, s1, T);
    T = __builtin_fmaf((float)(b2 & 15u) * 0.0625f, s2, T);
    T = __builtin_fmaf((float)(b3 & 15u) * 0.015625f, s3, T);
    float M = (float)(b0 >> 4) * X.x;
    M = __builtin_fmaf((float)(b1 >> 4), X.y, M);
    M = __builtin_fmaf((float)(b2 >> 4), X.z, M);
    M = __builtin_fmaf((float)(b3 >> 4), X.w, M);
    const float d = f16_ada(DD[rb] & 0xFFFFu) * 16777216.f, dmin = f16_ada(DD[rb] >> 16);
    acc[rb] = __builtin_fmaf(__builtin_fmaf(d, T, -(dmin * M)), invS, acc[rb]);
  }
}


// Q3_K (Decode_Q3K_Block, llm_dequant.adb:207-268): Q2_K's element layout
// with a high bit, code = low2 + 4 hbit, w = d (sc - 32) (code - 4).  Since
// code - 4 = low2 - 4 (1 - hbit), the low-bit fields take Q2_K's MFMAs and the
// inverted high bits (hmask bit 4 nh + k clear) one more MFMA each against
// the same fragments, left in place as the subnormals 2^(4nh+k-24) and scaled
// back per lane by -4 2^-(4nh+k).  No sum of x is subtracted: a zero weight
// (code 4) adds nothing to either sum, so a large activation there cannot
// leave the matrix cores' truncation error of a cancelled term behind.
template <int RB, int IL>
__device__ __forceinline__ void mv_dot(const MvCol<Q3_K, RB>& c, const uint4 (&img)[8][IL], const float* xsum,
                                       float invS, const MvLane& L, MvHdr<Q3_K>* hdr, int lane,
                                       float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15, nh = g >> 1, gg = g & 1;
  if (RB == 4) {
    hdr->sc[lane] = c.sc;
    hdr->d[lane] = c.d;
  }
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  uint4 SC[RB];
  uint32_t DD[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    SC[rb] = RB == 4 ? hdr->sc[16 * rb + n] : c.sc;
    DD[rb] = RB == 4 ? hdr->d[16 * rb + n] : c.d;
  }
  __builtin_amdgcn_wave_barrier();
  const uint32_t hb = 0x00010001u << (4 * nh);
  // Inverted high-bit sums carry 2^(4nh + k); code - 4 = low2 - 4 (1 - hbit).
  const float fh = -4.f * __builtin_ldexpf(1.f, -4 * nh);
  // One row block at a time: four accumulators live instead of 4 RB.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    mf4 D0{0.f, 0.f, 0.f, 0.f}, D1 = D0, E0 = D0, E1 = D0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t w = dword_of(c.q[rb], j), t = w >> 8;
      const uint32_t hm = ~dword_of(c.m[rb], j), ht = hm >> 8;
      D0 = mfma_f16(A[j], make_uint4(w & 0x00030003u, t & 0x00030003u, w & 0x000C000Cu, t & 0x000C000Cu), D0);
      E0 = mfma_f16(A[j], make_uint4(hm & hb, ht & hb, hm & (hb << 1), ht & (hb << 1)), E0);
      D1 = mfma_f16(A[4 + j], make_uint4(w & 0x00300030u, t & 0x00300030u, w & 0x00C000C0u, t & 0x00C000C0u), D1);
      E1 = mfma_f16(A[4 + j], make_uint4(hm & (hb << 2), ht & (hb << 2), hm & (hb << 3), ht & (hb << 3)), E1);
    }
    float cs[4];
    cs[0] = __builtin_fmaf(fh, __builtin_fmaf(E0[1], 1.f / 2048.f, E0[0]), __builtin_fmaf(D0[1], 1.f / 2048.f, D0[0]));
    cs[1] = __builtin_fmaf(fh * 0.5f, __builtin_fmaf(E0[3], 1.f / 2048.f, E0[2]),
                           0.25f * __builtin_fmaf(D0[3], 1.f / 2048.f, D0[2]));
    cs[2] = __builtin_fmaf(fh * 0.25f, __builtin_fmaf(E1[1], 1.f / 2048.f, E1[0]),
                           0.0625f * __builtin_fmaf(D1[1], 1.f / 2048.f, D1[0]));
    cs[3] = __builtin_fmaf(fh * 0.125f, __builtin_fmaf(E1[3], 1.f / 2048.f, E1[2]),
                           0.015625f * __builtin_fmaf(D1[3], 1.f / 2048.f, D1[2]));
    // 16 signed 6-bit scales (llm_dequant.adb:219-245): scale index 8 nh + 2k + g
    // is byte (g + 2 (k & 1)) of dword k >> 1, high bits from dword 2.
    const uint32_t sa[2] = {SC[rb].x, SC[rb].y}, tmp = SC[rb].z;
    float T = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int kk = k >> 1;
      const uint32_t bt = 8u * (uint32_t)(gg + 2 * (k & 1));
      const uint32_t sc6 = bfe(sa[kk], bt + 4u * nh, 4) | (bfe(tmp, bt + 4u * nh + 2u * kk, 2) << 4);
      T = __builtin_fmaf((float)((int)sc6 - 32), cs[k], T);
    }
    // cs[k] is sum (code - 4) x S in the codes' unit 2^-24.
    acc[rb] = __builtin_fmaf(f16_ada(DD[rb]) * 16777216.f * T, invS, acc[rb]);
  }
}


// One super-block column (weights c, activations xv of the column at xs,
// group grp of the packed layout, row block rb0 when RB = 1): the A image of
// the wave's 256 activations, then the kind's dot.
//
// Dominant activations.  The matrix cores do not round each addition of a
// product sum: a product much smaller than the largest one in the same sum
// keeps fewer bits (about 2^-18 of the largest).  Where a dominant
// activation's weight cancels against a min or code-offset term, that loss
// would stay behind against a small sum |w x| (with one 10^4x activation:
// up to 4.3e-4 of it for Q2_K, 2.6e-4 for Q6_K, 2.4e-4 for Q3_K; Q4_K and
// Q5_K stay below 1e-4).  For Q2_K, Q3_K and Q6_K, a column where at most 16
// activations are within 16x of its largest |x| (mv_dominant) has those
// activations zeroed in the image and its sub-block sums; mv_column returns
// true for it, and once its row sums are formed the wave adds w x for them
// in f32 (mv_dominant_exact), w its row's dequantized weight read from the
// packed group (dequant_elem, bit-exact).  Out of the column loop, the rare
// exact part costs the loop no registers; other columns pay only the test: four
// compares against max |x| / 16 and a count of the ballots (an ordinary
// column has most of its 256 activations within 16x of its largest).
template <int KIND> constexpr bool MV_EXACT_DOMINANT = KIND == Q2_K || KIND == Q3_K || KIND == Q6_K;

// The dominant set of a column whose max |x| bits are mx: ballots per float4
// component (bit l of bits[c] is element 4 l + c) and the test.  A
// non-finite maximum makes thr infinite or NaN: no set is taken out unless
// some |x| is infinite (their products are not finite either way).
struct MvDominant {
  uint64_t bits[4];
  bool take;
};
__device__ __forceinline__ MvDominant mv_dominant(float4 xv, uint32_t mx) {
  MvDominant d;
  const float thr = __builtin_bit_cast(float, mx) * 0.0625f;
  d.bits[0] = __ballot(__builtin_fabsf(xv.x) >= thr);
  d.bits[1] = __ballot(__builtin_fabsf(xv.y) >= thr);
  d.bits[2] = __ballot(__builtin_fabsf(xv.z) >= thr);
  d.bits[3] = __ballot(__builtin_fabsf(xv.w) >= thr);
  const int n = __builtin_popcountll(d.bits[0]) + __builtin_popcountll(d.bits[1]) +
                __builtin_popcountll(d.bits[2]) + __builtin_popcountll(d.bits[3]);
  d.take = __builtin_expect(n > 0 && n <= 16, 0);
  return d;
}

// Returns whether the column's dominant activations were left out (the
// caller adds them with mv_dominant_exact).
template <int KIND, int RB, int IL = (RB == 4 ? 64 : 17)>
__device__ __forceinline__ bool mv_column(const MvCol<KIND, RB>& c, float4 xv, const MvLane& L,
                                          uint4 (&img)[8][IL], float* xsum, MvHdr<KIND>* hdr, int lane,
                                          float (&acc)[RB]) {
  __builtin_amdgcn_wave_barrier();
  uint32_t mx = wave_max_abs_bits(xv);
  bool taken = false;
  if constexpr (MV_EXACT_DOMINANT<KIND>) {
    // mv_dominant's test, with the compares redone in the (rare) branch so
    // that no lane mask lives across it.
    const float thr = __builtin_bit_cast(float, mx) * 0.0625f;
    const int n = __builtin_popcountll(__ballot(__builtin_fabsf(xv.x) >= thr)) +
                  __builtin_popcountll(__ballot(__builtin_fabsf(xv.y) >= thr)) +
                  __builtin_popcountll(__ballot(__builtin_fabsf(xv.z) >= thr)) +
                  __builtin_popcountll(__ballot(__builtin_fabsf(xv.w) >= thr));
    if (__builtin_expect(n > 0 && n <= 16, 0)) {
      xv.x = __builtin_fabsf(xv.x) >= thr ? 0.f : xv.x;
      xv.y = __builtin_fabsf(xv.y) >= thr ? 0.f : xv.y;
      xv.z = __builtin_fabsf(xv.z) >= thr ? 0.f : xv.z;
      xv.w = __builtin_fabsf(xv.w) >= thr ? 0.f : xv.w;
      mx = wave_max_abs_bits(xv);
      taken = true;
    }
  }
  const float invS = build_image<KIND>(xv, L, xsum, mx);
  mv_dot<RB, IL>(c, img, xsum, invS, L, hdr, lane, acc);
  return taken;
}

// The exact part of the columns mv_column left dominant activations out of,
// for the lane's output row (RB = 4: row `lane`; RB = 1: row 16 rb0 +
// lane % 16).  Column s of the wave's run sits at xs0 + 256 s (activations)
// and grp0 + s gstride (packed group); bit s % 64 of `hint` is set for every
// such column, and each column s with its bit set is tested again (the same
// test, so the same set) -- a run of more than 64 columns shares bits.
template <int KIND, int RB>
__device__ __forceinline__ float mv_dominant_exact(uint64_t hint, int spw, const uint8_t* grp0, size_t gstride,
                                                   const float* xs0, int lane, int rb0) {
  float t = 0.f;
  if constexpr (MV_EXACT_DOMINANT<KIND>) {
#pragma nounroll
    for (uint64_t h = hint; h; h &= h - 1) {
#pragma nounroll
      for (int s = (int)__builtin_ctzll(h); s < spw; s += 64) {
        const float* xs = xs0 + (size_t)s * 256;
        float4 xv;
        __builtin_memcpy(&xv, __builtin_assume_aligned(xs + 4 * lane, 16), 16);
        const MvDominant d = mv_dominant(xv, wave_max_abs_bits(xv));
        if (!d.take) continue;
        const PackedBytes<KIND> wr(grp0 + (size_t)s * gstride, RB == 4 ? lane : 16 * rb0 + (lane & 15));
        // The component's ballot by selects: an indexed d.bits[cpt] would be
        // a private array, which the compiler places in LDS (40 B a thread).
#pragma nounroll
        for (int cpt = 0; cpt < 4; ++cpt)
#pragma nounroll
          for (uint64_t m = cpt == 0 ? d.bits[0] : cpt == 1 ? d.bits[1] : cpt == 2 ? d.bits[2] : d.bits[3]; m;
               m &= m - 1) {
            const int e = 4 * (int)__builtin_ctzll(m) + cpt;  // element e of the column
            t = __builtin_fmaf(dequant_elem<KIND>(wr, e), xs[e], t);
          }
      }
    }
  }
  return t;
}

// The LDS one wave uses: its A image, sub-block sums and row headers.
template <int KA, int KB>
struct MvShared {
  uint4 img[8][64];
  float xsum[16];
  union {
    MvHdr<KA> a;
    MvHdr<KB> b;
  } hdr;
};

// The LDS one wave of the 16-row kernels uses: the compact A image and the
// sub-block sums (headers come straight from the lane's own row).
struct MvShared16 {
  uint4 img[8][17];
  float xsum[16];
};

// Row `lane` of tile `tile`'s partial dot over super-block columns sb0 ..
// sb0 + spw - 1 of packed matrix P (nsb columns), computed by this wave.
// How a wave walks its columns: one column; two register sets in turn (the
// next column's loads in flight during this one's work); one register set,
// columns one after another (fewer registers, so more waves per CU).
constexpr int MV_ONE = 0, MV_PF = 1, MV_SEQ = 2;

//
// RB = 4: the wave covers the whole 64-row tile and lane l returns row l.
// RB = 1: it covers 16-row block rb0 of the tile and lane l returns row
// 16 rb0 + l % 16.
template <int KIND, int PIPE, int RB = 4>
__device__ __forceinline__ float mv_mfma_rows(const uint8_t* __restrict__ P, int nsb, int tile, int sb0, int spw,
                                              const float* __restrict__ x, uint4 (&img)[8][RB == 4 ? 64 : 17],
                                              float* xsum, MvHdr<KIND>* hdr, int lane, int rb0 = 0) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const uint8_t* gp = P + ((size_t)tile * nsb + sb0) * GB;
  const float* xc = x + (size_t)sb0 * 256;  // the wave's first column (uniform)
  const float* xp = xc + 4 * lane;

  // Each column's activations are requested before its weights: the loads
  // return in order, so the activation image can be built while the weights
  // are still on their way.  The first loads go out before anything else.
  MvCol<KIND, RB> c0;
  float4 x0;
  __builtin_memcpy(&x0, __builtin_assume_aligned(xp, 16), 16);
  c0.load(gp, lane, rb0);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (RB == 4 || lane < 17) img[j][lane] = make_uint4(0u, 0u, 0u, 0u);
  const MvLane L = mv_lane<KIND>(img, lane);

  float acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = 0.f;
  uint64_t hint = 0;  // bit s % 64: column s left dominant activations to mv_dominant_exact
  if (PIPE == MV_ONE) {
    hint |= (uint64_t)mv_column(c0, x0, L, img, xsum, hdr, lane, acc);
  } else if (PIPE == MV_SEQ) {  // columns one after another: one register set, more waves per CU
    for (int s = 0; s < spw; ++s) {
      if (s > 0) {
        asm volatile("" ::: "memory");  // the next column's loads stay after this column's work
        __builtin_memcpy(&x0, __builtin_assume_aligned(xp + (size_t)s * 256, 16), 16);
        c0.load(gp + (size_t)s * GB, lane, rb0);
      }
      hint |= (uint64_t)mv_column(c0, x0, L, img, xsum, hdr, lane, acc) << (s & 63);
    }
  } else {
    // Two register sets used in turn: the next column's loads are in flight
    // while the current one is multiplied, with no copies between them.
    MvCol<KIND, RB> c1;
    float4 x1;
    for (int s = 0; s < spw; s += 2) {
      const int s1 = s + 1 < spw ? s + 1 : s;
      __builtin_memcpy(&x1, __builtin_assume_aligned(xp + (size_t)s1 * 256, 16), 16);
      c1.load(gp + (size_t)s1 * GB, lane, rb0);
      asm volatile("" ::: "memory");  // keep these loads issued here
      hint |= (uint64_t)mv_column(c0, x0, L, img, xsum, hdr, lane, acc) << (s & 63);
      if (s + 2 < spw) {
        __builtin_memcpy(&x0, __builtin_assume_aligned(xp + (size_t)(s + 2) * 256, 16), 16);
        c0.load(gp + (size_t)(s + 2) * GB, lane, rb0);
        asm volatile("" ::: "memory");
      }
      if (s + 1 < spw) hint |= (uint64_t)mv_column(c1, x1, L, img, xsum, hdr, lane, acc) << (s1 & 63);
    }
  }

  // Lane (n, g) holds rows 16 rb + n over its quarter: add the four quarters
  // (ascending g), then the dominant activations' exact terms of the lane's
  // row.
  float* red = reinterpret_cast<float*>(&img[0][0]);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) red[rb * 64 + lane] = acc[rb];
  __builtin_amdgcn_wave_barrier();
  const float* rr = red + (RB == 4 ? (lane >> 4) * 64 : 0) + (lane & 15);
  const float y = ((rr[0] + rr[16]) + rr[32]) + rr[48];
  return y + mv_dominant_exact<KIND, RB>(hint, PIPE == MV_ONE ? 1 : spw, gp, GB, xc, lane, rb0);
}

__device__ __forceinline__ float4 ld_f4(const float* p) {
  float4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(p, 16), 16);
  return v;
}

// NV vectors x_v = x + v ldx at once (rows v >= nv repeat vector nv - 1;
// the caller does not write them): each column's weights are loaded once,
// then every vector gets its activation image and the column's MFMA dot
// (mv_column) against them, with the same arithmetic as mv_mfma_rows.  The
// columns are taken one after another.  out[v] is row `lane` (RB = 4) or
// row 16 rb0 + lane % 16 (RB = 1) of vector v.
template <int KIND, int RB, int NV>
__device__ __forceinline__ void mv_mfma_rows_nv(const uint8_t* __restrict__ P, int nsb, int tile, int sb0, int spw,
                                                const float* __restrict__ x, size_t ldx, int nv,
                                                uint4 (&img)[8][RB == 4 ? 64 : 17], float* xsum, MvHdr<KIND>* hdr,
                                                int lane, int rb0, float (&out)[NV]) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const uint8_t* gp = P + ((size_t)tile * nsb + sb0) * GB;
  const float* xp[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) xp[v] = x + (size_t)(v < nv ? v : nv - 1) * ldx + (size_t)sb0 * 256 + 4 * lane;
  MvCol<KIND, RB> c0;
  float4 xv[NV];
#pragma unroll
  for (int v = 0; v < NV; ++v) xv[v] = ld_f4(xp[v]);
  c0.load(gp, lane, rb0);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (RB == 4 || lane < 17) img[j][lane] = make_uint4(0u, 0u, 0u, 0u);
  const MvLane L = mv_lane<KIND>(img, lane);
  float acc[NV][RB];
#pragma unroll
  for (int v = 0; v < NV; ++v)
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[v][rb] = 0.f;
  uint64_t hint[NV];  // per vector, as in mv_mfma_rows
#pragma unroll
  for (int v = 0; v < NV; ++v) hint[v] = 0;
  for (int s = 0; s < spw; ++s) {
    if (s > 0) {
      asm volatile("" ::: "memory");  // the next column's loads stay after this column's work
#pragma unroll
      for (int v = 0; v < NV; ++v) xv[v] = ld_f4(xp[v] + (size_t)s * 256);
      c0.load(gp + (size_t)s * GB, lane, rb0);
    }
#pragma unroll
    for (int v = 0; v < NV; ++v) hint[v] |= (uint64_t)mv_column(c0, xv[v], L, img, xsum, hdr, lane, acc[v]) << (s & 63);
  }

  // Lane (n, g) holds rows 16 rb + n over its quarter: add the four quarters
  // (ascending g), vector by vector.
  float* red = reinterpret_cast<float*>(&img[0][0]);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) red[rb * 64 + lane] = acc[v][rb];
    __builtin_amdgcn_wave_barrier();
    const float* rr = red + (RB == 4 ? (lane >> 4) * 64 : 0) + (lane & 15);
    out[v] = ((rr[0] + rr[16]) + rr[32]) + rr[48] +
             mv_dominant_exact<KIND, RB>(hint[v], spw, gp, GB,
                                         x + (size_t)(v < nv ? v : nv - 1) * ldx + (size_t)sb0 * 256, lane, rb0);
  }
}

}  // namespace kq
