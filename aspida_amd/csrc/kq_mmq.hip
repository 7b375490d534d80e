// kq_mmq.hip -- small-batch (B = 2..64) K-quant products on MFMA, over the
// packed layout of kq_packed.h: Y[b][out] = sum_k W[out][k] X[b][k].
//
// Numerics.  The quantized codes q are exact small integers.  They enter the
// matrix cores as f16 (subnormals q * 2^-24, the same bit patterns the vector
// kernels feed v_fma_mix_f32), and MFMA products of f16 with f16 are exact in
// its f32 accumulator.  Activations are split into two f16 parts,
// x = s_b^-1 (hi + lo), where s_b is a per-row power of two that brings the
// row's largest |x| to about 2^14 (so neither part leaves f16's normal range
// for the values that matter), hi = f16(x s_b) and lo = f16(x s_b - hi).  Two
// MFMAs (hi, lo) per tile recover x to about 2^-22 relative -- f32-like, well
// inside the path's 1e-3 bar.  Per scale sub-block the kernel forms
// D_s = sum q x with fresh MFMA accumulators and adds (d * sc_s) * D_s in f32;
// the min / code-offset terms, (dmin * m_s) * sum_s x and 32 d sc_s sum_s x,
// are one more K=16 MFMA of the integer m_s (or sc_s) against the sub-block
// sums of x.  Every super-block column of a 64-row tile is read from HBM once
// for all B activation rows.
//
// MFMA lane layouts (v_mfma_f32_16x16x{16,32}_f16, checked on gfx950):
// A[i][k] in lane i + 16 (k / KL) element k % KL, B[k][j] in lane
// j + 16 (k / KL) element k % KL (KL = K / 4), D[i][j] in lane j + 16 (i / 4)
// element i % 4.  Here i = activation row, j = weight row, so each lane's D
// column is one weight row and its scales are per-lane values.
//
// Within every 4-element quad the codes arrive as the f16 pairs (e0, e2) and
// (e1, e3) -- two AND masks on one dword -- so the activation split stores
// each quad in the order (0, 2, 1, 3) to match.
#include <algorithm>

#include "kq_packed.h"
#include "kq_kernels.h"

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

template <int SUB>
__global__ __launch_bounds__(1024) void kq_xsplit(const float* __restrict__ X, int B, int in_dim,
                                                  _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                  _Float16* __restrict__ sh, _Float16* __restrict__ sl,
                                                  float* __restrict__ inv) {
  __shared__ float wmax[16];
  const int b = blockIdx.x, t = threadIdx.x;
  const bool live = b < B;
  const int nq = in_dim / 4, nsb = in_dim / 256;
  const float4* x4 = reinterpret_cast<const float4*>(X + (size_t)b * in_dim);
  float m = 0.f;
  if (live)
    for (int qd = t; qd < nq; qd += 1024) {
      const float4 v = x4[qd];
      m = fmaxf(m, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
  if ((t & 63) == 0) wmax[t >> 6] = m;
  __syncthreads();
  float amax = 0.f;
#pragma unroll
  for (int w = 0; w < 16; ++w) amax = fmaxf(amax, wmax[w]);
  // s_b = 2^(14 - e) with amax < 2^e; rows of zeros (or non-finite) use 1.
  const bool scaled = amax > 0.f && __builtin_isfinite(amax);
  int e = 0;
  if (scaled) (void)frexpf(amax, &e);
  const float sb = scaled ? ldexpf(1.f, 14 - e) : 1.f;
  if (t == 0) inv[b] = 1.f / sb;
  constexpr int QPS = SUB / 4;  // quads per sub-block
  for (int qd = t; qd < nq; qd += 1024) {
    float4 v = live ? x4[qd] : make_float4(0.f, 0.f, 0.f, 0.f);
    v.x *= sb; v.y *= sb; v.z *= sb; v.w *= sb;
    const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
    const _Float16 l0 = (_Float16)(v.x - (float)h0), l1 = (_Float16)(v.y - (float)h1);
    const _Float16 l2 = (_Float16)(v.z - (float)h2), l3 = (_Float16)(v.w - (float)h3);
    // quad order (0, 2, 1, 3)
    const uint2 ph = make_uint2(pack_h(h0, h2), pack_h(h1, h3));
    const uint2 pl = make_uint2(pack_h(l0, l2), pack_h(l1, l3));
    __builtin_memcpy(xh + (size_t)b * in_dim + 4 * qd, &ph, 8);
    __builtin_memcpy(xl + (size_t)b * in_dim + 4 * qd, &pl, 8);
    // sub-block sum over QPS consecutive lanes (consecutive quads)
    float s = (v.x + v.y) + (v.z + v.w);
#pragma unroll
    for (int o = 1; o < QPS; o <<= 1) s += __shfl_xor(s, o, 64);
    if (qd % QPS == 0) {
      const int u = qd / 64, slot = (qd % 64) / QPS;
      const size_t o = ((size_t)b * nsb + u) * 16;
      s *= XSUM_UNIT;  // |s| <= 32 * 2^14 before this: keep it inside f16's range
      const _Float16 shi = (_Float16)s;
      sh[o + slot] = shi;
      sl[o + slot] = (_Float16)(s - (float)shi);
      if (SUB == 32) {  // slots 8..15 of 32-element sub-blocks are zero padding
        sh[o + 8 + slot] = (_Float16)0.f;
        sl[o + 8 + slot] = (_Float16)0.f;
      }
    }
  }
}

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

struct MmArgs {
  const uint8_t* P;   // packed weights
  int nsb, out_dim, B, spw;
  const _Float16 *xh, *xl, *sh, *sl;
  const float* inv;
  float* Y;           // [B][out_dim]
  float* part;        // [ks][ntiles][Bp][64] partial sums (ks > 1)
  unsigned* count;    // [ntiles] arrival counters
  int nt;             // 1: weights read by this launch only (Q4_K: non-temporal loads;
                      // Q6_K measured slower with the per-load choice, 29.6 -> 30.1 us)
};

// Workgroup = 4 waves over 64 RB rows (RB tiles) and a range of spw
// super-block columns; wave w owns weight rows 64 RB tile + 16 (RB w + rb) +
// (lane % 16), rb < RB.  acc[rb][mb][r] holds activation row 16 mb +
// 4 (lane / 16) + r of that weight row.  With
// ks = gridDim.y > 1 column groups per tile, every workgroup stores its
// 64 x BP partial tile (device-scope stores) and the last to arrive adds the
// ks partials of each output in ascending order, all 256 threads with every
// load in flight at once (the host keeps ks <= 256 / BP).
template <int MB, int RB = 1>
__device__ __forceinline__ void mm_epilogue(const MmArgs& a, f4 (&acc)[RB][MB]) {
  __shared__ unsigned is_last;
  constexpr int BP = 16 * MB, ROWS = 64 * RB;
  constexpr int PER = BP * ROWS / 256;  // outputs per thread in the final sum
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, j = lane & 15, Q = lane >> 4;
  const int tile = blockIdx.x, ks = gridDim.y;
  const size_t ntiles = gridDim.x;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    f4 sc;
    __builtin_memcpy(&sc, a.inv + 16 * mb + 4 * Q, 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb][mb] *= sc;
  }
  if (ks == 1) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int row = ROWS * tile + 16 * (RB * w + rb) + j;
      if (row < a.out_dim)
#pragma unroll
        for (int mb = 0; mb < MB; ++mb)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int b = 16 * mb + 4 * Q + r;
            if (b < a.B) a.Y[(size_t)b * a.out_dim + row] = acc[rb][mb][r];
          }
    }
    return;
  }
  float* mine = a.part + ((size_t)blockIdx.y * ntiles + tile) * BP * ROWS;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        __hip_atomic_store(&mine[(16 * mb + 4 * Q + r) * ROWS + 16 * (RB * w + rb) + j], acc[rb][mb][r],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(&a.count[(size_t)tile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                      (unsigned)(ks - 1)
                  ? 1u
                  : 0u;
  __syncthreads();
  if (!is_last) return;
  // Output o = b * ROWS + row-in-block; thread t sums outputs t + 256 i over
  // the ks partials in ascending order, a partial's PER loads in flight together.
  const int t = threadIdx.x;
  float sum[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i)
    sum[i] = __hip_atomic_load(a.part + (size_t)tile * BP * ROWS + t + 256 * i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  for (int k = 1; k < ks; ++k) {
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i)
      v[i] = __hip_atomic_load(a.part + ((size_t)k * ntiles + tile) * BP * ROWS + t + 256 * i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int i = 0; i < PER; ++i) sum[i] += v[i];
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = t + 256 * i, b = o / ROWS, row = ROWS * tile + o % ROWS;
    if (b < a.B && row < a.out_dim) a.Y[(size_t)b * a.out_dim + row] = sum[i];
  }
  if (t == 0) __hip_atomic_store(&a.count[(size_t)tile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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

// Thread t's share of column s's activation tile: x chunks t + 256 u (row
// i / 64, chunk i % 64: hi 0..31, lo 32..63) and, for t < 4 BP, one chunk of
// sums (row t / 4: hi 0, 1, lo 2, 3).
// Register copies of the tile are native vectors: an array of the HIP
// uint4 class, copied with memcpy, stays in memory (then promoted to LDS,
// whose per-thread indexing reads the workgroup size from the dispatch
// packet at every launch).
typedef uint32_t xu4 __attribute__((ext_vector_type(4)));

template <int MB>
__device__ __forceinline__ void xtile_load(const MmArgs& a, int s, xu4 (&v)[XTile<MB>::NX], xu4& sv) {
  const int t = threadIdx.x, in_dim = a.nsb * 256;
#pragma unroll
  for (int u = 0; u < XTile<MB>::NX; ++u) {
    const int i = t + 256 * u, b = i >> 6, part = i & 63;
    const _Float16* src = (part < 32 ? a.xh : a.xl) + (size_t)b * in_dim + (size_t)s * 256 + 8 * (part & 31);
    v[u] = *reinterpret_cast<const xu4*>(src);
  }
  const int b = (t >> 2) & (XTile<MB>::BP - 1), part = t & 3;  // rows wrap for t >= 4 BP (not stored)
  const _Float16* src = (part < 2 ? a.sh : a.sl) + ((size_t)b * a.nsb + s) * 16 + 8 * (part & 1);
  sv = *reinterpret_cast<const xu4*>(src);
}

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

// RB 16-row blocks per wave: the workgroup covers 64 RB rows (RB tiles), so
// each staged activation tile serves RB times the rows, and each activation
// fragment read from LDS feeds RB matrix-core products.
template <int MB, int NB, int RB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void kq_mm_mfma_q4k(MmArgs a) {
  constexpr int GB = 64 * 144, BP = 16 * MB;
  __shared__ __attribute__((aligned(16))) _Float16 xb[NB][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[NB][BP * SROW];
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Row block RB w + rb of the workgroup: tile (4 RB bx + RB w + rb) / 4, rows
  // 16 ((RB w + rb) % 4) + (lane % 16) of it.
  auto load_w = [&](int s, Q4Regs (&r)[RB]) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const int G = 4 * RB * blockIdx.x + RB * w + rb, row = 16 * (G & 3) + j;
      const uint8_t* g = a.P + ((size_t)(G >> 2) * a.nsb + s) * GB;
      r[rb].h = a.nt ? ld16nt(g + 16 * row) : ld16(g + 16 * row);
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) {
        const uint8_t* src = g + (1 + 2 * gq + (q >> 1)) * 1024 + 16 * row + 8 * (q & 1);
        r[rb].wc[gq] = a.nt ? ld8nt(src) : ld8(src);
      }
    }
  };
  f4 acc[RB][MB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = f4{0.f, 0.f, 0.f, 0.f};
  const int s0 = blockIdx.y * a.spw;
  Q4Regs cur[RB], nxt[RB];
  xu4 xv[XTile<MB>::NX], xsv;
  load_w(s0, cur);
  xtile_load<MB>(a, s0, xv, xsv);
  xtile_store<MB>(xb[0], sb[0], xv, xsv);
  __syncthreads();
  for (int c = 0; c < a.spw; ++c) {
    const int buf = NB == 2 ? (c & 1) : 0;  // one buffer: a single column (host-checked)
    const bool more = c + 1 < a.spw;
    if (more) {
      load_w(s0 + c + 1, nxt);
      xtile_load<MB>(a, s0 + c + 1, xv, xsv);
    }
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
      const _Float16* xr = xb[buf] + (16 * mb + j) * XROW + 8 * q;
      const _Float16* sr = sb[buf] + (16 * mb + j) * SROW + 4 * q;
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
    if (more) {
      xtile_store<MB>(xb[(buf + 1) % NB], sb[(buf + 1) % NB], xv, xsv);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) cur[rb] = nxt[rb];
    }
    __syncthreads();
  }
  mm_epilogue<MB, RB>(a, acc);
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

template <int MB, int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void kq_mm_mfma_q6k(MmArgs a) {
  constexpr int GB = 64 * 210, BP = 16 * MB;
  __shared__ __attribute__((aligned(16))) _Float16 xb[NB][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[NB][BP * SROW];
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = 16 * w + j;
  const int tile = blockIdx.x;
  auto load_w = [&](int s, Q6Regs& r) {
    const uint8_t* g = a.P + ((size_t)tile * a.nsb + s) * GB;
    r.d = ld2(g + 13 * 1024 + 2 * row);
    r.sc = ld16(g + 12 * 1024 + 16 * row);
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      const int hh = ht >> 1, t = ht & 1, ro = 16 * row + 4 * q;
      r.wa[ht] = ld4(g + (4 * hh + t) * 1024 + ro);
      r.wb[ht] = ld4(g + (4 * hh + 2 + t) * 1024 + ro);
      r.wq[ht] = ld4(g + (8 + 2 * hh + t) * 1024 + ro);
    }
  };
  f4 acc[1][MB];
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) acc[0][mb] = f4{0.f, 0.f, 0.f, 0.f};
  const int s0 = blockIdx.y * a.spw;
  Q6Regs cur, nxt;
  xu4 xv[XTile<MB>::NX], xsv;
  load_w(s0, cur);
  xtile_load<MB>(a, s0, xv, xsv);
  xtile_store<MB>(xb[0], sb[0], xv, xsv);
  __syncthreads();
  for (int c = 0; c < a.spw; ++c) {
    const int buf = NB == 2 ? (c & 1) : 0;  // one buffer: a single column (host-checked)
    const bool more = c + 1 < a.spw;
    if (more) {
      load_w(s0 + c + 1, nxt);
      xtile_load<MB>(a, s0 + c + 1, xv, xsv);
    }
    const float d = f16_ada(cur.d);
    const uint4 scw = cur.sc;
    // lane group q: int8 scales 4q .. 4q+3 as f16 (exact), for the offset MFMA.
    const uint32_t w4 = q == 0 ? scw.x : q == 1 ? scw.y : q == 2 ? scw.z : scw.w;
    const h4 scb = as_h4(pack_h2((float)(int8_t)(w4 & 0xFF), (float)(int8_t)((w4 >> 8) & 0xFF)),
                         pack_h2((float)(int8_t)((w4 >> 16) & 0xFF), (float)(int8_t)(w4 >> 24)));
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      const _Float16* xr = xb[buf] + (16 * mb + j) * XROW + 4 * q;
      const _Float16* sr = sb[buf] + (16 * mb + j) * SROW + 4 * q;
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
          acc[0][mb] += (d * sc * 16777216.f) * D[k];
        }
      }
      // Code offset: acc -= 32 d sum_s sc_s xsum_s.
      f4 D = mfma16(lds_h4(sr), scb, f4{0.f, 0.f, 0.f, 0.f});
      D = mfma16(lds_h4(sr + 16), scb, D);
      acc[0][mb] -= (32.f * d * (1.f / XSUM_UNIT)) * D;
    }
    if (more) {
      xtile_store<MB>(xb[(buf + 1) % NB], sb[(buf + 1) % NB], xv, xsv);
      cur = nxt;
    }
    __syncthreads();
  }
  mm_epilogue<MB>(a, acc);
}

// ---- host side --------------------------------------------------------------

static int mm_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

bool mfma_kind(int kind) { return kind == Q4_K || kind == Q6_K; }

// 16-row blocks per wave of the Q4_K kernel: two (a workgroup covers 128
// rows) for 64 activation rows over at least 128 tiles, so each staged
// activation tile serves twice the rows (14336x4096, 64 rows: 61 -> 46 us).
// Smaller products keep one: with half the workgroups they ran slower
// (4096^2, 64 rows: 22.7 -> 26.9 us; 14336x4096, 32 rows: 31.4 -> 36.2 us).
static int mm_rb(int kind, int out_dim, int bp) {
  const int ntiles = (out_dim + 63) / 64;
  return kind == Q4_K && bp == 64 && ntiles >= 128 && ntiles % 2 == 0 ? 2 : 1;
}

// Super-block columns per workgroup: the divisor of nsb whose workgroup count
// (row groups x column groups) is closest to 4 per CU, with at most 256 / Bpad
// column groups per row group.
static int mm_spw(int in_dim, int out_dim, int bp, int rb) {
  static const int cus = mm_cus();
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64 / rb;
  const int oks = packed_plan_override_ks();
  if (oks > 0 && nsb % oks == 0 && oks <= 256 / bp) return nsb / oks;
  const double target = 4.0 * cus;
  int best_spw = nsb;
  double best = 1e30;
  for (int spw = 1; spw <= nsb; ++spw) {
    if (nsb % spw || nsb / spw > 256 / bp) continue;
    const double units = (double)ntiles * (nsb / spw);
    const double miss = units > target ? units / target : target / units;
    if (miss < best - 1e-9) { best = miss; best_spw = spw; }
  }
  return best_spw;
}

// Activation rows padded to 16, 32 or 64 (the three-block kernels would spill
// registers; 33..48 rows run as 64 with zero rows).
static int mm_bpad(int batch) { return batch <= 16 ? 16 : batch <= 32 ? 32 : 64; }

size_t mfma_workspace_bytes(int in_dim, int out_dim, int batch) {
  const int bp = mm_bpad(batch), nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  // The larger of the two kinds' plans (the buffer serves either).
  const int ks = std::max(nsb / mm_spw(in_dim, out_dim, bp, mm_rb(Q4_K, out_dim, bp)),
                          nsb / mm_spw(in_dim, out_dim, bp, 1));
  size_t n = 0;
  n += (size_t)bp * in_dim * 2 * 2;               // xh, xl
  n += (size_t)bp * nsb * 16 * 2 * 2;             // sh, sl
  n = (n + 255) / 256 * 256;
  n += (size_t)bp * 4;                            // inv
  n = (n + 255) / 256 * 256;
  if (ks > 1) n += (size_t)ks * ntiles * bp * 64 * 4;   // partials
  return n;
}

hipError_t launch_matmul_mfma_packed(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X,
                                     float* Y, void* work, unsigned* count, hipStream_t s, bool stream_once) {
  if (!mfma_kind(kind)) return hipErrorNotSupported;
  if (batch < 1 || batch > 64 || in_dim % 256 || out_dim <= 0) return hipErrorInvalidValue;
  const int bp = mm_bpad(batch), nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  const int rb = mm_rb(kind, out_dim, bp);
  const int spw = mm_spw(in_dim, out_dim, bp, rb), ks = nsb / spw;
  uint8_t* w = (uint8_t*)work;
  _Float16* xh = (_Float16*)w;
  _Float16* xl = xh + (size_t)bp * in_dim;
  _Float16* sh = xl + (size_t)bp * in_dim;
  _Float16* sl = sh + (size_t)bp * nsb * 16;
  size_t off = ((size_t)bp * in_dim * 4 + (size_t)bp * nsb * 16 * 4 + 255) / 256 * 256;
  float* inv = (float*)(w + off);
  off = (off + (size_t)bp * 4 + 255) / 256 * 256;
  float* part = (float*)(w + off);
  if (kind == Q4_K)
    hipLaunchKernelGGL(kq_xsplit<32>, dim3(bp), dim3(1024), 0, s, X, batch, in_dim, xh, xl, sh, sl, inv);
  else
    hipLaunchKernelGGL(kq_xsplit<16>, dim3(bp), dim3(1024), 0, s, X, batch, in_dim, xh, xl, sh, sl, inv);
  const MmArgs a{(const uint8_t*)P, nsb, out_dim, batch, spw, xh, xl, sh, sl, inv, Y, part, count, stream_once ? 1 : 0};
  const dim3 grid(ntiles / rb, ks);
  // One column per workgroup needs a single activation buffer: half the LDS,
  // so more workgroups are resident at once.
#define KQ_MM(MB)                                                                                         \
  if (bp == 16 * MB) {                                                                                    \
    if (kind == Q4_K && rb == 2) {                                                                        \
      if (spw == 1) hipLaunchKernelGGL((kq_mm_mfma_q4k<MB, 1, MB == 1 ? 1 : 2>), grid, dim3(256), 0, s, a); \
      else hipLaunchKernelGGL((kq_mm_mfma_q4k<MB, 2, MB == 1 ? 1 : 2>), grid, dim3(256), 0, s, a);          \
    } else if (spw == 1) {                                                                                \
      if (kind == Q4_K) hipLaunchKernelGGL((kq_mm_mfma_q4k<MB, 1, 1>), grid, dim3(256), 0, s, a);         \
      else hipLaunchKernelGGL((kq_mm_mfma_q6k<MB, 1>), grid, dim3(256), 0, s, a);                         \
    } else {                                                                                              \
      if (kind == Q4_K) hipLaunchKernelGGL((kq_mm_mfma_q4k<MB, 2, 1>), grid, dim3(256), 0, s, a);         \
      else hipLaunchKernelGGL((kq_mm_mfma_q6k<MB, 2>), grid, dim3(256), 0, s, a);                         \
    }                                                                                                     \
    return hipGetLastError();                                                                             \
  }
  KQ_MM(1) KQ_MM(2) KQ_MM(4)
#undef KQ_MM
  return hipErrorInvalidValue;
}

hipError_t launch_matmul_mfma(int kind, const void* W, int in_dim, int out_dim, int batch, const float* X,
                              float* Y, hipStream_t s) {
  (void)kind; (void)W; (void)in_dim; (void)out_dim; (void)batch; (void)X; (void)Y; (void)s;
  return hipErrorNotSupported;
}

}  // namespace kq
