// kq_mm16.hip -- small-batch products Y[b][out] = W X[b] for up to 16
// activation vectors per launch on the matrix cores, over packed Q4_K weights.
//
// Each v_mfma_f32_16x16x32_f16 takes one 32-element scale sub-block: A = the
// 16 vectors' activations of that sub-block (rows = vectors), B = the codes of
// 16 weight rows (f16 subnormals q 2^-24, as in the batch-1 kernels), so D[b][n]
// is sum_{k in sub-block} q x_b for row n -- dense in both dimensions.  The
// per-sub-block scale is applied in f32 on D (lane n + 16 (b / 4) holds rows n
// of vectors 4 (b / 4) .. + 3), and the minimum term dmin sum_t m_t X_{b,t}
// is one more K = 16 MFMA of the sub-block sums against the integer mins.
//
// The activations are prepared once per launch by kq_mm16_ximage: per
// super-block column and vector, x S (S a power of two putting the column's
// largest |x| just below 2^14) split into f16 hi and lo (lo times 2^11), laid
// out as the MFMA's A fragments (16 B per lane, 8 sub-blocks x 2 planes), plus
// the sub-block sums' fragment and 1/S.  The product kernel loads the
// fragments straight from L2 with one 16-byte load per lane each, so it needs
// no LDS staging or barrier per column.
//
// Lane (n, g) of a wave loads, per 16-row block rb and qs group g' = 0..3, the
// 8 qs bytes 32 g' + 8 g .. + 7 of row 16 rb + n (two f16 pairs per dword:
// elements 8 g + {0, 2, 1, 3, 4, 6, 5, 7} of sub-blocks 2g' (low nibbles) and
// 2g' + 1 (high nibbles, 16 q 2^-24)).  The activation fragments use the same
// element order.  A wave takes a 64-row tile (four row blocks) and a range of
// super-block columns, one after another; waves and workgroups meet as in
// the batch-1 kernels (LDS, then the last-arriving workgroup, ascending).
//
// Q6_K's sixteen 16-element sub-blocks carry signed 8-bit scales, and
// (q - 32) sc needs up to 13 bits, too many to fold into an exact f16 operand:
// each sub-block is one v_mfma_f32_16x16x16_f16 of the raw 6-bit codes (B =
// q 2^-24) against its own activation fragment, scaled in f32 on D, and the
// -32 offset is one more K = 16 MFMA of the sub-block sums against the
// scales (kq_mm16_ximage6 lays out that image: a fragment per sub-block).
//
// Accuracy as for the batch-1 MFMA kernels (kq_mv_mfma.hip): products exact,
// sums in the matrix cores' f32.  Result per row: Decode_Q4K_Block
// (src/llm/llm_dequant.adb:536-553) or Decode_Q6K_Block (122-184) dotted with
// each vector (QMatMul, llm_dequant.adb:808-932, once per vector).
#include <algorithm>

#include "kq_packed.h"
#include "kq_kernels.h"

namespace kq {

typedef _Float16 m16h8 __attribute__((ext_vector_type(8)));
typedef _Float16 m16h4 __attribute__((ext_vector_type(4)));
typedef float m16f4 __attribute__((ext_vector_type(4)));
typedef unsigned short m16u2 __attribute__((ext_vector_type(2)));

constexpr int MM16_NF = 17;            // A fragments per column: 8 sub-blocks x 2 planes, sums
constexpr float MM16_XSUM = 1.f / 64.f;  // sub-block sums (|.| <= 32 * 2^14) times this fit f16

__device__ __forceinline__ uint32_t mm16_pack(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// ---- activation images -----------------------------------------------------
//
// One workgroup of 256 threads per super-block column: thread (b, u) = vector
// b (< 16; rows >= B are zero), elements 16 u .. 16 u + 15 of the column.
__global__ __launch_bounds__(256) void kq_mm16_ximage(const float* __restrict__ X, int B, int in_dim,
                                                      uint4* __restrict__ img, float* __restrict__ inv) {
  __shared__ float sums[16][8];
  const int t = threadIdx.x, b = t >> 4, u = t & 15, c = blockIdx.x;
  float v[16];
  if (b < B) {
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)b * in_dim + (size_t)c * 256 + 16 * u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 q = p[i];
      v[4 * i] = q.x, v[4 * i + 1] = q.y, v[4 * i + 2] = q.z, v[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.f;
  }
  // Largest |x| of vector b in the column: the 16 threads of b are one DPP row.
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
  mx = fmaxf(mx, dpp_from<0x128>(mx, mx));  // row_ror:8
  mx = fmaxf(mx, dpp_from<0x124>(mx, mx));  // row_ror:4
  mx = fmaxf(mx, dpp_from<0x122>(mx, mx));  // row_ror:2
  mx = fmaxf(mx, dpp_from<0x121>(mx, mx));  // row_ror:1
  int e = 0;
  const bool scaled = mx > 0.f && __builtin_isfinite(mx);
  if (scaled) (void)frexpf(mx, &e);
  const int se = scaled ? std::min(std::max(14 - e, -120), 120) : 0;
  const float S = ldexpf(1.f, se);
  if (u == 0) inv[(size_t)c * 16 + b] = ldexpf(1.f, -se);
  // Fragments: sub-block s = u / 2, lanes b + 16 kg for kg = 2 (u % 2), +1;
  // each takes 8 elements in the order {0, 2, 1, 3, 4, 6, 5, 7}.
  float su = 0.f;
  uint32_t hw[8], lw[8];
#pragma unroll
  for (int i = 0; i < 16; i += 2) {
    const float a0 = v[i] * S, a1 = v[i + 1] * S;
    su += a0 + a1;
    (void)a1;
  }
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int o = 8 * kk;
    const int ord[8] = {0, 2, 1, 3, 4, 6, 5, 7};
    _Float16 hi[8], lo[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const float a = v[o + ord[i]] * S;
      hi[i] = (_Float16)a;
      lo[i] = (_Float16)((a - (float)hi[i]) * 2048.f);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      hw[4 * kk + i] = mm16_pack(hi[2 * i], hi[2 * i + 1]);
      lw[4 * kk + i] = mm16_pack(lo[2 * i], lo[2 * i + 1]);
    }
  }
  const int s = u >> 1;
  uint4* col = img + (size_t)c * MM16_NF * 64;
#pragma unroll
  for (int kk = 0; kk < 2; ++kk) {
    const int lane = b + 16 * (2 * (u & 1) + kk);
    col[(2 * s) * 64 + lane] = make_uint4(hw[4 * kk], hw[4 * kk + 1], hw[4 * kk + 2], hw[4 * kk + 3]);
    col[(2 * s + 1) * 64 + lane] = make_uint4(lw[4 * kk], lw[4 * kk + 1], lw[4 * kk + 2], lw[4 * kk + 3]);
  }
  // Sub-block sums of x S: the two threads of a sub-block are neighbours.
  su += dpp_from<0xB1>(su, 0.f);
  if ((u & 1) == 0) sums[b][s] = su;
  __syncthreads();
  // Sums fragment (K = 16 MFMA): lane b + 16 tq holds sub-blocks 4 tq .. +3
  // (tq < 2; zero above), hi in .x .y, lo (times 2^11) in .z .w.
  if (t < 64) {
    const int bb = t & 15, tq = t >> 4;
    _Float16 h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = tq < 2 ? sums[bb][4 * tq + i] * MM16_XSUM : 0.f;
      h[i] = (_Float16)a;
      l[i] = (_Float16)((a - (float)h[i]) * 2048.f);
    }
    col[16 * 64 + t] = make_uint4(mm16_pack(h[0], h[1]), mm16_pack(h[2], h[3]), mm16_pack(l[0], l[1]),
                                  mm16_pack(l[2], l[3]));
  }
}

// Q6_K's image: thread (b, u) holds sub-block u (elements 16 u .. + 15) of
// vector b.  Fragment u, lane b + 16 kq: elements 4 kq + {0, 2, 1, 3} of the
// sub-block, hi in .x .y, lo (times 2^11) in .z .w -- the x and y halves are
// one K = 16 A operand each.  Fragment 16: the sub-block sums, lane b + 16 kq
// holding sub-blocks 4 kq + {0, 2, 1, 3} in the same form.
__global__ __launch_bounds__(256) void kq_mm16_ximage6(const float* __restrict__ X, int B, int in_dim,
                                                       uint4* __restrict__ img, float* __restrict__ inv) {
  __shared__ float sums[16][16];
  const int t = threadIdx.x, b = t >> 4, u = t & 15, c = blockIdx.x;
  float v[16];
  if (b < B) {
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)b * in_dim + (size_t)c * 256 + 16 * u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 q = p[i];
      v[4 * i] = q.x, v[4 * i + 1] = q.y, v[4 * i + 2] = q.z, v[4 * i + 3] = q.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = 0.f;
  }
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(v[i]));
  mx = fmaxf(mx, dpp_from<0x128>(mx, mx));  // row_ror:8
  mx = fmaxf(mx, dpp_from<0x124>(mx, mx));  // row_ror:4
  mx = fmaxf(mx, dpp_from<0x122>(mx, mx));  // row_ror:2
  mx = fmaxf(mx, dpp_from<0x121>(mx, mx));  // row_ror:1
  int e = 0;
  const bool scaled = mx > 0.f && __builtin_isfinite(mx);
  if (scaled) (void)frexpf(mx, &e);
  const int se = scaled ? std::min(std::max(14 - e, -120), 120) : 0;
  const float S = ldexpf(1.f, se);
  if (u == 0) inv[(size_t)c * 16 + b] = ldexpf(1.f, -se);
  float su = 0.f;
  uint4* col = img + (size_t)c * MM16_NF * 64;
#pragma unroll
  for (int kq = 0; kq < 4; ++kq) {
    const int ord[4] = {0, 2, 1, 3};
    _Float16 hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = v[4 * kq + ord[i]] * S;
      su += a;
      hi[i] = (_Float16)a;
      lo[i] = (_Float16)((a - (float)hi[i]) * 2048.f);
    }
    col[u * 64 + b + 16 * kq] = make_uint4(mm16_pack(hi[0], hi[1]), mm16_pack(hi[2], hi[3]),
                                           mm16_pack(lo[0], lo[1]), mm16_pack(lo[2], lo[3]));
  }
  sums[b][u] = su;
  __syncthreads();
  if (t < 64) {
    const int bb = t & 15, kq = t >> 4;
    const int ord[4] = {0, 2, 1, 3};
    _Float16 h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a = sums[bb][4 * kq + ord[i]] * MM16_XSUM;
      h[i] = (_Float16)a;
      l[i] = (_Float16)((a - (float)h[i]) * 2048.f);
    }
    col[16 * 64 + t] = make_uint4(mm16_pack(h[0], h[1]), mm16_pack(h[2], h[3]), mm16_pack(l[0], l[1]),
                                  mm16_pack(l[2], l[3]));
  }
}

// ---- product ----------------------------------------------------------------

struct Mm16Args {
  const uint8_t* P;
  int nsb, out_rows, B, spw;
  const uint4* img;
  const float* inv;
  float* Y;          // [B][out_rows]
  float* part;       // ks > 1: [ks][ntiles][16][64]
  unsigned* count;   // per-tile arrival counters
};

__device__ __forceinline__ m16f4 mfma32(uint4 a, uint4 b, m16f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(m16h8, a), __builtin_bit_cast(m16h8, b), c, 0, 0, 0);
}
__device__ __forceinline__ m16f4 mfma16(uint2 a, uint2 b, m16f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(m16h4, a), __builtin_bit_cast(m16h4, b), c, 0, 0, 0);
}

// acc[rb][i] (row 16 rb + n of the tile, vector 4 q + i) of every wave to Y:
// waves meet in LDS, workgroups of a tile (ks > 1) through the partial sums
// and the last-arriving workgroup, in ascending order.
template <int NW>
__device__ __forceinline__ void mm16_finish(const Mm16Args& a, const float (&acc)[4][4], float (&red)[NW][16][64],
                                            unsigned& is_last, int w, int n, int q) {
  const int tile = blockIdx.x, ks = gridDim.y;
  // Each thread owns outputs o = threadIdx.x + 64 NW j (vector o / 64, row
  // o % 64) and adds the waves in ascending order.
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) red[w][4 * q + i][16 * rb + n] = acc[rb][i];
  __syncthreads();
  constexpr int PER = 1024 / (64 * NW);
  float outv[PER];
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int o = threadIdx.x + 64 * NW * j, b = o >> 6, r = o & 63;
    float t = red[0][b][r];
#pragma unroll
    for (int k = 1; k < NW; ++k) t += red[k][b][r];
    outv[j] = t;
  }
  if (ks > 1) {
    const size_t ntiles = gridDim.x;
    float* mine = a.part + ((size_t)blockIdx.y * ntiles + tile) * 1024;
#pragma unroll
    for (int j = 0; j < PER; ++j)
      __hip_atomic_store(&mine[threadIdx.x + 64 * NW * j], outv[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
      is_last = __hip_atomic_fetch_add(&a.count[(size_t)tile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ks - 1)
                    ? 1u
                    : 0u;
    __syncthreads();
    if (!is_last) return;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int o = threadIdx.x + 64 * NW * j;
      float t = 0.f;
      for (int k = 0; k < ks; ++k)
        t += __hip_atomic_load(a.part + ((size_t)k * ntiles + tile) * 1024 + o, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
      outv[j] = t;
    }
    if (threadIdx.x == 0)
      __hip_atomic_store(&a.count[(size_t)tile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int o = threadIdx.x + 64 * NW * j, b = o >> 6, row = tile * 64 + (o & 63);
    if (b < a.B && row < a.out_rows) a.Y[(size_t)b * a.out_rows + row] = outv[j];
  }
}

template <int NW, bool NT>
__global__ __launch_bounds__(64 * NW) void kq_mm16_q4k(Mm16Args a) {
  constexpr int GB = 64 * 144;
  __shared__ uint4 hdr[NW][64];
  __shared__ float red[NW][16][64];
  __shared__ unsigned is_last;
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * a.spw;
  // Scale extraction for lane group q's... every lane needs all 8 (sc, m) of
  // its row; mins go to the K = 16 MFMA as lane (n, q)'s four (q < 2).
  float acc[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rb][i] = 0.f;

  for (int s = 0; s < a.spw; ++s) {
    const int col = sb0 + s;
    const uint8_t* grp = a.P + ((size_t)tile * a.nsb + col) * GB;
    asm volatile("" ::: "memory");  // this column's loads after the previous column's work
    const uint4 h = ld16(grp + lane * 16);
    uint2 wq[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint8_t* src = grp + (1 + 2 * g + (q >> 1)) * 1024 + (16 * rb + n) * 16 + 8 * (q & 1);
        wq[rb][g] = NT ? ld8nt(src) : ld8(src);
      }
    const uint4* im = a.img + (size_t)col * MM16_NF * 64 + lane;
    uint4 A[MM16_NF];
#pragma unroll
    for (int f = 0; f < MM16_NF; ++f) A[f] = im[f * 64];
    float4 iv;
    __builtin_memcpy(&iv, __builtin_assume_aligned(a.inv + (size_t)col * 16 + 4 * q, 16), 16);
    __builtin_amdgcn_wave_barrier();
    hdr[w][lane] = h;
    __builtin_amdgcn_wave_barrier();
    uint4 H[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) H[rb] = hdr[w][16 * rb + n];
    __builtin_amdgcn_wave_barrier();
    const uint2 amin_hi = make_uint2(A[16].x, A[16].y), amin_lo = make_uint2(A[16].z, A[16].w);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint4 hh = H[rb];
      // Scales and mins as bytes (get_scale_min_k4, llm_dequant.adb:514-525):
      // sub-blocks 0-3 in scl/mnl, 4-7 in sch/mnh.
      const uint32_t scl = hh.y & 0x3F3F3F3Fu, mnl = hh.z & 0x3F3F3F3Fu;
      const uint32_t sch = (hh.w & 0x0F0F0F0Fu) | ((hh.y >> 2) & 0x30303030u);
      const uint32_t mnh = ((hh.w >> 4) & 0x0F0F0F0Fu) | ((hh.z >> 2) & 0x30303030u);
      // B = code x sub-block scale as f16 subnormals (q sc 2^-24, q sc <= 945),
      // so the column's 8 sub-blocks accumulate in the matrix cores: dh over
      // the hi plane, dl over the lo plane.
      m16f4 dh = {0.f, 0.f, 0.f, 0.f}, dl = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const uint32_t sc = g < 2 ? scl : sch;
        const uint32_t sel0 = (g & 1) ? 0x0C020C02u : 0x0C000C00u;
        const m16u2 p0 = __builtin_bit_cast(m16u2, __builtin_amdgcn_perm(0u, sc, sel0));
        const m16u2 p1 = __builtin_bit_cast(m16u2, __builtin_amdgcn_perm(0u, sc, sel0 + 0x00010001u));
        const uint32_t w0 = wq[rb][g].x, w1 = wq[rb][g].y;
        const uint32_t nib[8] = {w0, w0 >> 8, w1, w1 >> 8, w0 >> 4, w0 >> 12, w1 >> 4, w1 >> 12};
        uint32_t bq[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          bq[k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(m16u2, nib[k] & 0x000F000Fu) * (k < 4 ? p0 : p1));
        const uint4 blo = make_uint4(bq[0], bq[1], bq[2], bq[3]), bhi = make_uint4(bq[4], bq[5], bq[6], bq[7]);
        dh = mfma32(A[4 * g], blo, dh);
        dl = mfma32(A[4 * g + 1], blo, dl);
        dh = mfma32(A[4 * g + 2], bhi, dh);
        dl = mfma32(A[4 * g + 3], bhi, dl);
      }
      // Minimum terms dmin sum_t m_t X_{b,t}: lane (n, q) gives the mins of
      // sub-blocks 4 (q % 2) .. + 3 as f16 subnormals m 2^-24 (the sums
      // fragment is zero for q >= 2, so those lanes' values drop out).
      const uint32_t m4 = (q & 1) ? mnh : mnl;
      const uint2 bm = make_uint2(__builtin_amdgcn_perm(0u, m4, 0x0c010c00u), __builtin_amdgcn_perm(0u, m4, 0x0c030c02u));
      const m16f4 z = {0.f, 0.f, 0.f, 0.f};
      const m16f4 mh = mfma16(amin_hi, bm, z), ml = mfma16(amin_lo, bm, z);
      const float d = f16_ada(hh.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(hh.x >> 16);
      const float km = dmin * (16777216.f / MM16_XSUM);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float dt = __builtin_fmaf(dl[i], 1.f / 2048.f, dh[i]);
        const float mt = __builtin_fmaf(ml[i], 1.f / 2048.f, mh[i]);
        const float c = __builtin_fmaf(-km, mt, d * dt);
        acc[rb][i] = __builtin_fmaf(c, i == 0 ? iv.x : i == 1 ? iv.y : i == 2 ? iv.z : iv.w, acc[rb][i]);
      }
    }
  }

  mm16_finish<NW>(a, acc, red, is_last, w, n, q);
}

// Q6_K (Decode_Q6K_Block, llm_dequant.adb:122-184): sub-block sb = 8 h + 2 k
// + t of row r takes, at its element l (0..15), the ql byte 16 (4 h + 2 (k %
// 2) + t) + l (low nibble for k < 2, else high) and qh byte 16 (2 h + t) + l
// (bits 2k, 2k + 1); in the packed layout those are byte l of chunks
// 4 h + 2 (k % 2) + t and 8 + 2 h + t of the row.  Lane (n, kq) loads bytes
// 4 kq .. + 3 of each chunk of row 16 rb + n: the B operand of every
// sub-block's K = 16 MFMA.  The scale chunk (12) and d (the tail at 13 KB)
// of row `lane` come in one coalesced load each, shared through LDS.
template <int NW, bool NT>
__global__ __launch_bounds__(64 * NW) void kq_mm16_q6k(Mm16Args a) {
  constexpr int GB = 64 * 210;
  __shared__ uint4 hsc[NW][64];
  __shared__ uint32_t hd[NW][64];
  __shared__ float red[NW][16][64];
  __shared__ unsigned is_last;
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * a.spw;
  float acc[4][4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[rb][i] = 0.f;
  const m16f4 z4 = {0.f, 0.f, 0.f, 0.f};

  for (int s = 0; s < a.spw; ++s) {
    const int col = sb0 + s;
    const uint8_t* grp = a.P + ((size_t)tile * a.nsb + col) * GB;
    asm volatile("" ::: "memory");  // this column's loads after the previous column's work
    const uint4 h = ld16(grp + 12 * 1024 + lane * 16);
    const uint32_t dd = ld2(grp + 13 * 1024 + 2 * lane);
    uint32_t ql[4][8], qh[4][4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint8_t* r = grp + (16 * rb + n) * 16 + 4 * q;
#pragma unroll
      for (int c = 0; c < 8; ++c) ql[rb][c] = NT ? ld4nt(r + c * 1024) : ld4(r + c * 1024);
#pragma unroll
      for (int c = 0; c < 4; ++c) qh[rb][c] = NT ? ld4nt(r + (8 + c) * 1024) : ld4(r + (8 + c) * 1024);
    }
    const uint4* im = a.img + (size_t)col * MM16_NF * 64 + lane;
    uint4 A[MM16_NF];
#pragma unroll
    for (int f = 0; f < MM16_NF; ++f) A[f] = im[f * 64];
    float4 iv;
    __builtin_memcpy(&iv, __builtin_assume_aligned(a.inv + (size_t)col * 16 + 4 * q, 16), 16);
    __builtin_amdgcn_wave_barrier();
    hsc[w][lane] = h;
    hd[w][lane] = dd;
    __builtin_amdgcn_wave_barrier();
    uint4 H[4];
    uint32_t D[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      H[rb] = hsc[w][16 * rb + n];
      D[rb] = hd[w][16 * rb + n];
    }
    __builtin_amdgcn_wave_barrier();
    const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint32_t hs[4] = {H[rb].x, H[rb].y, H[rb].z, H[rb].w};
      float t[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int sb = 0; sb < 16; ++sb) {
        const int hh = sb >> 3, k = (sb >> 1) & 3, tt = sb & 1;
        const uint32_t lw = ql[rb][4 * hh + 2 * (k & 1) + tt], hw = qh[rb][2 * hh + tt];
        // 6-bit codes of elements 4 kq .. + 3 as bytes, then as f16 pairs
        // {0, 2}, {1, 3} (the image's order): subnormals q 2^-24.
        const uint32_t zc = (((k >> 1) ? (lw >> 4) : lw) & 0x0F0F0F0Fu) | (((hw >> (2 * k)) & 0x03030303u) << 4);
        const uint2 bq = make_uint2(__builtin_amdgcn_perm(zc, zc, 0x0C020C00u), __builtin_amdgcn_perm(zc, zc, 0x0C030C01u));
        const m16f4 dh = mfma16(make_uint2(A[sb].x, A[sb].y), bq, z4);
        const m16f4 dl = mfma16(make_uint2(A[sb].z, A[sb].w), bq, z4);
        const float sc = (float)(int)__builtin_amdgcn_sbfe(hs[sb >> 2], 8 * (sb & 3), 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) t[i] = __builtin_fmaf(sc, __builtin_fmaf(dl[i], 1.f / 2048.f, dh[i]), t[i]);
      }
      // The -32 offset: sum_sb sc_sb X_{b,sb}, lane (n, q) giving the scales
      // of sub-blocks 4 q + {0, 2, 1, 3} as f16 (exact integers).
      const uint32_t sw = hs[q];
      _Float16 f[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) f[i] = (_Float16)(float)(int)__builtin_amdgcn_sbfe(sw, 8 * i, 8);
      const uint2 bs = make_uint2(mm16_pack(f[0], f[2]), mm16_pack(f[1], f[3]));
      const m16f4 mh = mfma16(make_uint2(A[16].x, A[16].y), bs, z4);
      const m16f4 ml = mfma16(make_uint2(A[16].z, A[16].w), bs, z4);
      const float d = f16_ada(D[rb]);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float off = __builtin_fmaf(ml[i], 1.f / 2048.f, mh[i]) * (32.f / MM16_XSUM);
        acc[rb][i] = __builtin_fmaf(d * __builtin_fmaf(t[i], 16777216.f, -off), ivs[i], acc[rb][i]);
      }
    }
  }
  mm16_finish<NW>(a, acc, red, is_last, w, n, q);
}

// ---- host -----------------------------------------------------------------

// Split: columns one after another per wave; with a tile per CU or more, whole
// tiles by 4 waves, else one or two columns per wave in groups of up to 4.
static PackedPlan mm16_plan(int in_dim, int out_dim) {
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      cus <= 0)
    cus = 256;
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  PackedPlan p{1, 1, nsb};
  p.nw = 1;
  while (p.nw * 2 <= 4 && nsb % (p.nw * 2) == 0) p.nw *= 2;
  const int oks = packed_plan_override_ks();
  if (oks > 0 && nsb % (p.nw * oks) == 0) {
    p.ks = oks;
  } else if (ntiles >= cus) {
    p.ks = 1;
  } else {
    // about one workgroup per CU, at most 64 per tile
    p.ks = 1;
    while (p.ks * 2 <= 64 && nsb % (p.nw * p.ks * 2) == 0 && (long)ntiles * p.ks < cus) p.ks *= 2;
  }
  p.spw = nsb / (p.nw * p.ks);
  return p;
}

bool mm16_kind(int kind) { return kind == Q4_K || kind == Q6_K; }

size_t mm16_workspace_bytes(int in_dim, int out_dim) {
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  const PackedPlan p = mm16_plan(in_dim, out_dim);
  size_t n = (size_t)nsb * MM16_NF * 64 * 16;  // images
  n += (size_t)nsb * 16 * 4;                    // 1/S
  n = (n + 255) / 256 * 256;
  if (p.ks > 1) n += (size_t)p.ks * ntiles * 1024 * 4;
  return n;
}

hipError_t launch_matmul_mm16(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                              void* work, unsigned* count, hipStream_t s, bool stream_once) {
  if (!mm16_kind(kind)) return hipErrorNotSupported;
  if (batch < 1 || batch > 16 || in_dim % 256 || out_dim <= 0) return hipErrorInvalidValue;
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  const PackedPlan p = mm16_plan(in_dim, out_dim);
  uint8_t* wk = (uint8_t*)work;
  uint4* img = (uint4*)wk;
  float* inv = (float*)(wk + (size_t)nsb * MM16_NF * 64 * 16);
  float* part = (float*)(wk + ((size_t)nsb * MM16_NF * 64 * 16 + (size_t)nsb * 16 * 4 + 255) / 256 * 256);
  if (kind == Q6_K)
    hipLaunchKernelGGL(kq_mm16_ximage6, dim3(nsb), dim3(256), 0, s, X, batch, in_dim, img, inv);
  else
    hipLaunchKernelGGL(kq_mm16_ximage, dim3(nsb), dim3(256), 0, s, X, batch, in_dim, img, inv);
  const Mm16Args a{(const uint8_t*)P, nsb, out_dim, batch, p.spw, img, inv, Y, part, count};
  const dim3 grid(ntiles, p.ks);
  // Weights read by this launch only stream with non-temporal loads; when
  // further launches of the same batch re-read them (more than 16 vectors),
  // ordinary loads let the Infinity Cache serve the repeats (14336x4096,
  // 64 vectors: 69 us against 75 with non-temporal loads).
  const bool q6 = kind == Q6_K;
#define KQ_MM16(N)                                                                                                 \
  case N:                                                                                                          \
    if (stream_once)                                                                                               \
      hipLaunchKernelGGL((q6 ? kq_mm16_q6k<N, true> : kq_mm16_q4k<N, true>), grid, dim3(64 * N), 0, s, a);          \
    else                                                                                                           \
      hipLaunchKernelGGL((q6 ? kq_mm16_q6k<N, false> : kq_mm16_q4k<N, false>), grid, dim3(64 * N), 0, s, a);        \
    break;
  switch (p.nw) {
    KQ_MM16(4) KQ_MM16(2) KQ_MM16(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_MM16
  return hipGetLastError();
}

}  // namespace kq
