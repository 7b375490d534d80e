// kq_mv_mfma.hip -- batch-1 matvec of Q4_K weights on the matrix cores, over
// the packed layout (kq_packed.h).
//
// The VALU decode kernel (kq_packed.hip) spends one v_fma_mix_f32 per weight
// plus about 1.4 instructions of unpacking and scaling; at the HBM rate that
// would keep the vector ALUs ~85% busy, so weight loads and arithmetic cannot
// overlap.  Here the multiply-adds run on v_mfma_f32_16x16x32_f16 and the
// vector ALUs only unpack codes (5 instructions per 8 codes) and apply the
// per-sub-block scales: about half the vector work per weight.
//
// One MFMA (A 16x32, B 32x16, D 16x16; lane layouts as in kq_mmq.hip):
//   B[k][n]  n = a weight row of a 16-row block; k = 8 g + t are the 8 codes
//            one dword of qs holds for quarter g of that row: elements
//            4j + {0,2,1,3} of sub-block 2g (low nibbles, as the f16
//            subnormals q 2^-24) then of sub-block 2g+1 (high nibbles, 16 q
//            2^-24).  The packed layout already gives lane (n, g) those bytes.
//   A[m][k]  m = 2 s + p: plane p (hi, lo) of the scaled activation of the
//            element at k when k lies in sub-block s, zero otherwise.
//   D[m][n]  sum over sub-block s = m / 2 of q x (plane p) for row n, every
//            product exact and the sums f32.  D[m][n] sits in lane n + 16 (m/4)
//            element m % 4: lane (n, g) ends up with both planes of sub-blocks
//            2g and 2g+1, the sub-blocks whose codes and scales it loaded.
// Eight MFMAs (j = 0..7: qs dword j of the quarter) cover a 16-row block's
// super-block; a wave takes a 64-row tile (four blocks) and its range of
// super-block columns.
//
// A depends on x only.  Per column each wave builds it in its own 8 KB LDS
// image (one float4 of x per lane; the zero part is written once) and reads it
// back as 8 16-byte fragments per lane, shared by the tile's four row blocks.
// Activations are scaled per column: x' = x S, with S a power of two that puts
// the column's largest |x| just below 2^14 (and S / 16 for odd sub-blocks,
// which absorbs the high nibbles' factor 16), hi = f16(x'), lo = f16(x' - hi)
// -- x to about 2^-22 relative.  The minimum terms use the f32 sub-block sums
// of x'.
//
// Accuracy.  The matrix cores do not round each addition as IEEE f32 does:
// measured on MI355X, a product much smaller than the largest one in the same
// sum (and, in a chain of MFMAs, than the accumulator) keeps fewer bits.  So
// the result is within about 1e-6 of sum |w x| for ordinary activations, but
// within only ~3e-5 when a column holds outliers 10^4 times its other values
// (the VALU kernel: ~1e-7).  The lo plane is stored times 2^11 so that its
// products are as large as hi's.
//
// Result per row: sum over columns and sub-blocks of
// (d sc_s sum_s q x - dmin m_s sum_s x), the decode of Decode_Q4K_Block
// (src/llm/llm_dequant.adb:536-553) dotted with x, in a different summation
// order from the CPU's (QMatVec, llm_dequant.adb:808-932).
#include <algorithm>
#include <atomic>

#include "kq_packed.h"
#include "kq_kernels.h"

namespace kq {

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf4 __attribute__((ext_vector_type(4)));

// Codes, scales and d/dmin of one 64-row tile's super-block column for lane
// (n, g): rows 16 rb + n, header chunk 0 and qs chunks 1 + 2g, 2 + 2g.
struct MvColQ4 {
  uint4 h[4], a[4], b[4];
};

__device__ __forceinline__ void load_col_q4(MvColQ4& c, const uint8_t* __restrict__ grp, int n, int g) {
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const uint8_t* r = grp + (16 * rb + n) * 16;
    c.h[rb] = ld16(r);
    c.a[rb] = ld16(r + (1 + 2 * g) * 1024);
    c.b[rb] = ld16(r + (2 + 2 * g) * 1024);
  }
}

__device__ __forceinline__ uint32_t pack_f16x2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

// Per-lane constants of one wave.
struct MvLaneQ4 {
  uint32_t* wr_hi;  // this lane's image writes (plane hi; plane lo is 4 dwords on)
  float odd;        // 1/16 for odd sub-blocks
  int bs, bj;       // sub-block and 4-element slice this lane converts
  bool upper;       // scale extraction for sub-blocks 2g, 2g+1
  uint32_t b0, m1, m2, mshift;
};

// One super-block column of a 64-row tile: build the A image from the lane's
// float4 of x, run the four row blocks' MFMA chains interleaved (j outer, so
// consecutive MFMAs are independent), then apply each block's scales.
template <int NW>
__device__ __forceinline__ void column_q4(const MvColQ4& c, float4 xv, const MvLaneQ4& L, uint4 (&img)[8][64],
                                          float (&xsum)[8], int lane, int g, float (&acc)[4]) {
  float mx = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
  mx = wave_max(mx);
  int e = 0;
  const bool scaled = mx > 0.f && __builtin_isfinite(mx);
  if (scaled) (void)frexpf(mx, &e);
  const int se = scaled ? std::min(std::max(14 - e, -120), 120) : 0;
  const float S = ldexpf(1.f, se), invS = ldexpf(1.f, -se);
  const float sl = S * L.odd;
  const float v0 = xv.x * sl, v1 = xv.y * sl, v2 = xv.z * sl, v3 = xv.w * sl;
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1, h2 = (_Float16)v2, h3 = (_Float16)v3;
  // lo is stored times 2^11 (exact: a power of two), so that its products
  // stay as large as hi's inside the matrix cores' sums.
  const _Float16 l0 = (_Float16)((v0 - (float)h0) * 2048.f), l1 = (_Float16)((v1 - (float)h1) * 2048.f);
  const _Float16 l2 = (_Float16)((v2 - (float)h2) * 2048.f), l3 = (_Float16)((v3 - (float)h3) * 2048.f);
  // Sub-block sums of x S (without the odd sub-blocks' 1/16): quad sums,
  // then lane 4 of each 8-lane sub-block adds the quad below it (row_shr:4).
  float su = (xv.x + xv.y) + (xv.z + xv.w);
  su += dpp_from<0xB1>(su, 0.f);
  su += dpp_from<0x4E>(su, 0.f);
  su += dpp_from<0x114>(su, 0.f);
  __builtin_amdgcn_wave_barrier();
  *reinterpret_cast<uint2*>(L.wr_hi) = make_uint2(pack_f16x2(h0, h2), pack_f16x2(h1, h3));
  *reinterpret_cast<uint2*>(L.wr_hi + 4) = make_uint2(pack_f16x2(l0, l2), pack_f16x2(l1, l3));
  if (L.bj == 4) xsum[L.bs] = su * S;
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img[j][lane];
  const float2 X = *reinterpret_cast<const float2*>(&xsum[2 * g]);
  __builtin_amdgcn_wave_barrier();

  mf4 D[4];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) D[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint4& qv = j < 4 ? c.a[rb] : c.b[rb];
      const uint32_t q = (j & 3) == 0 ? qv.x : (j & 3) == 1 ? qv.y : (j & 3) == 2 ? qv.z : qv.w;
      const uint32_t t = q >> 8;
      const uint4 bq = make_uint4(q & 0x000F000Fu, t & 0x000F000Fu, q & 0x00F000F0u, t & 0x00F000F0u);
      D[rb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8, A[j]), __builtin_bit_cast(mh8, bq), D[rb],
                                                     0, 0, 0);
    }
  }
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const uint4 h = c.h[rb];
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

template <int NW, bool PF>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma_q4k(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                         const float* __restrict__ x, float* __restrict__ y, int spw,
                                                         float* __restrict__ part, unsigned* __restrict__ count) {
  constexpr int GB = 64 * 144;
  __shared__ uint4 img[NW][8][64];  // per wave: A fragments of MFMA j for each lane
  __shared__ float xsum[NW][8];     // per wave: sum of x S over each sub-block of the column
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  const int n = lane & 15, g = lane >> 4;

#pragma unroll
  for (int j = 0; j < 8; ++j) img[w][j][lane] = make_uint4(0u, 0u, 0u, 0u);

  // Image writes of this lane: it converts x[4 lane .. 4 lane + 3] = elements
  // 4 bj .. 4 bj + 3 of sub-block bs, which feed MFMA bj in the lanes of rows
  // m = 2 bs (hi) and 2 bs + 1 (lo) of k-group bs / 2, dwords 2 (bs % 2) + {0, 1}.
  MvLaneQ4 L;
  L.bs = lane >> 3;
  L.bj = lane & 7;
  L.wr_hi = reinterpret_cast<uint32_t*>(&img[w][L.bj][20 * (L.bs >> 1) + 2 * (L.bs & 1)]) + 2 * (L.bs & 1);
  L.odd = (L.bs & 1) ? 0.0625f : 1.f;
  // Scale extraction for sub-blocks 2g, 2g+1 (get_scale_min_k4,
  // llm_dequant.adb:514-525): both pairs sit in bytes b0, b0 + 1 of the scale
  // dwords; g >= 2 takes the low/high nibbles of the third dword plus two bits
  // from the first/second.
  L.upper = g >= 2;
  L.b0 = 16u * (uint32_t)(g & 1);
  L.m1 = L.upper ? 0x0F0Fu : 0x3F3Fu;
  L.m2 = L.upper ? 0x3030u : 0u;
  L.mshift = L.b0 + (L.upper ? 4u : 0u);

  float acc[4] = {0.f, 0.f, 0.f, 0.f};
  const uint8_t* gp = P + ((size_t)tile * nsb + sb0) * GB;
  const float* xp = x + (size_t)sb0 * 256 + 4 * lane;

  MvColQ4 c0;
  float4 x0;
  load_col_q4(c0, gp, n, g);
  __builtin_memcpy(&x0, __builtin_assume_aligned(xp, 16), 16);
  if (!PF) {  // one column per wave
    column_q4<NW>(c0, x0, L, img[w], xsum[w], lane, g, acc);
  } else {
    // Two register sets used in turn: the next column's loads are in flight
    // while the current one is multiplied, with no copies between them.
    MvColQ4 c1;
    float4 x1;
    for (int s = 0; s < spw; s += 2) {
      const int s1 = s + 1 < spw ? s + 1 : s;
      load_col_q4(c1, gp + (size_t)s1 * GB, n, g);
      __builtin_memcpy(&x1, __builtin_assume_aligned(xp + (size_t)s1 * 256, 16), 16);
      asm volatile("" ::: "memory");  // keep these loads issued here
      column_q4<NW>(c0, x0, L, img[w], xsum[w], lane, g, acc);
      if (s + 2 < spw) {
        load_col_q4(c0, gp + (size_t)(s + 2) * GB, n, g);
        __builtin_memcpy(&x0, __builtin_assume_aligned(xp + (size_t)(s + 2) * 256, 16), 16);
        asm volatile("" ::: "memory");
      }
      if (s + 1 < spw) column_q4<NW>(c1, x1, L, img[w], xsum[w], lane, g, acc);
    }
  }

  // Lane (n, g) holds rows 16 rb + n over sub-blocks 2g, 2g+1: add the four
  // quarters (ascending g) so that lane l holds row l of the tile.
  float* red = reinterpret_cast<float*>(&img[w][0][0]);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) red[rb * 64 + lane] = acc[rb];
  __builtin_amdgcn_wave_barrier();
  const float* rr = red + (lane >> 4) * 64 + (lane & 15);
  const float rowsum = ((rr[0] + rr[16]) + rr[32]) + rr[48];
  mv_epilogue<NW>(rowsum, tile, tile, out_rows, y, part, count);
}

// 0: the MFMA kernel for Q4_K, 1: the VALU kernel (comparison and tuning).
static std::atomic<int> g_engine{0};

void set_matvec_engine(int engine) { g_engine = engine; }

bool matvec_mfma_takes(int kind) { return kind == Q4_K && g_engine.load() == 0; }

hipError_t launch_matvec_mfma(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y, float* part,
                              unsigned* count, hipStream_t s) {
  if (kind != Q4_K) return hipErrorNotSupported;
  const PackedPlan p = mfma_plan(in_dim, out_dim);
  const dim3 grid((out_dim + 63) / 64, p.ks);
  const int nsb = in_dim / 256;
  const uint8_t* w = (const uint8_t*)P;
  switch (p.nw) {
#define KQ_MVM(N)                                                                                                  \
  case N:                                                                                                          \
    if (p.spw > 1)                                                                                                 \
      hipLaunchKernelGGL((kq_mv_mfma_q4k<N, true>), grid, dim3(64 * N), 0, s, w, nsb, out_dim, x, y, p.spw, part,  \
                         count);                                                                                   \
    else                                                                                                           \
      hipLaunchKernelGGL((kq_mv_mfma_q4k<N, false>), grid, dim3(64 * N), 0, s, w, nsb, out_dim, x, y, p.spw, part, \
                         count);                                                                                   \
    break;
    KQ_MVM(8) KQ_MVM(4) KQ_MVM(2) KQ_MVM(1)
#undef KQ_MVM
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kq
