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

#include "kq_kernels.h"
#include "kq_mmq.h"

namespace kq {

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

hipError_t launch_xsplit(int sub, const float* X, int B, int grid_rows, int in_dim, _Float16* xh, _Float16* xl,
                         _Float16* sh, _Float16* sl, float* inv, hipStream_t s) {
  if (sub == 32)
    hipLaunchKernelGGL(kq_xsplit<32>, dim3(grid_rows), dim3(1024), 0, s, X, B, in_dim, xh, xl, sh, sl, inv);
  else
    hipLaunchKernelGGL(kq_xsplit<16>, dim3(grid_rows), dim3(1024), 0, s, X, B, in_dim, xh, xl, sh, sl, inv);
  return hipGetLastError();
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

// Thread t's share of column s's activation tile (layout: kq_mmq.h, XTile).
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
      const int G = 4 * RB * blockIdx.x + RB * w + rb;
      q4k_load(a.P + ((size_t)(G >> 2) * a.nsb + s) * GB, 16 * (G & 3) + j, q, a.nt, r[rb]);
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
    q4k_column<MB, RB>(cur, xb[buf], sb[buf], j, q, acc);
    if (more) {
      xtile_store<MB>(xb[(buf + 1) % NB], sb[(buf + 1) % NB], xv, xsv);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) cur[rb] = nxt[rb];
    }
    __syncthreads();
  }
  mm_epilogue<MB, RB>(a, acc);
}

template <int MB, int NB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void kq_mm_mfma_q6k(MmArgs a) {
  constexpr int GB = 64 * 210, BP = 16 * MB;
  __shared__ __attribute__((aligned(16))) _Float16 xb[NB][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[NB][BP * SROW];
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = 16 * w + j;
  const int tile = blockIdx.x;
  auto load_w = [&](int s, Q6Regs& r) { q6k_load(a.P + ((size_t)tile * a.nsb + s) * GB, row, q, r); };
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
    q6k_column<MB>(cur, xb[buf], sb[buf], j, q, acc[0]);
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

// Super-block columns per workgroup: the divisor of nsb whose (64-row tile,
// column group) count is closest to 2 per CU, with at most 256 / Bpad column
// groups per tile.  Measured on MI355X (Q4_K, cold weights, every split):
// 14336x4096 at 64 vectors 42 us with two column groups against 46 us with
// the four a target of 4 workgroups per CU picked, 28672x4096 69 against 80 us
// with one, 14336x4096 at 32 vectors 26 against 28 us; 4096^2, 8192x4096 and
// 4096x14336 already sat at their best splits.
static int mm_spw(int in_dim, int out_dim, int bp, int rb) {
  static const int cus = mm_cus();
  (void)rb;  // a workgroup of two row tiles counts as two
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  const int oks = packed_plan_override_ks();
  if (oks > 0 && nsb % oks == 0 && oks <= 256 / bp) return nsb / oks;
  const double target = 2.0 * cus;
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
