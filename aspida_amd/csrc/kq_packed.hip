// kq_packed.hip -- batch-1 decode matvec over the lane-interleaved layout
// (kq_packed.h), and the kernels that move weights into and out of it.
//
// kq_mv_packed: lane l of a wave owns row 64 * tile + l and walks a range of
// super-block columns; per column it loads its row's whole super-block (one
// 1 KB-coalesced 16-byte load per chunk plane), and all lanes multiply the
// same 256 activations, which the compiler keeps in scalar registers
// (s_load), so the vector registers hold only weights and accumulators.  The
// per-16 activation sums for the min/offset terms are formed in the kernel
// (one 16-byte load per lane, a DPP quad sum, readlane), so a matvec is a
// single launch.
//
// The columns of a tile are split over the NW waves of a workgroup and over
// `ks` workgroups (grid.y).  Waves meet in LDS; workgroups write partial
// sums to a workspace, and the last workgroup of a tile to arrive (an atomic
// arrival counter per tile) adds them in ascending order, writes y and
// re-arms the counter -- so results are deterministic and the launch needs no
// memset.
#include <algorithm>

#include <atomic>

#include "kq_packed.h"
#include "kq_kernels.h"

namespace kq {

// Row `lane`'s dot over spw consecutive super-block columns starting at the
// group g (activations xs).  With PF the next column's loads are issued
// before the current column's arithmetic (twice the weight registers).
template <int KIND, bool PF>
__device__ __forceinline__ float columns_dot(const uint8_t* __restrict__ g, const float* __restrict__ xs, int lane,
                                             int spw) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  typename Packed<KIND>::R r = Packed<KIND>::load(g, lane);
  float acc = 0.f;
  if (!PF) {  // one column per wave: no second register set, so more waves fit
    for (int s = 0; s + 1 < spw; ++s) {
      acc += sb_dot<KIND>(r, xs + (size_t)s * 256, lane);
      r = Packed<KIND>::load(g + (size_t)(s + 1) * GB, lane);
    }
    return acc + sb_dot<KIND>(r, xs + (size_t)(spw - 1) * 256, lane);
  }
  for (int s = 0; s + 1 < spw; ++s) {
    const typename Packed<KIND>::R nr = Packed<KIND>::load(g + (size_t)(s + 1) * GB, lane);
    // Keep those loads issued here: without the barrier the compiler sinks
    // them to their use in the next iteration and nothing overlaps.
    asm volatile("" ::: "memory");
    acc += sb_dot<KIND>(r, xs + (size_t)s * 256, lane);
    r = nr;
  }
  return acc + sb_dot<KIND>(r, xs + (size_t)(spw - 1) * 256, lane);
}

template <int KIND, int NW, bool PF>
__global__ __launch_bounds__(64 * NW) void kq_mv_packed(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                       const float* __restrict__ x, float* __restrict__ y, int spw,
                                                       float* __restrict__ part, unsigned* __restrict__ count) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  const float acc = columns_dot<KIND, PF>(P + ((size_t)tile * nsb + sb0) * GB, x + (size_t)sb0 * 256, lane, spw);
  mv_epilogue<NW>(acc, tile, tile, out_rows, y, part, count);
}

// Two matrices that multiply the same x in one launch: tiles [0, tiles_a) of
// the grid are matrix A's (kind KA), the rest matrix B's (kind KB).  Both use
// the launch's column split.
template <int KA, int KB, int NW, bool PF>
__global__ __launch_bounds__(64 * NW) void kq_mv_packed2(const uint8_t* __restrict__ Pa, int out_a, float* __restrict__ ya,
                                                        const uint8_t* __restrict__ Pb, int out_b, float* __restrict__ yb,
                                                        int tiles_a, int nsb, const float* __restrict__ x, int spw,
                                                        float* __restrict__ part, unsigned* __restrict__ count) {
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gtile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  const float* xs = x + (size_t)sb0 * 256;
  if (gtile < tiles_a) {
    const float acc = columns_dot<KA, PF>(Pa + ((size_t)gtile * nsb + sb0) * (64 * Block<KA>::BYTES), xs, lane, spw);
    mv_epilogue<NW>(acc, gtile, gtile, out_a, ya, part, count);
  } else {
    const int tile = gtile - tiles_a;
    const float acc = columns_dot<KB, PF>(Pb + ((size_t)tile * nsb + sb0) * (64 * Block<KB>::BYTES), xs, lane, spw);
    mv_epilogue<NW>(acc, gtile, tile, out_b, yb, part, count);
  }
}

// Byte moves between the ggml layout W[out][nsb] and the packed layout; one
// thread per byte of the packed image (rows past out_rows pack as zeros and
// are skipped when unpacking).
template <int KIND>
__global__ void kq_pack(const uint8_t* __restrict__ src, uint8_t* __restrict__ dst, int nsb, int out_rows,
                        size_t total, int unpack) {
  constexpr int BB = Block<KIND>::BYTES;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < total; i += (size_t)gridDim.x * blockDim.x) {
    const int b = (int)(i % BB);
    const size_t rest = i / BB;
    const int r = (int)(rest % 64);
    const size_t grp = rest / 64;  // tile * nsb + sb
    const int sb = (int)(grp % nsb);
    const size_t tile = grp / nsb;
    const size_t row = tile * 64 + r;
    const size_t off_p = grp * (size_t)(64 * BB) + (size_t)packed_offset(KIND, r, b);
    const size_t off_g = (row * nsb + sb) * BB + b;
    if (!unpack)
      dst[off_p] = row < (size_t)out_rows ? src[off_g] : (uint8_t)0;
    else if (row < (size_t)out_rows)
      dst[off_g] = src[off_p];
  }
}

// ---- launchers --------------------------------------------------------------

static int device_cus() {
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  return cus;
}

size_t packed_bytes(int kind, int in_dim, int out_dim) {
  const int bb = block_bytes(kind);
  if (bb <= 0 || in_dim <= 0 || in_dim % 256 || out_dim <= 0) return 0;
  return (size_t)((out_dim + 63) / 64) * 64 * (size_t)(in_dim / 256) * bb;
}

// Columns per wave, waves per workgroup and workgroups per tile.  A
// workgroup of up to 16 waves covering a whole tile needs no cross-workgroup
// sum, and is the fastest split whenever there are enough tiles to occupy
// the chip: with >= 256 tiles the columns per wave are chosen for about 14
// waves per CU, with 128..255 tiles and <= 16 columns every wave takes one
// column.  Below 128 tiles of <= 16 columns a tile is spread over up to 8
// workgroups (about 256 in all), and other narrow matrices split each tile
// over ks workgroups of up to 8 waves (4 below 32 tiles), one column per wave.
static int pow2_divisor_upto(int n, int cap) {
  int d = 1;
  while (d * 2 <= cap && n % (d * 2) == 0) d *= 2;
  return d;
}

// Per-thread override of the split (tuning): waves per workgroup and
// workgroups per tile, 0 = the built-in choice.
// Test and tuning overrides, per calling thread.
static thread_local int g_plan_nw = 0, g_plan_ks = 0;

void set_packed_plan_override(int nw, int ks) {
  g_plan_nw = nw;
  g_plan_ks = ks;
}

int packed_plan_override_ks() { return g_plan_ks; }

PackedPlan packed_plan(int in_dim, int out_dim) {
  static const int cus = device_cus();
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  PackedPlan p{1, 1, nsb};
  {
    const int onw = g_plan_nw, oks = g_plan_ks;
    if (onw > 0 && oks > 0 && (onw & (onw - 1)) == 0 && nsb % (onw * oks) == 0 &&
      (onw <= 8 || (onw == 16 && nsb == onw * oks))) {
      p.nw = onw;
      p.ks = oks;
      p.spw = nsb / (onw * oks);
      return p;
    }
  }
  if (ntiles >= 256) {
    const double target = 14.0 * cus;
    double best = 1e30;
    for (int spw = 1; spw <= nsb; ++spw) {
      if (nsb % spw || nsb / spw > 16) continue;
      const double waves = (double)ntiles * (nsb / spw);
      const double miss = waves > target ? waves / target : target / waves;
      if (miss < best - 1e-9) { best = miss; p.spw = spw; }
    }
    p.nw = pow2_divisor_upto(nsb / p.spw, 16);
    p.spw = nsb / p.nw;
    return p;
  }
  if (nsb <= 16 && ntiles < 128) {
    // Narrow and short (o, q|k, v of a decoder): spread each tile over up to
    // 8 workgroups so that about 256 take part; measured on MI355X, 11% faster
    // on 4096^2 than one workgroup per tile.
    int want = 1;
    while (want * 2 <= 8 && ntiles * want * 2 <= 256) want *= 2;
    p.ks = pow2_divisor_upto(nsb, want);
    p.nw = pow2_divisor_upto(nsb / p.ks, 16);
    p.spw = nsb / (p.ks * p.nw);
    return p;
  }
  if (ntiles >= 64 && nsb <= 16) {
    p.nw = pow2_divisor_upto(nsb, 16);
    p.spw = nsb / p.nw;
    return p;
  }
  p.spw = 1;
  p.nw = pow2_divisor_upto(nsb, ntiles < 32 ? 4 : 8);
  p.ks = nsb / p.nw;
  return p;
}

// Split of the MFMA matvec (kq_mv_mfma.hip), fitted to measurements on
// MI355X at the Llama-3-8B Q4_K_M shapes (launch time per split, cold HBM):
//   * a tile per CU or more: whole tiles (no cross-workgroup sum, whose atomic
//     round trip holds every workgroup ~1 us longer) by 4 waves, each taking
//     its columns one after another with one register set (~140 registers,
//     3 workgroups per CU, so all tiles run in one round): 28672x4096 14.5 us
//     against 15.3 for 16 one-column waves and 16.2 for 4 groups per tile;
//     128256x4096 75.7 us against 81;
//   * narrower matrices: one column per wave, the most waves per workgroup
//     (<= 8) that still leave >= 150 workgroups, at least 2 (4096x14336 Q6_K
//     8 x 7 groups: 12.6 us against 14.1 for 4 x 14; 4096x4096: 4 x 4, 5.5 us;
//     1024x4096: 2 x 8).
static thread_local int g_mfma_pipe = 0;

void set_mfma_pipeline(int mode) { g_mfma_pipe = mode; }

static thread_local int g_mfma_rows = 0;

void set_mfma_rows(int mode) { g_mfma_rows = mode; }

// 16-row workgroups (kq_mv_mfma16): as many waves as divide the columns, up
// to 16 (the instantiated counts), several columns per wave taken one after
// another (measured faster than prefetching on MI355X).
static PackedPlan mfma16_plan(int nsb, int max_nw = 16) {
  PackedPlan p{1, 1, nsb};
  for (int n : {16, 14, 8, 4, 2, 1})
    if (n <= max_nw && nsb % n == 0) {
      p.nw = n;
      break;
    }
  p.spw = nsb / p.nw;
  p.seq = p.spw > 1;
  p.blk16 = true;
  return p;
}

static PackedPlan mfma_plan_choice(int kind, int in_dim, int out_dim);
static PackedPlan mfma64_plan(int kind, int in_dim, int out_dim);

PackedPlan mfma_plan(int kind, int in_dim, int out_dim) {
  const int nsb = in_dim / 256;
  const int pipe = g_mfma_pipe, rows = g_mfma_rows;
  PackedPlan p = mfma_plan_choice(kind, in_dim, out_dim);
  if (rows == 2 || (rows == 0 && p.blk16)) {
    if (!p.blk16) p = mfma16_plan(nsb);
    const int onw = g_plan_nw;
    if ((onw == 16 || onw == 14 || onw == 8 || onw == 4 || onw == 2 || onw == 1) && nsb % onw == 0) {
      p.nw = onw;
      p.spw = nsb / onw;
    }
    if (pipe == 1) p.seq = false;
    if (pipe == 2) p.seq = p.spw > 1;
    return p;
  }
  if (p.blk16) p = mfma64_plan(kind, in_dim, out_dim);
  const int onw = g_plan_nw, oks = g_plan_ks;
  if (onw > 0 && oks > 0 && (onw & (onw - 1)) == 0 && nsb % (onw * oks) == 0 &&
      (onw <= 8 || (onw == 16 && nsb == onw * oks))) {
    p.nw = onw;
    p.ks = oks;
    p.spw = nsb / (onw * oks);
    p.seq = false;
  }
  if (pipe == 1) p.seq = false;
  if (pipe == 2) p.seq = true;
  // Prefetching waves (two register sets) fit at most 8 per workgroup, 4 for Q6_K, Q5_K and Q3_K.
  if (p.spw > 1 && !p.seq && p.nw > (kind == Q6_K || kind == Q5_K || kind == Q3_K ? 4 : 8)) p.seq = true;
  return p;
}

static PackedPlan mfma_plan_choice(int kind, int in_dim, int out_dim) {
  static const int cus = device_cus();
  const int ntiles = (out_dim + 63) / 64;
  // The 16-row kernels (no partial sums through memory) for up to two 16-row
  // blocks per CU, when a wave takes at most one column or the blocks fill
  // every CU (otherwise few CUs would walk long column runs).  Measured on
  // MI355X: Q4_K 4096x4096 4.3 us against 5.8 us on 64-row workgroups with
  // partial sums; 1024x14336 5.9 us on 64-row workgroups against 8.1 us.
  // Q2_K streams fewer bytes per column for the same arithmetic, so its long
  // column runs walked one after another stay on 64-row workgroups
  // (4096x14336: 8.6 us against 9.1; the prefetching 16-row rule above takes
  // that shape now); so do Q3_K rows of more than 32 blocks (8192x28672: 29.4
  // us against 31.3).
  // With more 16-row blocks than CUs, two blocks share a CU: when 16 waves
  // would still walk several columns each, 8 waves keep both resident (Q4_K
  // 8192x8192: 9.2 us against 10.1 with 16 waves; Q6_K 8192x28672: 35.7
  // against 36.8); with rows of up to 16 blocks a column per wave stays
  // better (q|k+v 6144x4096: 6.0 against 6.3).
  const int nsb = in_dim / 256;
  // Q2_K and Q3_K (more unpacking per byte) on 16-row blocks whose waves
  // prefetch their next column (two register sets: 95 and 124 VGPRs, no
  // spill): with rows of up to 64 blocks and one block per CU, or with 1.5 to
  // 2 blocks per CU.  Measured on MI355X against the 64-row plans below:
  // Q2_K 4096x14336 7.7 us against 8.8, 8192x8192 7.9 against 8.7,
  // 8192x14336 12.0 against 12.7; Q3_K 4096x14336 9.8 against 10.3,
  // 8192x8192 10.1 against 10.4; and against 16 one-column waves (which leave
  // one Q3_K workgroup per CU at 65 VGPRs) Q3_K 8192x4096 6.2 against 7.4,
  // 6144x4096 6.1 against 6.8.  Not at 1.25 blocks per CU (Q2_K 5120x14336
  // slower than 64-row workgroups at 9.9 us).
  if ((kind == Q2_K || kind == Q3_K) && nsb <= 64 && 4L * ntiles <= 2L * cus &&
      (2 * 4L * ntiles >= 3L * cus || (nsb > 16 && 4L * ntiles == cus))) {
    PackedPlan p = mfma16_plan(nsb, 4L * ntiles > cus ? 8 : 16);
    p.seq = false;
    return p;
  }
  if (4L * ntiles <= 2L * cus &&
      (nsb <= 16 || (4L * ntiles >= cus && kind != Q2_K && (kind != Q3_K || nsb <= 32))))
    return mfma16_plan(nsb, 4L * ntiles > cus && nsb > 16 ? 8 : 16);
  // Tall matrices with long rows (the 70B FFN) and very tall Q6_K ones (the
  // output heads): 16-row workgroups of 8 waves walking 2+ columns each
  // (Q4_K 57344x8192: 47.9 us against 55.9 on 4-wave 64-row workgroups;
  // Q6_K 128256x4096: 71.5 us against 77.3).
  if ((kind == Q4_K || kind == Q6_K) && ntiles >= cus && (nsb >= 32 || (kind == Q6_K && ntiles >= 4L * cus)))
    return mfma16_plan(nsb, 8);
  return mfma64_plan(kind, in_dim, out_dim);
}

static PackedPlan mfma64_plan(int kind, int in_dim, int out_dim) {
  static const int cus = device_cus();
  const int nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  PackedPlan p{1, 1, nsb};
  // Q2_K and Q3_K, measured on MI355X against the general choices below:
  //   * a tile per CU or more, rows of 32+ blocks: Q2_K 4 waves prefetching
  //     their next column (28672x8192: 19.6 us against 21.2; 57344x8192: 33.7
  //     against 34.6);
  //   * 1 to 4 tiles per CU: Q3_K a column per wave, 4 waves per workgroup,
  //     the row split over nsb/4 workgroups (57344x4096: 24.7 us against 25.9;
  //     57344x8192: 44.5 against 46.9), but not on more tiles (128256x4096:
  //     54 against 50);
  //   * fewer tiles than CUs but two or more groups of 4 per CU, rows of 64+
  //     blocks: Q2_K 4 groups per tile of 4 waves prefetching nsb/16 columns
  //     each (8192x28672: 19.5-19.9 us against 21.7-22.2 on one-column waves;
  //     Q3_K measured 27.1 against 28.5 on one box, 27.2 against 26.3 on
  //     another, so it keeps one-column waves).
  if (kind == Q2_K && ntiles >= cus && nsb >= 32 && nsb % 4 == 0) {
    p.ks = 1;
    p.nw = 4;
    p.spw = nsb / 4;
    return p;
  }
  if (kind == Q3_K && ntiles >= cus && ntiles < 4 * cus && nsb % 4 == 0) {
    p.spw = 1;
    p.nw = 4;
    p.ks = nsb / 4;
    return p;
  }
  if (kind == Q2_K && ntiles < cus && 2 * ntiles >= cus && nsb > 64 && nsb % 16 == 0) {
    p.ks = 4;
    p.nw = 4;
    p.spw = nsb / 16;
    return p;
  }
  if (ntiles >= cus) {
    p.ks = 1;
    p.nw = pow2_divisor_upto(nsb, 4);
    p.spw = nsb / p.nw;
    p.seq = true;
    return p;
  }
  p.spw = 1;
  if (2L * ntiles >= cus && nsb <= 16 && (nsb & (nsb - 1)) == 0) {
    // A tile per workgroup and a column per wave: no partial sums (Q4_K
    // 14336x4096: 8.6 us against 9.8 us with two workgroups per tile).
    p.nw = nsb;
    p.ks = 1;
    return p;
  }
  int nw = pow2_divisor_upto(nsb, 8);
  while (nw > 2 && (long)ntiles * (nsb / nw) < 150) nw /= 2;
  p.nw = nw;
  p.ks = nsb / nw;
  return p;
}

size_t packed_workspace_floats(int in_dim, int out_dim) {
  const int ks = std::max({packed_plan(in_dim, out_dim).ks, mfma_plan(Q4_K, in_dim, out_dim).ks,
                           mfma_plan(Q6_K, in_dim, out_dim).ks, mfma_plan(Q2_K, in_dim, out_dim).ks,
                           mfma_plan(Q5_K, in_dim, out_dim).ks, mfma_plan(Q3_K, in_dim, out_dim).ks});
  return ks > 1 ? (size_t)ks * ((out_dim + 63) / 64) * 64 : 0;
}

size_t packed_counters(int out_dim) { return (size_t)(out_dim + 63) / 64 * COUNTER_STRIDE; }

// Whether the prefetching walk (two weight register sets) fits without
// spilling: not for Q8_0's 17 chunks per row at 16 waves per workgroup, which
// walk their columns one after another instead.
static constexpr bool pf_fits(int ka, int kb, int nw) { return !(nw == 16 && (ka == Q8_0 || kb == Q8_0)); }

template <int KIND>
static hipError_t launch_mvp_kind(const uint8_t* P, int in_dim, int out_dim, const float* x, float* y, float* part,
                                  unsigned* count, hipStream_t s) {
  const PackedPlan p = packed_plan(in_dim, out_dim);
  const dim3 grid((out_dim + 63) / 64, p.ks);
  const int nsb = in_dim / 256;
  switch (p.nw) {
#define KQ_MVP(N)                                                                                              \
  case N:                                                                                                      \
    if constexpr (pf_fits(KIND, KIND, N))                                                                      \
      if (p.spw > 1) {                                                                                         \
        hipLaunchKernelGGL((kq_mv_packed<KIND, N, true>), grid, dim3(64 * N), 0, s, P, nsb, out_dim, x, y,      \
                           p.spw, part, count);                                                                \
        break;                                                                                                 \
      }                                                                                                        \
    hipLaunchKernelGGL((kq_mv_packed<KIND, N, false>), grid, dim3(64 * N), 0, s, P, nsb, out_dim, x, y, p.spw,  \
                       part, count);                                                                           \
    break;
    KQ_MVP(16) KQ_MVP(8) KQ_MVP(4) KQ_MVP(2) KQ_MVP(1)
#undef KQ_MVP
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_matvec_packed(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y,
                                float* part, unsigned* count, hipStream_t s) {
  if (matvec_mfma_takes(kind)) return launch_matvec_mfma(kind, P, in_dim, out_dim, x, y, part, count, s);
  const uint8_t* w = (const uint8_t*)P;
  switch (kind) {
    case Q4_K: return launch_mvp_kind<Q4_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q6_K: return launch_mvp_kind<Q6_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q5_K: return launch_mvp_kind<Q5_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q3_K: return launch_mvp_kind<Q3_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q2_K: return launch_mvp_kind<Q2_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q8_0: return launch_mvp_kind<Q8_0>(w, in_dim, out_dim, x, y, part, count, s);
    default: return hipErrorInvalidValue;
  }
}

// Kind pairs with a fused two-matrix kernel (the attention input projections
// of the common quantization mixes).
#define KQ_PAIRS(X) X(Q4_K, Q6_K) X(Q5_K, Q6_K) X(Q4_K, Q4_K) X(Q6_K, Q6_K) X(Q5_K, Q5_K) X(Q8_0, Q8_0)

bool matvec2_supported(int kind_a, int kind_b) {
#define KQ_PAIR_OK(A, B) if (kind_a == A && kind_b == B) return true;
  KQ_PAIRS(KQ_PAIR_OK)
#undef KQ_PAIR_OK
  return false;
}

template <int KA, int KB>
static hipError_t launch_mv2_pair(const void* Pa, int out_a, float* ya, const void* Pb, int out_b, float* yb,
                                  int in_dim, const float* x, float* part, unsigned* count, hipStream_t s) {
  const int tiles_a = (out_a + 63) / 64, tiles_b = (out_b + 63) / 64;
  const PackedPlan p = packed_plan(in_dim, (tiles_a + tiles_b) * 64);
  const dim3 grid(tiles_a + tiles_b, p.ks);
  const int nsb = in_dim / 256;
  const uint8_t* a = (const uint8_t*)Pa;
  const uint8_t* b = (const uint8_t*)Pb;
  switch (p.nw) {
#define KQ_MV2(N)                                                                                             \
  case N:                                                                                                     \
    if constexpr (pf_fits(KA, KB, N))                                                                         \
      if (p.spw > 1) {                                                                                        \
        hipLaunchKernelGGL((kq_mv_packed2<KA, KB, N, true>), grid, dim3(64 * N), 0, s, a, out_a, ya, b, out_b, \
                           yb, tiles_a, nsb, x, p.spw, part, count);                                          \
        break;                                                                                                \
      }                                                                                                       \
    hipLaunchKernelGGL((kq_mv_packed2<KA, KB, N, false>), grid, dim3(64 * N), 0, s, a, out_a, ya, b, out_b, yb, \
                       tiles_a, nsb, x, p.spw, part, count);                                                  \
    break;
    KQ_MV2(16) KQ_MV2(8) KQ_MV2(4) KQ_MV2(2) KQ_MV2(1)
#undef KQ_MV2
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_matvec2_packed(int kind_a, const void* Pa, int out_a, float* ya, int kind_b, const void* Pb,
                                 int out_b, float* yb, int in_dim, const float* x, float* part, unsigned* count,
                                 hipStream_t s) {
  if (matvec2_mfma_takes(kind_a, kind_b))
    return launch_matvec2_mfma(kind_a, Pa, out_a, ya, kind_b, Pb, out_b, yb, in_dim, x, part, count, s);
#define KQ_PAIR_GO(A, B) \
  if (kind_a == A && kind_b == B) return launch_mv2_pair<A, B>(Pa, out_a, ya, Pb, out_b, yb, in_dim, x, part, count, s);
  KQ_PAIRS(KQ_PAIR_GO)
#undef KQ_PAIR_GO
  return hipErrorNotSupported;
}

hipError_t launch_pack(int kind, const void* src, int in_dim, int out_dim, void* dst, bool unpack, hipStream_t s) {
  const size_t total = packed_bytes(kind, in_dim, out_dim);
  if (total == 0) return hipErrorInvalidValue;
  const int nsb = in_dim / 256;
  const unsigned blocks = (unsigned)std::min<size_t>((total + 255) / 256, (size_t)1 << 20);
  const uint8_t* a = (const uint8_t*)src;
  uint8_t* b = (uint8_t*)dst;
#define KQ_PACK(K) \
  case K: hipLaunchKernelGGL(kq_pack<K>, dim3(blocks), dim3(256), 0, s, a, b, nsb, out_dim, total, unpack ? 1 : 0); break;
  switch (kind) {
    KQ_PACK(Q4_K) KQ_PACK(Q6_K) KQ_PACK(Q5_K) KQ_PACK(Q3_K) KQ_PACK(Q2_K) KQ_PACK(Q8_0)
    default: return hipErrorInvalidValue;
  }
#undef KQ_PACK
  return hipGetLastError();
}

}  // namespace kq
