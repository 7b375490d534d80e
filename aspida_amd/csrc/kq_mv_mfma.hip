// kq_mv_mfma.hip -- batch-1 matvec of Q4_K and Q6_K weights on the matrix
// cores, over the packed layout (kq_packed.h).
//
// The VALU decode kernel (kq_packed.hip) spends one v_fma_mix_f32 per weight
// plus 0.6-1.5 instructions of unpacking and scaling, which keeps the vector
// ALUs too busy for weight loads and arithmetic to overlap.  Here the
// multiply-adds run on v_mfma_f32_16x16x32_f16 and the vector ALUs only unpack
// codes and apply the per-sub-block scales.
//
// One MFMA (A 16x32, B 32x16, D 16x16; lane layouts as in kq_mmq.hip):
//   B[k][n]  n = a weight row of a 16-row block; k = 8 g + t: 8 codes of
//            "quarter" g of that row, as f16 subnormals (q 2^-24, or 16 q
//            2^-24 for a high nibble left in place).  Lane (n, g) loads
//            exactly the packed bytes its codes come from.
//   A[m][k]  m = 4 g + 2 kappa + p: plane p (hi, lo) of the scaled activation
//            at k when k lies in sub-block kappa of lane group g's pair of
//            sub-blocks, zero otherwise (only lanes 20 g + r hold data).
//   D[m][n]  sum over that sub-block of q x (plane p) for row n; it sits in
//            lane n + 16 (m / 4) element m % 4, so lane (n, g) ends up with
//            both planes of the two sub-blocks whose codes and scales it read.
// Q4_K: quarter g = qs bytes 32 g .. 32 g + 31, sub-blocks 2g (low nibbles)
// and 2g + 1 (high nibbles); MFMA j takes qs dword j (elements 4j + {0,2,1,3}
// of both).  Eight MFMAs per 16-row block and super-block, one accumulator.
// Q6_K: quarter g = 2h + t holds sub-blocks 8h + t + 2k (k = 0..3) -- the
// quarter split of Block<Q6_K>; MFMA (T, j) takes 4 elements of sub-blocks
// k = 2T, 2T + 1, built from ql/qh dword j; two accumulators (T = 0, 1).
// A wave takes a 64-row tile (four blocks) and a range of super-block columns.
//
// A depends on x only.  Per column each wave builds it in its own 8 KB LDS
// image (one float4 of x per lane; the zero part is written once) and reads it
// back as 8 16-byte fragments per lane, shared by the tile's four row blocks.
// Activations are scaled per column: x' = x S, with S a power of two that puts
// the column's largest |x| just below 2^14 (Q4_K's high-nibble sub-blocks take
// S / 16, which absorbs their codes' factor 16), hi = f16(x'), lo = f16(x' - hi)
// -- x to about 2^-22 relative.  The minimum / code-offset terms use the f32
// sub-block sums of x S.  Row headers (Q4_K d, dmin, scales; Q6_K scales, d)
// are loaded once per row and shared through LDS by the row's four quarters.
//
// Accuracy.  The matrix cores do not round each addition as IEEE f32 does:
// measured on MI355X, a product much smaller than the largest one in the same
// sum (and, in a chain of MFMAs, than the accumulator) keeps fewer bits.  So
// the result is within about 1e-6 of sum |w x| for ordinary activations, but
// within only ~1e-4 when a column holds outliers 10^4 times its other values
// (the VALU kernel: ~1e-7).  The lo plane is stored times 2^11 so that its
// products are as large as hi's.
//
// Result per row: the decodes of Decode_Q4K_Block / Decode_Q6K_Block
// (src/llm/llm_dequant.adb:536-553, 140-181) dotted with x, in a different
// summation order from the CPU's (QMatVec, llm_dequant.adb:808-932).
#include <algorithm>
#include <atomic>

#include "kq_host.h"
#include "kq_kernels.h"
#include "kq_mv_mfma.h"

namespace kq {

template <int KIND, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                     const float* __restrict__ x, float* __restrict__ y, int spw,
                                                     float* __restrict__ part, unsigned* __restrict__ count) {
  __shared__ MvShared<KIND, KIND> sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const float rowsum = mv_mfma_rows<KIND, PIPE>(P, nsb, tile, (blockIdx.y * NW + w) * spw, spw, x, sh[w].img,
                                              sh[w].xsum, &sh[w].hdr.a, lane);
  mv_epilogue<NW>(rowsum, tile, tile, out_rows, y, part, count);
}

// Two matrices that multiply the same x (q|k and v of attention): tiles
// [0, tiles_a) of the grid are matrix A's (kind KA), the rest matrix B's.
template <int KA, int KB, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma2(const uint8_t* __restrict__ Pa, int out_a, float* __restrict__ ya,
                                                      const uint8_t* __restrict__ Pb, int out_b, float* __restrict__ yb,
                                                      int tiles_a, int nsb, const float* __restrict__ x, int spw,
                                                      float* __restrict__ part, unsigned* __restrict__ count) {
  __shared__ MvShared<KA, KB> sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gtile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  if (gtile < tiles_a) {
    const float r = mv_mfma_rows<KA, PIPE>(Pa, nsb, gtile, sb0, spw, x, sh[w].img, sh[w].xsum, &sh[w].hdr.a, lane);
    mv_epilogue<NW>(r, gtile, gtile, out_a, ya, part, count);
  } else {
    const float r =
        mv_mfma_rows<KB, PIPE>(Pb, nsb, gtile - tiles_a, sb0, spw, x, sh[w].img, sh[w].xsum, &sh[w].hdr.b, lane);
    mv_epilogue<NW>(r, gtile, gtile - tiles_a, out_b, yb, part, count);
  }
}

// 16-row workgroups: workgroup b takes rows 16 b .. 16 b + 15 (block b % 4
// of tile b / 4) over every super-block column, its NW waves splitting the
// columns, and the waves meet in LDS only -- no partial sums through memory,
// whose device-coherent store, counter and reload cost about 1.5 us per
// launch on MI355X.  Each wave builds its own activation image per column, so
// the image is amortised over 16 rows instead of 64: the choice for matrices
// too small to need the 64-row kernels' throughput.
template <int NW>
__device__ __forceinline__ void mv16_epilogue(float r, int blk, int out_rows, float* __restrict__ y) {
  __shared__ float red16[NW][16];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (NW > 1) {
    if (lane < 16) red16[w][lane] = r;
    __syncthreads();
    if (w != 0) return;
    float t = red16[0][lane & 15];
#pragma unroll
    for (int k = 1; k < NW; ++k) t += red16[k][lane & 15];
    r = t;
  }
  const int row = 16 * blk + lane;
  if (lane < 16 && row < out_rows) y[row] = r;
}

// Six waves per SIMD for the Q6_K 16-row kernels of 8 or more waves walking
// their columns one after another (the output head's plan: three 8-wave
// workgroups per CU), which the registers of the dominant-activation path
// (kq_mv_mfma.h) would otherwise cut to five (head 65 -> 75 us); they fit
// without spilling (79 VGPRs).  Q3_K would spill and keeps five.
constexpr int mv16_waves(int kind, int nw, int pipe) { return kind == Q6_K && nw >= 8 && pipe == MV_SEQ ? 6 : 1; }

template <int KIND, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(mv16_waves(KIND, NW, PIPE))))
void kq_mv_mfma16(const uint8_t* __restrict__ P, int nsb, int out_rows, const float* __restrict__ x,
                  float* __restrict__ y, int spw) {
  __shared__ MvShared16 sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = mv16_block(blockIdx.x, gridDim.x);
  const float r = mv_mfma_rows<KIND, PIPE, 1>(P, nsb, blk >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KIND>*)nullptr, lane, blk & 3);
  mv16_epilogue<NW>(r, blk, out_rows, y);
}

// The same with x formed in the launch: x = RMSNorm(H + r) with weights g
// (LLM_RMSNorm.Forward, src/llm/llm_rmsnorm.adb:10-41, Epsilon 1e-6 of
// llm_rmsnorm.ads:19), as a model's attention norm before its first
// projection.  Every workgroup forms x in LDS -- threads 0-255 sum the
// squares in the order of a one-workgroup norm of 256 threads, so x is that
// norm's bit for bit -- and reads its columns from there; H is not written.
constexpr int MV_NORM_MAX_DIM = 4096;
template <int KIND, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma16_norm(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                            const float* __restrict__ H, const float* __restrict__ r,
                                                            const float* __restrict__ g, float* __restrict__ y,
                                                            int spw) {
  static_assert(NW >= 4, "the norm's sums take 256 threads");
  __shared__ MvShared16 sh[NW];
  __shared__ float4 xs4[MV_NORM_MAX_DIM / 4];
  __shared__ float part[4];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = mv16_block(blockIdx.x, gridDim.x), dim = nsb * 256, n4 = dim / 4;
  const float4* h4 = reinterpret_cast<const float4*>(H);
  const float4* r4 = reinterpret_cast<const float4*>(r);
  if (threadIdx.x < 256) {
    float ss = 0.f;
    for (int i = threadIdx.x; i < n4; i += 256) {
      float4 v = h4[i];
      if (r4) {
        const float4 a = r4[i];
        v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
      }
      xs4[i] = v;
      ss += v.x * v.x;
      ss += v.y * v.y;
      ss += v.z * v.z;
      ss += v.w * v.w;
    }
    ss = wave_total(ss);
    if (lane == 0) part[w] = ss;
  }
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) tot += part[k];
  const float rms = sqrtf(tot / (float)dim + 1e-6f);
  const float4* g4 = reinterpret_cast<const float4*>(g);
  for (int i = threadIdx.x; i < n4; i += 64 * NW) {
    const float4 v = xs4[i], gg = g4[i];
    xs4[i] = make_float4((v.x / rms) * gg.x, (v.y / rms) * gg.y, (v.z / rms) * gg.z, (v.w / rms) * gg.w);
  }
  __syncthreads();
  const float res = mv_mfma_rows<KIND, PIPE, 1>(P, nsb, blk >> 2, w * spw, spw, reinterpret_cast<const float*>(xs4),
                                                sh[w].img, sh[w].xsum, (MvHdr<KIND>*)nullptr, lane, blk & 3);
  mv16_epilogue<NW>(res, blk, out_rows, y);
}

// Two matrices that multiply the same x: blocks [0, blocks_a) are matrix A's.
template <int KA, int KB, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma2_16(const uint8_t* __restrict__ Pa, int out_a,
                                                         float* __restrict__ ya, const uint8_t* __restrict__ Pb,
                                                         int out_b, float* __restrict__ yb, int blocks_a, int nsb,
                                                         const float* __restrict__ x, int spw) {
  __shared__ MvShared16 sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = mv16_block(blockIdx.x, gridDim.x);
  if (blk < blocks_a) {
    const float r = mv_mfma_rows<KA, PIPE, 1>(Pa, nsb, blk >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KA>*)nullptr, lane, blk & 3);
    mv16_epilogue<NW>(r, blk, out_a, ya);
  } else {
    const int b = blk - blocks_a;
    const float r = mv_mfma_rows<KB, PIPE, 1>(Pb, nsb, b >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KB>*)nullptr, lane, b & 3);
    mv16_epilogue<NW>(r, b, out_b, yb);
  }
}

// Small batches of NV <= 4 vectors with the batch-1 arithmetic: each
// column's weights are read once for every vector (mv_mfma_rows_nv), on
// 16-row workgroups as kq_mv_mfma16 (on 64-row ones the vectors' registers
// do not fit 16 waves).  Y[v][out_rows] for v < nv.
template <int KIND, int NW, int NV>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma16n(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                        const float* __restrict__ x, float* __restrict__ y, int spw,
                                                        int nv) {
  __shared__ MvShared16 sh[NW];
  __shared__ float red16[NW][NV][16];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = mv16_block(blockIdx.x, gridDim.x);
  float r[NV];
  mv_mfma_rows_nv<KIND, 1, NV>(P, nsb, blk >> 2, w * spw, spw, x, (size_t)nsb * 256, nv, sh[w].img, sh[w].xsum,
                               (MvHdr<KIND>*)nullptr, lane, blk & 3, r);
  if (lane < 16)
#pragma unroll
    for (int v = 0; v < NV; ++v) red16[w][v][lane] = r[v];
  __syncthreads();
  if (w != 0 || lane >= 16) return;
  const int row = 16 * blk + lane;
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    float t = red16[0][v][lane];
#pragma unroll
    for (int k = 1; k < NW; ++k) t += red16[k][v][lane];
    if (v < nv && row < out_rows) y[(size_t)v * out_rows + row] = t;
  }
}

// 0: the MFMA kernel for Q4_K and Q6_K, 1: the VALU kernel (comparison and tuning).
// Per calling thread (a test or tuning override).
static thread_local int g_engine = 0;

void set_matvec_engine(int engine) { g_engine = engine; }

bool matvec_mfma_takes(int kind) {
  return (kind == Q4_K || kind == Q6_K || kind == Q2_K || kind == Q5_K || kind == Q3_K) && g_engine == 0;
}

// The kernel a plan runs: NW waves per workgroup and the column walk.
static int mv_pipe(const PackedPlan& p) { return p.spw == 1 ? MV_ONE : p.seq ? MV_SEQ : MV_PF; }

// Dynamic LDS that leaves room for at most ceil(blocks / CUs) workgroups per
// CU: the dispatcher otherwise stacks several small workgroups on one CU
// while others idle (Q4_K 4096x4096, 256 blocks: 4.7 us stacked, 4.3 us one
// per CU).  The kernels do not use it.  Per kernel, once: its static LDS and
// the dynamic LDS it may take (the device's per-workgroup limit minus the
// static part, opted into; 0 if any query fails, which only turns the
// spreading off).
struct LdsRoom {
  size_t stat = 0, dyn_max = 0;
};

// min_static: the kernel's static LDS as this file lays it out, a floor in
// case the runtime reports less; 1 KB of the limit is left unused.  Run
// through OnceQuery (kq_host.h), which clears the error a failed query leaves.
static LdsRoom lds_room_of(const void* kernel, size_t min_static) {
  LdsRoom r;
  hipFuncAttributes fa;
  int dev = 0, smem = 0;
  if (hipFuncGetAttributes(&fa, kernel) == hipSuccess && hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&smem, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess) {
    const size_t stat = std::max<size_t>(fa.sharedSizeBytes, min_static);
    if ((size_t)smem > stat + 1024 &&
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, smem - (int)stat - 1024) ==
            hipSuccess) {
      r.stat = stat;
      r.dyn_max = (size_t)smem - stat - 1024;
    }
  }
  return r;
}

// One per kernel (K is the kernel itself, so each instantiation has its own).
template <auto K, int NW>
static LdsRoom lds_room() {
  static OnceQuery<LdsRoom> q;
  return q.get(
      [] { return lds_room_of(reinterpret_cast<const void*>(K), (size_t)NW * (sizeof(MvShared16) + 16 * sizeof(float))); },
      LdsRoom{});
}

static int device_attr(hipDeviceAttribute_t a, int fallback) {
  int dev = 0, v = 0;
  const bool ok = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, a, dev) == hipSuccess && v > 0;
  return ok ? v : fallback;
}

// Never more than the kernel's own dynamic allowance (room.dyn_max), so static
// plus dynamic LDS stays within the per-workgroup limit.
static size_t mv16_spread_lds(int blocks, const LdsRoom& room) {
  static OnceQuery<int> qc, ql;
  const int cus = qc.get([] { return device_attr(hipDeviceAttributeMultiprocessorCount, 256); }, 256);
  const int lds_cu =
      ql.get([] { return device_attr(hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, 160 * 1024); }, 160 * 1024);
  const size_t per_cu = std::max<size_t>(1, ((size_t)blocks + cus - 1) / cus);
  const size_t share = (size_t)lds_cu / per_cu, need = room.stat + 2048;
  if (share <= need) return 0;
  return std::min(room.dyn_max, (share - need) / 1024 * 1024);
}

template <int KIND>
static hipError_t launch_mfma16_kind(const PackedPlan& p, const uint8_t* w, int in_dim, int out_dim, const float* x,
                                     float* y, hipStream_t s) {
  const dim3 grid((out_dim + 15) / 16);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
#define KQ_GO(N, PIPE)                                                                                     \
  hipLaunchKernelGGL((kq_mv_mfma16<KIND, N, PIPE>), grid, dim3(64 * N),                                    \
                     mv16_spread_lds((int)grid.x, lds_room<kq_mv_mfma16<KIND, N, PIPE>, N>()), s, w, nsb, out_dim, x, \
                     y, p.spw)
#define KQ_NW(N)                                  \
  case N:                                         \
    if (pipe == MV_ONE) {                         \
      KQ_GO(N, MV_ONE);                           \
    } else if (pipe == MV_SEQ) {                  \
      KQ_GO(N, MV_SEQ);                           \
    } else {                                      \
      KQ_GO(N, MV_PF);                            \
    }                                             \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(14) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_mfma_kind(const uint8_t* w, int in_dim, int out_dim, const float* x, float* y, float* part,
                                   unsigned* count, hipStream_t s) {
  const PackedPlan p = mfma_plan(KIND, in_dim, out_dim);
  if (p.blk16) return launch_mfma16_kind<KIND>(p, w, in_dim, out_dim, x, y, s);
  const dim3 grid((out_dim + 63) / 64, p.ks);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
#define KQ_GO(N, PIPE) \
  hipLaunchKernelGGL((kq_mv_mfma<KIND, N, PIPE>), grid, dim3(64 * N), 0, s, w, nsb, out_dim, x, y, p.spw, part, count)
#define KQ_NW(N)                                                                                \
  case N:                                                                                       \
    if (pipe == MV_ONE) KQ_GO(N, MV_ONE);                                                       \
    else if constexpr (N == 16) return hipErrorInvalidValue; /* 16 waves: one column only */    \
    else if (pipe == MV_SEQ) KQ_GO(N, MV_SEQ);                                                  \
    else if constexpr (N <= 4 || (N == 8 && KIND != Q6_K && KIND != Q5_K && KIND != Q3_K)) KQ_GO(N, MV_PF); \
    else return hipErrorInvalidValue; /* two register sets: <= 8 waves, 4 for Q6_K/Q5_K */      \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

// The pair kernels are built for Q4_K and Q6_K.
bool matvec2_mfma_takes(int kind_a, int kind_b) {
  return (kind_a == Q4_K || kind_a == Q6_K) && (kind_b == Q4_K || kind_b == Q6_K) && matvec_mfma_takes(kind_a) &&
         matvec_mfma_takes(kind_b);
}

template <int KA, int KB>
static hipError_t launch_mfma_pair(const uint8_t* a, int out_a, float* ya, const uint8_t* b, int out_b, float* yb,
                                   int in_dim, const float* x, float* part, unsigned* count, hipStream_t s) {
  const int tiles_a = (out_a + 63) / 64, tiles_b = (out_b + 63) / 64;
  // The split of the wider kind's registers (Q6_K when either is).
  constexpr int KW = KA == Q6_K || KB == Q6_K ? Q6_K : Q4_K;
  const PackedPlan p = mfma_plan(KW, in_dim, (tiles_a + tiles_b) * 64);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
  if (p.blk16) {
    const int blocks_a = (out_a + 15) / 16;
    const dim3 grid16(blocks_a + (out_b + 15) / 16);
#define KQ_GO(N, PIPE)                                                                                  \
  hipLaunchKernelGGL((kq_mv_mfma2_16<KA, KB, N, PIPE>), grid16, dim3(64 * N),                            \
                     mv16_spread_lds((int)grid16.x, lds_room<kq_mv_mfma2_16<KA, KB, N, PIPE>, N>()), s, a, out_a, \
                     ya, b, out_b, yb, blocks_a, nsb, x, p.spw)
#define KQ_NW(N)                                  \
  case N:                                         \
    if (pipe == MV_ONE) {                         \
      KQ_GO(N, MV_ONE);                           \
    } else if (pipe == MV_SEQ) {                  \
      KQ_GO(N, MV_SEQ);                           \
    } else {                                      \
      KQ_GO(N, MV_PF);                            \
    }                                             \
    break;
    switch (p.nw) {
      KQ_NW(16) KQ_NW(14) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
      default: return hipErrorInvalidValue;
    }
#undef KQ_NW
#undef KQ_GO
    return hipGetLastError();
  }
  const dim3 grid(tiles_a + tiles_b, p.ks);
#define KQ_GO(N, PIPE)                                                                                            \
  hipLaunchKernelGGL((kq_mv_mfma2<KA, KB, N, PIPE>), grid, dim3(64 * N), 0, s, a, out_a, ya, b, out_b, yb, tiles_a, \
                     nsb, x, p.spw, part, count)
#define KQ_NW(N)                                                          \
  case N:                                                                 \
    if (pipe == MV_ONE) KQ_GO(N, MV_ONE);                                 \
    else if constexpr (N == 16) return hipErrorInvalidValue;              \
    else if (pipe == MV_SEQ) KQ_GO(N, MV_SEQ);                            \
    else if constexpr (N <= 4 || (N == 8 && KW != Q6_K)) KQ_GO(N, MV_PF); \
    else return hipErrorInvalidValue;                                     \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

hipError_t launch_matvec2_mfma(int kind_a, const void* Pa, int out_a, float* ya, int kind_b, const void* Pb, int out_b,
                               float* yb, int in_dim, const float* x, float* part, unsigned* count, hipStream_t s) {
  const uint8_t* a = (const uint8_t*)Pa;
  const uint8_t* b = (const uint8_t*)Pb;
  if (kind_a == Q4_K && kind_b == Q6_K) return launch_mfma_pair<Q4_K, Q6_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q4_K && kind_b == Q4_K) return launch_mfma_pair<Q4_K, Q4_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q6_K && kind_b == Q6_K) return launch_mfma_pair<Q6_K, Q6_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q6_K && kind_b == Q4_K) return launch_mfma_pair<Q6_K, Q4_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  return hipErrorNotSupported;
}

// Waves per 16-row workgroup: the most of 16, 14, 8, 4, 2, 1 dividing the
// columns; each takes its columns one after another.
template <int KIND, int NV>
static hipError_t launch_mfma_nv_kind(const uint8_t* w, int in_dim, int out_dim, int nv, const float* x, float* y,
                                      hipStream_t s) {
  const int nsb = in_dim / 256;
  int nw = 1;
  for (int c : {16, 14, 8, 4, 2})
    if (nsb % c == 0) {
      nw = c;
      break;
    }
  const int spw = nsb / nw;
  const dim3 grid((out_dim + 15) / 16);
#define KQ_GO(N)                                                                                                 \
  case N:                                                                                                        \
    hipLaunchKernelGGL((kq_mv_mfma16n<KIND, N, NV>), grid, dim3(64 * N),                                         \
                       mv16_spread_lds((int)grid.x, lds_room<kq_mv_mfma16n<KIND, N, NV>, N>()), s, w, nsb, out_dim, x, \
                       y, spw, nv);                                                                              \
    break;
  switch (nw) {
    KQ_GO(16) KQ_GO(14) KQ_GO(8) KQ_GO(4) KQ_GO(2) KQ_GO(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_GO
  return hipGetLastError();
}

bool matvec_nv_takes(int kind, int in_dim, int out_dim) {
  return (kind == Q4_K || kind == Q6_K) && in_dim > 0 && in_dim % 256 == 0 && out_dim > 0;
}

hipError_t launch_matvec_mfma_nv(int kind, const void* P, int in_dim, int out_dim, int nv, const float* x, float* y,
                                 hipStream_t s) {
  const uint8_t* w = (const uint8_t*)P;
  if (nv < 1 || nv > 4) return hipErrorInvalidValue;
  if (kind == Q4_K) return nv <= 2 ? launch_mfma_nv_kind<Q4_K, 2>(w, in_dim, out_dim, nv, x, y, s)
                                   : launch_mfma_nv_kind<Q4_K, 4>(w, in_dim, out_dim, nv, x, y, s);
  if (kind == Q6_K) return nv <= 2 ? launch_mfma_nv_kind<Q6_K, 2>(w, in_dim, out_dim, nv, x, y, s)
                                   : launch_mfma_nv_kind<Q6_K, 4>(w, in_dim, out_dim, nv, x, y, s);
  return hipErrorNotSupported;
}

template <int KIND>
static hipError_t launch_norm16_kind(const PackedPlan& p, const uint8_t* w, int in_dim, int out_dim, const float* H,
                                     const float* r, const float* g, float* y, hipStream_t s) {
  const dim3 grid((out_dim + 15) / 16);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
#define KQ_GO(N, PIPE)                                                                                      \
  hipLaunchKernelGGL((kq_mv_mfma16_norm<KIND, N, PIPE>), grid, dim3(64 * N), 0, s, w, nsb, out_dim, H, r, g, y, \
                     p.spw)
#define KQ_NW(N)                                  \
  case N:                                         \
    if (pipe == MV_ONE) {                         \
      KQ_GO(N, MV_ONE);                           \
    } else if (pipe == MV_SEQ) {                  \
      KQ_GO(N, MV_SEQ);                           \
    } else {                                      \
      KQ_GO(N, MV_PF);                            \
    }                                             \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(14) KQ_NW(8) KQ_NW(4)
    default: return hipErrorNotSupported;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

bool matvec_norm_takes(int kind, int in_dim, int out_dim) {
  if (!(kind == Q4_K || kind == Q6_K) || !matvec_mfma_takes(kind) || in_dim <= 0 || in_dim % 256 ||
      in_dim > MV_NORM_MAX_DIM || out_dim <= 0)
    return false;
  const PackedPlan p = mfma_plan(kind, in_dim, out_dim);
  return p.blk16 && p.nw >= 4 && p.nw != 2 && p.nw != 1;
}

hipError_t launch_matvec_norm(int kind, const void* P, int in_dim, int out_dim, const float* H, const float* r,
                              const float* g, float* y, hipStream_t s) {
  if (!matvec_norm_takes(kind, in_dim, out_dim)) return hipErrorNotSupported;
  const PackedPlan p = mfma_plan(kind, in_dim, out_dim);
  const uint8_t* w = (const uint8_t*)P;
  return kind == Q4_K ? launch_norm16_kind<Q4_K>(p, w, in_dim, out_dim, H, r, g, y, s)
                      : launch_norm16_kind<Q6_K>(p, w, in_dim, out_dim, H, r, g, y, s);
}

hipError_t launch_matvec_mfma(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y, float* part,
                              unsigned* count, hipStream_t s) {
  const uint8_t* w = (const uint8_t*)P;
  switch (kind) {
    case Q4_K: return launch_mfma_kind<Q4_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q6_K: return launch_mfma_kind<Q6_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q2_K: return launch_mfma_kind<Q2_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q5_K: return launch_mfma_kind<Q5_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q3_K: return launch_mfma_kind<Q3_K>(w, in_dim, out_dim, x, y, part, count, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace kq
