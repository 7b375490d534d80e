// kq_packed_multi.hip -- Y[b][out] = W X[b] for up to 8 activation vectors at
// once over the packed layout: the small-batch product on VALU.
//
// The batch-1 kernel's structure (kq_packed.hip): lane = row, a wave walks
// spw super-block columns, NW waves per workgroup meet in LDS and ks
// workgroups per tile meet in the fence-free cross-workgroup sum.  Each
// column's weights are loaded once and multiplied by every vector in turn
// (each vector repeats the per-weight arithmetic, one v_fma_mix_f32 plus
// unpacking, but not the HBM read), so nb vectors cost far less than nb
// launches while VALU time stays below the launch's fixed cost: measured on
// MI355X, faster than the MFMA kernel up to 4 vectors on Q4_K and Q6_K.  Activations
// stay
// f32 and every vector's sums are formed in the batch-1 kernel's order under
// the same split plan, so row b of the result is bit-identical to the batch-1
// matvec of X[b].
//
// QMatMul on the CPU (llm_dequant.adb:808-932, once per vector) and the
// reference's batched kernels (gpu/gpu_matvec.cu:234-382) compute the same
// products.
#include "kq_kernels.h"
#include "kq_packed.h"

namespace kq {

constexpr int MV_MULTI_MAX = 8;  // vectors per launch

template <int KIND, int NW, int BMAX, bool PF>
__global__ __launch_bounds__(64 * NW) void kq_mm_packed_valu(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                            const float* __restrict__ X, int in_dim, int nb,
                                                            float* __restrict__ Y, int spw,
                                                            float* __restrict__ part, unsigned* __restrict__ count) {
  using R = typename Packed<KIND>::R;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  __shared__ float red[BMAX][NW][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x, ks = gridDim.y;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  const uint8_t* g = P + ((size_t)tile * nsb + sb0) * GB;
  float acc[BMAX];
#pragma unroll
  for (int b = 0; b < BMAX; ++b) acc[b] = 0.f;
  R r = Packed<KIND>::load(g, lane);
  for (int s = 0; s < spw; ++s) {
    R nr = r;
    if (PF && s + 1 < spw) {
      nr = Packed<KIND>::load(g + (size_t)(s + 1) * GB, lane);
      asm volatile("" ::: "memory");  // keep the next column's loads issued here
    }
    const float* xs = X + (size_t)(sb0 + s) * 256;
#pragma unroll
    for (int b = 0; b < BMAX; ++b)
      if (b < nb) {
        // Decode per vector: hoisted out of this loop, a whole decoded column
        // (256 floats per lane) would not fit in registers.
        opaque_regs(r);
        acc[b] += sb_dot<KIND>(r, xs + (size_t)b * in_dim, lane);
      }
    if (PF) r = nr;
    else if (s + 1 < spw) r = Packed<KIND>::load(g + (size_t)(s + 1) * GB, lane);
  }
  // Waves of the workgroup, then workgroups of the tile (ascending order).
#pragma unroll
  for (int b = 0; b < BMAX; ++b) red[b][w][lane] = acc[b];
  __syncthreads();
  if (w != 0) return;  // no barrier follows
  float t[BMAX];
#pragma unroll
  for (int b = 0; b < BMAX; ++b) {
    t[b] = red[b][0][lane];
#pragma unroll
    for (int k = 1; k < NW; ++k) t[b] += red[b][k][lane];
  }
  const int row = tile * 64 + lane;
  if (ks > 1) {
    const size_t ntiles = gridDim.x;
#pragma unroll
    for (int b = 0; b < BMAX; ++b)
      if (b < nb)
        __hip_atomic_store(&part[(((size_t)blockIdx.y * ntiles + tile) * BMAX + b) * 64 + lane], t[b],
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the partials are out before the arrival counts
    unsigned old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(&count[(size_t)tile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(old) != (unsigned)(ks - 1)) return;
#pragma unroll
    for (int b = 0; b < BMAX; ++b) t[b] = 0.f;
    for (int k = 0; k < ks; ++k) {
      float v[BMAX];
#pragma unroll
      for (int b = 0; b < BMAX; ++b)
        v[b] = b < nb ? __hip_atomic_load(&part[(((size_t)k * ntiles + tile) * BMAX + b) * 64 + lane],
                                          __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                      : 0.f;
#pragma unroll
      for (int b = 0; b < BMAX; ++b) t[b] += v[b];
    }
    if (lane == 0)
      __hip_atomic_store(&count[(size_t)tile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (row < out_rows) {
#pragma unroll
    for (int b = 0; b < BMAX; ++b)
      if (b < nb) Y[(size_t)b * out_rows + row] = t[b];
  }
}

size_t multi_workspace_floats(int in_dim, int out_dim) {
  return packed_workspace_floats(in_dim, out_dim) * MV_MULTI_MAX;
}

template <int KIND, int BMAX>
static hipError_t launch_multi_kind(const uint8_t* P, int in_dim, int out_dim, int nb, const float* X, float* Y,
                                    float* part, unsigned* count, hipStream_t s) {
  const PackedPlan p = packed_plan(in_dim, out_dim);
  const dim3 grid((out_dim + 63) / 64, p.ks);
  const int nsb = in_dim / 256;
  switch (p.nw) {
// The prefetching walk holds two weight register sets: at 16 waves per
// workgroup Q6_K and Q8_0 spill with it (16-77 registers), so they walk their
// columns one after another.
#define KQ_MM(N)                                                                                                 \
  case N:                                                                                                        \
    if constexpr (!(N == 16 && (KIND == Q6_K || KIND == Q8_0)))                                                  \
      if (p.spw > 1) {                                                                                           \
        hipLaunchKernelGGL((kq_mm_packed_valu<KIND, N, BMAX, true>), grid, dim3(64 * N), 0, s, P, nsb, out_dim,  \
                           X, in_dim, nb, Y, p.spw, part, count);                                                \
        break;                                                                                                   \
      }                                                                                                          \
    hipLaunchKernelGGL((kq_mm_packed_valu<KIND, N, BMAX, false>), grid, dim3(64 * N), 0, s, P, nsb, out_dim, X,  \
                       in_dim, nb, Y, p.spw, part, count);                                                       \
    break;
    KQ_MM(16) KQ_MM(8) KQ_MM(4) KQ_MM(2) KQ_MM(1)
#undef KQ_MM
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_multi_b(const uint8_t* P, int in_dim, int out_dim, int nb, const float* X, float* Y,
                                 float* part, unsigned* count, hipStream_t s) {
  if (nb <= 4) return launch_multi_kind<KIND, 4>(P, in_dim, out_dim, nb, X, Y, part, count, s);
  return launch_multi_kind<KIND, 8>(P, in_dim, out_dim, nb, X, Y, part, count, s);
}

hipError_t launch_matmul_packed_valu(int kind, const void* P, int in_dim, int out_dim, int nb, const float* X, float* Y,
                                     float* part, unsigned* count, hipStream_t s) {
  if (nb < 1 || nb > MV_MULTI_MAX) return hipErrorInvalidValue;
  const uint8_t* w = (const uint8_t*)P;
  switch (kind) {
    case Q4_K: return launch_multi_b<Q4_K>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    case Q6_K: return launch_multi_b<Q6_K>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    case Q5_K: return launch_multi_b<Q5_K>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    case Q3_K: return launch_multi_b<Q3_K>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    case Q2_K: return launch_multi_b<Q2_K>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    case Q8_0: return launch_multi_b<Q8_0>(w, in_dim, out_dim, nb, X, Y, part, count, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kq
