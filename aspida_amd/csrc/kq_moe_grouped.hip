// kq_moe_grouped.hip -- the MoE expert FFN over packed expert weights,
// grouped by expert: every expert's weights are read from HBM once per
// layer, however many of the T tokens chose it.
//
//   moe_gate_up   one workgroup per (expert, 64-row tile of the intermediate
//                 dimension); the routed experts and the shared expert
//                 (index n_exp, every token's slot top_k).  It lists the
//                 (token, slot) jobs that use its expert, keeps the tile's
//                 gate and up super-blocks in registers (wave w: column w) and
//                 writes h = silu(gate . x) * (up . x) per job
//                 (llm_moe.adb:124-132).  The shared expert's first tile also
//                 computes the shared gate g_t = sigmoid(shared_gate_inp . x_t)
//                 (llm_moe.adb:285-293) and zeroes the combine counters.
//   moe_down      one workgroup per (expert, 64-row tile of dim): the down
//                 projection of each job's h into yk[t][slot], then per
//                 (token, tile) an arrival count; the last of a token's
//                 top_k + 1 slots to arrive forms
//                 y = sum_k top_w[k] yk[k] (ascending k) + g_t yk[top_k]
//                 (llm_moe.adb:270-299), so the result does not depend on
//                 arrival order.
// Each (token, slot) product is the packed batch-1 matvec's arithmetic
// (kq_packed.hip: per-column sums formed in-kernel, f16-subnormal codes on
// v_fma_mix_f32), so no xsum launch is needed.
#include <math.h>

#include "kq_moe.h"
#include "kq_packed.h"

namespace kq {

constexpr int MOE_JOBS_PER_PASS = 8;  // jobs whose partial sums share LDS at once

// s16[j] = sum of xs[16j .. 16j+15] (wave-uniform); xs 16-byte aligned.
__device__ __forceinline__ void moe_sb_sums(const float* __restrict__ xs, int lane, float (&s16)[16]) {
  float4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(xs + 4 * lane, 16), 16);
  float t = (v.x + v.y) + (v.z + v.w);
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0xB1, 0xF, 0xF, false));
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x4E, 0xF, 0xF, false));
#pragma unroll
  for (int j = 0; j < 16; ++j)
    s16[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), 4 * j));
}

template <int KIND>
__device__ __forceinline__ float moe_sb_dot(const typename Packed<KIND>::R& r, const float* __restrict__ xs,
                                            int lane) {
  using B = Block<KIND>;
  float s16[16];
  moe_sb_sums(xs, lane, s16);
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    XQuarter X;
    B::load_x(xs, s16, q, X);
    acc += B::dot(Packed<KIND>::quarter(r, q), q, X);
  }
  return acc;
}

// The gate and up dots of one super-block column over the same activations:
// each quarter of x is loaded once (64 SGPRs) and feeds both matrices.
template <int KIND>
__device__ __forceinline__ float2 moe_sb_dot2(const typename Packed<KIND>::R& rg, const typename Packed<KIND>::R& ru,
                                              const float* __restrict__ xs, int lane) {
  using B = Block<KIND>;
  float s16[16];
  moe_sb_sums(xs, lane, s16);
  float g = 0.f, u = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    XQuarter X;
    B::load_x(xs, s16, q, X);
    g += B::dot(Packed<KIND>::quarter(rg, q), q, X);
    u += B::dot(Packed<KIND>::quarter(ru, q), q, X);
    // Keep the next quarter's scalar loads below this one's arithmetic:
    // hoisted, the four quarters (256 SGPRs) spill into vector lanes.
    asm volatile("" ::: "memory");
  }
  return make_float2(g, u);
}

// Jobs (t * slots + k) of expert e, in ascending job order: routed slots with
// top_idx[t][k] == e, or every token's shared slot for e == n_exp.  Wave 0
// compacts 64 routing entries per step with a ballot.
__device__ __forceinline__ int moe_jobs(const int* __restrict__ idx, int T, int top_k, int n_exp, int e,
                                        int* __restrict__ jobs) {
  __shared__ int nj;
  const int slots = top_k + 1;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    if (e == n_exp) {
      for (int t = lane; t < T; t += 64) jobs[t] = t * slots + top_k;
      if (lane == 0) nj = T;
    } else {
      int base = 0;
      const int n = T * top_k;
      for (int i0 = 0; i0 < n; i0 += 64) {
        const int i = i0 + lane;
        const bool m = i < n && idx[i] == e;
        const unsigned long long mask = __ballot(m);
        const int pos = base + __popcll(mask & ((1ull << lane) - 1ull));
        if (m && pos < MOE_MAX_JOBS) jobs[pos] = (i / top_k) * slots + i % top_k;
        base += __popcll(mask);
      }
      if (lane == 0) nj = base < MOE_MAX_JOBS ? base : MOE_MAX_JOBS;
    }
  }
  __syncthreads();
  return nj;
}

// Wave w of NW owns super-block columns w, w + NW, ..., (cpw of them); its
// partial sums over them are accumulated in LDS and the NW partials of a
// row summed in ascending wave order.  With cpw == 1 the weights stay in
// registers for all of the expert's jobs; otherwise every pass of
// MOE_JOBS_PER_PASS jobs reloads its columns (from L2 after the first pass).
template <int KIND, int NW>
__global__ __launch_bounds__(64 * NW) void moe_gate_up(MoeGroupedArgs a, int cpw, const float* __restrict__ x,
                                                      float* __restrict__ h) {
  __shared__ int jobs[MOE_MAX_JOBS];
  __shared__ float part[MOE_JOBS_PER_PASS][NW][2][64];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = blockIdx.x, tile = blockIdx.y;
  const bool shared = e == a.n_exp;
  const int slots = a.top_k + 1;
  if (shared && tile == 0) {
    for (int i = threadIdx.x; i < a.T * a.tiles_dim; i += blockDim.x) a.count[(size_t)i * COUNTER_STRIDE] = 0u;
    if (w == 0)
      for (int t = 0; t < a.T; ++t) {
        float s = 0.f;
        if (a.sgi)
          for (int d = lane; d < a.dim; d += 64) s = __builtin_fmaf(a.sgi[d], x[(size_t)t * a.dim + d], s);
        s = wave_sum(s);
        if (lane == 0) a.gsh[t] = a.sgi ? 1.0f / (1.0f + expf(-s)) : 1.0f;
      }
  }
  const int nj = moe_jobs(a.idx, a.T, a.top_k, a.n_exp, e, jobs);
  if (nj == 0) return;  // uniform over the workgroup
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const size_t nsb = (size_t)NW * cpw;
  const uint8_t* G = (shared ? a.sh_gate : a.gate + (size_t)e * a.gu_stride) + (size_t)tile * nsb * GB;
  const uint8_t* U = (shared ? a.sh_up : a.up + (size_t)e * a.gu_stride) + (size_t)tile * nsb * GB;
  typename Packed<KIND>::R rg = Packed<KIND>::load(G + (size_t)w * GB, lane);
  typename Packed<KIND>::R ru = Packed<KIND>::load(U + (size_t)w * GB, lane);
  const int row = tile * 64 + lane;
  for (int j0 = 0; j0 < nj; j0 += MOE_JOBS_PER_PASS) {
    const int n = nj - j0 < MOE_JOBS_PER_PASS ? nj - j0 : MOE_JOBS_PER_PASS;
    for (int j = 0; j < n; ++j) part[j][w][0][lane] = part[j][w][1][lane] = 0.f;  // this wave's slots only
    for (int c = 0; c < cpw; ++c) {
      const int col = w + c * NW;
      if (cpw > 1 && (c > 0 || j0 > 0)) {
        rg = Packed<KIND>::load(G + (size_t)col * GB, lane);
        ru = Packed<KIND>::load(U + (size_t)col * GB, lane);
      }
#pragma unroll 1
      for (int j = 0; j < n; ++j) {
        // The job index is the same in every lane: say so, so that x is read
        // with scalar loads into SGPRs rather than once per lane.
        const int t = __builtin_amdgcn_readfirstlane(jobs[j0 + j]) / slots;
        opaque_regs(rg);
        opaque_regs(ru);
        const float2 gu = moe_sb_dot2<KIND>(rg, ru, x + (size_t)t * a.dim + (size_t)col * 256, lane);
        part[j][w][0][lane] += gu.x;
        part[j][w][1][lane] += gu.y;
      }
    }
    __syncthreads();
    for (int j = w; j < n; j += NW) {
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        g += part[j][k][0][lane];
        u += part[j][k][1][lane];
      }
      if (row < a.I) h[(size_t)jobs[j0 + j] * a.I + row] = (g / (1.0f + expf(-g))) * u;
    }
    __syncthreads();
  }
}

template <int KIND, int NW>
__global__ __launch_bounds__(64 * NW) void moe_down(MoeGroupedArgs a, int cpw, const float* __restrict__ h,
                                                   float* __restrict__ yk, float* __restrict__ y) {
  __shared__ int jobs[MOE_MAX_JOBS];
  __shared__ float part[MOE_JOBS_PER_PASS][NW][64];
  __shared__ int last[MOE_JOBS_PER_PASS];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = blockIdx.x, tile = blockIdx.y;
  const bool shared = e == a.n_exp;
  const int slots = a.top_k + 1;
  const int nj = moe_jobs(a.idx, a.T, a.top_k, a.n_exp, e, jobs);
  if (nj == 0) return;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const size_t nsb = (size_t)NW * cpw;
  const uint8_t* D = (shared ? a.sh_down : a.down + (size_t)e * a.d_stride) + (size_t)tile * nsb * GB;
  typename Packed<KIND>::R rd = Packed<KIND>::load(D + (size_t)w * GB, lane);
  const int row = tile * 64 + lane;
  for (int j0 = 0; j0 < nj; j0 += MOE_JOBS_PER_PASS) {
    const int n = nj - j0 < MOE_JOBS_PER_PASS ? nj - j0 : MOE_JOBS_PER_PASS;
    for (int j = 0; j < n; ++j) part[j][w][lane] = 0.f;  // this wave's slots only
    for (int c = 0; c < cpw; ++c) {
      const int col = w + c * NW;
      if (cpw > 1 && (c > 0 || j0 > 0)) rd = Packed<KIND>::load(D + (size_t)col * GB, lane);
#pragma unroll 1
      for (int j = 0; j < n; ++j) {
        const int job = __builtin_amdgcn_readfirstlane(jobs[j0 + j]);  // uniform: scalar loads of h
        opaque_regs(rd);
        const float v = moe_sb_dot<KIND>(rd, h + (size_t)job * a.I + (size_t)col * 256, lane);
        part[j][w][lane] += v;
      }
    }
    __syncthreads();
    // yk of each job (device-scope stores: the combine may run on another XCD).
    for (int j = w; j < n; j += NW) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) v += part[j][k][lane];
      __hip_atomic_store(&yk[(size_t)jobs[j0 + j] * a.dim + row], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < n) {
      const int t = jobs[j0 + threadIdx.x] / slots;
      last[threadIdx.x] = __hip_atomic_fetch_add(&a.count[((size_t)t * a.tiles_dim + tile) * COUNTER_STRIDE], 1u,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(slots - 1);
    }
    __syncthreads();
    // Combine every token whose last slot arrived here.
    for (int j = w; j < n; j += NW)
      if (last[j]) {
        const int t = jobs[j0 + j] / slots;
        const float* yt = yk + (size_t)t * slots * a.dim + row;
        float acc = 0.f;
        for (int k = 0; k < a.top_k; ++k)
          acc = acc + a.top_w[t * a.top_k + k] *
                          __hip_atomic_load(yt + (size_t)k * a.dim, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        acc = acc + a.gsh[t] * __hip_atomic_load(yt + (size_t)a.top_k * a.dim, __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT);
        y[(size_t)t * a.dim + row] = acc;
      }
    __syncthreads();
  }
}

// ---- launchers ------------------------------------------------------------------

// Work layout: h [T][slots][I] | yk [T][slots][dim] | gsh [T] (256-byte
// rounded) | counters [T][tiles_dim] x COUNTER_STRIDE.  Every part starts on
// a 256-byte boundary when work does (I and dim are multiples of 256).
size_t moe_grouped_work_bytes(int T, int dim, int I, int top_k) {
  const size_t slots = (size_t)top_k + 1;
  size_t n = 0;
  n += (size_t)T * slots * I * 4;                             // h
  n += (size_t)T * slots * dim * 4;                           // yk
  n += ((size_t)T * 4 + 255) / 256 * 256;                     // gsh
  n += (size_t)T * ((dim + 63) / 64) * COUNTER_STRIDE * 4;    // counters
  return n;
}

void moe_grouped_bind(MoeGroupedArgs& a, void* work) {
  const size_t slots = (size_t)a.top_k + 1;
  uint8_t* p = (uint8_t*)work;
  a.h = (float*)p;
  p += (size_t)a.T * slots * a.I * 4;
  a.yk = (float*)p;
  p += (size_t)a.T * slots * a.dim * 4;
  a.gsh = (float*)p;
  p += ((size_t)a.T * 4 + 255) / 256 * 256;
  a.count = (unsigned*)p;
  a.tiles_dim = (a.dim + 63) / 64;
}

// Waves per workgroup for nsb super-block columns: the largest of 8, 4, 3,
// 2, 1 dividing nsb (each wave then walks nsb / NW columns).
static int moe_waves(int nsb) {
  for (int nw : {8, 4, 3, 2})
    if (nsb % nw == 0) return nw;
  return 1;
}

template <int KIND>
static hipError_t launch_gate_up_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const dim3 grid(a.n_exp + 1, (a.I + 63) / 64);
  const int nsb = a.dim / 256, nw = moe_waves(nsb);
  switch (nw) {
#define KQ_GU(N) case N: hipLaunchKernelGGL((moe_gate_up<KIND, N>), grid, dim3(64 * N), 0, s, a, nsb / N, a.x, a.h); break;
    KQ_GU(1) KQ_GU(2) KQ_GU(3) KQ_GU(4) KQ_GU(8)
#undef KQ_GU
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_down_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const dim3 grid(a.n_exp + 1, a.tiles_dim);
  const int nsb = a.I / 256, nw = moe_waves(nsb);
  switch (nw) {
#define KQ_DN(N) case N: hipLaunchKernelGGL((moe_down<KIND, N>), grid, dim3(64 * N), 0, s, a, nsb / N, a.h, a.yk, a.y); break;
    KQ_DN(1) KQ_DN(2) KQ_DN(3) KQ_DN(4) KQ_DN(8)
#undef KQ_DN
    default: return hipErrorNotSupported;
  }
  return hipGetLastError();
}

bool moe_grouped_supported(int dim, int I, int T, int top_k) {
  return dim > 0 && I > 0 && dim % 256 == 0 && I % 256 == 0 && T > 0 && top_k > 0 && top_k <= MOE_MAX_TOPK &&
         (size_t)T * top_k <= MOE_MAX_JOBS && T <= MOE_MAX_JOBS;
}

hipError_t launch_moe_grouped(const MoeGroupedArgs& a, int gu_kind, int down_kind, hipStream_t s) {
  hipError_t e;
  switch (gu_kind) {
    case Q4_K: e = launch_gate_up_kind<Q4_K>(a, s); break;
    case Q6_K: e = launch_gate_up_kind<Q6_K>(a, s); break;
    case Q5_K: e = launch_gate_up_kind<Q5_K>(a, s); break;
    case Q3_K: e = launch_gate_up_kind<Q3_K>(a, s); break;
    case Q2_K: e = launch_gate_up_kind<Q2_K>(a, s); break;
    case Q8_0: e = launch_gate_up_kind<Q8_0>(a, s); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  switch (down_kind) {
    case Q4_K: return launch_down_kind<Q4_K>(a, s);
    case Q6_K: return launch_down_kind<Q6_K>(a, s);
    case Q5_K: return launch_down_kind<Q5_K>(a, s);
    case Q3_K: return launch_down_kind<Q3_K>(a, s);
    case Q2_K: return launch_down_kind<Q2_K>(a, s);
    case Q8_0: return launch_down_kind<Q8_0>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kq
