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

#include <algorithm>
#include <map>
#include <mutex>

#include "kq_host.h"
#include "kq_kernels.h"
#include "kq_moe.h"
#include "kq_moe_sched.h"
#include "kq_mv_mfma.h"
#include "kq_packed.h"

namespace kq {


// The schedule of work items (moe_schedule, moe_item) and the gate/up
// prologue are in kq_moe_sched.h; these kernels take chunks of MOE_JPW jobs.
constexpr int MOE_JPW = 4;

// ---- kernels ------------------------------------------------------------------------
//
// Wave w of NW owns super-block columns w, w + NW, ... (cpw of them) of the
// item's tile; its partial sums over them are accumulated in LDS and the NW
// partials of a row summed in ascending wave order.

// Two workgroups per CU (four waves per SIMD at NW = 8), so one's weight
// loads overlap the other's arithmetic -- for the kinds whose gate and up
// registers fit in 128 VGPRs without spilling.
constexpr int moe_gu_waves(int kind, int nw) {
  return (kind == Q6_K || kind == Q8_0 || nw < 4) ? 1 : nw / 2;
}

template <int KIND, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(moe_gu_waves(KIND, NW)))) void moe_gate_up(MoeGroupedArgs a, int cpw, const float* __restrict__ x,
                                                      float* __restrict__ h) {
  __shared__ MoeSched S;
  __shared__ float part[MOE_JPW][NW][2][64];
  __shared__ __attribute__((aligned(16))) float xst[NW][256];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slots = a.top_k + 1, ne = a.n_exp + 1, tiles = a.I / 64;
  moe_gu_prologue(a, x, NW, w, lane);
  const int items = moe_schedule<MOE_JPW>(a, S) * tiles;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const size_t nsb = (size_t)NW * cpw;
  for (int i = blockIdx.x; i < items; i += gridDim.x) {
    const MoeItem it = moe_item<MOE_JPW>(S, ne, tiles, i);
    const bool shared = it.e == a.n_exp;
    const uint8_t* G = (shared ? a.sh_gate : a.gate + (size_t)it.e * a.gu_stride) + (size_t)it.tile * nsb * GB;
    const uint8_t* U = (shared ? a.sh_up : a.up + (size_t)it.e * a.gu_stride) + (size_t)it.tile * nsb * GB;
    for (int j = 0; j < it.nj; ++j) part[j][w][0][lane] = part[j][w][1][lane] = 0.f;  // this wave's slots only
    for (int c = 0; c < cpw; ++c) {
      const int col = w + c * NW;
      const float4* xc = reinterpret_cast<const float4*>(x + (size_t)col * 256) + lane;
      float4 xv = xc[(size_t)(S.jobs[it.j0] / slots) * (a.dim / 4)];
      // Ordinary loads: an expert tile of more than MOE_JPW jobs is read again
      // by the adjacent items, and the caches serve those repeats.
      typename Packed<KIND>::R rg = Packed<KIND>::template load<false>(G + (size_t)col * GB, lane);
      typename Packed<KIND>::R ru = Packed<KIND>::template load<false>(U + (size_t)col * GB, lane);
#pragma unroll 1
      for (int j = 0; j < it.nj; ++j) {
        const float4 cur = xv;
        if (j + 1 < it.nj) xv = xc[(size_t)(S.jobs[it.j0 + j + 1] / slots) * (a.dim / 4)];  // next job's slice
        float s16[16];
        stage_x256(cur, xst[w], lane, s16);
        opaque_regs(rg);
        opaque_regs(ru);
        const float2 gu = staged_dot2<KIND>(rg, ru, xst[w], s16);
        part[j][w][0][lane] += gu.x;
        part[j][w][1][lane] += gu.y;
      }
    }
    __syncthreads();
    const int row = it.tile * 64 + lane;
    for (int j = w; j < it.nj; j += NW) {
      float g = 0.f, u = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) {
        g += part[j][k][0][lane];
        u += part[j][k][1][lane];
      }
      h[(size_t)S.jobs[it.j0 + j] * a.I + row] = (g / (1.0f + expf(-g))) * u;
    }
    __syncthreads();
  }
}

template <int KIND, int NW>
__global__ __launch_bounds__(64 * NW) void moe_down(MoeGroupedArgs a, int cpw, const float* __restrict__ h,
                                                   float* __restrict__ yk, float* __restrict__ y) {
  __shared__ MoeSched S;
  __shared__ float part[MOE_JPW][NW][64];
  __shared__ __attribute__((aligned(16))) float xst[NW][256];
  __shared__ int last[MOE_JPW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slots = a.top_k + 1, ne = a.n_exp + 1, tiles = a.tiles_dim;
  const int items = moe_schedule_load<MOE_JPW>(a, S) * tiles;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const size_t nsb = (size_t)NW * cpw;
  for (int i = blockIdx.x; i < items; i += gridDim.x) {
    const MoeItem it = moe_item<MOE_JPW>(S, ne, tiles, i);
    const bool shared = it.e == a.n_exp;
    const uint8_t* D = (shared ? a.sh_down : a.down + (size_t)it.e * a.d_stride) + (size_t)it.tile * nsb * GB;
    for (int j = 0; j < it.nj; ++j) part[j][w][lane] = 0.f;  // this wave's slots only
    for (int c = 0; c < cpw; ++c) {
      const int col = w + c * NW;
      const float4* hc = reinterpret_cast<const float4*>(h + (size_t)col * 256) + lane;
      float4 hv = hc[(size_t)S.jobs[it.j0] * (a.I / 4)];
      typename Packed<KIND>::R rd = Packed<KIND>::template load<false>(D + (size_t)col * GB, lane);
#pragma unroll 1
      for (int j = 0; j < it.nj; ++j) {
        const float4 cur = hv;
        if (j + 1 < it.nj) hv = hc[(size_t)S.jobs[it.j0 + j + 1] * (a.I / 4)];  // next job's slice
        float s16[16];
        stage_x256(cur, xst[w], lane, s16);
        opaque_regs(rd);
        part[j][w][lane] += staged_dot<KIND>(rd, xst[w], s16);
      }
    }
    __syncthreads();
    // yk of each job (device-scope stores: the combine may run on another XCD).
    const int row = it.tile * 64 + lane;
    for (int j = w; j < it.nj; j += NW) {
      float v = 0.f;
#pragma unroll
      for (int k = 0; k < NW; ++k) v += part[j][k][lane];
      __hip_atomic_store(&yk[(size_t)S.jobs[it.j0 + j] * a.dim + row], v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x < it.nj) {
      const int t = S.jobs[it.j0 + threadIdx.x] / slots;
      last[threadIdx.x] = __hip_atomic_fetch_add(&a.count[((size_t)t * tiles + it.tile) * COUNTER_STRIDE], 1u,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(slots - 1);
    }
    __syncthreads();
    // Combine every token whose last slot arrived here.
    for (int j = w; j < it.nj; j += NW)
      if (last[j]) {
        const int t = S.jobs[it.j0 + j] / slots;
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

// ---- one token on the matrix cores (Q4_K, Q6_K) ---------------------------------
//
// With T = 1 each slot is its own expert matrix and the projections are
// batch-1 matvecs: per wave the 16-row matrix-core matvec's arithmetic
// (kq_mv_mfma.h: the activation image, MFMA on f16-subnormal codes, scales in
// f32), with no schedule and no partial sums through memory.
//   moe_gate_up1  workgroup (slot k, 16-row block b of I): waves [0, NWG) take
//                 the gate matrix's columns, [NWG, 2 NWG) the up matrix's;
//                 h[k][16 b + r] = silu(g) u (llm_moe.adb:124-132).
//                 Workgroup 0 also forms g_t (moe_gu_prologue).
//   moe_down1     workgroup b (16 rows of dim) takes every (slot, column)
//                 pair of those rows, NW waves over the pairs, and forms
//                 y = sum_k top_w[k] y_k (ascending k) + g_t y_shared in LDS
//                 (llm_moe.adb:270-299).
// Expert ids outside [0, n_exp) are clamped for the loads, and such a
// token's y is not written.
constexpr int MOE1_MAX_UNITS = 64;  // (slot, down column) pairs per down workgroup

__device__ __forceinline__ int moe_expert(const MoeGroupedArgs& a, int k) {
  return min(max(a.idx[k], 0), a.n_exp - 1);
}

template <int KIND, int NWG, int PIPE>
__global__ __launch_bounds__(128 * NWG) void moe_gate_up1(MoeGroupedArgs a, int cpw) {
  constexpr int NW = 2 * NWG;
  __shared__ MvShared16 sh[NW];
  __shared__ float part[NW][16];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blocks = a.I / 16, k = blockIdx.x / blocks, b = blockIdx.x % blocks;
  moe_gu_prologue(a, a.x, NW, w, lane);
  const bool up = w >= NWG;
  const int wc = up ? w - NWG : w;
  const uint8_t* M = k < a.top_k ? (up ? a.up : a.gate) + (size_t)moe_expert(a, k) * a.gu_stride
                                 : (up ? a.sh_up : a.sh_gate);
  const float r = mv_mfma_rows<KIND, PIPE, 1>(M, a.dim / 256, b >> 2, wc * cpw, cpw, a.x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KIND>*)nullptr, lane, b & 3);
  if (lane < 16) part[w][lane] = r;
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    float g = 0.f, u = 0.f;
#pragma unroll
    for (int q = 0; q < NWG; ++q) {
      g += part[q][t];
      u += part[NWG + q][t];
    }
    a.h[(size_t)k * a.I + 16 * b + t] = (g / (1.0f + expf(-g))) * u;
  }
}

// One (slot, column) unit of a 16-row block whose weights c and activations
// xv are loaded: the arithmetic of mv_mfma_rows<KIND, MV_ONE, 1> from the
// image build on (the same results).
template <int KIND>
__device__ __forceinline__ float moe1_unit(const MvCol<KIND, 1>& c, float4 xv, MvShared16& sh, int lane,
                                           const uint8_t* grp, const float* xs, int rb0) {
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (lane < 17) sh.img[j][lane] = make_uint4(0u, 0u, 0u, 0u);
  const MvLane L = mv_lane<KIND>(sh.img, lane);
  float acc[1] = {0.f};
  const bool taken = mv_column<KIND, 1, 17>(c, xv, L, sh.img, sh.xsum, (MvHdr<KIND>*)nullptr, lane, acc);
  float* red = reinterpret_cast<float*>(&sh.img[0][0]);
  __builtin_amdgcn_wave_barrier();
  red[lane] = acc[0];
  __builtin_amdgcn_wave_barrier();
  const float* rr = red + (lane & 15);
  return ((rr[0] + rr[16]) + rr[32]) + rr[48] + mv_dominant_exact<KIND, 1>(taken ? 1u : 0u, 1, grp, 0, xs, lane, rb0);
}

template <int KIND, int NW>
__global__ __launch_bounds__(64 * NW) void moe_down1(MoeGroupedArgs a) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  __shared__ MvShared16 sh[NW];
  __shared__ float part[MOE1_MAX_UNITS][16];
  __shared__ float wk[MOE_MAX_TOPK + 1];  // the combine's slot weights, top_w[k] and g last
  __shared__ int ids[MOE_MAX_TOPK];       // the slots' expert ids (a token with an invalid one keeps y unwritten)
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b = blockIdx.x, nsb = a.I / 256, units = (a.top_k + 1) * nsb;
  // Requested now, with the first loads, rather than one after another in the combine.
  if ((int)threadIdx.x <= a.top_k) wk[threadIdx.x] = (int)threadIdx.x < a.top_k ? a.top_w[threadIdx.x] : a.gsh[0];
  if ((int)threadIdx.x < a.top_k) ids[threadIdx.x] = a.idx[threadIdx.x];
  // Units u and u + NW of a wave: both units' weights and activations are
  // requested before either is multiplied, so their loads overlap.
  for (int u = w; u < units; u += 2 * NW) {
    const int v = u + NW < units ? u + NW : u;
    const int k0 = u / nsb, c0 = u % nsb, k1 = v / nsb, c1 = v % nsb;
    const uint8_t* M0 = k0 < a.top_k ? a.down + (size_t)moe_expert(a, k0) * a.d_stride : a.sh_down;
    const uint8_t* M1 = k1 < a.top_k ? a.down + (size_t)moe_expert(a, k1) * a.d_stride : a.sh_down;
    MvCol<KIND, 1> w0, w1;
    const float4 x0 = ld_f4(a.h + (size_t)k0 * a.I + (size_t)c0 * 256 + 4 * lane);
    w0.load(M0 + ((size_t)(b >> 2) * nsb + c0) * GB, lane, b & 3);
    const float4 x1 = ld_f4(a.h + (size_t)k1 * a.I + (size_t)c1 * 256 + 4 * lane);
    w1.load(M1 + ((size_t)(b >> 2) * nsb + c1) * GB, lane, b & 3);
    const float r0 = moe1_unit<KIND>(w0, x0, sh[w], lane, M0 + ((size_t)(b >> 2) * nsb + c0) * GB,
                                     a.h + (size_t)k0 * a.I + (size_t)c0 * 256, b & 3);
    if (lane < 16) part[u][lane] = r0;
    if (v != u) {
      const float r1 = moe1_unit<KIND>(w1, x1, sh[w], lane, M1 + ((size_t)(b >> 2) * nsb + c1) * GB,
                                       a.h + (size_t)k1 * a.I + (size_t)c1 * 256, b & 3);
      if (lane < 16) part[v][lane] = r1;
    }
  }
  __syncthreads();
  if (threadIdx.x < 16) {
    const int t = threadIdx.x;
    float acc = 0.f;
    bool valid = true;
    for (int k = 0; k <= a.top_k; ++k) {
      float s = 0.f;
      for (int c = 0; c < nsb; ++c) s += part[k * nsb + c][t];
      acc = acc + wk[k] * s;
      if (k < a.top_k) valid = valid && ids[k] >= 0 && ids[k] < a.n_exp;
    }
    if (valid) a.y[16 * b + t] = acc;
  }
}

// ---- launchers ------------------------------------------------------------------

// Work layout: h [T][slots][I] | yk [T][slots][dim] | gsh [T] (256-byte
// rounded) | counters [T][blocks_dim] x COUNTER_STRIDE (16-row blocks of dim:
// enough for either down projection).  Every part starts on
// a 256-byte boundary when work does (I and dim are multiples of 256).
size_t moe_grouped_work_bytes(int T, int dim, int I, int top_k) {
  const size_t slots = (size_t)top_k + 1;
  size_t n = 0;
  n += (size_t)T * slots * I * 4;                             // h
  n += (size_t)T * slots * dim * 4;                           // yk
  n += ((size_t)T * 4 + 255) / 256 * 256;                     // gsh
  n += (size_t)T * ((dim + 15) / 16) * COUNTER_STRIDE * 4;    // counters
  n += ((MOE_MAX_EXP + 2 + (size_t)T * slots) * 4 + 255) / 256 * 256;  // schedule
  n += (size_t)(1 + moe_max_chunks(T, top_k, T * top_k, MOE_MFMA_JPW)) * 16;  // chunk table
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
  p += (size_t)a.T * ((a.dim + 15) / 16) * COUNTER_STRIDE * 4;
  a.sched = (int*)p;
  p += ((MOE_MAX_EXP + 2 + (size_t)a.T * slots) * 4 + 255) / 256 * 256;
  a.units = (int4*)p;
  a.tiles_dim = (a.dim + 63) / 64;
  a.blocks_dim = (a.dim + 15) / 16;
}

// Waves per workgroup for nsb super-block columns: the largest of 8, 4, 3,
// 2, 1 dividing nsb (each wave then walks nsb / NW columns).
static int moe_waves(int nsb) {
  for (int nw : {8, 4, 3, 2})
    if (nsb % nw == 0) return nw;
  return 1;
}

// Workgroups of a launch: enough for every item the schedule can produce
// (chunks <= jobs / MOE_JPW + non-empty experts), at most what the device
// keeps resident at once; the kernels loop over items beyond the grid, so
// no workgroup waits for a slot only to build the schedule again.
static int moe_resident(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  int dev = 0;
  if (hipPeekAtLastError() != hipSuccess || hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({kernel, dev});
  if (it != cache.end()) return it->second;
  int cus = 0, per = 0;
  // The occupancy query fails ("unknown error") for some kernels of 256 VGPRs
  // on this runtime, the Q8_0 grouped ones among them; their launches are
  // fine.  Then one resident workgroup per CU is assumed, and the query's own
  // error is cleared (query_clean, kq_host.h) so that the launch's check does
  // not report it; an error pending from earlier work is left in place.
  if (!query_clean([&] {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
          cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || per <= 0) per = 1;
      }))
    return 256;
  return cache[{kernel, dev}] = per * cus;
}

static int moe_grid(const MoeGroupedArgs& a, int tiles, int cap) {
  const long slots = a.top_k + 1;
  const long nonempty = std::min<long>(a.n_exp, (long)a.T * a.top_k) + 1;
  const long bound = (long)tiles * (((long)a.T * slots + MOE_JPW - 1) / MOE_JPW + nonempty);
  return (int)std::max<long>(1, std::min<long>(bound, cap));
}

template <int KIND>
static hipError_t launch_gate_up_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const int nsb = a.dim / 256, nw = moe_waves(nsb);
#define KQ_GU(N)                                                                                        \
  case N: {                                                                                             \
    const dim3 grid(moe_grid(a, a.I / 64, moe_resident((const void*)moe_gate_up<KIND, N>, 64 * N)));    \
    hipLaunchKernelGGL((moe_gate_up<KIND, N>), grid, dim3(64 * N), 0, s, a, nsb / N, a.x, a.h);        \
    break;                                                                                              \
  }
  switch (nw) {
    KQ_GU(1) KQ_GU(2) KQ_GU(3) KQ_GU(4) KQ_GU(8)
    default: return hipErrorNotSupported;
  }
#undef KQ_GU
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_down_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const int nsb = a.I / 256, nw = moe_waves(nsb);
#define KQ_DN(N)                                                                                        \
  case N: {                                                                                             \
    const dim3 grid(moe_grid(a, a.tiles_dim, moe_resident((const void*)moe_down<KIND, N>, 64 * N)));    \
    hipLaunchKernelGGL((moe_down<KIND, N>), grid, dim3(64 * N), 0, s, a, nsb / N, a.h, a.yk, a.y);     \
    break;                                                                                              \
  }
  switch (nw) {
    KQ_DN(1) KQ_DN(2) KQ_DN(3) KQ_DN(4) KQ_DN(8)
    default: return hipErrorNotSupported;
  }
#undef KQ_DN
  return hipGetLastError();
}

bool moe_grouped_supported(int dim, int I, int T, int top_k) {
  return dim > 0 && I > 0 && dim % 256 == 0 && I % 256 == 0 && T > 0 && top_k > 0 && top_k <= MOE_MAX_TOPK &&
         (size_t)T * top_k <= MOE_MAX_JOBS && T <= MOE_MAX_JOBS;
}

bool moe_grouped_experts_ok(int n_exp) { return n_exp > 0 && n_exp <= MOE_MAX_EXP; }

static hipError_t launch_gate_up_valu(const MoeGroupedArgs& a, int gu_kind, hipStream_t s);
static hipError_t launch_down_valu(const MoeGroupedArgs& a, int down_kind, hipStream_t s);

// One-token launches: gate/up waves per matrix NWG (8, 4, 2 or 1, dividing
// dim / 256, columns one after another beyond one per wave); down waves up to
// 16 over the (slot, column) pairs.
template <int KIND>
static hipError_t launch_gate_up1_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const int nsb = a.dim / 256;
  int nwg = 1;
  for (int n : {8, 4, 2})
    if (nsb % n == 0) {
      nwg = n;
      break;
    }
  const int cpw = nsb / nwg;
  const dim3 grid((a.top_k + 1) * (a.I / 16));
#define KQ_GU1(N)                                                                                          \
  case N:                                                                                                  \
    if (cpw == 1)                                                                                          \
      hipLaunchKernelGGL((moe_gate_up1<KIND, N, MV_ONE>), grid, dim3(128 * N), 0, s, a, cpw);            \
    else                                                                                                   \
      hipLaunchKernelGGL((moe_gate_up1<KIND, N, MV_SEQ>), grid, dim3(128 * N), 0, s, a, cpw);            \
    break;
  switch (nwg) {
    KQ_GU1(1) KQ_GU1(2) KQ_GU1(4) KQ_GU1(8)
    default: return hipErrorNotSupported;
  }
#undef KQ_GU1
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_down1_kind(const MoeGroupedArgs& a, hipStream_t s) {
  const int units = (a.top_k + 1) * (a.I / 256);
  const int nw = units >= 16 ? 16 : units >= 8 ? 8 : units >= 4 ? 4 : units >= 2 ? 2 : 1;
  const dim3 grid(a.dim / 16);
#define KQ_DN1(N) \
  case N: hipLaunchKernelGGL((moe_down1<KIND, N>), grid, dim3(64 * N), 0, s, a); break;
  switch (nw) {
    KQ_DN1(1) KQ_DN1(2) KQ_DN1(4) KQ_DN1(8) KQ_DN1(16)
    default: return hipErrorNotSupported;
  }
#undef KQ_DN1
  return hipGetLastError();
}

hipError_t launch_moe_grouped(const MoeGroupedArgs& a, int gu_kind, int down_kind, hipStream_t s) {
  // One token with matrix-core kinds throughout: the one-token kernels.
  const auto mfma_moe = [](int k) { return (k == Q4_K || k == Q6_K) && matvec_mfma_takes(k); };
  if (a.T == 1 && mfma_moe(gu_kind) && mfma_moe(down_kind) &&
      (a.top_k + 1) * (a.I / 256) <= MOE1_MAX_UNITS) {
    const hipError_t e = gu_kind == Q4_K ? launch_gate_up1_kind<Q4_K>(a, s) : launch_gate_up1_kind<Q6_K>(a, s);
    if (e != hipSuccess) return e;
    return down_kind == Q4_K ? launch_down1_kind<Q4_K>(a, s) : launch_down1_kind<Q6_K>(a, s);
  }
  // More tokens: grouped by expert, on the matrix cores for Q4_K / Q6_K.
  if (mfma_moe(gu_kind) && mfma_moe(down_kind)) return launch_moe_grouped_mfma(a, gu_kind, down_kind, s);
  const hipError_t e = launch_gate_up_valu(a, gu_kind, s);
  if (e != hipSuccess) return e;
  return launch_down_valu(a, down_kind, s);
}

static hipError_t launch_gate_up_valu(const MoeGroupedArgs& a, int gu_kind, hipStream_t s) {
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
  return e;
}

static hipError_t launch_down_valu(const MoeGroupedArgs& a, int down_kind, hipStream_t s) {
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
