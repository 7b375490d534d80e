// kq_moe.hip -- MoE expert FFN and router kernels for gfx950.
//
// The expert FFN of LLM_MoE.Forward (src/llm/llm_moe.adb:249-299) runs as:
//   xsum16(x)                 per-16 activation sums (kq_matvec.hip)
//   moe_proj<gate/up kinds>   one K-quant matvec per (token, slot), the expert
//                             index read from device memory
//   moe_swiglu                h = silu(g) * u, and h's per-16 sums
//   moe_proj<down kind>       down projection per (token, slot)
//   moe_shared_gate           g_t = sigmoid(shared_gate_inp . x_t) (optional)
//   moe_combine               y = sum_k top_w[k] * yk[k] (ascending k)
//                                 + g_t * y_shared
// Slot top_k of every token is the shared expert.
#include <math.h>

#include "kq_blocks.h"
#include "kq_kernels.h"
#include "kq_moe.h"
#include "kq_packed.h"

namespace kq {

// One wave computes R consecutive output rows of one (token, slot) job.
// Job j = t * slots + k reads expert idx[t * top_k + k] of `base` for k <
// top_k, and the matrix `shared` for k >= top_k (skipped when it is null).
struct ProjJob {
  const uint8_t* base;     // routed experts
  const uint8_t* shared;   // shared expert, or null to skip slots >= top_k
  long stride;             // bytes per routed expert
  const int* idx;          // [T][top_k]; ids outside [0, n_exp) are clamped
  int n_exp;
  int top_k, slots;        // slots = top_k (+1 with the shared expert)
  const float* x;          // activations
  long x_tok, x_slot;      // element strides of x per token / per slot
  float* y;
  long y_tok, y_slot;
  int in_dim, out_rows;
};

template <int KIND, int R>
__global__ __launch_bounds__(256) void moe_proj(ProjJob J, const float* __restrict__ xq_base) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (row0 >= J.out_rows) return;
  const int j = blockIdx.y;
  const int t = j / J.slots, k = j % J.slots;
  const uint8_t* W;
  if (k < J.top_k) {
    const int e = min(max(J.idx[t * J.top_k + k], 0), J.n_exp - 1);
    W = J.base + (size_t)e * (size_t)J.stride;
  } else {
    if (!J.shared) return;
    W = J.shared;
  }
  const int nsb = J.in_dim / 256;
  const size_t row_bytes = (size_t)nsb * Block<KIND>::BYTES;
  const long xoff = (long)t * J.x_tok + (long)k * J.x_slot;
  const float* x = J.x + xoff;
  const float* xq = xq_base + xoff / 16;
  const int c = lane & 3, slot = lane >> 2;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int sb = slot; sb < nsb; sb += 16) {
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] += quarter<KIND>(W + (size_t)min(row0 + r, J.out_rows - 1) * row_bytes +
                                         (size_t)sb * Block<KIND>::BYTES,
                                c, x + (size_t)sb * 256, xq + (size_t)sb * 16);
  }
  float* y = J.y + (long)t * J.y_tok + (long)k * J.y_slot;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < J.out_rows) y[row0 + r] = v;
  }
}

template <int KIND>
static void launch_proj(const ProjJob& J, int njobs, const float* xq, hipStream_t s) {
  constexpr int R = 2;
  const int waves = (J.out_rows + R - 1) / R;
  hipLaunchKernelGGL((moe_proj<KIND, R>), dim3((waves + 3) / 4, njobs), dim3(256), 0, s, J, xq);
}

static hipError_t proj(int kind, const ProjJob& J, int njobs, const float* xq, hipStream_t s) {
  switch (kind) {
    case Q4_K: launch_proj<Q4_K>(J, njobs, xq, s); break;
    case Q6_K: launch_proj<Q6_K>(J, njobs, xq, s); break;
    case Q5_K: launch_proj<Q5_K>(J, njobs, xq, s); break;
    case Q3_K: launch_proj<Q3_K>(J, njobs, xq, s); break;
    case Q2_K: launch_proj<Q2_K>(J, njobs, xq, s); break;
    case Q8_0: launch_proj<Q8_0>(J, njobs, xq, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// h = silu(g) * u with silu(v) = v / (1 + exp(-v)) (llm_moe.adb:88, 124-132);
// each thread handles 16 consecutive elements and writes their sum to hq.
__global__ void moe_swiglu(const float* __restrict__ g, const float* __restrict__ u, float* __restrict__ h,
                           float* __restrict__ hq, int n16) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n16) return;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 16; ++e) {
    const float gv = g[(size_t)i * 16 + e];
    const float v = (gv / (1.0f + expf(-gv))) * u[(size_t)i * 16 + e];
    h[(size_t)i * 16 + e] = v;
    s += v;
  }
  hq[i] = s;
}

// gsh[t] = sigmoid(sum_d sgi[d] x[t][d]) (llm_moe.adb:285-293), or 1.
__global__ void moe_shared_gate(const float* __restrict__ sgi, const float* __restrict__ x, int dim,
                                float* __restrict__ gsh) {
  const int t = blockIdx.x, lane = threadIdx.x;
  float a = 0.f;
  if (sgi)
    for (int d = lane; d < dim; d += 64) a = __builtin_fmaf(sgi[d], x[(size_t)t * dim + d], a);
  a = wave_sum(a);
  if (lane == 0) gsh[t] = sgi ? 1.0f / (1.0f + expf(-a)) : 1.0f;
}

// y[t][i] = ((0 + w0*yk0) + w1*yk1 + ...) + gsh[t] * yk[top_k]  (llm_moe.adb:270-299).
__global__ void moe_combine(const float* __restrict__ yk, const float* __restrict__ top_w,
                            const float* __restrict__ gsh, int top_k, int dim, int T, float* __restrict__ y) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= dim * T) return;
  const int t = i / dim, d = i % dim;
  const float* base = yk + (size_t)t * (top_k + 1) * dim + d;
  float acc = 0.f;
  for (int k = 0; k < top_k; ++k) acc = acc + top_w[t * top_k + k] * base[(size_t)k * dim];
  y[i] = acc + gsh[t] * base[(size_t)top_k * dim];
}

size_t moe_scratch_floats(const MoeWeights& w, int T, int top_k) {
  const size_t slots = (size_t)top_k + 1;
  return moe_staging_floats(w.dim, T, top_k)           // x | top_w | top_idx staging (host ABI)
         + (size_t)T * (w.dim / 16)                   // xq
         + 3 * (size_t)T * slots * w.intermed         // g, u, h
         + (size_t)T * slots * (w.intermed / 16)      // hq
         + (size_t)T * slots * w.dim                  // yk
         + (size_t)T + 64;                            // gsh
}

hipError_t launch_moe_experts(const MoeWeights& w, int T, int top_k, const float* x, const int* top_idx,
                              const float* top_w, const float* sgi, float* work, float* y, hipStream_t s) {
  const int slots = top_k + 1, dim = w.dim, I = w.intermed;
  float* xq = work;
  float* g = xq + (size_t)T * (dim / 16);
  float* u = g + (size_t)T * slots * I;
  float* h = u + (size_t)T * slots * I;
  float* hq = h + (size_t)T * slots * I;
  float* yk = hq + (size_t)T * slots * (I / 16);
  float* gsh = yk + (size_t)T * slots * dim;
  hipError_t e = launch_xsum(x, dim, T, xq, s);
  if (e != hipSuccess) return e;

  ProjJob J{};
  J.idx = top_idx; J.n_exp = w.n_exp; J.top_k = top_k; J.slots = slots;
  J.x = x; J.x_tok = dim; J.x_slot = 0; J.in_dim = dim; J.out_rows = I;
  J.y_tok = (long)slots * I; J.y_slot = I;
  // Routed slots and, when its kind matches, the shared slot in one launch;
  // otherwise the shared slot in a launch of its own kind.
  auto run = [&](const ProjJob& P0, const uint8_t* base, long stride, const uint8_t* shared, int kind,
                 int sh_kind, float* out, const float* xq_in, const float* x_sh, const float* xq_sh,
                 float* y_sh) -> hipError_t {
    ProjJob P = P0;
    P.base = base; P.stride = stride; P.shared = kind == sh_kind ? shared : nullptr; P.y = out;
    hipError_t r = proj(kind, P, T * slots, xq_in, s);
    if (r != hipSuccess || kind == sh_kind) return r;
    ProjJob Q = P;
    Q.base = nullptr; Q.idx = nullptr; Q.shared = shared; Q.top_k = 0; Q.slots = 1;
    Q.x = x_sh; Q.y = y_sh;
    return proj(sh_kind, Q, T, xq_sh, s);
  };
  e = run(J, w.gate, w.gate_stride, w.sh_gate, w.gate_kind, w.sh_gate_kind, g, xq, x, xq,
          g + (size_t)top_k * I);
  if (e == hipSuccess)
    e = run(J, w.up, w.up_stride, w.sh_up, w.up_kind, w.sh_up_kind, u, xq, x, xq, u + (size_t)top_k * I);
  if (e != hipSuccess) return e;
  const int n16 = T * slots * (I / 16);
  hipLaunchKernelGGL(moe_swiglu, dim3((n16 + 255) / 256), dim3(256), 0, s, g, u, h, hq, n16);

  ProjJob D = J;
  D.x = h; D.x_tok = (long)slots * I; D.x_slot = I; D.in_dim = I; D.out_rows = dim;
  D.y_tok = (long)slots * dim; D.y_slot = dim;
  e = run(D, w.down, w.down_stride, w.sh_down, w.down_kind, w.sh_down_kind, yk, hq, h + (size_t)top_k * I,
          hq + (size_t)top_k * (I / 16), yk + (size_t)top_k * dim);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(moe_shared_gate, dim3(T), dim3(64), 0, s, sgi, x, dim, gsh);
  hipLaunchKernelGGL(moe_combine, dim3((dim * T + 255) / 256), dim3(256), 0, s, yk, top_w, gsh, top_k, dim, T, y);
  return hipGetLastError();
}

// ---- router -------------------------------------------------------------------
//
// logits[t][e] = W[e] . x[t], stable softmax, greedy top-k and
// renormalisation (llm_moe.adb:136-197).  Workgroup (i, j) of 4 waves takes
// experts 4i..4i+3 (one per wave) for tokens ROUTE_TT j .. ROUTE_TT j + 3, so
// the router matrix is spread over many CUs and each row is read once per
// token group.  The logits are published with device-scope stores; the last
// workgroup of a token group to arrive (a per-group counter, reset by that
// workgroup) runs the selection, one wave per token.  The selection follows
// the CPU's rule exactly -- strict >, so the lowest index wins among equal
// probabilities -- on probabilities that may differ from the CPU's in the last
// bits (the exponential and the order of the exp-sum differ), as any GPU
// softmax does.
constexpr int ROUTE_MAX_EXP = 1024;
constexpr int ROUTE_TT = 4;

// Softmax + top-k of one token's logits lg[0..n_exp) by one wave; lane l holds
// experts l, l + 64, ..., PER of them (n_exp <= 64 PER).  Lane k < top_k
// writes slot k.  GLOBAL: lg is device memory another workgroup wrote (read
// with device-scope loads), else this workgroup's LDS.
template <int PER, bool GLOBAL = true>
__device__ __forceinline__ void route_select(const float* lg, int n_exp, int top_k, int lane, int* __restrict__ idx,
                                             float* __restrict__ tw) {
  float p[PER];
  float m = -INFINITY;
  // All loads issued before any use: indices clamped instead of branched on.
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    const float* q = lg + (e < n_exp ? e : n_exp - 1);
    p[i] = GLOBAL ? __hip_atomic_load(q, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : *q;
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (lane + 64 * i >= n_exp) p[i] = -INFINITY;
    m = fmaxf(m, p[i]);
  }
  m = wave_max(m);
  float part = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    p[i] = lane + 64 * i < n_exp ? expf(p[i] - m) : 0.f;
    part += p[i];
  }
  const float sum = wave_total(part);
#pragma unroll
  for (int i = 0; i < PER; ++i) p[i] = lane + 64 * i < n_exp ? p[i] / sum : -INFINITY;
  float mine_v = 0.f;
  int mine_i = 0;
  for (int k = 0; k < top_k; ++k) {
    // This lane's best (strict >: the lowest of its experts among equals,
    // never NaN), then the wave's.
    float bv = -INFINITY;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (p[i] > bv) { bv = p[i]; bi = lane + 64 * i; }
    wave_argmax(bv, bi);
    if (bi >= n_exp) bi = 0;  // only when every remaining value is NaN
#pragma unroll
    for (int i = 0; i < PER; ++i)
      if (bi == lane + 64 * i) p[i] = -INFINITY;
    if (lane == k) { mine_v = bv; mine_i = bi; }
  }
  // Renormalise by the sum of the selected probabilities, in ascending k.
  float sw = 0.f;
  for (int k = 0; k < top_k; ++k) sw = sw + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine_v), k));
  if (lane < top_k) {
    idx[lane] = mine_i;
    tw[lane] = mine_v / sw;
  }
}

// The same selection by the four waves of the last workgroup, for
// n_exp <= 64 PER <= 256: the greedy rounds above are a chain of dependent
// cross-lane steps (8 rounds took 3 us on MI355X), while this is a rank count
// whose steps are independent.  The nt <= 4 tokens of the workgroup share its
// waves: G = 4, 2 or 1 waves per token.  Every wave computes its token's
// probabilities exactly as route_select does (same loads, max, exp, sum and
// division), so they are bit-identical.  Expert e gets the key
// (bits(p_e) << 32) | ~e: the probabilities are >= 0, so comparing keys as
// unsigned integers orders by p and puts the lower index first among equal
// p -- the CPU's strict > rule -- and rank(e) = #{j : key_j > key_e} is the
// round in which the greedy loop picks e.  The G waves of a token count over
// 1 / G of the experts each; the experts of rank < top_k are the selection,
// renormalised in ascending rank as route_select does.  A token with a NaN
// probability takes route_select (its rule for NaN is not a rank).  All 256
// threads call this; the logits are another workgroup's output (device-scope
// loads).
constexpr int ROUTE_RANK_MAX = 256;
struct RouteLds {
  unsigned long long key[ROUTE_TT][ROUTE_RANK_MAX];
  unsigned short part[4][ROUTE_RANK_MAX];
  float selp[ROUTE_TT][64];
  int seli[ROUTE_TT][64];
  int has_nan[ROUTE_TT];
};

template <int PER, int G>
__device__ __forceinline__ void route_select_wg(RouteLds& L, const float* logits, int n_exp, int top_k, int t0,
                                                int nt, int* __restrict__ top_idx, float* __restrict__ top_w) {
  constexpr int NE = 64 * PER;
  static_assert(NE <= ROUTE_RANK_MAX, "rank selection up to 256 experts");
  auto& key = L.key;
  auto& part = L.part;
  auto& selp = L.selp;
  auto& seli = L.seli;
  auto& has_nan = L.has_nan;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tt = w / G, sw = w % G;
  const bool active = tt < nt;
  const float* lg = logits + (size_t)(t0 + (active ? tt : 0)) * n_exp;
  float p[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    p[i] = __hip_atomic_load(lg + (e < n_exp ? e : n_exp - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    if (lane + 64 * i >= n_exp) p[i] = -INFINITY;
    m = fmaxf(m, p[i]);
  }
  m = wave_max(m);
  float part_sum = 0.f;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    p[i] = lane + 64 * i < n_exp ? expf(p[i] - m) : 0.f;
    part_sum += p[i];
  }
  const float sum = wave_total(part_sum);
  bool nan = false;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int e = lane + 64 * i;
    p[i] = p[i] / sum;
    nan = nan || (e < n_exp && __builtin_isnan(p[i]));
    if (active && sw == 0) key[tt][e] = e < n_exp ? ((unsigned long long)__float_as_uint(p[i]) << 32) | (unsigned)~e : 0ull;
  }
  if (threadIdx.x < ROUTE_TT) has_nan[threadIdx.x] = 0;
  __syncthreads();
  if (active && sw == 0 && nan) has_nan[tt] = 1;
  __syncthreads();
  const bool rank = active && !has_nan[tt];
  // Wave (tt, sw) counts the keys j in [q sw, q sw + q) above each of its
  // lane's keys.
  if (rank) {
    constexpr int Q = NE / G;  // keys per wave: a compile-time count, so the LDS reads are issued ahead
    unsigned cnt[PER];
    unsigned long long mine[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      cnt[i] = 0;
      mine[i] = key[tt][lane + 64 * i];
    }
    const unsigned long long* kq = &key[tt][Q * sw];
#pragma unroll 16
    for (int j = 0; j < Q; ++j) {
      const unsigned long long kj = kq[j];
#pragma unroll
      for (int i = 0; i < PER; ++i) cnt[i] += kj > mine[i] ? 1u : 0u;
    }
#pragma unroll
    for (int i = 0; i < PER; ++i) part[w][lane + 64 * i] = (unsigned short)cnt[i];
  }
  __syncthreads();
  if (rank && sw == 0) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int e = lane + 64 * i;
      int r = 0;
      for (int g = 0; g < G; ++g) r += part[w + g][e];
      if (e < n_exp && r < top_k) {
        selp[tt][r] = p[i];
        seli[tt][r] = e;
      }
    }
  }
  __syncthreads();
  if (!active || sw != 0) return;
  int* idx = top_idx + (size_t)(t0 + tt) * top_k;
  float* tw = top_w + (size_t)(t0 + tt) * top_k;
  if (!rank) {
    route_select<PER>(lg, n_exp, top_k, lane, idx, tw);
    return;
  }
  // Renormalise by the sum of the selected probabilities, in ascending k
  // (lane k holds the k-th; top_k <= 64).
  const float pk = lane < top_k ? selp[tt][lane] : 0.f;
  const int ik = lane < top_k ? seli[tt][lane] : 0;
  float swt = 0.f;
  for (int k = 0; k < top_k; ++k) swt = swt + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pk), k));
  if (lane < top_k) {
    idx[lane] = ik;
    tw[lane] = pk / swt;
  }
}

// The router's input formed in the same launch (NORM): x = RMSNorm(H + r
// (+ r2)) with weights g, as a model's post-attention norm (LLM_RMSNorm.Forward,
// src/llm/llm_rmsnorm.adb:10-41, Epsilon 1e-6 of llm_rmsnorm.ads:19): every
// workgroup forms its tokens' x in LDS -- the sum of squares in the order of
// a one-workgroup norm of 256 threads, so x is the same -- and the last
// workgroup of a token group to arrive writes H + r back to H and x to nx
// (no workgroup of the launch reads those rows after it).
constexpr int ROUTE_NORM_MAX_DIM = 4096;
struct RouteNorm {
  const float* r;  // residual to add to H, or null
  const float* r2; // a second one, added after r, or null
  const float* g;  // norm weights [dim]
  float* H;        // [T][dim], read (and written back when r is given)
  float* nx;       // [T][dim] the normalised input
};

__device__ __forceinline__ void route_norm_rows(const RouteNorm& nm, float (&xs)[ROUTE_TT][ROUTE_NORM_MAX_DIM],
                                                float* part, int t0, int nt, int dim) {
  const int n4 = dim / 4;
  for (int tt = 0; tt < nt; ++tt) {
    const float4* h = reinterpret_cast<const float4*>(nm.H + (size_t)(t0 + tt) * dim);
    const float4* rr = nm.r ? reinterpret_cast<const float4*>(nm.r + (size_t)(t0 + tt) * dim) : nullptr;
    const float4* rr2 = nm.r2 ? reinterpret_cast<const float4*>(nm.r2 + (size_t)(t0 + tt) * dim) : nullptr;
    float4* xs4 = reinterpret_cast<float4*>(xs[tt]);
    float s = 0.f;
    for (int i = threadIdx.x; i < n4; i += 256) {
      float4 v = h[i];
      if (rr) {
        const float4 a = rr[i];
        v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
      }
      if (rr2) {
        const float4 a = rr2[i];
        v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
      }
      xs4[i] = v;
      s += v.x * v.x;
      s += v.y * v.y;
      s += v.z * v.z;
      s += v.w * v.w;
    }
    s = wave_total(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    float tot = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) tot += part[k];
    const float rms = sqrtf(tot / (float)dim + 1e-6f);
    const float4* g4 = reinterpret_cast<const float4*>(nm.g);
    for (int i = threadIdx.x; i < n4; i += 256) {
      const float4 v = xs4[i], g = g4[i];
      xs4[i] = make_float4((v.x / rms) * g.x, (v.y / rms) * g.y, (v.z / rms) * g.z, (v.w / rms) * g.w);
    }
    __syncthreads();
  }
}

template <bool NORM>
__global__ __launch_bounds__(256) void moe_route(const float* __restrict__ W, int n_exp, int dim, int T,
                                                 const float* __restrict__ x, int top_k, float* __restrict__ logits,
                                                 int* __restrict__ top_idx, float* __restrict__ top_w,
                                                 unsigned* __restrict__ count, RouteNorm nm) {
  __shared__ int last;
  __shared__ RouteLds sel;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = blockIdx.x * 4 + w;
  const int t0 = blockIdx.y * ROUTE_TT;
  const int nt = T - t0 < ROUTE_TT ? T - t0 : ROUTE_TT;
  const int n4 = dim / 4;
  __shared__ float normpart[4];
  __shared__ float xs[NORM ? ROUTE_TT : 1][NORM ? ROUTE_NORM_MAX_DIM : 4];
  if constexpr (NORM) route_norm_rows(nm, xs, normpart, t0, nt, dim);
  if (e < n_exp) {
    // Rows are read in blocks of RB float4 per lane, all loads of a block in
    // flight together: indices are clamped (and the products of the padding
    // zeroed) instead of branched on, and absent tokens re-read token t0.
    constexpr int RB = 8;
    const float4* w4 = reinterpret_cast<const float4*>(W + (size_t)e * dim);
    const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)t0 * dim);
    float acc[ROUTE_TT] = {0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < n4; b += 64 * RB) {
      float4 q[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const int i = b + 64 * r + lane;
        const float4 v = w4[i < n4 ? i : n4 - 1];
        q[r] = i < n4 ? v : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int tt = 0; tt < ROUTE_TT; ++tt) {
        const float4* xt = NORM ? reinterpret_cast<const float4*>(xs[tt < nt ? tt : 0]) : x4 + (size_t)(tt < nt ? tt : 0) * n4;
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const int i = b + 64 * r + lane;
          const float4 v = xt[i < n4 ? i : n4 - 1];
          acc[tt] = __builtin_fmaf(q[r].x, v.x, acc[tt]);
          acc[tt] = __builtin_fmaf(q[r].y, v.y, acc[tt]);
          acc[tt] = __builtin_fmaf(q[r].z, v.z, acc[tt]);
          acc[tt] = __builtin_fmaf(q[r].w, v.w, acc[tt]);
        }
      }
    }
#pragma unroll
    for (int tt = 0; tt < ROUTE_TT; ++tt) {
      const float s = wave_total(acc[tt]);
      if (lane == 0 && tt < nt)
        __hip_atomic_store(&logits[(size_t)(t0 + tt) * n_exp + e], s, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  // Last-arrival handoff of the logits, by the rule stated at mv_epilogue
  // (kq_packed.h): sc1 atomic stores, retired before the arrival is counted;
  // the last workgroup reads them with sc1 atomic loads after its count.
  __builtin_amdgcn_s_waitcnt(0);  // the logits stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned* c = count + (size_t)blockIdx.y * COUNTER_STRIDE;
    const bool l = __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    if (l) __hip_atomic_store(c, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next launch
    last = l;
  }
  __syncthreads();
  if (!last) return;
  if constexpr (NORM) {
    // This token group's rows: H + r back to H, x to nx.
    for (int tt = 0; tt < nt; ++tt) {
      float4* h = reinterpret_cast<float4*>(nm.H + (size_t)(t0 + tt) * dim);
      const float4* rr = nm.r ? reinterpret_cast<const float4*>(nm.r + (size_t)(t0 + tt) * dim) : nullptr;
      const float4* rr2 = nm.r2 ? reinterpret_cast<const float4*>(nm.r2 + (size_t)(t0 + tt) * dim) : nullptr;
      float4* y = reinterpret_cast<float4*>(nm.nx + (size_t)(t0 + tt) * dim);
      const float4* xs4 = reinterpret_cast<const float4*>(xs[tt]);
      for (int i = threadIdx.x; i < n4; i += 256) {
        if (rr || rr2) {
          float4 v = h[i];
          if (rr) {
            const float4 a = rr[i];
            v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
          }
          if (rr2) {
            const float4 a = rr2[i];
            v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
          }
          h[i] = v;
        }
        y[i] = xs4[i];
      }
    }
  }
  if (n_exp <= 256) {
    // G waves per token: all four for one token, two each for two, one each for more.
#define KQ_SEL(PER)                                                                                 \
  {                                                                                                 \
    if (nt == 1) route_select_wg<PER, 4>(sel, logits, n_exp, top_k, t0, nt, top_idx, top_w);        \
    else if (nt == 2) route_select_wg<PER, 2>(sel, logits, n_exp, top_k, t0, nt, top_idx, top_w);   \
    else route_select_wg<PER, 1>(sel, logits, n_exp, top_k, t0, nt, top_idx, top_w);                \
    return;                                                                                         \
  }
    if (n_exp <= 128) KQ_SEL(2)
    KQ_SEL(4)
#undef KQ_SEL
  }
  if (w >= nt) return;
  const int t = t0 + w;
  const float* lg = logits + (size_t)t * n_exp;
  int* ti = top_idx + (size_t)t * top_k;
  float* tw = top_w + (size_t)t * top_k;
  if (n_exp <= 64) route_select<1>(lg, n_exp, top_k, lane, ti, tw);
  else if (n_exp <= 128) route_select<2>(lg, n_exp, top_k, lane, ti, tw);
  else if (n_exp <= 256) route_select<4>(lg, n_exp, top_k, lane, ti, tw);
  else route_select<ROUTE_MAX_EXP / 64>(lg, n_exp, top_k, lane, ti, tw);
}

// Many tokens (prefill): a workgroup of RT_WAVES waves takes RT_TOK tokens and
// every expert, so each token's activations are read once per workgroup (the
// token-group launch above reads them once per four experts) and the selection
// needs no hand-off between workgroups.  Each lane keeps its slices of the
// tokens' activations in registers (dim <= RT_MAX_DIM); wave w takes experts
// w, w + RT_WAVES, ..., reading each router row from L2; the logits meet in
// LDS and wave t selects token t's experts.
constexpr int RT_TOK = 4;
constexpr int RT_WAVES = 8;
constexpr int RT_MAX_DIM = 2048;

__global__ __launch_bounds__(64 * RT_WAVES) void moe_route_tokens(const float* __restrict__ W, int n_exp, int dim,
                                                                  int T, const float* __restrict__ x, int top_k,
                                                                  float* __restrict__ logits,
                                                                  int* __restrict__ top_idx,
                                                                  float* __restrict__ top_w) {
  constexpr int R = RT_MAX_DIM / 256;  // float4 per lane per token
  __shared__ float lg[RT_TOK][ROUTE_MAX_EXP];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int t0 = blockIdx.x * RT_TOK, nt = T - t0 < RT_TOK ? T - t0 : RT_TOK;
  const int n4 = dim / 4;
  float4 xv[RT_TOK][R];
#pragma unroll
  for (int tt = 0; tt < RT_TOK; ++tt) {
    const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)(t0 + (tt < nt ? tt : 0)) * dim);
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = lane + 64 * r;
      xv[tt][r] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  for (int e = w; e < n_exp; e += RT_WAVES) {
    const float4* w4 = reinterpret_cast<const float4*>(W + (size_t)e * dim);
    float4 q[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int i = lane + 64 * r;
      q[r] = i < n4 ? w4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float acc[RT_TOK];
#pragma unroll
    for (int tt = 0; tt < RT_TOK; ++tt) {
      float s = 0.f;
#pragma unroll
      for (int r = 0; r < R; ++r) {
        s = __builtin_fmaf(q[r].x, xv[tt][r].x, s);
        s = __builtin_fmaf(q[r].y, xv[tt][r].y, s);
        s = __builtin_fmaf(q[r].z, xv[tt][r].z, s);
        s = __builtin_fmaf(q[r].w, xv[tt][r].w, s);
      }
      acc[tt] = s;
    }
#pragma unroll
    for (int tt = 0; tt < RT_TOK; ++tt) {
      const float s = wave_total(acc[tt]);
      if (lane == 0) lg[tt][e] = s;
    }
  }
  __syncthreads();
  for (int i = threadIdx.x; i < nt * n_exp; i += 64 * RT_WAVES)
    logits[(size_t)(t0 + i / n_exp) * n_exp + i % n_exp] = lg[i / n_exp][i % n_exp];
  if (w >= nt) return;
  const int t = t0 + w;
  int* ti = top_idx + (size_t)t * top_k;
  float* tw = top_w + (size_t)t * top_k;
  if (n_exp <= 64) route_select<1, false>(lg[w], n_exp, top_k, lane, ti, tw);
  else if (n_exp <= 128) route_select<2, false>(lg[w], n_exp, top_k, lane, ti, tw);
  else if (n_exp <= 256) route_select<4, false>(lg[w], n_exp, top_k, lane, ti, tw);
  else route_select<ROUTE_MAX_EXP / 64, false>(lg[w], n_exp, top_k, lane, ti, tw);
}

// From this many tokens the token-group router takes over.  Its workgroups
// each take about 26 us whatever T (a wave's 16 experts one after another),
// against 14.9, 20.8, 30.6 and 52 us for T = 128, 256, 512 and 1024 on the
// expert-split launch.
constexpr int ROUTE_TOKENS_MIN_T = 384;

static bool route_tokens_takes(int T, int dim) { return T >= ROUTE_TOKENS_MIN_T && dim <= RT_MAX_DIM; }

int moe_route_groups(int T) { return (T + ROUTE_TT - 1) / ROUTE_TT; }

hipError_t launch_moe_route(const float* router_w, int n_exp, int dim, int T, int top_k, const float* x,
                            float* logits, int* top_idx, float* top_w, unsigned* count, hipStream_t s) {
  if (n_exp > ROUTE_MAX_EXP || top_k > MOE_MAX_TOPK || top_k > n_exp || top_k > 64 || dim % 4 || !logits || !count)
    return hipErrorInvalidValue;
  if (route_tokens_takes(T, dim)) {
    hipLaunchKernelGGL(moe_route_tokens, dim3((T + RT_TOK - 1) / RT_TOK), dim3(64 * RT_WAVES), 0, s, router_w, n_exp,
                       dim, T, x, top_k, logits, top_idx, top_w);
    return hipGetLastError();
  }
  const dim3 grid((n_exp + 3) / 4, (T + ROUTE_TT - 1) / ROUTE_TT);
  hipLaunchKernelGGL(moe_route<false>, grid, dim3(256), 0, s, router_w, n_exp, dim, T, x, top_k, logits, top_idx,
                     top_w, count, RouteNorm{});
  return hipGetLastError();
}

// Up to 2 tokens: every workgroup normalises its group's rows, so the
// prologue grows with the tokens of a group (measured at 8 tokens: 16.3 us
// against 10.6 us for the router and 4.7 us for a norm launch).
constexpr int ROUTE_NORM_MAX_T = 2;
bool moe_route_norm_takes(int n_exp, int dim, int T, int top_k) {
  return n_exp > 0 && n_exp <= ROUTE_MAX_EXP && top_k > 0 && top_k <= MOE_MAX_TOPK && top_k <= n_exp && top_k <= 64 &&
         dim > 0 && dim % 4 == 0 && dim <= ROUTE_NORM_MAX_DIM && T > 0 && T <= ROUTE_NORM_MAX_T &&
         !route_tokens_takes(T, dim);
}

hipError_t launch_moe_route_norm(const float* router_w, int n_exp, int dim, int T, int top_k, float* H, const float* r,
                                 const float* r2, const float* g, float* nx, float* logits, int* top_idx, float* top_w,
                                 unsigned* count, hipStream_t s) {
  if (!moe_route_norm_takes(n_exp, dim, T, top_k) || !H || !g || !nx || !logits || !count) return hipErrorInvalidValue;
  const dim3 grid((n_exp + 3) / 4, (T + ROUTE_TT - 1) / ROUTE_TT);
  hipLaunchKernelGGL(moe_route<true>, grid, dim3(256), 0, s, router_w, n_exp, dim, T, (const float*)nullptr, top_k,
                     logits, top_idx, top_w, count, RouteNorm{r, r2, g, H, nx});
  return hipGetLastError();
}

}  // namespace kq
