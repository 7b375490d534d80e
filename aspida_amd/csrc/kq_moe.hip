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
// One workgroup (4 waves) per token: logits[t][e] = W[e] . x[t] (wave w takes
// experts w, w + 4, ...; each a coalesced dot over dim), stable softmax,
// greedy top-k and renormalisation (llm_moe.adb:136-197).  The exp-sum and
// the renormalising sum run sequentially in ascending order, as on the CPU,
// so equal probabilities arise exactly where the CPU's do; the arg-max takes
// the lowest index among equal values.
constexpr int ROUTE_MAX_EXP = 1024;
constexpr int ROUTE_MAX_DIM4 = 64 * 16;  // dim / 4 cached in registers: dim <= 4096

// CACHE_X: dim <= 4096, x held in registers for all experts; otherwise x is
// re-read (from cache) per expert.  Both add in the same order.
template <bool CACHE_X>
__global__ __launch_bounds__(256) void moe_route(const float* __restrict__ W, int n_exp, int dim,
                                                 const float* __restrict__ x, int top_k,
                                                 float* __restrict__ logits, int* __restrict__ top_idx,
                                                 float* __restrict__ top_w) {
  __shared__ float p[ROUTE_MAX_EXP];
  __shared__ float bestv[MOE_MAX_TOPK];
  __shared__ float sum_s;
  const int t = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int n4 = dim / 4;
  const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)t * dim);
  float4 xv[CACHE_X ? 16 : 1];
  if (CACHE_X) {
#pragma unroll
    for (int i = 0; i < 16; ++i) xv[i] = lane + 64 * i < n4 ? x4[lane + 64 * i] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  for (int e = w; e < n_exp; e += 4) {
    const float4* w4 = reinterpret_cast<const float4*>(W + (size_t)e * dim);
    float a = 0.f;
    if (CACHE_X) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (lane + 64 * i < n4) {
          const float4 q = w4[lane + 64 * i];
          a = __builtin_fmaf(q.x, xv[i].x, a);
          a = __builtin_fmaf(q.y, xv[i].y, a);
          a = __builtin_fmaf(q.z, xv[i].z, a);
          a = __builtin_fmaf(q.w, xv[i].w, a);
        }
    } else {
      for (int i = lane; i < n4; i += 64) {
        const float4 q = w4[i], v = x4[i];
        a = __builtin_fmaf(q.x, v.x, a);
        a = __builtin_fmaf(q.y, v.y, a);
        a = __builtin_fmaf(q.z, v.z, a);
        a = __builtin_fmaf(q.w, v.w, a);
      }
    }
    a = wave_sum(a);
    if (lane == 0) {
      p[e] = a;
      if (logits) logits[(size_t)t * n_exp + e] = a;
    }
  }
  __syncthreads();
  // Softmax and top-k on wave 0 (lanes hold e = lane + 64 i); every wave
  // passes every barrier.
  if (w == 0) {
    float m = -INFINITY;
    for (int e = lane; e < n_exp; e += 64) m = fmaxf(m, p[e]);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    for (int e = lane; e < n_exp; e += 64) p[e] = expf(p[e] - m);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float sum = 0.f;
    for (int e = 0; e < n_exp; ++e) sum = sum + p[e];
    sum_s = sum;
  }
  __syncthreads();
  if (w == 0) {
    const float sum = sum_s;
    for (int e = lane; e < n_exp; e += 64) p[e] = p[e] / sum;
  }
  __syncthreads();
  for (int k = 0; k < top_k; ++k) {
    if (w == 0) {
      float bv = -INFINITY;
      int bi = 0x7fffffff;
      for (int e = lane; e < n_exp; e += 64)
        if (p[e] > bv) { bv = p[e]; bi = e; }
#pragma unroll
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
      }
      if (bi >= n_exp) bi = 0;   // only when every remaining value is NaN
      if (lane == 0) {
        top_idx[t * top_k + k] = bi;
        bestv[k] = bv;
        p[bi] = -INFINITY;
      }
    }
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    float sw = 0.f;
    for (int k = 0; k < top_k; ++k) sw = sw + bestv[k];
    for (int k = 0; k < top_k; ++k) top_w[t * top_k + k] = bestv[k] / sw;
  }
}

hipError_t launch_moe_route(const float* router_w, int n_exp, int dim, int T, int top_k, const float* x,
                            float* logits, int* top_idx, float* top_w, hipStream_t s) {
  if (n_exp > ROUTE_MAX_EXP || top_k > MOE_MAX_TOPK || top_k > n_exp || dim % 4) return hipErrorInvalidValue;
  if (dim / 4 <= ROUTE_MAX_DIM4)
    hipLaunchKernelGGL(moe_route<true>, dim3(T), dim3(256), 0, s, router_w, n_exp, dim, x, top_k, logits, top_idx,
                       top_w);
  else
    hipLaunchKernelGGL(moe_route<false>, dim3(T), dim3(256), 0, s, router_w, n_exp, dim, x, top_k, logits, top_idx,
                       top_w);
  return hipGetLastError();
}

}  // namespace kq
