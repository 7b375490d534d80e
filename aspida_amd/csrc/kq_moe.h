// kq_moe.h -- MoE expert FFN on the GPU (host-side launchers, namespace kq).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kq {

constexpr int MOE_MAX_TOPK = 32;

// Device-resident MoE layer weights.  Routed experts are [n_exp][rows][cols]
// with `*_stride` bytes per expert (gate/up: intermed x dim, down: dim x
// intermed); the shared expert is one [rows][cols] matrix per projection.
struct MoeWeights {
  const uint8_t *gate = nullptr, *up = nullptr, *down = nullptr;
  const uint8_t *sh_gate = nullptr, *sh_up = nullptr, *sh_down = nullptr;
  long gate_stride = 0, up_stride = 0, down_stride = 0;
  int gate_kind = 0, up_kind = 0, down_kind = 1;
  int sh_gate_kind = 0, sh_up_kind = 0, sh_down_kind = 1;
  int dim = 0, intermed = 0, n_exp = 0;
};

// Floats at the front of the work space reserved for staging x | top_w |
// top_idx (host ABI), rounded up to 16 bytes.
inline size_t moe_staging_floats(int dim, int T, int top_k) {
  return ((size_t)T * dim + 2 * (size_t)T * top_k + 3) & ~(size_t)3;
}

// Floats of work space (staging included) launch_moe_experts needs for T tokens.
size_t moe_scratch_floats(const MoeWeights& w, int T, int top_k);

// y[t] = sum_k top_w[t][k] * Down_e(silu(Gate_e x_t) * Up_e x_t)  (e = top_idx[t][k],
// ascending k) + g_t * SharedDown(silu(SharedGate x_t) * SharedUp x_t), where
// g_t = sigmoid(shared_gate_inp . x_t) when shared_gate_inp is non-null, else 1
// (LLM_MoE.Forward steps 4-5, src/llm/llm_moe.adb:249-299).  x: [T][dim],
// top_idx/top_w: [T][top_k] (0-based experts), all device pointers.
hipError_t launch_moe_experts(const MoeWeights& w, int T, int top_k, const float* x, const int* top_idx,
                              const float* top_w, const float* shared_gate_inp, float* work, float* y,
                              hipStream_t s);

// ---- grouped path over packed expert weights (kq_moe_grouped.hip) ----

// Routed jobs (token, slot) per launch (T * top_k bound; also T <= it).
constexpr int MOE_MAX_JOBS = 1024;
// Routed experts the grouped path schedules (LDS tables per workgroup).
constexpr int MOE_MAX_EXP = 1024;
// Bitmask words of the schedule's slot ranks ((n_exp + 1) * ceil(T top_k /
// 32) of them; more than this and it counts ranks by scanning instead).
constexpr int MOE_SCHED_MASK_WORDS = 2048;
// Jobs per chunk of the matrix-core grouped launches (kq_moe_mfma.hip).
constexpr int MOE_MFMA_JPW = 2;

// Chunks of up to jpw jobs a schedule can produce: T (top_k + 1) jobs over
// at most `routed` routed experts plus the shared one.
inline long moe_max_chunks(int T, int top_k, int routed, int jpw) {
  return ((long)T * (top_k + 1) + jpw - 1) / jpw + routed + 1;
}

// Packed expert tensors: expert e's matrix at base + e * stride (stride =
// packed bytes of one [rows][cols] matrix); the shared expert's matrices
// separately, same kinds.  Work arrays are device memory the caller owns
// (moe_grouped_work_bytes).
struct MoeGroupedArgs {
  const uint8_t *gate, *up, *down, *sh_gate, *sh_up, *sh_down;
  size_t gu_stride, d_stride;
  const int* idx;        // [T][top_k] expert ids (0-based)
  const float* top_w;    // [T][top_k]
  const float* x;        // [T][dim], 16-byte aligned rows
  const float* sgi;      // shared gate input [dim] or null
  float *h, *yk, *gsh, *y;
  unsigned* count;       // [T][blocks_dim] arrival counters, one per 256 bytes
  int* sched;            // the schedule the gate/up launch publishes: joff[n_exp + 2], jobs[T (top_k + 1)]
  int4* units;           // matrix-core launches: [0].x = chunk count, [1 + c] = chunk c {expert, job, job | -1}
  int T, top_k, n_exp, dim, I;
  int tiles_dim;         // 64-row tiles of dim (vector-ALU down projection)
  int blocks_dim;        // 16-row blocks of dim (matrix-core down projection)
  // Optional (a model chain's next norm in the combine launch): when norm_h is
  // set and the launch path combines in a launch of its own (matrix cores,
  // T >= 2), that launch also adds y[t] into norm_h[t] and writes
  // norm_nx[t] = RMSNorm(norm_h[t]) with weights norm_w, and sets the host
  // flag *norm_done.  Other paths leave the three alone.
  float* norm_h = nullptr;
  const float* norm_w = nullptr;
  float* norm_nx = nullptr;
  bool* norm_done = nullptr;
};

size_t moe_grouped_work_bytes(int T, int dim, int I, int top_k);
// Points h, yk, gsh, count, sched, units into `work` (moe_grouped_work_bytes of a.T, a.dim,
// a.I, a.top_k, 256-byte aligned) and sets tiles_dim, blocks_dim.  The counters need no
// clearing: the gate/up launch zeroes them.
void moe_grouped_bind(MoeGroupedArgs& a, void* work);
bool moe_grouped_supported(int dim, int I, int T, int top_k);
bool moe_grouped_experts_ok(int n_exp);
// Two launches: gate/up + SwiGLU, then down + combine (gate and up of one
// kind, down of another; the shared expert's kinds equal the routed ones).
// Q4_K and Q6_K projections run on the matrix cores (16-row blocks), the
// other kinds -- and every kind under aspida_kq_set_mv_engine(1) -- on the
// vector ALUs (64-row tiles).
hipError_t launch_moe_grouped(const MoeGroupedArgs& a, int gu_kind, int down_kind, hipStream_t s);
// aspida_moe_experts_packed_dev with the model chain's next norm taken into
// the combine launch where the path has one (MoeGroupedArgs::norm_h): then
// y[t] is also added into norm_h[t], norm_nx[t] = RMSNorm(norm_h[t]) with
// weights norm_w, and *norm_done is set; otherwise *norm_done is false and
// norm_h, norm_nx are untouched.  Null norm pointers: the plain entry point.
int moe_experts_packed_norm(const float* x, int T, int dim, int top_k, int intermed, int n_exp, const int* top_idx,
                            const float* top_w, const void* gate_p, const void* up_p, int gu_kind,
                            const void* down_p, int down_kind, const void* shg_p, const void* shu_p,
                            const void* shd_p, const float* shared_gate_inp, void* work, float* y, void* stream,
                            float* norm_h, const float* norm_w, float* norm_nx, bool* norm_done);
// The grouped launches on the matrix cores (kq_moe_mfma.hip): Q4_K and Q6_K
// projections, any T; hipErrorNotSupported for other kinds.
bool moe_mfma_kind(int kind);
hipError_t launch_moe_grouped_mfma(const MoeGroupedArgs& a, int gu_kind, int down_kind, hipStream_t s);

// ---- prefill: many tokens per launch (kq_moe_prefill.hip) ----

// Tokens from which Q4_K gate/up with Q6_K down run the grouped GEMM of
// kq_moe_prefill.hip, and the most tokens one of its launch sequences takes.
constexpr int MOE_PREFILL_MIN_TOKENS = 96;  // measured: 64 tokens 256 us here vs 239 us grouped
constexpr int MOE_PREFILL_MAX_TOKENS = 1024;
bool moe_prefill_takes(int T, int gu_kind, int down_kind, int dim, int I, int top_k, int n_exp);
// Work bytes of one launch sequence of T <= MOE_PREFILL_MAX_TOKENS tokens
// (any n_exp up to MOE_MAX_EXP).
size_t moe_prefill_work_bytes(int T, int dim, int I, int top_k);
// a: the weights, idx, top_w, x, sgi, y, T, top_k, n_exp, dim, I of
// MoeGroupedArgs (its work pointers are not used); work 256-byte aligned.
hipError_t launch_moe_prefill(const MoeGroupedArgs& a, void* work, hipStream_t s);

// Router: logits[t] = router_w[n_exp][dim] . x[t] (f32), stable softmax,
// greedy top-k (strict >, lowest index wins ties), renormalised weights
// (llm_moe.adb:136-197).  Writes top_idx/top_w [T][top_k].
// count: moe_route_groups(T) zeroed counters, 64 unsigned (256 bytes) apart;
// every launch leaves them zero again.  Launches sharing counters must be
// ordered (one stream).  logits is required (the selection reads it back).
hipError_t launch_moe_route(const float* router_w, int n_exp, int dim, int T, int top_k, const float* x,
                            float* logits, int* top_idx, float* top_w, unsigned* count, hipStream_t s);
int moe_route_groups(int T);
// The router with its input normalised in the same launch: x = RMSNorm(H +
// r + r2) with weights g (r, r2 may be null; added in that order); the sum
// is written back to H and x to nx.  Arguments otherwise as
// launch_moe_route; dim <= 4096 and up to 2 tokens (moe_route_norm_takes).
bool moe_route_norm_takes(int n_exp, int dim, int T, int top_k);
hipError_t launch_moe_route_norm(const float* router_w, int n_exp, int dim, int T, int top_k, float* H, const float* r,
                                 const float* r2, const float* g, float* nx, float* logits, int* top_idx, float* top_w,
                                 unsigned* count, hipStream_t s);

}  // namespace kq
