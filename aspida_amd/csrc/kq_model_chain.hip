// kq_model_chain.hip -- the resident model chain: one decode step of a whole
// MoE model (embedding row; per layer a mixer and the routed + shared expert
// FFN with its router; final norm and output head) run on device-resident
// weights as one fixed sequence of launches, captured once per lane count
// into a HIP graph and replayed for every token after that.
//
// The entry points take the C shapes of the reference's chain
// (gpu/gpu_matvec.cu:2063-2066 reset, 2143-2199 moe, 2201-2213 model and
// ready, 2328-2340 begin / end, 2356-2400 forward, 2783-2961 forward_batch).
// The reference registers each layer's mixer -- gated attention or a
// delta-net recurrence -- through chain_fattn / chain_dnet; those mixers are
// not part of this library, and a layer's mixer here is one matvec of any
// supported kind (aspida_kq_chain_layer), the stand-in with which the chain's
// MoE steps run behind the reference ABI.  Without chain_fattn / chain_dnet the
// Ada host's Chain_Available (src/llm/llm_qwen_gpu.adb:554-560) stays false
// and it keeps its per-layer paths.
//
// Per layer, as LLM_Qwen_Blk.Step (src/llm/llm_qwen_blk.adb:125-170):
//   nx = RMSNorm(H, attn_norm); H += Mix nx;
//   nr = RMSNorm(H, post_norm); H += MoE(nr)        (LLM_MoE.Forward)
// and logits = LM RMSNorm(H, final_norm) (src/llm/llm_qwen.adb:1199-1203).
// Every residual add is fused into the norm launch that follows it.  The
// router is f32: a quantised router is dequantised once at registration
// (bit-exact decoders), so its logits are the f32 dot products QMatVec forms
// from the decoded values, up to summation order.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <set>
#include <vector>

#include "../../include/aspidagpu.h"
#include "kq_common.h"
#include "kq_moe.h"

namespace kq {
void abi_report(int code, const char* what);  // aspidagpu.hip: the calling thread's aspida_gpu_last_error
// aspidagpu.hip: the router with the norm before it in one launch, and the
// one-lane mixer with the norm before it (0, -ENOTSUP or an error).
int route_norm_dev(const float* router_w, int n_exp, int dim, int T, int top_k, float* H, const float* r,
                   const float* r2, const float* g, float* nx, float* logits, int* top_idx, float* top_w,
                   void* stream);
int matvec_norm_dev(int kind, const void* P, int in_dim, int out_dim, const float* H, const float* r, const float* g,
                    float* y, void* stream);
bool moe_route_norm_takes(int n_exp, int dim, int T, int top_k);  // kq_moe.hip
}  // namespace kq

namespace {

using kq::MOE_MAX_JOBS;
using kq::MOE_MAX_TOPK;

constexpr int CHAIN_THREADS = 256;
constexpr int CHAIN_MAX_LANES = 64;

// ---- kernels ------------------------------------------------------------------

// H[b] = E[rows[b]]: the embedding rows of the B lanes (rows checked on the
// host before they are copied to the device).
__global__ __launch_bounds__(CHAIN_THREADS) void chain_embed(const float* __restrict__ E, const int* __restrict__ rows,
                                                             int dim, float* __restrict__ H) {
  const int b = blockIdx.y, i = blockIdx.x * CHAIN_THREADS + threadIdx.x, n4 = dim / 4;
  if (i >= n4) return;
  const float4* e = reinterpret_cast<const float4*>(E + (size_t)rows[b] * dim);
  reinterpret_cast<float4*>(H + (size_t)b * dim)[i] = e[i];
}

// H[b] += r[b] (when r is non-null), then nx[b] = (H[b] / rms) * w with
// rms = sqrt(mean(H[b]^2) + 1e-6) (LLM_RMSNorm.Forward,
// src/llm/llm_rmsnorm.adb:10-41, Epsilon of llm_rmsnorm.ads:19).  One
// workgroup per lane; the sum of squares in a fixed order.
__global__ __launch_bounds__(CHAIN_THREADS) void chain_add_norm(float* __restrict__ H, const float* __restrict__ r,
                                                                const float* __restrict__ w, float* __restrict__ nx,
                                                                int dim) {
  __shared__ float part[CHAIN_THREADS / 64];
  const int n4 = dim / 4;
  float4* h = reinterpret_cast<float4*>(H + (size_t)blockIdx.x * dim);
  const float4* rr = r ? reinterpret_cast<const float4*>(r + (size_t)blockIdx.x * dim) : nullptr;
  float s = 0.f;
  for (int i = threadIdx.x; i < n4; i += CHAIN_THREADS) {
    float4 v = h[i];
    if (rr) {
      const float4 a = rr[i];
      v = make_float4(v.x + a.x, v.y + a.y, v.z + a.z, v.w + a.w);
      h[i] = v;
    }
    s += v.x * v.x;
    s += v.y * v.y;
    s += v.z * v.z;
    s += v.w * v.w;
  }
  s = kq::wave_total(s);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < CHAIN_THREADS / 64; ++k) tot += part[k];
  const float rms = sqrtf(tot / (float)dim + 1e-6f);
  const float4* w4 = reinterpret_cast<const float4*>(w);
  float4* y = reinterpret_cast<float4*>(nx + (size_t)blockIdx.x * dim);
  for (int i = threadIdx.x; i < n4; i += CHAIN_THREADS) {
    const float4 v = h[i], g = w4[i];
    y[i] = make_float4((v.x / rms) * g.x, (v.y / rms) * g.y, (v.z / rms) * g.z, (v.w / rms) * g.w);
  }
}

// ---- registered model --------------------------------------------------------

// A matrix of the chain: dense f32 [out][in] (kind -1) or the packed layout of
// a quantised kind.
struct Mat {
  void* d = nullptr;
  int kind = -1, in = 0, out = 0;
};

struct Layer {
  int dim = 0;
  float *attn_norm = nullptr, *post_norm = nullptr;
  bool has_mix = false, has_moe = false;
  Mat mix;
  // MoE block.
  float* router = nullptr;  // f32 [n_exp][dim]
  float* sgi = nullptr;     // shared-expert gate input [dim] or null
  bool grouped = false;     // packed experts (aspida_moe_experts_packed_dev)
  const void *g = nullptr, *u = nullptr, *dn = nullptr, *sg = nullptr, *su = nullptr, *sd = nullptr;
  long g_stride = 0, u_stride = 0, d_stride = 0;
  int gk = 0, uk = 0, dk = 0, sgk = 0, suk = 0, sdk = 0;
  int n_exp = 0, top_k = 0, intermed = 0;
};

struct Chain {
  std::mutex mu;
  std::vector<Layer> layers;
  std::vector<void*> mem;  // every device allocation of the registered model
  bool broken = false;     // a registration failed: not ready until reset
  bool model = false;
  float *embed = nullptr, *fnorm = nullptr;
  long embed_rows = 0;
  Mat lm;
  int dim = 0, vocab = 0;
  // Run state: buffers for CHAIN_MAX_LANES lanes, the stream, graphs.
  hipStream_t st = nullptr;
  bool bufs = false;
  std::vector<void*> run_mem;  // the buffers, sized for the registered layers
  float *H = nullptr, *nx = nullptr, *ao = nullptr, *y = nullptr, *rl = nullptr, *tw = nullptr, *dlog = nullptr;
  int *idx = nullptr, *rows = nullptr;
  void* work = nullptr;
  float* hlog = nullptr;  // pinned: logits of every lane
  int* hrows = nullptr;   // pinned: the lanes' rows
  std::map<int, hipGraphExec_t> graphs;  // per lane count
  std::set<int> warmed;                  // lane counts run eagerly at least once
  int use_graphs = -1;                   // -1: from ASPIDA_NO_GRAPH at the first forward
};

Chain& chain() {
  static Chain* c = new Chain();  // never destroyed: the process may still call in at exit
  return *c;
}

long block_bytes(int kind) {
  switch (kind) {
    case 0: return 144;
    case 1: return 210;
    case 2: return 176;
    case 3: return 110;
    case 4: return 84;
    case 5: return 272;
    default: return 0;
  }
}

// Bytes of a row-major [out][in / 256 blocks] weight (kind >= 0) or a dense
// f32 [out][in] one (kind -1); 0 for an unknown kind.
long mat_bytes(int kind, int in, int out) {
  if (kind == -1) return (long)in * out * 4;
  return (long)out * (in / 256) * block_bytes(kind);
}

int fail(int code, const char* what) {
  kq::abi_report(code, what);
  return code;
}

int hip(hipError_t e, const char* what) { return e == hipSuccess ? 0 : fail((int)e, what); }

// A device entry point's status: its errors are recorded as the chain's.
int ep(int rc, const char* what) { return rc ? fail(rc, what) : 0; }

void destroy_graphs(Chain& c) {
  for (auto& kv : c.graphs) (void)hipGraphExecDestroy(kv.second);
  c.graphs.clear();
}

int alloc(Chain& c, void** p, size_t bytes, const char* what, bool run = false) {
  *p = nullptr;
  if (int rc = hip(hipMalloc(p, bytes), what)) return rc;
  (run ? c.run_mem : c.mem).push_back(*p);
  return 0;
}

// Drops the run buffers and the graphs that point into them: every
// registration change does (the buffers are sized for the layers).
void drop_run_state(Chain& c) {
  destroy_graphs(c);
  if (c.st) (void)hipStreamSynchronize(c.st);
  for (void* p : c.run_mem) (void)hipFree(p);
  c.run_mem.clear();
  if (c.hlog) (void)hipHostFree(c.hlog);
  if (c.hrows) (void)hipHostFree(c.hrows);
  c.hlog = nullptr;
  c.hrows = nullptr;
  c.bufs = false;
}

int upload(Chain& c, void** d, const void* host, size_t bytes, const char* what) {
  if (int rc = alloc(c, d, bytes, what)) return rc;
  return hip(hipMemcpy(*d, host, bytes, hipMemcpyHostToDevice), what);
}

int ensure_stream(Chain& c) {
  if (c.st) return 0;
  return hip(hipStreamCreateWithFlags(&c.st, hipStreamNonBlocking), "chain stream");
}

// A [out][in] matrix of `kind` from host bytes: dense f32 as is, a quantised
// kind repacked into the packed layout (the raw copy freed after).
int upload_mat(Chain& c, Mat& m, const void* host, long bytes, int kind, int in, int out, const char* what) {
  m.kind = kind;
  m.in = in;
  m.out = out;
  const long need = mat_bytes(kind, in, out);
  if (!host || need <= 0 || bytes < need || in % 256) return fail(-EINVAL, what);
  if (kind == -1) return upload(c, &m.d, host, (size_t)need, what);
  const long long pb = aspida_kq_packed_bytes(kind, in, out);
  if (pb <= 0) return fail(-EINVAL, what);
  void* raw = nullptr;
  if (int rc = hip(hipMalloc(&raw, (size_t)need), what)) return rc;
  int rc = hip(hipMemcpy(raw, host, (size_t)need, hipMemcpyHostToDevice), what);
  if (!rc) rc = alloc(c, &m.d, (size_t)pb, what);
  if (!rc) rc = ep(aspida_kq_pack_dev(kind, raw, in, out, m.d, c.st), what);
  if (!rc) rc = hip(hipStreamSynchronize(c.st), what);
  (void)hipFree(raw);
  return rc;
}

// n routed experts of a projection: packed (each expert's matrix at
// e * packed_bytes) or raw GGML bytes (stride bytes / n, gpu_matvec.cu:1702-1703).
int upload_experts(Chain& c, const void** d, const void* host, long bytes, int kind, int in, int out, int n,
                   bool packed, const char* what) {
  const long per = bytes / n, need = mat_bytes(kind, in, out);
  if (!host || kind < 0 || need <= 0 || per < need) return fail(-EINVAL, what);
  void* dst = nullptr;
  if (!packed) {
    if (int rc = upload(c, &dst, host, (size_t)per * n, what)) return rc;
    *d = dst;
    return 0;
  }
  const long long pb = aspida_kq_packed_bytes(kind, in, out);
  void* raw = nullptr;
  if (int rc = hip(hipMalloc(&raw, (size_t)per * n), what)) return rc;
  int rc = hip(hipMemcpy(raw, host, (size_t)per * n, hipMemcpyHostToDevice), what);
  if (!rc) rc = alloc(c, &dst, (size_t)pb * n, what);
  if (!rc) rc = ep(aspida_moe_pack_experts_dev(kind, raw, per, in, out, n, dst, c.st), what);
  if (!rc) rc = hip(hipStreamSynchronize(c.st), what);
  (void)hipFree(raw);
  if (rc) return rc;
  *d = dst;
  return 0;
}

// ---- one step ---------------------------------------------------------------------

int mat_apply(Chain& c, const Mat& m, int B, const float* x, float* y) {
  if (m.kind == -1) {
    for (int b = 0; b < B; ++b)
      if (int rc = ep(aspida_dense_matvec_dev((const float*)m.d, m.in, m.out, x + (size_t)b * m.in,
                                              y + (size_t)b * m.out, c.st),
                      "chain dense matvec"))
        return rc;
    return 0;
  }
  if (B == 1) return ep(aspida_kq_matvec_packed_dev(m.kind, m.d, m.in, m.out, x, y, c.st), "chain matvec");
  return ep(aspida_kq_matmul_packed_dev(m.kind, m.d, m.in, m.out, B, x, y, c.st), "chain matmul");
}

int add_norm(Chain& c, int B, const float* r, const float* w) {
  hipLaunchKernelGGL(chain_add_norm, dim3(B), dim3(CHAIN_THREADS), 0, c.st, c.H, r, w, c.nx, c.dim);
  return hip(hipGetLastError(), "chain norm");
}

// The post-attention norm and the router: one launch where the router can
// form its own input (every workgroup normalises its tokens' rows of H +
// pend + pend2; the last one writes the sum and the norm's output back),
// else norm launches and then the router.
int norm_route(Chain& c, const Layer& L, int B, const float* pend, const float* pend2) {
  const int rc = kq::route_norm_dev(L.router, L.n_exp, c.dim, B, L.top_k, c.H, pend, pend2, L.post_norm, c.nx, c.rl,
                                    c.idx, c.tw, c.st);
  if (rc != -ENOTSUP) return ep(rc, "chain router with norm");
  if (int rc2 = add_norm(c, B, pend, L.post_norm)) return rc2;
  if (pend2)
    if (int rc2 = add_norm(c, B, pend2, L.post_norm)) return rc2;
  return ep(aspida_moe_route_dev(L.router, L.n_exp, c.dim, B, L.top_k, c.nx, c.rl, c.idx, c.tw, c.st), "chain router");
}

// The experts of one layer into c.y.  With next_norm set, the combine launch
// (when the experts' path has one) also adds c.y into H and forms
// nx = RMSNorm(H) with those weights -- the step's next add_norm -- and
// *normed says whether it did.
int moe_apply(Chain& c, const Layer& L, int B, const float* next_norm = nullptr, bool* normed = nullptr) {
  if (normed) *normed = false;
  if (L.grouped)
    return ep(kq::moe_experts_packed_norm(c.nx, B, c.dim, L.top_k, L.intermed, L.n_exp, c.idx, c.tw, L.g, L.u, L.gk,
                                          L.dn, L.dk, L.sg, L.su, L.sd, L.sgi, c.work, c.y, c.st,
                                          next_norm ? c.H : nullptr, next_norm, next_norm ? c.nx : nullptr, normed),
              "chain experts");
  return ep(aspida_moe_experts_dev(c.nx, B, c.dim, L.top_k, L.intermed, L.n_exp, c.idx, c.tw, L.g, L.g_stride, L.gk,
                                   L.u, L.u_stride, L.uk, L.dn, L.d_stride, L.dk, L.sg, L.sgk, L.su, L.suk, L.sd, L.sdk,
                                   L.sgi, (float*)c.work, c.y, c.st),
            "chain experts");
}

// Records (or launches) the step for B lanes whose rows are in c.rows:
// embedding, the first n_layers layers, the final norm and, when `logits`,
// the output head into c.dlog.  Afterwards H holds the residual stream.
int record(Chain& c, int B, int n_layers, bool logits) {
  hipLaunchKernelGGL(chain_embed, dim3((c.dim / 4 + CHAIN_THREADS - 1) / CHAIN_THREADS, B), dim3(CHAIN_THREADS), 0,
                     c.st, c.embed, c.rows, c.dim, c.H);
  if (int rc = hip(hipGetLastError(), "chain embed")) return rc;
  const float* pend = nullptr;  // the residual still to be added to H
  bool normed = false;          // H holds its residual and nx its next norm already (the experts' combine)
  // The norm that follows layer l's experts: the next layer's attention norm
  // (or its post-attention norm when it has no mixer), else the final norm.
  const auto next_norm = [&](int l) -> const float* {
    if (l + 1 >= n_layers) return c.fnorm;
    const Layer& N = c.layers[l + 1];
    return N.has_mix ? N.attn_norm : N.has_moe ? N.post_norm : nullptr;
  };
  for (int l = 0; l < n_layers; ++l) {
    const Layer& L = c.layers[l];
    if (L.has_mix && B == 1 && L.has_moe && L.mix.kind >= 0 &&
        kq::moe_route_norm_takes(L.n_exp, c.dim, B, L.top_k)) {
      // One lane: the attention norm inside the mixer launch (H not written)
      // and the router adding both residuals, pend then the mixer's output.
      const int rc = kq::matvec_norm_dev(L.mix.kind, L.mix.d, L.mix.in, L.mix.out, c.H, pend, L.attn_norm, c.ao, c.st);
      if (rc == 0) {
        if (int rc2 = norm_route(c, L, B, pend, c.ao)) return rc2;
        if (int rc2 = moe_apply(c, L, B)) return rc2;
        pend = c.y;
        continue;
      }
      if (rc != -ENOTSUP) return ep(rc, "chain mixer with norm");
    }
    if (L.has_mix) {
      if (!normed)
        if (int rc = add_norm(c, B, pend, L.attn_norm)) return rc;
      normed = false;
      if (int rc = mat_apply(c, L.mix, B, c.nx, c.ao)) return rc;
      pend = c.ao;
    }
    if (L.has_moe) {
      if (normed) {
        if (int rc = ep(aspida_moe_route_dev(L.router, L.n_exp, c.dim, B, L.top_k, c.nx, c.rl, c.idx, c.tw, c.st),
                        "chain router"))
          return rc;
      } else if (int rc = norm_route(c, L, B, pend, nullptr)) {
        return rc;
      }
      // From 2 lanes the experts' combine is a launch of its own, which then
      // also takes the next add_norm.
      const float* nn = B > 1 ? next_norm(l) : nullptr;
      if (int rc = moe_apply(c, L, B, nn, &normed)) return rc;
      pend = normed ? nullptr : c.y;
    }
  }
  if (!normed)
    if (int rc = add_norm(c, B, pend, c.fnorm)) return rc;
  return logits ? mat_apply(c, c.lm, B, c.nx, c.dlog) : 0;
}

bool ready(const Chain& c) { return c.model && !c.broken && !c.layers.empty(); }

// Device buffers for CHAIN_MAX_LANES lanes (allocated once per registered
// model, so graphs captured earlier keep valid pointers).
int ensure_bufs(Chain& c) {
  if (c.bufs) return 0;
  const size_t D = (size_t)CHAIN_MAX_LANES * c.dim;
  int n_exp = 1, top_k = 1;
  size_t work = 256;
  for (const Layer& L : c.layers) {
    if (!L.has_moe) continue;
    n_exp = std::max(n_exp, L.n_exp);
    top_k = std::max(top_k, L.top_k);
    const int T = std::min(CHAIN_MAX_LANES, MOE_MAX_JOBS / L.top_k);
    const long wb = L.grouped ? aspida_moe_packed_work_bytes(T, c.dim, L.intermed, L.top_k)
                              : aspida_moe_work_floats(T, c.dim, L.top_k, L.intermed) * 4;
    if (wb <= 0) return fail(-EINVAL, "chain work size");
    work = std::max(work, (size_t)wb);
  }
  void* p[9];
  const size_t bytes[9] = {D * 4, D * 4, D * 4, D * 4, (size_t)CHAIN_MAX_LANES * n_exp * 4,
                           (size_t)CHAIN_MAX_LANES * top_k * 4, (size_t)CHAIN_MAX_LANES * c.vocab * 4,
                           (size_t)CHAIN_MAX_LANES * top_k * 4, (size_t)CHAIN_MAX_LANES * 4};
  for (int i = 0; i < 9; ++i)
    if (int rc = alloc(c, &p[i], bytes[i], "chain buffers", true)) return rc;
  c.H = (float*)p[0];
  c.nx = (float*)p[1];
  c.ao = (float*)p[2];
  c.y = (float*)p[3];
  c.rl = (float*)p[4];
  c.tw = (float*)p[5];
  c.dlog = (float*)p[6];
  c.idx = (int*)p[7];
  c.rows = (int*)p[8];
  if (int rc = alloc(c, &c.work, work, "chain work", true)) return rc;
  if (int rc = hip(hipHostMalloc((void**)&c.hlog, (size_t)CHAIN_MAX_LANES * c.vocab * 4, hipHostMallocDefault),
                   "chain pinned logits"))
    return rc;
  if (int rc = hip(hipHostMalloc((void**)&c.hrows, CHAIN_MAX_LANES * 4, hipHostMallocDefault), "chain pinned rows"))
    return rc;
  c.bufs = true;
  return 0;
}

void free_all(Chain& c) {
  drop_run_state(c);
  // A new registration starts with no lane count run eagerly, so that the
  // first forward of every lane count sizes the workspaces again before a
  // graph is captured (forward()).
  c.warmed.clear();
  for (void* p : c.mem) (void)hipFree(p);
  c.mem.clear();
  c.layers.clear();
  c.model = c.broken = false;
  c.embed = c.fnorm = nullptr;
  c.embed_rows = 0;
  c.lm = Mat();
  c.dim = c.vocab = 0;
}

// The lanes' rows to the device, checked against the embedding table.
int stage_rows(Chain& c, int B, const int* rows) {
  for (int b = 0; b < B; ++b)
    if (rows[b] < 0 || rows[b] >= c.embed_rows) return fail(-EINVAL, "chain forward: embedding row out of range");
  std::memcpy(c.hrows, rows, (size_t)B * 4);
  return hip(hipMemcpyAsync(c.rows, c.hrows, (size_t)B * 4, hipMemcpyHostToDevice, c.st), "chain rows");
}

// One forward of B lanes into logits[B][vocab] (host).  The first run of a
// lane count is eager (its library workspaces are sized then); every later
// one replays the graph captured after it.  A lane count run eagerly for the
// first time may have grown a workspace that earlier graphs point into, so
// it drops them.
int forward(Chain& c, int B, const int* rows, float* logits) {
  if (!ready(c)) return fail(-EINVAL, "chain forward: no model registered (chain_model, layers, chain_moe)");
  if (B < 1 || B > CHAIN_MAX_LANES) return fail(-EINVAL, "chain forward: lane count out of range");
  for (const Layer& L : c.layers)
    if (L.has_moe && (long)B * L.top_k > MOE_MAX_JOBS) return fail(-EINVAL, "chain forward: too many lanes for top_k");
  if (int rc = ensure_stream(c)) return rc;
  if (int rc = ensure_bufs(c)) return rc;
  if (c.use_graphs < 0) c.use_graphs = getenv("ASPIDA_NO_GRAPH") ? 0 : 1;
  if (int rc = stage_rows(c, B, rows)) return rc;
  auto it = c.graphs.find(B);
  if (it != c.graphs.end()) {
    if (int rc = hip(hipGraphLaunch(it->second, c.st), "chain graph launch")) return rc;
  } else {
    if (int rc = record(c, B, (int)c.layers.size(), true)) return rc;
    if (int rc = hip(hipStreamSynchronize(c.st), "chain forward")) return rc;
    if (!c.warmed.count(B)) {
      destroy_graphs(c);
      c.warmed.insert(B);
    }
    if (c.use_graphs) {
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      if (int rc = hip(hipStreamBeginCapture(c.st, hipStreamCaptureModeThreadLocal), "chain capture")) return rc;
      const int rr = record(c, B, (int)c.layers.size(), true);
      const hipError_t ee = hipStreamEndCapture(c.st, &g);
      if (rr || ee != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return rr ? rr : hip(ee, "chain capture");
      }
      const hipError_t ie = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
      (void)hipGraphDestroy(g);
      if (int rc = hip(ie, "chain graph instantiate")) return rc;
      c.graphs[B] = ge;
    }
  }
  const size_t n = (size_t)B * c.vocab;
  if (int rc = hip(hipMemcpyAsync(c.hlog, c.dlog, n * 4, hipMemcpyDeviceToHost, c.st), "chain logits")) return rc;
  if (int rc = hip(hipStreamSynchronize(c.st), "chain forward")) return rc;
  std::memcpy(logits, c.hlog, n * 4);
  return 0;
}

void fill_nan(float* y, size_t n) {
  if (!y) return;
  const float q = std::nanf("");
  for (size_t i = 0; i < n; ++i) y[i] = q;
}

}  // namespace

// ---- reference chain ABI ---------------------------------------------------------

extern "C" void aspida_gpu_chain_reset(void) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  free_all(c);
}

extern "C" int aspida_kq_chain_layer(const float* attn_norm, long an_b, const float* post_norm, long pn_b,
                                     const void* mix_w, long mix_b, int mix_k) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  const int dim = (int)(an_b / 4);
  if (!attn_norm || !post_norm || an_b <= 0 || an_b % 1024 || pn_b != an_b || (c.dim && dim != c.dim) ||
      (mix_w && mix_k != -1 && block_bytes(mix_k) == 0)) {
    c.broken = true;
    return fail(-EINVAL, "aspida_kq_chain_layer: bad arguments");
  }
  drop_run_state(c);
  if (int rc = ensure_stream(c)) return c.broken = true, rc;
  Layer L;
  L.dim = dim;
  int rc = upload(c, (void**)&L.attn_norm, attn_norm, (size_t)an_b, "chain attn norm");
  if (!rc) rc = upload(c, (void**)&L.post_norm, post_norm, (size_t)pn_b, "chain post norm");
  if (!rc && mix_w) {
    L.has_mix = true;
    rc = upload_mat(c, L.mix, mix_w, mix_b, mix_k, dim, dim, "chain mixer");
  }
  if (rc) {
    c.broken = true;
    return rc;
  }
  c.dim = dim;
  c.layers.push_back(L);
  return 0;
}

extern "C" void aspida_gpu_chain_moe(const void* router_w, long router_b, int router_k, const void* gate_w, long gate_b,
                                     int gate_k, const void* up_w, long up_b, int up_k, const void* down_w,
                                     long down_b, int down_k, const void* shg_w, long shg_b, int shg_k,
                                     const void* shu_w, long shu_b, int shu_k, const void* shd_w, long shd_b,
                                     int shd_k, const float* sgi, long sgi_b, int sgi_len, int n_exp, int top_k,
                                     int intermed) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  if (c.layers.empty()) return;  // as the reference: nothing to attach to
  Layer& L = c.layers.back();
  const int dim = L.dim;
  const bool gated = sgi_len > 1 && sgi;
  const int kinds[6] = {gate_k, up_k, down_k, shg_k, shu_k, shd_k};
  bool ok = !L.has_moe && n_exp >= 1 && n_exp <= 1024 && top_k >= 1 && top_k <= MOE_MAX_TOPK && top_k <= n_exp &&
            intermed > 0 && intermed % 256 == 0 && (router_k == -1 || block_bytes(router_k) > 0) &&
            (!gated || (sgi_len == dim && sgi_b >= (long)dim * 4));
  for (int k : kinds) ok = ok && block_bytes(k) > 0;
  if (!ok) {
    c.broken = true;
    fail(-EINVAL, "aspida_gpu_chain_moe: bad arguments");
    return;
  }
  drop_run_state(c);
  L.n_exp = n_exp;
  L.top_k = top_k;
  L.intermed = intermed;
  L.gk = gate_k;
  L.uk = up_k;
  L.dk = down_k;
  L.sgk = shg_k;
  L.suk = shu_k;
  L.sdk = shd_k;
  L.grouped = gate_k == up_k && shg_k == gate_k && shu_k == gate_k && shd_k == down_k &&
              kq::moe_grouped_supported(dim, intermed, 1, top_k) && kq::moe_grouped_experts_ok(n_exp);
  // Router: f32 [n_exp][dim]; a quantised one is decoded to f32 once.
  int rc = 0;
  if (router_k == -1) {
    rc = router_w && router_b >= (long)n_exp * dim * 4
             ? upload(c, (void**)&L.router, router_w, (size_t)n_exp * dim * 4, "chain router")
             : fail(-EINVAL, "aspida_gpu_chain_moe: router bytes");
  } else {
    const long need = mat_bytes(router_k, dim, n_exp);
    void* raw = nullptr;
    rc = router_w && router_b >= need ? hip(hipMalloc(&raw, (size_t)need), "chain router")
                                      : fail(-EINVAL, "aspida_gpu_chain_moe: router bytes");
    if (!rc) rc = hip(hipMemcpy(raw, router_w, (size_t)need, hipMemcpyHostToDevice), "chain router");
    if (!rc) rc = alloc(c, (void**)&L.router, (size_t)n_exp * dim * 4, "chain router");
    if (!rc) rc = ep(aspida_kq_dequant_dev(router_k, raw, dim, n_exp, L.router, c.st), "chain router");
    if (!rc) rc = hip(hipStreamSynchronize(c.st), "chain router");
    if (raw) (void)hipFree(raw);
  }
  if (!rc) rc = upload_experts(c, &L.g, gate_w, gate_b, gate_k, dim, intermed, n_exp, L.grouped, "chain gate experts");
  if (!rc) rc = upload_experts(c, &L.u, up_w, up_b, up_k, dim, intermed, n_exp, L.grouped, "chain up experts");
  if (!rc) rc = upload_experts(c, &L.dn, down_w, down_b, down_k, intermed, dim, n_exp, L.grouped, "chain down experts");
  if (!rc) rc = upload_experts(c, &L.sg, shg_w, shg_b, shg_k, dim, intermed, 1, L.grouped, "chain shared gate");
  if (!rc) rc = upload_experts(c, &L.su, shu_w, shu_b, shu_k, dim, intermed, 1, L.grouped, "chain shared up");
  if (!rc) rc = upload_experts(c, &L.sd, shd_w, shd_b, shd_k, intermed, dim, 1, L.grouped, "chain shared down");
  if (!rc && gated) rc = upload(c, (void**)&L.sgi, sgi, (size_t)dim * 4, "chain shared gate input");
  if (rc) {
    c.broken = true;
    return;
  }
  L.g_stride = gate_b / n_exp;
  L.u_stride = up_b / n_exp;
  L.d_stride = down_b / n_exp;
  L.has_moe = true;
}

extern "C" void aspida_gpu_chain_model(const float* embed, long embed_b, const float* fnorm, long fnorm_b,
                                       const void* lm, long lm_b, int lm_k, int dim, int vocab) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!embed || !fnorm || dim <= 0 || dim % 256 || vocab <= 0 || (c.dim && dim != c.dim) ||
      embed_b < (long)dim * 4 || fnorm_b < (long)dim * 4 || (lm_k != -1 && block_bytes(lm_k) == 0) || c.model) {
    c.broken = true;
    fail(-EINVAL, "aspida_gpu_chain_model: bad arguments");
    return;
  }
  drop_run_state(c);
  int rc = ensure_stream(c);
  const long rows = embed_b / ((long)dim * 4);
  if (!rc) rc = upload(c, (void**)&c.embed, embed, (size_t)rows * dim * 4, "chain embedding");
  if (!rc) rc = upload(c, (void**)&c.fnorm, fnorm, (size_t)dim * 4, "chain final norm");
  if (!rc) rc = upload_mat(c, c.lm, lm, lm_b, lm_k, dim, vocab, "chain output head");
  if (rc) {
    c.broken = true;
    return;
  }
  c.embed_rows = rows;
  c.dim = dim;
  c.vocab = vocab;
  c.model = true;
}

extern "C" int aspida_gpu_chain_ready(void) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  return ready(c) ? 1 : 0;
}

// A generation's start and end drop the captured graphs, as the reference's
// do (the handles name per-generation attention state, which this chain's
// mixers do not have).
extern "C" void aspida_gpu_chain_begin(const int* attn_handles) {
  (void)attn_handles;
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  destroy_graphs(c);
}

extern "C" void aspida_gpu_chain_end(void) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  destroy_graphs(c);
}

// pos and attn_handles index the attention state of the reference's mixers;
// the matvec mixers here are stateless, so both are unused.
extern "C" void aspida_gpu_chain_forward(int embed_row, int pos, const int* attn_handles, float* logits) {
  (void)pos;
  (void)attn_handles;
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  if (forward(c, 1, &embed_row, logits)) fill_nan(logits, (size_t)c.vocab);
}

extern "C" void aspida_gpu_chain_forward_batch(int B, const int* rows, const int* pos, const int* handles,
                                               float* logits) {
  (void)pos;
  (void)handles;
  if (B < 1) return;  // as the reference
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!rows || forward(c, B, rows, logits)) fill_nan(logits, (size_t)std::max(B, 0) * c.vocab);
}

// ---- this library's additions --------------------------------------------------

extern "C" int aspida_kq_chain_forward_layers(int B, const int* rows, int n_layers, float* hidden) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  if (!ready(c) || !rows || !hidden || B < 1 || B > CHAIN_MAX_LANES || n_layers < 0 ||
      n_layers > (int)c.layers.size())
    return fail(-EINVAL, "aspida_kq_chain_forward_layers: bad arguments");
  for (const Layer& L : c.layers)
    if (L.has_moe && (long)B * L.top_k > MOE_MAX_JOBS) return fail(-EINVAL, "chain: too many lanes for top_k");
  if (int rc = ensure_stream(c)) return rc;
  if (int rc = ensure_bufs(c)) return rc;
  if (int rc = stage_rows(c, B, rows)) return rc;
  if (int rc = record(c, B, n_layers, false)) return rc;
  if (!c.warmed.count(B)) {
    if (int rc = hip(hipStreamSynchronize(c.st), "chain forward")) return rc;
    destroy_graphs(c);
    c.warmed.insert(B);
  }
  const size_t n = (size_t)B * c.dim;
  if (int rc = hip(hipMemcpyAsync(hidden, c.H, n * 4, hipMemcpyDeviceToHost, c.st), "chain hidden")) return rc;
  return hip(hipStreamSynchronize(c.st), "chain forward");
}

extern "C" int aspida_kq_chain_set_graphs(int on) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  destroy_graphs(c);
  c.use_graphs = on ? 1 : 0;
  return 0;
}

extern "C" int aspida_kq_chain_graphs(void) {
  Chain& c = chain();
  std::lock_guard<std::mutex> lk(c.mu);
  return (int)c.graphs.size();
}
