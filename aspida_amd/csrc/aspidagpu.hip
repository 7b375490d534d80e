// aspidagpu.hip -- the drop-in C ABI (libaspidagpu.so).
//
// Exports the symbols Aspida's Ada host resolves with dlopen/dlsym
// (src/llm/llm_gpu.adb:80-146, src/llm/llm_qwen_gpu.adb:257-266), with the
// reference shim's signatures (gpu/gpu_matvec.cu:494-553, 925, 1673), plus
// device-pointer entry points for callers whose activations already live in
// HBM.  Declarations and contracts: include/aspidagpu.h.
//
// Host-ABI calls are synchronous, like the reference's: on return y is fully
// written.  Unlike the reference they are thread-safe: each calling thread
// gets its own HIP stream, device scratch and pinned staging buffers, and the
// VRAM weight cache is guarded by a mutex.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <atomic>
#include <cstdint>
#include <mutex>
#include <shared_mutex>
#include <unordered_map>
#include <vector>

#include "../../include/aspidagpu.h"
#include "kq_common.h"
#include "kq_kernels.h"
#include "kq_moe.h"
#include "kq_chain.h"

namespace {

// ---- errors -----------------------------------------------------------------

thread_local int t_last_error = 0;

void report(int code, const char* fmt, ...) {
  t_last_error = code;
  va_list ap;
  va_start(ap, fmt);
  fprintf(stderr, "[aspida_gpu] ");
  vfprintf(stderr, fmt, ap);
  fprintf(stderr, "\n");
  va_end(ap);
}

int check(hipError_t e, const char* where) {
  if (e == hipSuccess) return 0;
  report((int)e, "%s: %s", where, hipGetErrorString(e));
  return (int)e;
}

void fill_nan(float* y, long n) {
  if (!y || n <= 0) return;
  const float q = std::nanf("");
  for (long i = 0; i < n; ++i) y[i] = q;
}

long need_bytes(int kind, int in_dim, int rows) {
  return (long)rows * (long)(in_dim / 256) * (long)kq::block_bytes(kind);
}

// ---- VRAM weight cache keyed by host pointer --------------------------------
//
// Two mirrors per host pointer: the ggml layout (ggml bytes) and the packed
// layout of the batch-1 kernels.  A host-ABI call holds g_wmu shared from its
// lookup until its stream has been synchronised, so no mirror it uses can be
// freed or re-packed under it: aspida_gpu_free_weight and every upload or
// re-pack take g_wmu exclusively and so wait for the calls in flight.

struct WEnt {
  void* d;
  long bytes;
};
// Packed mirror: n matrices of kind / in_dim / out_dim, packed_bytes apart.
struct PEnt {
  void* d;
  int kind, in_dim, out_dim, n;
};
std::shared_mutex g_wmu;
std::unordered_map<const void*, WEnt> g_wcache;
std::unordered_map<const void*, PEnt> g_pcache;

// One weight a call needs in HBM: the ggml mirror of [w, w + bytes), or
// (packed) the packed mirror of n matrices the host holds src_stride bytes
// apart (MoE experts; n = 1 for a plain matrix).
struct WReq {
  const void* w = nullptr;
  bool packed = false;
  long bytes = 0;
  int kind = 0, in_dim = 0, out_dim = 0, n = 1;
  size_t src_stride = 0;
  void* d = nullptr;  // the mirror, once acquired
};

WReq ggml_req(const void* w, long bytes) {
  WReq r;
  r.w = w;
  r.bytes = bytes;
  return r;
}

WReq packed_req(const void* w, int kind, int in_dim, int out_dim, int n = 1, size_t src_stride = 0) {
  WReq r;
  r.w = w;
  r.packed = true;
  r.kind = kind;
  r.in_dim = in_dim;
  r.out_dim = out_dim;
  r.n = n;
  r.src_stride = src_stride;
  return r;
}

// The cached mirror satisfying r, or null (g_wmu held, either way).  A ggml
// mirror at least r.bytes long serves; a packed one must match exactly.
void* lookup(const WReq& r) {
  if (!r.packed) {
    auto it = g_wcache.find(r.w);
    return it != g_wcache.end() && it->second.bytes >= r.bytes ? it->second.d : nullptr;
  }
  auto it = g_pcache.find(r.w);
  if (it == g_pcache.end()) return nullptr;
  const PEnt& e = it->second;
  return e.kind == r.kind && e.in_dim == r.in_dim && e.out_dim == r.out_dim && e.n == r.n ? e.d : nullptr;
}

// Uploads r's mirror, replacing a smaller or differently shaped one (g_wmu
// held exclusively).  0 or -1.
int create(const WReq& r) {
  if (!r.packed) {
    auto it = g_wcache.find(r.w);
    if (it != g_wcache.end()) {
      (void)hipFree(it->second.d);
      g_wcache.erase(it);
    }
    void* d = nullptr;
    if (check(hipMalloc(&d, (size_t)r.bytes), "weight upload: hipMalloc")) return -1;
    if (check(hipMemcpy(d, r.w, (size_t)r.bytes, hipMemcpyHostToDevice), "weight upload: hipMemcpy")) {
      (void)hipFree(d);
      return -1;
    }
    g_wcache[r.w] = {d, r.bytes};
    return 0;
  }
  auto it = g_pcache.find(r.w);
  if (it != g_pcache.end()) {
    (void)hipFree(it->second.d);
    g_pcache.erase(it);
  }
  // Packed on the device from a temporary ggml copy.
  const size_t one = (size_t)need_bytes(r.kind, r.in_dim, r.out_dim);
  const size_t stride = r.n == 1 ? one : r.src_stride;
  const size_t raw = stride * (size_t)(r.n - 1) + one;
  const size_t pb = kq::packed_bytes(r.kind, r.in_dim, r.out_dim);
  void *tmp = nullptr, *d = nullptr;
  int rc = check(hipMalloc(&tmp, raw), "weight upload: hipMalloc");
  if (!rc) rc = check(hipMalloc(&d, pb * (size_t)r.n), "weight upload: hipMalloc packed");
  if (!rc) rc = check(hipMemcpy(tmp, r.w, raw, hipMemcpyHostToDevice), "weight upload: hipMemcpy");
  for (int i = 0; i < r.n && !rc; ++i)
    rc = check(kq::launch_pack(r.kind, (const uint8_t*)tmp + stride * i, r.in_dim, r.out_dim, (uint8_t*)d + pb * i,
                               false, nullptr),
               "weight upload: pack");
  if (!rc) rc = check(hipStreamSynchronize(nullptr), "weight upload: sync");
  if (tmp) (void)hipFree(tmp);
  if (rc) {
    if (d) (void)hipFree(d);
    return -1;
  }
  g_pcache[r.w] = {d, r.kind, r.in_dim, r.out_dim, r.n};
  return 0;
}

// Sets every r[i].d and returns 0 with `rd` (a deferred shared lock of
// g_wmu) locked: the mirrors stay valid until the caller releases it.  Missing
// mirrors are uploaded under the exclusive lock, then looked up again (another
// thread may free or replace one in between; a few rounds settle it).  -1,
// with rd unlocked, if an upload fails.
int acquire(std::shared_lock<std::shared_mutex>& rd, WReq* r, int n) {
  for (int round = 0; round < 8; ++round) {
    rd.lock();
    bool all = true;
    for (int i = 0; i < n; ++i) all = (r[i].d = lookup(r[i])) != nullptr && all;
    if (all) return 0;
    rd.unlock();
    std::unique_lock<std::shared_mutex> wr(g_wmu);
    for (int i = 0; i < n; ++i)
      if (!lookup(r[i]) && create(r[i])) return -1;
  }
  report(-EAGAIN, "weight upload: the cache kept changing under concurrent frees");
  return -1;
}

// ---- per-thread execution context -------------------------------------------

// Device buffer that only grows.  By default it never frees a buffer it has
// handed out: a HIP graph captured while an older, smaller buffer was current
// keeps its pointer, so a later growth must leave that memory valid.  Growth
// at least doubles, so the superseded buffers together stay smaller than the
// current one; all of them live until the process ends.  Buffers that no
// graph can hold (the host ABI's per-thread ones, used only inside a call
// that ends with a stream synchronisation) set keep_old = false and free the
// superseded buffer when they grow.
template <class T>
struct DevBuf {
  T* p = nullptr;
  size_t n = 0;
  bool keep_old = true;
  std::vector<T*> old;
  // 0 or -1; *grew says whether p is a new, uninitialised buffer.
  int ensure(size_t want, const char* what, bool* grew = nullptr) {
    if (grew) *grew = false;
    if (want <= n) return 0;
    const size_t sz = std::max(want, 2 * n);
    T* q = nullptr;
    if (check(hipMalloc(&q, sz * sizeof(T)), what)) return -1;
    if (p && keep_old) old.push_back(p);
    else if (p) (void)hipFree(p);
    p = q;
    n = sz;
    if (grew) *grew = true;
    return 0;
  }
};

template <class T>
struct HostBuf {
  T* p = nullptr;
  size_t n = 0;
  int ensure(size_t want, const char* what) {
    if (want <= n) return 0;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
    if (check(hipHostMalloc((void**)&p, want * sizeof(T), hipHostMallocDefault), what)) return -1;
    n = want;
    return 0;
  }
};

// Bytes of MvWorkspace::mm for every launch matmul_packed may issue for up
// to `batch` vectors: the 16-vector kernel, and the 64-vector kernel at each
// padding (16, 32, 64 vectors) a launch of at most min(batch, 64) vectors
// takes -- a smaller padding can mean a finer column split and so more
// partial sums.
size_t mm_work_bytes(int in_dim, int out_dim, int batch) {
  size_t n = kq::mm16_workspace_bytes(in_dim, out_dim);
  for (int bp = 16; bp <= 64; bp *= 2) {
    n = std::max(n, kq::mfma_workspace_bytes(in_dim, out_dim, bp));
    if (bp >= batch) break;
  }
  if (in_dim % 1024 == 0) n = std::max(n, kq::mmw_workspace_bytes(in_dim, out_dim, std::min(batch, 64)));
  return n;
}

// Partial sums and per-tile arrival counters of the packed matvec
// (kq::launch_matvec_packed).  Counters start zeroed and every launch leaves
// them zero; launches sharing a workspace must be ordered on one stream.
struct MvWorkspace {
  DevBuf<float> part;
  DevBuf<unsigned> count;
  DevBuf<uint8_t> mm;  // activation split and partials of the MFMA product
  int ensure(int in_dim, int out_dim, int batch = 1) {
    const size_t pf = batch > 1 ? kq::multi_workspace_floats(in_dim, out_dim) : kq::packed_workspace_floats(in_dim, out_dim);
    if (part.ensure(std::max<size_t>(pf, 64), "hipMalloc partials")) return -1;
    if (batch > 1 && mm.ensure(mm_work_bytes(in_dim, out_dim, batch), "hipMalloc mfma")) return -1;
    bool grew = false;
    if (count.ensure(kq::packed_counters(out_dim), "hipMalloc counters", &grew)) return -1;
    return grew ? check(hipMemset(count.p, 0, count.n * sizeof(unsigned)), "hipMemset counters") : 0;
  }
};

// Y[batch][out] = X W^T over packed W on `st`.  Batch 1 is the matvec.
// Otherwise, by g_mm_engine: 0 picks, 1 forces the multi-vector VALU kernel,
// 2 the 64-vector and 3 the 16-vector MFMA kernel, 4 the one-pass kernel
// (kq_mmv.hip), 5 the batch-1 kernel for up to 4 vectors per launch and 6
// the wave-per-column kernel (kq_mmw.hip), where the kind has one.
// The pick for Q4_K and Q6_K (measured on MI355X at 4096x4096 and
// 14336x4096, `small_batch` of bench.py):
//   up to 4 vectors: the batch-1 kernel on 4 vectors where its batch-1
//     plan is 16-row workgroups (and Q6_K at 2 vectors), else one pass;
//   5-16 vectors: one pass;
//   on matrices of at least MM16_TALL_UNITS pairs up to 16 vectors: the
//     16-vector kernel (Q6_K up to 4 vectors: the batch-1 kernel on 4);
//   above 16: one pass for Q6_K (launches of 32 vectors on 64-row tiles;
//     above 32 on at most MMW_MAX_UNITS pairs the wave-per-column kernel);
//     Q4_K on the 64-vector kernel in one launch.
// The 16-vector kernel stays an engine of its own (3).
constexpr int MULTI_MAX_BATCH = 8;
constexpr int MULTI_MAX_BATCH_MFMA_KINDS = 4;
constexpr long MM16_MIN_UNITS = 2048;
// From this many (64-row tile, super-block column) pairs, batches of up to 16
// take the 16-vector kernel (Q4_K from 2 vectors, Q6_K from 5).  Measured on
// MI355X, 8 vectors: Q6_K 151936x2048 98 against 129 us on the one-pass
// kernel, 65536x2048 48 against 55, 32768x4096 45 against 55; Q4_K
// 151936x2048 at 2 vectors 54 against 70, 65536x4096 45 against 47; below,
// at 14336x4096 (3584 pairs), the one-pass kernel is ahead (Q4_K 8 vectors
// 15.2 against 19.1 us).
constexpr long MM16_TALL_UNITS = 8192;
constexpr long MMW_MAX_UNITS = 1024;
// Test and tuning overrides (aspida_kq_set_*) are per calling thread: a
// thread's override changes only the launches that thread makes.
thread_local int g_mm_engine = 0;

// The kernel family of a batched product and how many vectors each launch
// takes: 0 the multi-vector VALU kernel, 1 the 16-vector and 2 the 64-vector
// MFMA kernel.
struct MmRoute {
  int family, step;
};
MmRoute mm_route(int kind, int in_dim, int out_dim, int batch) {
  const int eng = g_mm_engine;
  const long units = (long)((out_dim + 63) / 64) * (in_dim / 256);
  // Q4_K above 16 vectors: one pass of the 64-vector kernel rather than 16
  // vectors per launch (14336x4096: 32 vectors 37 -> 31 us, 64 vectors
  // 69 -> 46 us).  Q6_K keeps the 16-vector launches on big matrices (the
  // 64-vector Q6_K kernel measured equal or slower there).
  const bool mm16 = kq::mm16_kind(kind) &&
                    (eng == 3 || (eng == 0 && batch > MULTI_MAX_BATCH_MFMA_KINDS &&
                                  (batch <= 16 || (units >= MM16_MIN_UNITS && kind != kq::Q4_K))));
  const bool mm64 = !mm16 && kq::mfma_kind(kind) && (eng == 2 || (eng == 0 && batch > MULTI_MAX_BATCH_MFMA_KINDS));
  // Q6_K in launches of at most 32 vectors: the 64-vector kernel's Q6_K
  // variant runs out of registers above 32 (14336x4096: 359 us for 64
  // vectors in one launch, 82 us per 32).
  if (eng == 4 && kq::mmv_kind(kind)) return {3, 64};
  if (eng == 5 && kq::matvec_nv_takes(kind, in_dim, out_dim)) return {4, 4};
  if (eng == 6 && kq::mmw_takes(kind, in_dim)) return {5, 64};
  // Q6_K above 32 vectors on at most MMW_MAX_UNITS (tile, column) pairs:
  // the wave-per-column kernel in one launch (4096^2, 64 vectors: 32.8
  // against 36.1 us for two 32-vector one-pass launches; at 14336x4096 the
  // one-pass launches stay ahead, 86 against 95-110 us).
  if (eng == 0 && kind == kq::Q6_K && batch > 32 && units <= MMW_MAX_UNITS && kq::mmw_takes(kind, in_dim))
    return {5, 64};
  if (eng == 0 && kq::mmv_kind(kind) && kq::matvec_nv_takes(kind, in_dim, out_dim)) {
    // Very tall matrices (output heads): the 16-vector kernel, whose
    // activation pre-pass is amortised over many rows.
    const bool tall = units >= MM16_TALL_UNITS && kq::mm16_kind(kind);
    if (batch <= 4) {
      if (tall) return kind == kq::Q6_K ? MmRoute{4, 4} : MmRoute{1, 16};
      if (kq::mfma_plan(kind, in_dim, out_dim).blk16 || (kind == kq::Q6_K && batch <= 2)) return {4, 4};
      return {3, 64};
    }
    if (batch <= 16 && tall) return {1, 16};
    if (batch <= 16 || kind == kq::Q6_K) return {3, kq::mmv_step(kind, in_dim, out_dim)};
  }
  if (mm16) return {1, 16};
  if (mm64) return {2, kind == kq::Q6_K ? 32 : 64};
  return {0, MULTI_MAX_BATCH};
}

// The largest MvWorkspace::mm any launch of matmul_packed needs for this
// product (launches of `step` vectors and a last one of the remainder).
size_t mm_launch_need(int kind, int in_dim, int out_dim, int batch) {
  if (batch <= 1) return 0;
  const MmRoute r = mm_route(kind, in_dim, out_dim, batch);
  if (r.family == 5) return kq::mmw_workspace_bytes(in_dim, out_dim, std::min(batch, r.step));
  if (r.family == 0 || r.family >= 3) return 0;
  if (r.family == 1) return kq::mm16_workspace_bytes(in_dim, out_dim);
  size_t n = kq::mfma_workspace_bytes(in_dim, out_dim, std::min(batch, r.step));
  if (batch > r.step && batch % r.step) n = std::max(n, kq::mfma_workspace_bytes(in_dim, out_dim, batch % r.step));
  return n;
}

hipError_t matmul_packed(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                         MvWorkspace& ws, hipStream_t st) {
  if (batch == 1)
    return kq::launch_matvec_packed(kind, P, in_dim, out_dim, X, Y, ws.part.p, ws.count.p, st);
  const MmRoute r = mm_route(kind, in_dim, out_dim, batch);
  for (int b0 = 0; b0 < batch; b0 += r.step) {
    const int nb = std::min(r.step, batch - b0);
    const float* xb = X + (size_t)b0 * in_dim;
    float* yb = Y + (size_t)b0 * out_dim;
    hipError_t e;
    if (r.family == 4)
      e = kq::launch_matvec_mfma_nv(kind, P, in_dim, out_dim, nb, xb, yb, st);
    else if (r.family == 3)
      e = kq::launch_matmul_mmv(kind, P, in_dim, out_dim, nb, xb, yb, st);
    else if (r.family == 5)
      e = kq::launch_matmul_mmw(kind, P, in_dim, out_dim, nb, xb, yb, ws.mm.p, ws.count.p, st);
    else if (r.family == 1)
      e = kq::launch_matmul_mm16(kind, P, in_dim, out_dim, nb, xb, yb, ws.mm.p, ws.count.p, st, batch <= r.step);
    else if (r.family == 2)
      e = kq::launch_matmul_mfma_packed(kind, P, in_dim, out_dim, nb, xb, yb, ws.mm.p, ws.count.p, st,
                                        batch <= r.step);
    else
      e = kq::launch_matmul_packed_valu(kind, P, in_dim, out_dim, nb, xb, yb, ws.part.p, ws.count.p, st);
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

// Buffers live until the process ends (thread exit does not release them).
struct Ctx {
  hipStream_t st = nullptr;
  DevBuf<float> dx, dy, dq, dh;
  HostBuf<float> hx, hy;
  DevBuf<int> di;
  MvWorkspace ws;
  // Every call on this context ends with hipStreamSynchronize and none is
  // captured into a graph, so a superseded buffer is idle when it is freed.
  Ctx() {
    dx.keep_old = dy.keep_old = dq.keep_old = dh.keep_old = di.keep_old = false;
    ws.part.keep_old = ws.count.keep_old = ws.mm.keep_old = false;
  }
  int init() {
    if (st) return 0;
    return check(hipStreamCreateWithFlags(&st, hipStreamNonBlocking), "hipStreamCreate");
  }
};

Ctx& ctx() {
  static thread_local Ctx* c = new Ctx();
  return *c;
}

// Launch-shape override for batch-1 matvecs (tuning and tests, per calling
// thread); rows <= 0 means "use kq::default_mv_config".
thread_local int g_cfg_rows = 0, g_cfg_wpc = 16;

kq::MvConfig mv_config(int kind, int in_dim, int out_dim) {
  if (g_cfg_rows <= 0) return kq::default_mv_config(kind, in_dim, out_dim);
  kq::MvConfig c;
  c.rows_per_wave = g_cfg_rows;
  c.waves_per_cu = g_cfg_wpc;
  return c;
}

bool valid_kind(int kind) { return kind >= 0 && kind <= 5; }

int validate_mv(const char* fn, const void* w, long wbytes, int kind, int in_dim, int out_dim, int batch,
                const float* x, const float* y) {
  if (!w || !x || !y) { report(-EINVAL, "%s: null pointer argument", fn); return -EINVAL; }
  if (!valid_kind(kind)) { report(-EINVAL, "%s: unsupported kind %d", fn, kind); return -EINVAL; }
  if (in_dim <= 0 || out_dim <= 0 || batch <= 0) {
    report(-EINVAL, "%s: bad shape in=%d out=%d batch=%d", fn, in_dim, out_dim, batch);
    return -EINVAL;
  }
  if (in_dim % 256 != 0) {
    report(-EINVAL, "%s: in_dim %d is not a multiple of 256", fn, in_dim);
    return -EINVAL;
  }
  if (wbytes < need_bytes(kind, in_dim, out_dim)) {
    report(-EINVAL, "%s: wbytes %ld < %ld needed for %d x %d kind %d", fn, wbytes,
           need_bytes(kind, in_dim, out_dim), out_dim, in_dim, kind);
    return -EINVAL;
  }
  return 0;
}

// The host ABI's x, staged from its pinned host buffer by the GPU itself: a
// kernel's reads of pinned host memory return sooner than a copy-engine
// transfer of the same 16-57 KB (drop-in 8B decode, 225 calls per token:
// 151 -> 177 tok/s together with y written straight to pinned memory).
__global__ void stage_copy(const float4* __restrict__ src, float4* __restrict__ dst, int n4) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n4; i += gridDim.x * blockDim.x) dst[i] = src[i];
}

// x -> device (through pinned staging), per-group sums (when `sums`), then
// `launch`, then y <- device; synchronous.  With y_host the launch writes y
// into the pinned buffer c.hy itself (the matvec and small-batch kernels
// store each output once, with plain stores), so no device-to-host copy is
// queued.
template <class F>
int run_host(Ctx& c, const float* x, long nx, float* y, long ny, int in_dim, int rows, bool sums, F&& launch,
             bool y_host = false) {
  if (c.init()) return -1;
  if (c.dx.ensure((size_t)nx, "hipMalloc x") || (!y_host && c.dy.ensure((size_t)ny, "hipMalloc y")) ||
      c.dq.ensure((size_t)(nx / 16 + 1), "hipMalloc xsum") || c.hx.ensure((size_t)nx, "pinned x") ||
      c.hy.ensure((size_t)ny, "pinned y"))
    return -1;
  std::memcpy(c.hx.p, x, (size_t)nx * sizeof(float));
  if (nx % 4 == 0) {
    const int n4 = (int)(nx / 4);
    hipLaunchKernelGGL(stage_copy, dim3(std::min(64, (n4 + 255) / 256)), dim3(256), 0, c.st,
                       (const float4*)c.hx.p, (float4*)c.dx.p, n4);
    if (check(hipGetLastError(), "stage x")) return -1;
  } else if (check(hipMemcpyAsync(c.dx.p, c.hx.p, (size_t)nx * sizeof(float), hipMemcpyHostToDevice, c.st), "H2D x"))
    return -1;
  if (sums && check(kq::launch_xsum(c.dx.p, in_dim, rows, c.dq.p, c.st), "xsum launch")) return -1;
  if (check(launch(), "kernel launch")) return -1;
  if (!y_host &&
      check(hipMemcpyAsync(c.hy.p, c.dy.p, (size_t)ny * sizeof(float), hipMemcpyDeviceToHost, c.st), "D2H y"))
    return -1;
  if (check(hipStreamSynchronize(c.st), "hipStreamSynchronize")) return -1;
  std::memcpy(y, c.hy.p, (size_t)ny * sizeof(float));
  return 0;
}

}  // namespace

namespace kq {
// Errors of the resident model chain (kq_model_chain.hip), recorded like this
// file's own.
void abi_report(int code, const char* what) { report(code, "%s", what); }
}  // namespace kq

// =============================================================================
// Reference ABI
// =============================================================================

extern "C" void aspida_gpu_matvec(const void* w, long wbytes, int kind, int in_dim, int out_dim,
                                  const float* x, float* y) {
  if (validate_mv("aspida_gpu_matvec", w, wbytes, kind, in_dim, out_dim, 1, x, y)) {
    fill_nan(y, out_dim);
    return;
  }
  std::shared_lock<std::shared_mutex> rd(g_wmu, std::defer_lock);
  WReq req = packed_req(w, kind, in_dim, out_dim);
  Ctx& c = ctx();
  int rc = acquire(rd, &req, 1);
  if (!rc) rc = c.init() || c.ws.ensure(in_dim, out_dim) ? -1 : 0;
  if (!rc)
    rc = run_host(c, x, in_dim, y, out_dim, in_dim, 1, false, [&]() {
      return kq::launch_matvec_packed(kind, req.d, in_dim, out_dim, c.dx.p, c.hy.p, c.ws.part.p, c.ws.count.p, c.st);
    }, true);
  if (rc) fill_nan(y, out_dim);
}

extern "C" void aspida_gpu_matmul(const void* w, long wbytes, int kind, int in_dim, int out_dim, int batch,
                                  const float* x, float* y) {
  if (batch < 1) return;  // nothing to compute (gpu_matvec.cu:538)
  if (validate_mv("aspida_gpu_matmul", w, wbytes, kind, in_dim, out_dim, batch, x, y)) {
    fill_nan(y, (long)out_dim * batch);
    return;
  }
  Ctx& c = ctx();
  // Packed HBM mirror (shared with aspida_gpu_matvec): the multi-vector VALU
  // kernel up to 8 vectors at a time, MFMA for larger Q4_K / Q6_K batches.
  std::shared_lock<std::shared_mutex> rd(g_wmu, std::defer_lock);
  WReq req = packed_req(w, kind, in_dim, out_dim);
  int rc = acquire(rd, &req, 1);
  if (!rc) rc = c.init() || c.ws.ensure(in_dim, out_dim, batch) ? -1 : 0;
  if (!rc)
    rc = run_host(c, x, (long)in_dim * batch, y, (long)out_dim * batch, in_dim, batch, false, [&]() {
      return matmul_packed(kind, req.d, in_dim, out_dim, batch, c.dx.p, c.hy.p, c.ws, c.st);
    }, true);
  if (rc) fill_nan(y, (long)out_dim * batch);
}

extern "C" void aspida_gpu_dense_matvec(const void* w, long wbytes, int in_dim, int out_dim, const float* x,
                                        float* y) {
  if (!w || !x || !y || in_dim <= 0 || out_dim <= 0 || wbytes < (long)in_dim * out_dim * 4) {
    report(-EINVAL, "aspida_gpu_dense_matvec: bad arguments (in=%d out=%d wbytes=%ld)", in_dim, out_dim, wbytes);
    fill_nan(y, out_dim);
    return;
  }
  std::shared_lock<std::shared_mutex> rd(g_wmu, std::defer_lock);
  WReq req = ggml_req(w, (long)in_dim * out_dim * 4);
  Ctx& c = ctx();
  int rc = acquire(rd, &req, 1);
  if (!rc) {
    if (c.init() || c.dx.ensure((size_t)in_dim, "hipMalloc x") || c.dy.ensure((size_t)out_dim, "hipMalloc y") ||
        c.hx.ensure((size_t)in_dim, "pinned x") || c.hy.ensure((size_t)out_dim, "pinned y"))
      rc = -1;
  }
  if (!rc) {
    std::memcpy(c.hx.p, x, (size_t)in_dim * 4);
    rc = check(hipMemcpyAsync(c.dx.p, c.hx.p, (size_t)in_dim * 4, hipMemcpyHostToDevice, c.st), "H2D x");
    if (!rc) rc = check(kq::launch_dense((const float*)req.d, in_dim, out_dim, c.dx.p, c.dy.p, c.st), "dense");
    if (!rc) rc = check(hipMemcpyAsync(c.hy.p, c.dy.p, (size_t)out_dim * 4, hipMemcpyDeviceToHost, c.st), "D2H");
    if (!rc) rc = check(hipStreamSynchronize(c.st), "sync");
    if (!rc) std::memcpy(y, c.hy.p, (size_t)out_dim * 4);
  }
  if (rc) fill_nan(y, out_dim);
}

// Waits (exclusive lock) for every host-ABI call that holds a mirror of w.
extern "C" void aspida_gpu_free_weight(const void* w) {
  std::unique_lock<std::shared_mutex> wr(g_wmu);
  auto it = g_wcache.find(w);
  if (it != g_wcache.end()) {
    (void)hipFree(it->second.d);
    g_wcache.erase(it);
  }
  auto pt = g_pcache.find(w);
  if (pt != g_pcache.end()) {
    (void)hipFree(pt->second.d);
    g_pcache.erase(pt);
  }
}

extern "C" void aspida_gpu_moe_experts(const float* x, int dim, int top_k, int intermed, int n_exp,
                                       const int* top_idx, const float* top_w, const void* gate_w,
                                       long gate_bytes, int gate_kind, const void* up_w, long up_bytes,
                                       int up_kind, const void* down_w, long down_bytes, int down_kind,
                                       const void* shg_w, long shg_bytes, int shg_kind, const void* shu_w,
                                       long shu_bytes, int shu_kind, const void* shd_w, long shd_bytes,
                                       int shd_kind, const float* shared_gate_inp, int gate_inp_len,
                                       float* y) {
  const char* fn = "aspida_gpu_moe_experts";
  if (!x || !y || !top_idx || !top_w || !gate_w || !up_w || !down_w || !shg_w || !shu_w || !shd_w) {
    report(-EINVAL, "%s: null pointer argument", fn);
    fill_nan(y, dim);
    return;
  }
  const int kinds[6] = {gate_kind, up_kind, down_kind, shg_kind, shu_kind, shd_kind};
  bool ok = dim > 0 && intermed > 0 && n_exp > 0 && top_k > 0 && top_k <= n_exp && top_k <= kq::MOE_MAX_TOPK &&
            dim % 256 == 0 && intermed % 256 == 0;
  for (int k : kinds) ok = ok && valid_kind(k);
  if (ok) {
    const long gb = need_bytes(gate_kind, dim, intermed), ub = need_bytes(up_kind, dim, intermed),
               db = need_bytes(down_kind, intermed, dim);
    ok = gate_bytes / n_exp >= gb && up_bytes / n_exp >= ub && down_bytes / n_exp >= db &&
         shg_bytes >= need_bytes(shg_kind, dim, intermed) && shu_bytes >= need_bytes(shu_kind, dim, intermed) &&
         shd_bytes >= need_bytes(shd_kind, intermed, dim);
  }
  if (ok)
    for (int k = 0; k < top_k; ++k) ok = ok && top_idx[k] >= 0 && top_idx[k] < n_exp;
  if (!ok) {
    report(-EINVAL, "%s: bad arguments (dim=%d intermed=%d n_exp=%d top_k=%d)", fn, dim, intermed, n_exp, top_k);
    fill_nan(y, dim);
    return;
  }
  Ctx& c = ctx();
  const bool gated = gate_inp_len > 1 && shared_gate_inp;
  // Per call, one pinned buffer and one copy carry x | top_w | top_idx and,
  // when gated, the shared gate's input vector.  That vector is not a cached
  // weight: the Ada host never frees it through aspida_gpu_free_weight
  // (LLM_MoE.Free, src/llm/llm_moe.adb:74-79), so a mirror keyed by its
  // address could outlive it.
  const size_t nstage = (size_t)dim + 2 * top_k + (gated ? (size_t)dim : 0);
  const size_t stage = (nstage + 63) & ~(size_t)63;
  auto stage_inputs = [&]() {
    std::memcpy(c.hx.p, x, (size_t)dim * 4);
    std::memcpy(c.hx.p + dim, top_w, (size_t)top_k * 4);
    std::memcpy(c.hx.p + dim + top_k, top_idx, (size_t)top_k * 4);
    if (gated) std::memcpy(c.hx.p + dim + 2 * top_k, shared_gate_inp, (size_t)dim * 4);
    // The stage is a whole number of float4s (64-float aligned; the pinned
    // buffer is allocated to that length), copied by the GPU (stage_copy).
    const int n4 = (int)(stage / 4);
    hipLaunchKernelGGL(stage_copy, dim3(std::min(64, (n4 + 255) / 256)), dim3(256), 0, c.st, (const float4*)c.hx.p,
                       (float4*)c.dh.p, n4);
    return check(hipGetLastError(), "stage inputs");
  };
  std::shared_lock<std::shared_mutex> rd(g_wmu, std::defer_lock);
  // Grouped path over packed experts when gate, up and the shared gate/up
  // share one kind and both downs another (the Q4_K_M layouts do).
  if (gate_kind == up_kind && shg_kind == gate_kind && shu_kind == gate_kind && shd_kind == down_kind &&
      kq::moe_grouped_supported(dim, intermed, 1, top_k) && kq::moe_grouped_experts_ok(n_exp)) {
    // The per-expert stride of the host tensors is bytes / n_exp (gpu_matvec.cu:1702-1703).
    WReq req[6] = {packed_req(gate_w, gate_kind, dim, intermed, n_exp, (size_t)(gate_bytes / n_exp)),
                   packed_req(up_w, up_kind, dim, intermed, n_exp, (size_t)(up_bytes / n_exp)),
                   packed_req(down_w, down_kind, intermed, dim, n_exp, (size_t)(down_bytes / n_exp)),
                   packed_req(shg_w, shg_kind, dim, intermed), packed_req(shu_w, shu_kind, dim, intermed),
                   packed_req(shd_w, shd_kind, intermed, dim)};
    int rc = acquire(rd, req, 6);
    kq::MoeGroupedArgs a{};
    a.gate = (const uint8_t*)req[0].d;
    a.up = (const uint8_t*)req[1].d;
    a.down = (const uint8_t*)req[2].d;
    a.sh_gate = (const uint8_t*)req[3].d;
    a.sh_up = (const uint8_t*)req[4].d;
    a.sh_down = (const uint8_t*)req[5].d;
    a.gu_stride = kq::packed_bytes(gate_kind, dim, intermed);
    a.d_stride = kq::packed_bytes(down_kind, intermed, dim);
    a.T = 1; a.top_k = top_k; a.n_exp = n_exp; a.dim = dim; a.I = intermed;
    // The staged inputs, then the grouped work on a 256-byte boundary.
    const size_t scratch = stage + (kq::moe_grouped_work_bytes(1, dim, intermed, top_k) + 3) / 4;
    if (!rc && (c.init() || c.dy.ensure((size_t)dim, "hipMalloc y") || c.dh.ensure(scratch, "hipMalloc moe scratch") ||
                c.hx.ensure(stage, "pinned x") || c.hy.ensure((size_t)dim, "pinned y")))
      rc = -1;
    if (!rc) {
      rc = stage_inputs();
      if (!rc) {
        a.x = c.dh.p;
        a.top_w = c.dh.p + dim;
        a.idx = (const int*)(c.dh.p + dim + top_k);
        a.sgi = gated ? c.dh.p + dim + 2 * top_k : nullptr;
        a.y = c.dy.p;
        kq::moe_grouped_bind(a, c.dh.p + stage);
        rc = check(kq::launch_moe_grouped(a, gate_kind, down_kind, c.st), "moe launch");
      }
      if (!rc) rc = check(hipMemcpyAsync(c.hy.p, c.dy.p, (size_t)dim * 4, hipMemcpyDeviceToHost, c.st), "D2H");
      if (!rc) rc = check(hipStreamSynchronize(c.st), "sync");
      if (!rc) std::memcpy(y, c.hy.p, (size_t)dim * 4);
    }
    if (rc) fill_nan(y, dim);
    return;
  }
  // The per-expert stride is bytes / n_exp (gpu_matvec.cu:1702-1703).
  WReq req[6] = {ggml_req(gate_w, gate_bytes), ggml_req(up_w, up_bytes),   ggml_req(down_w, down_bytes),
                 ggml_req(shg_w, shg_bytes),   ggml_req(shu_w, shu_bytes), ggml_req(shd_w, shd_bytes)};
  int rc = acquire(rd, req, 6);
  kq::MoeWeights mw;
  mw.gate = (const uint8_t*)req[0].d;
  mw.up = (const uint8_t*)req[1].d;
  mw.down = (const uint8_t*)req[2].d;
  mw.sh_gate = (const uint8_t*)req[3].d;
  mw.sh_up = (const uint8_t*)req[4].d;
  mw.sh_down = (const uint8_t*)req[5].d;
  mw.gate_stride = gate_bytes / n_exp;
  mw.up_stride = up_bytes / n_exp;
  mw.down_stride = down_bytes / n_exp;
  mw.gate_kind = gate_kind; mw.up_kind = up_kind; mw.down_kind = down_kind;
  mw.sh_gate_kind = shg_kind; mw.sh_up_kind = shu_kind; mw.sh_down_kind = shd_kind;
  mw.dim = dim; mw.intermed = intermed; mw.n_exp = n_exp;
  // The per-slot work follows the staged inputs (moe_staging_floats of them
  // are set aside at the front of the scratch).
  const size_t front = std::max(stage, kq::moe_staging_floats(dim, 1, top_k));
  const size_t scratch = front + kq::moe_scratch_floats(mw, 1, top_k) - kq::moe_staging_floats(dim, 1, top_k);
  if (!rc && (c.init() || c.dy.ensure((size_t)dim, "hipMalloc y") || c.dh.ensure(scratch, "hipMalloc moe scratch") ||
              c.hx.ensure(stage, "pinned x") || c.hy.ensure((size_t)dim, "pinned y")))
    rc = -1;
  if (!rc) {
    rc = stage_inputs();
    if (!rc) {
      const float* dxx = c.dh.p;
      const float* dtw = c.dh.p + dim;
      const int* dti = (const int*)(c.dh.p + dim + top_k);
      const float* dsgi = gated ? c.dh.p + dim + 2 * top_k : nullptr;
      float* work = c.dh.p + front;
      rc = check(kq::launch_moe_experts(mw, 1, top_k, dxx, dti, dtw, dsgi, work, c.dy.p, c.st), "moe launch");
    }
    if (!rc) rc = check(hipMemcpyAsync(c.hy.p, c.dy.p, (size_t)dim * 4, hipMemcpyDeviceToHost, c.st), "D2H");
    if (!rc) rc = check(hipStreamSynchronize(c.st), "sync");
    if (!rc) std::memcpy(y, c.hy.p, (size_t)dim * 4);
  }
  if (rc) fill_nan(y, dim);
}

extern "C" int aspida_gpu_last_error(void) {
  const int e = t_last_error;
  t_last_error = 0;
  return e;
}

// =============================================================================
// Device-pointer entry points (activations already in HBM; asynchronous on
// `stream`, which may be NULL for the null stream).
// =============================================================================

extern "C" int aspida_kq_xsum_dev(const float* x, int in_dim, int rows, float* xq, void* stream) {
  if (!x || !xq || in_dim <= 0 || in_dim % 16 || rows <= 0) return -EINVAL;
  return check(kq::launch_xsum(x, in_dim, rows, xq, (hipStream_t)stream), "aspida_kq_xsum_dev");
}

extern "C" int aspida_kq_matvec_dev(int kind, const void* w, int in_dim, int out_dim, const float* x,
                                    const float* xq, float* y, void* stream) {
  if (!w || !x || !xq || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0) return -EINVAL;
  const kq::MvConfig cfg = mv_config(kind, in_dim, out_dim);
  return check(kq::launch_matvec(kind, w, in_dim, out_dim, x, xq, y, (hipStream_t)stream, cfg),
               "aspida_kq_matvec_dev");
}

extern "C" long long aspida_kq_packed_bytes(int kind, int in_dim, int out_dim) {
  if (!valid_kind(kind)) return 0;
  return (long long)kq::packed_bytes(kind, in_dim, out_dim);
}

extern "C" int aspida_kq_packed_plan(int in_dim, int out_dim, int* waves_per_group, int* groups_per_tile,
                                     int* columns_per_wave) {
  if (in_dim <= 0 || in_dim % 256 || out_dim <= 0 || !waves_per_group || !groups_per_tile || !columns_per_wave)
    return -EINVAL;
  const kq::PackedPlan p = kq::packed_plan(in_dim, out_dim);
  *waves_per_group = p.nw;
  *groups_per_tile = p.ks;
  *columns_per_wave = p.spw;
  return 0;
}

extern "C" int aspida_kq_matvec_plan(int kind, int in_dim, int out_dim, int* waves_per_group, int* groups_per_tile,
                                     int* columns_per_wave) {
  if (!valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || !waves_per_group || !groups_per_tile ||
      !columns_per_wave)
    return -EINVAL;
  const bool mfma = kq::matvec_mfma_takes(kind);
  const kq::PackedPlan p = mfma ? kq::mfma_plan(kind, in_dim, out_dim) : kq::packed_plan(in_dim, out_dim);
  *waves_per_group = p.nw;
  *groups_per_tile = p.ks;
  *columns_per_wave = p.spw;
  if (!mfma) return 0;
  const int seq = p.seq && p.spw > 1 ? 1 : 0;
  return p.blk16 ? 3 + seq : 1 + seq;
}

extern "C" int aspida_kq_pack_dev(int kind, const void* w, int in_dim, int out_dim, void* packed, void* stream) {
  if (!w || !packed || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0) return -EINVAL;
  return check(kq::launch_pack(kind, w, in_dim, out_dim, packed, false, (hipStream_t)stream), "aspida_kq_pack_dev");
}

extern "C" int aspida_kq_unpack_dev(int kind, const void* packed, int in_dim, int out_dim, void* w, void* stream) {
  if (!w || !packed || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0) return -EINVAL;
  return check(kq::launch_pack(kind, packed, in_dim, out_dim, w, true, (hipStream_t)stream),
               "aspida_kq_unpack_dev");
}

namespace {
// Packed-matvec workspaces of the device entry point, one per stream.
std::mutex g_ws_mu;
std::unordered_map<void*, MvWorkspace*> g_ws;
}  // namespace

static MvWorkspace* stream_workspace(void* stream, int in_dim, int out_dim, int batch) {
  std::lock_guard<std::mutex> lk(g_ws_mu);
  MvWorkspace*& slot = g_ws[stream];
  if (!slot) slot = new MvWorkspace();
  if (slot->ensure(in_dim, out_dim, batch)) return nullptr;
  return slot;
}

extern "C" int aspida_kq_matmul_packed_dev(int kind, const void* packed, int in_dim, int out_dim, int batch,
                                           const float* x, float* y, void* stream) {
  if (!packed || !x || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || batch <= 0 ||
      ((uintptr_t)x & 15))
    return -EINVAL;
  MvWorkspace* ws = stream_workspace(stream, in_dim, out_dim, batch);
  if (!ws) return t_last_error ? t_last_error : -1;
  return check(matmul_packed(kind, packed, in_dim, out_dim, batch, x, y, *ws, (hipStream_t)stream),
               "aspida_kq_matmul_packed_dev");
}

extern "C" int aspida_kq_matvec2_packed_dev(int kind_a, const void* packed_a, int out_a, float* y_a, int kind_b,
                                            const void* packed_b, int out_b, float* y_b, int in_dim, const float* x,
                                            void* stream) {
  if (!packed_a || !packed_b || !x || !y_a || !y_b || !valid_kind(kind_a) || !valid_kind(kind_b) || in_dim <= 0 ||
      in_dim % 256 || out_a <= 0 || out_b <= 0 || ((uintptr_t)x & 15))
    return -EINVAL;
  const int rows = ((out_a + 63) / 64 + (out_b + 63) / 64) * 64;
  MvWorkspace* ws = stream_workspace(stream, in_dim, rows, 1);
  if (!ws) return t_last_error ? t_last_error : -1;
  const hipStream_t st = (hipStream_t)stream;
  if (kq::matvec2_supported(kind_a, kind_b))
    return check(kq::launch_matvec2_packed(kind_a, packed_a, out_a, y_a, kind_b, packed_b, out_b, y_b, in_dim, x,
                                           ws->part.p, ws->count.p, st),
                 "aspida_kq_matvec2_packed_dev");
  hipError_t e = kq::launch_matvec_packed(kind_a, packed_a, in_dim, out_a, x, y_a, ws->part.p, ws->count.p, st);
  if (e == hipSuccess)
    e = kq::launch_matvec_packed(kind_b, packed_b, in_dim, out_b, x, y_b, ws->part.p, ws->count.p, st);
  return check(e, "aspida_kq_matvec2_packed_dev");
}

extern "C" int aspida_kq_matvec_packed_dev(int kind, const void* packed, int in_dim, int out_dim, const float* x,
                                           float* y, void* stream) {
  if (!packed || !x || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 ||
      ((uintptr_t)x & 15))
    return -EINVAL;
  MvWorkspace* ws = stream_workspace(stream, in_dim, out_dim, 1);
  if (!ws) return t_last_error ? t_last_error : -1;
  return check(kq::launch_matvec_packed(kind, packed, in_dim, out_dim, x, y, ws->part.p, ws->count.p,
                                        (hipStream_t)stream),
               "aspida_kq_matvec_packed_dev");
}

// ---- allocation-free batch-1 matvec --------------------------------------------
//
// aspida_kq_matvec_packed_noalloc_dev runs aspida_kq_matvec_packed_dev's
// kernels with their workspace in `scratch`, a fixed device array of this
// library (one copy per GPU, held until the process ends), so a call never
// allocates: for code under HIP graph capture, tight serving loops and
// harnesses that forbid hipMalloc.  Layout: per-tile arrival counters, then
// the cross-workgroup partial sums.
constexpr size_t NOALLOC_COUNTER_BYTES = (size_t)1 << 20;  // 4096 64-row tiles (262,144 rows)
constexpr size_t NOALLOC_PART_BYTES = (size_t)5 << 20;     // 1,310,720 partial sums
constexpr size_t NOALLOC_SCRATCH_BYTES = NOALLOC_COUNTER_BYTES + NOALLOC_PART_BYTES;
static __device__ __align__(256) uint8_t scratch[NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int NOALLOC_MAX_DEVICES = 64;

// `scratch`'s device address on each GPU (its host-side name is not one).
struct NoAllocDevice {
  std::once_flag once;
  void* ptr = nullptr;
  hipError_t err = hipSuccess;
};
NoAllocDevice g_noalloc[NOALLOC_MAX_DEVICES];

// The current device's copy of `scratch`, looked up once per device with that
// device current; null (and t_last_error set) on failure.
void* noalloc_scratch() {
  int dev = -1;
  if (check(hipGetDevice(&dev), "aspida_kq_matvec_packed_noalloc_dev: hipGetDevice")) return nullptr;
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    report(-ENODEV, "aspida_kq_matvec_packed_noalloc_dev: device %d beyond the %d supported", dev,
           NOALLOC_MAX_DEVICES);
    return nullptr;
  }
  NoAllocDevice& d = g_noalloc[dev];
  std::call_once(d.once, [&d]() {
    void* p = nullptr;
    d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (d.err == hipSuccess) d.ptr = p;
  });
  if (d.err != hipSuccess) {
    check(d.err, "aspida_kq_matvec_packed_noalloc_dev: hipGetSymbolAddress(scratch)");
    return nullptr;
  }
  return d.ptr;
}

__global__ void fill_u32(unsigned* __restrict__ p, unsigned v, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

}  // namespace

extern "C" int aspida_kq_matvec_packed_noalloc_dev(int kind, const void* packed, int in_dim, int out_dim,
                                                   const float* x, float* y, void* stream) {
  const char* fn = "aspida_kq_matvec_packed_noalloc_dev";
  if (!packed || !x || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 ||
      ((uintptr_t)x & 15))
    return -EINVAL;
  const size_t ncount = kq::packed_counters(out_dim);
  const size_t npart = kq::packed_workspace_floats(in_dim, out_dim);
  if (ncount * sizeof(unsigned) > NOALLOC_COUNTER_BYTES || npart * sizeof(float) > NOALLOC_PART_BYTES) {
    report(-E2BIG, "%s: %d x %d needs %zu counter and %zu partial-sum bytes; the fixed scratch holds %zu and %zu",
           fn, out_dim, in_dim, ncount * sizeof(unsigned), npart * sizeof(float), NOALLOC_COUNTER_BYTES,
           NOALLOC_PART_BYTES);
    return -E2BIG;
  }
  uint8_t* base = (uint8_t*)noalloc_scratch();
  if (!base) return t_last_error ? t_last_error : -1;
  unsigned* count = (unsigned*)base;
  float* part = (float*)(base + NOALLOC_COUNTER_BYTES);
  const hipStream_t st = (hipStream_t)stream;
  // The arrival counters must be zero when the launch starts.  Every launch
  // leaves them zero, but the array is shared with every other call on this
  // GPU, so they are cleared here -- with a kernel, not a memset node, so the
  // call may be captured into a HIP graph -- whenever the launch splits a
  // tile over workgroups (the only case that uses them).
  const bool mfma = kq::matvec_mfma_takes(kind);
  const kq::PackedPlan p = mfma ? kq::mfma_plan(kind, in_dim, out_dim) : kq::packed_plan(in_dim, out_dim);
  if (p.ks > 1 && !p.blk16) {
    const int blocks = (int)std::min<size_t>((ncount + 255) / 256, 1024);
    hipLaunchKernelGGL(fill_u32, dim3(blocks), dim3(256), 0, st, count, 0u, ncount);
    if (check(hipGetLastError(), fn)) return t_last_error;
  }
  return check(kq::launch_matvec_packed(kind, packed, in_dim, out_dim, x, y, part, count, st), fn);
}

extern "C" int aspida_kq_matmul_dev(int kind, const void* w, int in_dim, int out_dim, int batch, const float* x,
                                    const float* xq, float* y, void* stream) {
  if (!w || !x || !xq || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || batch <= 0)
    return -EINVAL;
  hipError_t e = kq::launch_matmul_mfma(kind, w, in_dim, out_dim, batch, x, y, (hipStream_t)stream);
  if (e == hipErrorNotSupported)
    e = kq::launch_matmul_valu(kind, w, in_dim, out_dim, batch, x, xq, y, (hipStream_t)stream);
  return check(e, "aspida_kq_matmul_dev");
}

extern "C" int aspida_kq_matmul_valu_dev(int kind, const void* w, int in_dim, int out_dim, int batch,
                                         const float* x, const float* xq, float* y, void* stream) {
  if (!w || !x || !xq || !y || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || batch <= 0)
    return -EINVAL;
  return check(kq::launch_matmul_valu(kind, w, in_dim, out_dim, batch, x, xq, y, (hipStream_t)stream),
               "aspida_kq_matmul_valu_dev");
}

extern "C" int aspida_kq_dequant_dev(int kind, const void* w, int in_dim, int out_dim, float* dst, void* stream) {
  if (!w || !dst || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0) return -EINVAL;
  return check(kq::launch_dequant(kind, w, in_dim, out_dim, dst, (hipStream_t)stream), "aspida_kq_dequant_dev");
}

extern "C" int aspida_dense_matvec_dev(const float* w, int in_dim, int out_dim, const float* x, float* y,
                                       void* stream) {
  if (!w || !x || !y || in_dim <= 0 || out_dim <= 0) return -EINVAL;
  return check(kq::launch_dense(w, in_dim, out_dim, x, y, (hipStream_t)stream), "aspida_dense_matvec_dev");
}

extern "C" int aspida_moe_route_dev(const float* router_w, int n_exp, int dim, int T, int top_k, const float* x,
                                    float* logits, int* top_idx, float* top_w, void* stream) {
  if (!router_w || !x || !logits || !top_idx || !top_w || n_exp <= 0 || dim <= 0 || dim % 4 || T <= 0 ||
      top_k <= 0 || ((uintptr_t)router_w & 15) || ((uintptr_t)x & 15))
    return -EINVAL;
  // Arrival counters from the stream's matvec workspace (one per 64 "rows",
  // kept zero between launches).
  MvWorkspace* ws = stream_workspace(stream, 256, kq::moe_route_groups(T) * 64, 1);
  if (!ws) return t_last_error ? t_last_error : -1;
  return check(kq::launch_moe_route(router_w, n_exp, dim, T, top_k, x, logits, top_idx, top_w, ws->count.p,
                                    (hipStream_t)stream),
               "aspida_moe_route_dev");
}

namespace kq {
// The model chain's router step with the post-attention norm in the same
// launch (launch_moe_route_norm): 0, -ENOTSUP when the shape does not take
// it, or the error.
int route_norm_dev(const float* router_w, int n_exp, int dim, int T, int top_k, float* H, const float* r,
                   const float* r2, const float* g, float* nx, float* logits, int* top_idx, float* top_w,
                   void* stream) {
  if (!moe_route_norm_takes(n_exp, dim, T, top_k)) return -ENOTSUP;
  if (!router_w || !H || !g || !nx || !logits || !top_idx || !top_w || ((uintptr_t)router_w & 15) ||
      ((uintptr_t)H & 15) || ((uintptr_t)nx & 15) || ((uintptr_t)g & 15) || (r && ((uintptr_t)r & 15)) ||
      (r2 && ((uintptr_t)r2 & 15)))
    return -EINVAL;
  MvWorkspace* ws = stream_workspace(stream, 256, moe_route_groups(T) * 64, 1);
  if (!ws) return t_last_error ? t_last_error : -1;
  return check(launch_moe_route_norm(router_w, n_exp, dim, T, top_k, H, r, r2, g, nx, logits, top_idx, top_w,
                                     ws->count.p, (hipStream_t)stream),
               "chain router with norm");
}

// The model chain's one-lane mixer with the attention norm in the same
// launch (launch_matvec_norm): 0, -ENOTSUP when the shape does not take it,
// or the error.
int matvec_norm_dev(int kind, const void* P, int in_dim, int out_dim, const float* H, const float* r, const float* g,
                    float* y, void* stream) {
  if (!matvec_norm_takes(kind, in_dim, out_dim)) return -ENOTSUP;
  if (!P || !H || !g || !y || ((uintptr_t)H & 15) || ((uintptr_t)g & 15) || (r && ((uintptr_t)r & 15)))
    return -EINVAL;
  return check(launch_matvec_norm(kind, P, in_dim, out_dim, H, r, g, y, (hipStream_t)stream), "chain mixer with norm");
}
}  // namespace kq

extern "C" long aspida_moe_work_floats(int T, int dim, int top_k, int intermed) {
  kq::MoeWeights w;
  w.dim = dim;
  w.intermed = intermed;
  return (long)kq::moe_scratch_floats(w, T, top_k);
}

extern "C" int aspida_moe_experts_dev(const float* x, int T, int dim, int top_k, int intermed, int n_exp,
                                      const int* top_idx, const float* top_w, const void* gate_w, long gate_stride,
                                      int gate_kind, const void* up_w, long up_stride, int up_kind,
                                      const void* down_w, long down_stride, int down_kind, const void* shg_w,
                                      int shg_kind, const void* shu_w, int shu_kind, const void* shd_w,
                                      int shd_kind, const float* shared_gate_inp, float* work, float* y,
                                      void* stream) {
  const int kinds[6] = {gate_kind, up_kind, down_kind, shg_kind, shu_kind, shd_kind};
  bool ok = x && top_idx && top_w && gate_w && up_w && down_w && shg_w && shu_w && shd_w && work && y && T > 0 &&
            dim > 0 && intermed > 0 && dim % 256 == 0 && intermed % 256 == 0 && top_k > 0 && top_k <= n_exp &&
            top_k <= kq::MOE_MAX_TOPK;
  for (int k : kinds) ok = ok && valid_kind(k);
  if (!ok) return -EINVAL;
  kq::MoeWeights mw;
  mw.gate = (const uint8_t*)gate_w; mw.up = (const uint8_t*)up_w; mw.down = (const uint8_t*)down_w;
  mw.sh_gate = (const uint8_t*)shg_w; mw.sh_up = (const uint8_t*)shu_w; mw.sh_down = (const uint8_t*)shd_w;
  mw.gate_stride = gate_stride; mw.up_stride = up_stride; mw.down_stride = down_stride;
  mw.gate_kind = gate_kind; mw.up_kind = up_kind; mw.down_kind = down_kind;
  mw.sh_gate_kind = shg_kind; mw.sh_up_kind = shu_kind; mw.sh_down_kind = shd_kind;
  mw.dim = dim; mw.intermed = intermed; mw.n_exp = n_exp;
  // The staging prefix of the work layout is only used by the host ABI.
  float* wk = work + kq::moe_staging_floats(dim, T, top_k);
  return check(kq::launch_moe_experts(mw, T, top_k, x, top_idx, top_w, shared_gate_inp, wk, y,
                                      (hipStream_t)stream),
               "aspida_moe_experts_dev");
}

// Tokens per grouped launch: every expert lists at most MOE_MAX_JOBS jobs.
static int moe_chunk(int T, int top_k) { return std::min(T, kq::MOE_MAX_JOBS / top_k); }

extern "C" long aspida_moe_packed_work_bytes(int T, int dim, int intermed, int top_k) {
  if (T <= 0 || dim <= 0 || intermed <= 0 || top_k <= 0 || top_k > kq::MOE_MAX_TOPK) return -EINVAL;
  size_t n = kq::moe_grouped_work_bytes(moe_chunk(T, top_k), dim, intermed, top_k);
  // From MOE_PREFILL_MIN_TOKENS tokens the Q4_K / Q6_K experts may take the
  // prefill products, in launch sequences of up to MOE_PREFILL_MAX_TOKENS.
  if (T >= kq::MOE_PREFILL_MIN_TOKENS && dim % 256 == 0 && intermed % 256 == 0)
    n = std::max(n, kq::moe_prefill_work_bytes(std::min(T, kq::MOE_PREFILL_MAX_TOKENS), dim, intermed, top_k));
  return (long)n;
}

extern "C" int aspida_moe_pack_experts_dev(int kind, const void* src, long src_stride, int in_dim, int out_dim,
                                           int n, void* dst, void* stream) {
  if (!src || !dst || !valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || n <= 0 ||
      src_stride < need_bytes(kind, in_dim, out_dim))
    return -EINVAL;
  const size_t pb = kq::packed_bytes(kind, in_dim, out_dim);
  for (int i = 0; i < n; ++i) {
    const int rc = check(kq::launch_pack(kind, (const uint8_t*)src + (size_t)src_stride * i, in_dim, out_dim,
                                         (uint8_t*)dst + pb * i, false, (hipStream_t)stream),
                         "aspida_moe_pack_experts_dev");
    if (rc) return rc;
  }
  return 0;
}

extern "C" int aspida_moe_experts_packed_dev(const float* x, int T, int dim, int top_k, int intermed, int n_exp,
                                             const int* top_idx, const float* top_w, const void* gate_p,
                                             const void* up_p, int gu_kind, const void* down_p, int down_kind,
                                             const void* shg_p, const void* shu_p, const void* shd_p,
                                             const float* shared_gate_inp, void* work, float* y, void* stream) {
  return kq::moe_experts_packed_norm(x, T, dim, top_k, intermed, n_exp, top_idx, top_w, gate_p, up_p, gu_kind, down_p,
                                     down_kind, shg_p, shu_p, shd_p, shared_gate_inp, work, y, stream, nullptr,
                                     nullptr, nullptr, nullptr);
}

int kq::moe_experts_packed_norm(const float* x, int T, int dim, int top_k, int intermed, int n_exp,
                                const int* top_idx, const float* top_w, const void* gate_p, const void* up_p,
                                int gu_kind, const void* down_p, int down_kind, const void* shg_p, const void* shu_p,
                                const void* shd_p, const float* shared_gate_inp, void* work, float* y, void* stream,
                                float* norm_h, const float* norm_w, float* norm_nx, bool* norm_done) {
  if (norm_done) *norm_done = false;
  const bool ok = x && top_idx && top_w && gate_p && up_p && down_p && shg_p && shu_p && shd_p && work && y &&
                  valid_kind(gu_kind) && valid_kind(down_kind) && T > 0 && n_exp > 0 && top_k > 0 &&
                  top_k <= n_exp && kq::moe_grouped_supported(dim, intermed, 1, top_k) &&
                  kq::moe_grouped_experts_ok(n_exp) &&
                  ((uintptr_t)x & 15) == 0 && ((uintptr_t)work & 255) == 0;
  if (!ok) return -EINVAL;
  // An error left pending by earlier work on this thread is returned (and
  // recorded) as such before anything is launched: the call does no work, and
  // its return code and aspida_gpu_last_error agree.
  if (const hipError_t pend = hipGetLastError(); pend != hipSuccess) {
    report((int)pend, "aspida_moe_experts_packed_dev: error pending from earlier work: %s", hipGetErrorString(pend));
    return (int)pend;
  }
  kq::MoeGroupedArgs a{};
  a.gate = (const uint8_t*)gate_p; a.up = (const uint8_t*)up_p; a.down = (const uint8_t*)down_p;
  a.sh_gate = (const uint8_t*)shg_p; a.sh_up = (const uint8_t*)shu_p; a.sh_down = (const uint8_t*)shd_p;
  a.gu_stride = kq::packed_bytes(gu_kind, dim, intermed);
  a.d_stride = kq::packed_bytes(down_kind, intermed, dim);
  a.sgi = shared_gate_inp;
  a.top_k = top_k; a.n_exp = n_exp; a.dim = dim; a.I = intermed;
  if (kq::moe_prefill_takes(T, gu_kind, down_kind, dim, intermed, top_k, n_exp) && kq::matvec_mfma_takes(gu_kind) &&
      kq::matvec_mfma_takes(down_kind)) {
    // Many tokens: the grouped products of kq_moe_prefill.hip, in sequences of
    // up to MOE_PREFILL_MAX_TOKENS tokens (a last short one included).
    for (int t0 = 0; t0 < T; t0 += kq::MOE_PREFILL_MAX_TOKENS) {
      a.T = std::min(kq::MOE_PREFILL_MAX_TOKENS, T - t0);
      a.x = x + (size_t)t0 * dim;
      a.idx = top_idx + (size_t)t0 * top_k;
      a.top_w = top_w + (size_t)t0 * top_k;
      a.y = y + (size_t)t0 * dim;
      const int rc = check(kq::launch_moe_prefill(a, work, (hipStream_t)stream), "aspida_moe_experts_packed_dev");
      if (rc) return rc;
    }
    return 0;
  }
  const int chunk = moe_chunk(T, top_k);
  for (int t0 = 0; t0 < T; t0 += chunk) {
    a.T = std::min(chunk, T - t0);
    a.x = x + (size_t)t0 * dim;
    a.idx = top_idx + (size_t)t0 * top_k;
    a.top_w = top_w + (size_t)t0 * top_k;
    a.y = y + (size_t)t0 * dim;
    kq::moe_grouped_bind(a, work);
    // The norm goes into the combine only when every chunk's launch takes it.
    bool done = false;
    if (norm_h && norm_w && norm_nx && chunk >= T) {
      a.norm_h = norm_h + (size_t)t0 * dim;
      a.norm_w = norm_w;
      a.norm_nx = norm_nx + (size_t)t0 * dim;
      a.norm_done = &done;
    }
    const int rc = check(kq::launch_moe_grouped(a, gu_kind, down_kind, (hipStream_t)stream),
                         "aspida_moe_experts_packed_dev");
    if (rc) return rc;
    if (norm_done) *norm_done = done;
  }
  return 0;
}

extern "C" void* aspida_kq_chain_create(const aspida_kq_step* steps, int nsteps) {
  if (!steps || nsteps <= 0) {
    report(-EINVAL, "aspida_kq_chain_create: no steps");
    return nullptr;
  }
  std::vector<kq::ChainStepDesc> d((size_t)nsteps);
  for (int i = 0; i < nsteps; ++i) {
    if (!valid_kind(steps[i].kind)) {
      report(-EINVAL, "aspida_kq_chain_create: step %d: bad kind %d", i, steps[i].kind);
      return nullptr;
    }
    d[i] = {steps[i].kind, steps[i].in_dim, steps[i].out_dim, steps[i].packed, steps[i].x, steps[i].y};
  }
  kq::Chain* c = nullptr;
  const char* why = "";
  const hipError_t e = kq::chain_create(d.data(), nsteps, &c, &why);
  if (e != hipSuccess) {
    report((int)e, "aspida_kq_chain_create: %s (%s)", why, hipGetErrorString(e));
    return nullptr;
  }
  return c;
}

extern "C" int aspida_kq_chain_run(void* chain, void* stream) {
  if (!chain) return -EINVAL;
  return check(kq::chain_run((kq::Chain*)chain, (hipStream_t)stream), "aspida_kq_chain_run");
}

extern "C" int aspida_kq_chain_check(void* chain) {
  if (!chain) return -EINVAL;
  unsigned failed = 0;
  const int rc = check(kq::chain_check((kq::Chain*)chain, &failed), "aspida_kq_chain_check");
  return rc ? rc : (failed ? 1 : 0);
}

extern "C" int aspida_kq_chain_workgroups(void* chain) {
  return chain ? kq::chain_workgroups((kq::Chain*)chain) : -EINVAL;
}

extern "C" void aspida_kq_chain_destroy(void* chain) { kq::chain_destroy((kq::Chain*)chain); }

extern "C" int aspida_kq_matmul_workspace(int kind, int in_dim, int out_dim, int batch, long long* allocated,
                                          long long* needed) {
  if (!valid_kind(kind) || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || batch <= 0 || !allocated || !needed)
    return -EINVAL;
  *allocated = batch > 1 ? (long long)mm_work_bytes(in_dim, out_dim, batch) : 0;
  *needed = (long long)mm_launch_need(kind, in_dim, out_dim, batch);
  return 0;
}

extern "C" int aspida_kq_set_packed_plan(int waves_per_group, int groups_per_tile) {
  if (waves_per_group < 0 || groups_per_tile < 0) return -EINVAL;
  kq::set_packed_plan_override(waves_per_group, groups_per_tile);
  return 0;
}

extern "C" int aspida_kq_set_mfma_pipeline(int mode) {
  if (mode < 0 || mode > 2) return -EINVAL;
  kq::set_mfma_pipeline(mode);
  return 0;
}

extern "C" int aspida_kq_set_mfma_rows(int mode) {
  if (mode < 0 || mode > 2) return -EINVAL;
  kq::set_mfma_rows(mode);
  return 0;
}

extern "C" int aspida_kq_set_mv_engine(int engine) {
  if (engine < 0 || engine > 1) return -EINVAL;
  kq::set_matvec_engine(engine);
  return 0;
}

extern "C" int aspida_kq_set_mm_engine(int engine) {
  if (engine < 0 || engine > 6) return -EINVAL;
  g_mm_engine = engine;
  return 0;
}

extern "C" int aspida_kq_set_mv_config(int rows_per_wave, int waves_per_cu) {
  if (rows_per_wave > 0 && !(rows_per_wave == 1 || rows_per_wave == 2 || rows_per_wave == 4)) return -EINVAL;
  if (rows_per_wave > 0 && (waves_per_cu < 1 || waves_per_cu > 64)) return -EINVAL;
  g_cfg_rows = rows_per_wave;
  g_cfg_wpc = waves_per_cu;
  return 0;
}
