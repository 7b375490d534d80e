// kq_moe_prefill.hip -- the grouped MoE experts for many tokens at once
// (prefill chunks) on the matrix cores: a grouped GEMM over the experts'
// packed Q4_K gate / up and Q6_K down matrices, for Q4_K_M-style layers.
//
// Per launch sequence of up to PF_MAX_TOKENS tokens (LLM_MoE.Forward steps 4-5,
// src/llm/llm_moe.adb:249-299, for every token; the reference's prefill runs
// K-quant experts per token, gpu/gpu_matvec.cu:4237-4239):
//
//   kq_xsplit<32>   the tokens' activations as f16 hi / lo images (kq_mmq.h)
//   moe_pf_plan     one workgroup: every (token, slot) job bucketed by expert
//                   (shared expert first), cut into groups of up to BP jobs
//   moe_pf_gate_up  per (group, 64-row tile): gate and up rows of the group's
//                   expert against the group's activation rows, gathered by
//                   token; h[job][row] = silu(gate) * up
//   moe_pf_gates    the tokens' shared-expert gates g_t, one wave per token
//   kq_xsplit<16>   h as f16 hi / lo images, one row per job
//   moe_pf_down     per (group, 64-row tile of dim): yk[job][row] = down . h[job]
//   moe_pf_combine  y[t] = sum_k top_w[t][k] yk[t, k] (ascending k) +
//                   g_t yk[t, shared], g_t = sigmoid(shared_gate_inp . x_t)
//                   (1 without shared_gate_inp)
//
// Each product tile reads its 64 weight rows once for up to BP = 64 jobs, so
// the weights of an expert are read once per BP of its jobs rather than once
// per job, and the matrix cores do the f16 products with the small-batch
// arithmetic (exact integer codes, activations split into hi + lo; kq_mmq.h).
// Within an expert's bucket the jobs' order is not fixed (atomic placement),
// but every output element is one job's own dot product over all columns in
// a fixed order, and the combine sums in ascending k: the results are
// deterministic.
#include <math.h>

#include <algorithm>

#include "kq_kernels.h"
#include "kq_mmq.h"
#include "kq_moe.h"

namespace kq {

struct PfArgs {
  const uint8_t *gate, *up, *down, *sh_gate, *sh_up, *sh_down;
  size_t gu_stride, d_stride;
  const int* idx;
  const float *top_w, *x, *sgi;
  float* y;
  int T, top_k, n_exp, dim, I;
  // work
  _Float16 *xh, *xl, *xsh, *xsl;
  float* xinv;
  float* gsh;   // [T] shared-expert gates
  float* h;
  _Float16 *hh, *hl, *hsh, *hsl;
  float* hinv;
  float* yk;
  int* jobs;    // [T slots]: job = t slots + k, bucketed by expert position
  int4* units;  // [0].x = group count; [1 + c] = group c: {expert, first job (into jobs), job count, 0}
};

__device__ __forceinline__ int pf_expert_at(int p, int n_exp) { return p == 0 ? n_exp : p - 1; }

// ---- plan -------------------------------------------------------------------------

template <int BP>
__global__ __launch_bounds__(1024) void moe_pf_plan(PfArgs a) {
  __shared__ int cnt[MOE_MAX_EXP + 1], off[MOE_MAX_EXP + 2], coff[MOE_MAX_EXP + 2], cur[MOE_MAX_EXP + 1];
  const int ne = a.n_exp + 1, n = a.T * a.top_k, slots = a.top_k + 1, tid = threadIdx.x;
  for (int p = tid; p < ne; p += 1024) cnt[p] = p == 0 ? a.T : 0;
  __syncthreads();
  for (int i = tid; i < n; i += 1024) {
    const int e = a.idx[i];
    if (e >= 0 && e < a.n_exp) atomicAdd(&cnt[e + 1], 1);
  }
  __syncthreads();
  // Exclusive sums of the jobs and of the groups per position (one wave).
  if (tid < 64) {
    int rj = 0, rc = 0;
    for (int base = 0; base < ne; base += 64) {
      const int p = base + tid;
      const int c = p < ne ? cnt[p] : 0, g = (c + BP - 1) / BP;
      const int sj = wave_scan_add(c), sg = wave_scan_add(g);  // inclusive
      if (p < ne) {
        off[p] = rj + sj - c;
        coff[p] = rc + sg - g;
      }
      rj += __builtin_amdgcn_readlane(sj, 63);
      rc += __builtin_amdgcn_readlane(sg, 63);
    }
    if (tid == 0) {
      off[ne] = rj;
      coff[ne] = rc;
    }
  }
  __syncthreads();
  for (int p = tid; p < ne; p += 1024) cur[p] = off[p] + (p == 0 ? a.T : 0);
  __syncthreads();
  for (int t = tid; t < a.T; t += 1024) a.jobs[t] = t * slots + a.top_k;  // position 0: the shared expert
  for (int i = tid; i < n; i += 1024) {
    const int e = a.idx[i];
    if (e >= 0 && e < a.n_exp) a.jobs[atomicAdd(&cur[e + 1], 1)] = (i / a.top_k) * slots + i % a.top_k;
  }
  const int groups = coff[ne];
  for (int c = tid; c < groups; c += 1024) {
    int lo = 0, hi = ne - 1;  // the position p with coff[p] <= c < coff[p + 1]
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (coff[mid] <= c) lo = mid;
      else hi = mid - 1;
    }
    const int k = c - coff[lo];
    a.units[1 + c] = make_int4(pf_expert_at(lo, a.n_exp), off[lo] + k * BP, std::min(BP, cnt[lo] - k * BP), 0);
  }
  if (tid == 0) a.units[0] = make_int4(groups, 0, 0, 0);
}

// ---- products ---------------------------------------------------------------------

// Thread t's share of column s's activation tile, its rows gathered: tile
// row b is row rows[b] of the split images (kq_mmq.h, XTile).
template <int MB>
__device__ __forceinline__ void pf_xload(const _Float16* xh, const _Float16* xl, const _Float16* sh, const _Float16* sl,
                                         int nsb, const int* rows, int s, xu4 (&v)[XTile<MB>::NX], xu4& sv) {
  const int t = threadIdx.x, in_dim = nsb * 256;
#pragma unroll
  for (int u = 0; u < XTile<MB>::NX; ++u) {
    const int i = t + 256 * u, b = i >> 6, part = i & 63;
    const _Float16* src = (part < 32 ? xh : xl) + (size_t)rows[b] * in_dim + (size_t)s * 256 + 8 * (part & 31);
    v[u] = *reinterpret_cast<const xu4*>(src);
  }
  const int b = (t >> 2) & (XTile<MB>::BP - 1), part = t & 3;
  const _Float16* src = (part < 2 ? sh : sl) + ((size_t)rows[b] * nsb + s) * 16 + 8 * (part & 1);
  sv = *reinterpret_cast<const xu4*>(src);
}

// The group of unit u (tiles per group): false when u lies past the plan's
// groups.  Fills jb (the group's jobs, -1 past its count) and rows (the
// activation row of each tile row: the job's token for gate / up, the job
// for down; row 0 past the count).
template <int BP>
__device__ __forceinline__ bool pf_group(const PfArgs& a, int c, bool by_token, int* jb, int* rows, int4& G) {
  if (c >= a.units[0].x) return false;
  G = a.units[1 + c];
  const int t = threadIdx.x;
  if (t < BP) {
    const int j = t < G.z ? a.jobs[G.y + t] : -1;
    jb[t] = j;
    rows[t] = j < 0 ? 0 : by_token ? j / (a.top_k + 1) : j;
  }
  __syncthreads();
  return true;
}

// The shared-expert gates g_t = sigmoid(sgi . x_t), or 1 without sgi
// (llm_moe.adb:285-293), one wave per token.  A launch of its own: inside the
// gate/up kernel its registers cost the 32-job variant its second wave per
// SIMD (T = 512: 470 -> 541 us per layer).
__global__ __launch_bounds__(256) void moe_pf_gates(PfArgs a) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  for (int t = blockIdx.x * 4 + w; t < a.T; t += gridDim.x * 4) {
    float s = 0.f;
    if (a.sgi) {
      const float4* g4 = reinterpret_cast<const float4*>(a.sgi);
      const float4* x4 = reinterpret_cast<const float4*>(a.x + (size_t)t * a.dim);
      for (int i = lane; i < a.dim / 4; i += 64) {
        const float4 gv = g4[i], xv = x4[i];
        s = __builtin_fmaf(gv.x, xv.x, s);
        s = __builtin_fmaf(gv.y, xv.y, s);
        s = __builtin_fmaf(gv.z, xv.z, s);
        s = __builtin_fmaf(gv.w, xv.w, s);
      }
      s = wave_total(s);
    }
    if (lane == 0) a.gsh[t] = a.sgi ? 1.0f / (1.0f + expf(-s)) : 1.0f;
  }
}

// Gate and up of one (group, 64-row tile): wave w takes rows 16 w .. 16 w + 15
// of both matrices (acc[0] gate, acc[1] up) over every column.
template <int MB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void moe_pf_gate_up(PfArgs a) {
  constexpr int GB = 64 * 144, BP = 16 * MB;
  __shared__ __attribute__((aligned(16))) _Float16 xb[2][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[2][BP * SROW];
  __shared__ int jb[BP], rows[BP];
  const int tiles = a.I / 64, nsb = a.dim / 256;
  const int c = blockIdx.x / tiles, tile = blockIdx.x % tiles;
  int4 G;
  if (!pf_group<BP>(a, c, true, jb, rows, G)) return;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = G.x, row = 16 * w + j;
  const uint8_t* Wg = (e == a.n_exp ? a.sh_gate : a.gate + (size_t)e * a.gu_stride) + (size_t)tile * nsb * GB;
  const uint8_t* Wu = (e == a.n_exp ? a.sh_up : a.up + (size_t)e * a.gu_stride) + (size_t)tile * nsb * GB;
  auto load_w = [&](int s, Q4Regs (&r)[2]) {
    q4k_load(Wg + (size_t)s * GB, row, q, false, r[0]);
    q4k_load(Wu + (size_t)s * GB, row, q, false, r[1]);
  };
  f4 acc[2][MB];
#pragma unroll
  for (int rb = 0; rb < 2; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = f4{0.f, 0.f, 0.f, 0.f};
  Q4Regs cur[2], nxt[2];
  xu4 xv[XTile<MB>::NX], xsv;
  load_w(0, cur);
  pf_xload<MB>(a.xh, a.xl, a.xsh, a.xsl, nsb, rows, 0, xv, xsv);
  xtile_store<MB>(xb[0], sb[0], xv, xsv);
  __syncthreads();
  for (int s = 0; s < nsb; ++s) {
    const int buf = s & 1;
    const bool more = s + 1 < nsb;
    if (more) {
      load_w(s + 1, nxt);
      pf_xload<MB>(a.xh, a.xl, a.xsh, a.xsl, nsb, rows, s + 1, xv, xsv);
    }
    q4k_column<MB, 2>(cur, xb[buf], sb[buf], j, q, acc);
    if (more) {
      xtile_store<MB>(xb[buf ^ 1], sb[buf ^ 1], xv, xsv);
      cur[0] = nxt[0];
      cur[1] = nxt[1];
    }
    __syncthreads();
  }
  // acc[.][mb][r]: activation row b = 16 mb + 4 q + r, weight row `row`.
  const int orow = 64 * tile + row;
#pragma unroll
  for (int mb = 0; mb < MB; ++mb)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int b = 16 * mb + 4 * q + r, job = jb[b];
      if (job >= 0) {
        const float sx = a.xinv[rows[b]];
        const float g = acc[0][mb][r] * sx, v = acc[1][mb][r] * sx;
        a.h[(size_t)job * a.I + orow] = (g / (1.0f + expf(-g))) * v;
      }
    }
}

// Down of one (group, 64-row tile of dim): yk[job][row], for groups of up to
// BPG jobs in passes of 16 MB (the Q6_K column arithmetic at 64 rows would
// spill registers; the second pass reads the tile's weights from cache).
template <int MB, int BPG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void moe_pf_down(PfArgs a) {
  constexpr int GB = 64 * 210, BP = 16 * MB;
  __shared__ __attribute__((aligned(16))) _Float16 xb[2][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[2][BP * SROW];
  __shared__ int jb[BPG], rows[BPG];
  const int tiles = a.dim / 64, nsb = a.I / 256;
  const int c = blockIdx.x / tiles, tile = blockIdx.x % tiles;
  int4 G;
  if (!pf_group<BPG>(a, c, false, jb, rows, G)) return;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = G.x, row = 16 * w + j;
  const uint8_t* Wd = (e == a.n_exp ? a.sh_down : a.down + (size_t)e * a.d_stride) + (size_t)tile * nsb * GB;
  const int orow = 64 * tile + row;
  for (int base = 0; base < G.z; base += BP) {
    const int* prow = rows + base;
    f4 acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
    Q6Regs cur, nxt;
    xu4 xv[XTile<MB>::NX], xsv;
    q6k_load(Wd, row, q, cur);
    pf_xload<MB>(a.hh, a.hl, a.hsh, a.hsl, nsb, prow, 0, xv, xsv);
    xtile_store<MB>(xb[0], sb[0], xv, xsv);
    __syncthreads();
    for (int s = 0; s < nsb; ++s) {
      const int buf = s & 1;
      const bool more = s + 1 < nsb;
      if (more) {
        q6k_load(Wd + (size_t)(s + 1) * GB, row, q, nxt);
        pf_xload<MB>(a.hh, a.hl, a.hsh, a.hsl, nsb, prow, s + 1, xv, xsv);
      }
      q6k_column<MB>(cur, xb[buf], sb[buf], j, q, acc);
      if (more) {
        xtile_store<MB>(xb[buf ^ 1], sb[buf ^ 1], xv, xsv);
        cur = nxt;
      }
      __syncthreads();
    }
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int b = base + 16 * mb + 4 * q + r, job = b < BPG ? jb[b] : -1;
        if (job >= 0) a.yk[(size_t)job * a.dim + orow] = acc[mb][r] * a.hinv[job];
      }
  }
}

// Down for intermediate sizes of at most PF_DN_COLS super-block columns: the
// group's activations for every column are staged in LDS once per pass of
// 16 MB jobs, then the workgroup walks PF_DN_TILES 64-row tiles of dim
// against them -- the next tile's weights in flight while the current one is
// multiplied, and no barrier between tiles.
constexpr int PF_DN_COLS = 3;
constexpr int PF_DN_TILES = 8;

template <int MB, int BPG>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void moe_pf_down_wide(PfArgs a) {
  constexpr int GB = 64 * 210, BP = 16 * MB, NC = PF_DN_COLS;
  __shared__ __attribute__((aligned(16))) _Float16 xb[NC][BP * XROW];
  __shared__ __attribute__((aligned(16))) _Float16 sb[NC][BP * SROW];
  __shared__ int jb[BPG], rows[BPG];
  const int tiles = a.dim / 64, blocks = (tiles + PF_DN_TILES - 1) / PF_DN_TILES, nsb = a.I / 256;
  const int c = blockIdx.x / blocks, tb = blockIdx.x % blocks;
  int4 G;
  if (!pf_group<BPG>(a, c, false, jb, rows, G)) return;
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int e = G.x, row = 16 * w + j;
  const uint8_t* Wd = e == a.n_exp ? a.sh_down : a.down + (size_t)e * a.d_stride;
  const int t0 = tb * PF_DN_TILES, t1 = std::min(tiles, t0 + PF_DN_TILES);
  auto load_tile = [&](int tile, Q6Regs (&r)[NC]) {
#pragma unroll
    for (int s = 0; s < NC; ++s)
      if (s < nsb) q6k_load(Wd + ((size_t)tile * nsb + s) * GB, row, q, r[s]);
  };
  for (int base = 0; base < G.z; base += BP) {
    Q6Regs cur[NC], nxt[NC];
    load_tile(t0, cur);
    {
      xu4 xv[XTile<MB>::NX], xsv;
#pragma unroll
      for (int s = 0; s < NC; ++s)
        if (s < nsb) {
          pf_xload<MB>(a.hh, a.hl, a.hsh, a.hsl, nsb, rows + base, s, xv, xsv);
          xtile_store<MB>(xb[s], sb[s], xv, xsv);
        }
    }
    __syncthreads();
    for (int tile = t0; tile < t1; ++tile) {
      if (tile + 1 < t1) load_tile(tile + 1, nxt);
      f4 acc[MB];
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[mb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < NC; ++s)
        if (s < nsb) q6k_column<MB>(cur[s], xb[s], sb[s], j, q, acc);
      const int orow = 64 * tile + row;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int b = base + 16 * mb + 4 * q + r, job = b < BPG ? jb[b] : -1;
          if (job >= 0) a.yk[(size_t)job * a.dim + orow] = acc[mb][r] * a.hinv[job];
        }
      if (tile + 1 < t1)
#pragma unroll
        for (int s = 0; s < NC; ++s) cur[s] = nxt[s];
    }
    __syncthreads();  // the next pass overwrites the staged activations
  }
}

// y[t][row] = sum_k top_w[t][k] yk[t slots + k][row] (ascending k) +
// g_t yk[t slots + top_k][row] (llm_moe.adb:270-299), g_t from
// moe_pf_gates.  Workgroup (i, t): rows 256 i .. 256 i + 255 of token t.  A token
// with a routed expert outside [0, n_exp) keeps its y unwritten.
__global__ __launch_bounds__(256) void moe_pf_combine(PfArgs a) {
  const int t = blockIdx.y, row = blockIdx.x * 256 + threadIdx.x, slots = a.top_k + 1;
  bool ok = true;
  for (int k = 0; k < a.top_k; ++k) {
    const int e = a.idx[(size_t)t * a.top_k + k];
    ok = ok && e >= 0 && e < a.n_exp;
  }
  if (!ok || row >= a.dim) return;
  const float gs = a.gsh[t];
  const float* yt = a.yk + (size_t)t * slots * a.dim + row;
  float acc = 0.f;
  for (int k0 = 0; k0 < a.top_k; k0 += 8) {
    float v[8], wk[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + i < a.top_k ? k0 + i : k0;
      v[i] = yt[(size_t)k * a.dim];
      wk[i] = a.top_w[(size_t)t * a.top_k + k];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (k0 + i < a.top_k) acc = acc + wk[i] * v[i];
  }
  a.y[(size_t)t * a.dim + row] = acc + gs * yt[(size_t)a.top_k * a.dim];
}

// ---- host side --------------------------------------------------------------

static size_t pf_round(size_t n) { return (n + 255) / 256 * 256; }

// Groups a plan can produce: ceil(jobs / BP) plus one partial group per
// non-empty position.
static size_t pf_max_groups(int T, int top_k, int n_exp, int bp) {
  const size_t jobs = (size_t)T * (top_k + 1);
  return (jobs + bp - 1) / bp + std::min<size_t>((size_t)n_exp, (size_t)T * top_k) + 1;
}

size_t moe_prefill_work_bytes(int T, int dim, int I, int top_k) {
  const size_t J = (size_t)T * (top_k + 1), nd = dim / 256, ni = I / 256;
  size_t n = 0;
  n += 2 * pf_round((size_t)T * dim * 2);       // xh, xl
  n += 2 * pf_round((size_t)T * nd * 16 * 2);   // xsh, xsl
  n += pf_round((size_t)T * 4);                 // xinv
  n += pf_round((size_t)T * 4);                 // gsh
  n += pf_round(J * I * 4);                     // h
  n += 2 * pf_round(J * I * 2);                 // hh, hl
  n += 2 * pf_round(J * ni * 16 * 2);           // hsh, hsl
  n += pf_round(J * 4);                         // hinv
  n += pf_round(J * dim * 4);                   // yk
  n += pf_round(J * 4);                         // jobs
  n += pf_round((1 + pf_max_groups(T, top_k, MOE_MAX_EXP, 16)) * 16);  // units (for the smallest groups)
  return n;
}

static void pf_bind(PfArgs& a, void* work) {
  const size_t J = (size_t)a.T * (a.top_k + 1), nd = a.dim / 256, ni = a.I / 256;
  uint8_t* p = (uint8_t*)work;
  auto take = [&](size_t bytes) {
    uint8_t* r = p;
    p += pf_round(bytes);
    return r;
  };
  a.xh = (_Float16*)take((size_t)a.T * a.dim * 2);
  a.xl = (_Float16*)take((size_t)a.T * a.dim * 2);
  a.xsh = (_Float16*)take((size_t)a.T * nd * 16 * 2);
  a.xsl = (_Float16*)take((size_t)a.T * nd * 16 * 2);
  a.xinv = (float*)take((size_t)a.T * 4);
  a.gsh = (float*)take((size_t)a.T * 4);
  a.h = (float*)take(J * a.I * 4);
  a.hh = (_Float16*)take(J * a.I * 2);
  a.hl = (_Float16*)take(J * a.I * 2);
  a.hsh = (_Float16*)take(J * ni * 16 * 2);
  a.hsl = (_Float16*)take(J * ni * 16 * 2);
  a.hinv = (float*)take(J * 4);
  a.yk = (float*)take(J * a.dim * 4);
  a.jobs = (int*)take(J * 4);
  a.units = (int4*)p;
}

// Activation rows per product tile from the expected jobs per routed expert.
static int pf_mb(int T, int top_k, int n_exp) {
  const double per = (double)T * top_k / n_exp;
  return per >= 40 ? 4 : per >= 20 ? 2 : 1;
}

bool moe_prefill_takes(int T, int gu_kind, int down_kind, int dim, int I, int top_k, int n_exp) {
  return T >= MOE_PREFILL_MIN_TOKENS && gu_kind == Q4_K && down_kind == Q6_K && dim % 256 == 0 && I % 256 == 0 &&
         top_k >= 1 && top_k <= MOE_MAX_TOPK && n_exp >= 1 && n_exp <= MOE_MAX_EXP;
}

hipError_t launch_moe_prefill(const MoeGroupedArgs& g, void* work, hipStream_t s) {
  if (g.T < 1 || g.T > MOE_PREFILL_MAX_TOKENS) return hipErrorInvalidValue;
  PfArgs a{};
  a.gate = g.gate; a.up = g.up; a.down = g.down;
  a.sh_gate = g.sh_gate; a.sh_up = g.sh_up; a.sh_down = g.sh_down;
  a.gu_stride = g.gu_stride; a.d_stride = g.d_stride;
  a.idx = g.idx; a.top_w = g.top_w; a.x = g.x; a.sgi = g.sgi; a.y = g.y;
  a.T = g.T; a.top_k = g.top_k; a.n_exp = g.n_exp; a.dim = g.dim; a.I = g.I;
  pf_bind(a, work);
  const int J = a.T * (a.top_k + 1);
  const int mb = pf_mb(a.T, a.top_k, a.n_exp), bp = 16 * mb;
  const size_t groups = pf_max_groups(a.T, a.top_k, a.n_exp, bp);
  hipError_t e = launch_xsplit(32, a.x, a.T, a.T, a.dim, a.xh, a.xl, a.xsh, a.xsl, a.xinv, s);
  if (e != hipSuccess) return e;
  switch (mb) {
    case 1: hipLaunchKernelGGL(moe_pf_plan<16>, dim3(1), dim3(1024), 0, s, a); break;
    case 2: hipLaunchKernelGGL(moe_pf_plan<32>, dim3(1), dim3(1024), 0, s, a); break;
    default: hipLaunchKernelGGL(moe_pf_plan<64>, dim3(1), dim3(1024), 0, s, a); break;
  }
  const dim3 gu((unsigned)(groups * (a.I / 64))), dn((unsigned)(groups * (a.dim / 64)));
  const bool wide = a.I / 256 <= PF_DN_COLS;
  const dim3 dnw((unsigned)(groups * ((a.dim / 64 + PF_DN_TILES - 1) / PF_DN_TILES)));
  switch (mb) {
    case 1: hipLaunchKernelGGL(moe_pf_gate_up<1>, gu, dim3(256), 0, s, a); break;
    case 2: hipLaunchKernelGGL(moe_pf_gate_up<2>, gu, dim3(256), 0, s, a); break;
    default: hipLaunchKernelGGL(moe_pf_gate_up<4>, gu, dim3(256), 0, s, a); break;
  }
  e = launch_xsplit(16, a.h, J, J, a.I, a.hh, a.hl, a.hsh, a.hsl, a.hinv, s);
  if (e != hipSuccess) return e;
  if (wide) {
    switch (mb) {
      case 1: hipLaunchKernelGGL((moe_pf_down_wide<1, 16>), dnw, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((moe_pf_down_wide<2, 32>), dnw, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((moe_pf_down_wide<2, 64>), dnw, dim3(256), 0, s, a); break;
    }
  } else {
    switch (mb) {
      case 1: hipLaunchKernelGGL((moe_pf_down<1, 16>), dn, dim3(256), 0, s, a); break;
      case 2: hipLaunchKernelGGL((moe_pf_down<2, 32>), dn, dim3(256), 0, s, a); break;
      default: hipLaunchKernelGGL((moe_pf_down<2, 64>), dn, dim3(256), 0, s, a); break;
    }
  }
  hipLaunchKernelGGL(moe_pf_gates, dim3((a.T + 3) / 4), dim3(256), 0, s, a);
  hipLaunchKernelGGL(moe_pf_combine, dim3((a.dim + 255) / 256, a.T), dim3(256), 0, s, a);
  return hipGetLastError();
}

}  // namespace kq
