// kq_moe_sched.h -- the schedule of the grouped MoE kernels (the vector-ALU
// ones in kq_moe_grouped.hip and the matrix-core ones in kq_moe_mfma.hip):
// every workgroup derives the same list of work items from top_idx in LDS,
// and the gate/up launch's prologue.
#pragma once
#include <math.h>

#include "kq_moe.h"
#include "kq_packed.h"

namespace kq {

// ---- schedule ---------------------------------------------------------------------
//
// Work items are (expert, 64-row tile, chunk of up to JPW jobs), the
// shared expert being expert n_exp with every token's slot top_k.  Experts
// are taken in the order of their positions p: the shared expert first
// (p = 0: it has a job for every token, the most of any expert, so its items
// start first and do not form the launch's tail), then routed expert e at
// p = e + 1.  Items are numbered position-major, then tile, then chunk, so
// the chunks that share an expert tile are adjacent and run close together
// in time (their weights are read from HBM about once).
//
// Jobs per expert are bucketed in ascending slot order: a slot's place is
// the number of earlier slots routed to the same expert, counted from a
// bitmask of the slots of each expert (one LDS atomic OR per slot, then
// popcounts) -- or, when the masks do not fit, by scanning the earlier
// slots.  Every workgroup derives the same buckets.  The gate/up launch
// computes them, and its workgroup 0 publishes the job offsets and the job
// list to the workspace (a.sched), from which the down launch reads them.
struct MoeSched {
  int idx[MOE_MAX_JOBS];                // top_idx, flat
  union {
    unsigned mask[MOE_SCHED_MASK_WORDS];  // [position][slot / 32]: bit slot % 32
    int fill[MOE_MAX_EXP + 1];            // jobs per position (when the masks do not fit)
  };
  int coff[MOE_MAX_EXP + 2];            // exclusive sum of chunks per position
  int joff[MOE_MAX_EXP + 2];            // exclusive sum of jobs per position
  int jobs[2 * MOE_MAX_JOBS];           // t * slots + k, bucketed by position, ascending
};

__device__ __forceinline__ int moe_expert_at(int p, int n_exp) { return p == 0 ? n_exp : p - 1; }
__device__ __forceinline__ int moe_position(int e, int n_exp) { return e == n_exp ? 0 : e + 1; }

// coff from joff (one wave): chunks of up to JPW jobs per position.
template <int JPW>
__device__ __forceinline__ void moe_chunk_offsets(MoeSched& S, int ne) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x;
  int run = 0;
  for (int base = 0; base < ne; base += 64) {
    const int p = base + lane;
    const int c = p < ne ? (S.joff[p + 1] - S.joff[p] + JPW - 1) / JPW : 0;
    const int ch = wave_scan_add(c);  // inclusive
    if (p < ne) S.coff[p] = run + ch - c;
    run += __builtin_amdgcn_readlane(ch, 63);
  }
  if (lane == 0) S.coff[ne] = run;
}

// Returns the number of chunks (items per tile) of up to JPW jobs.
template <int JPW>
__device__ int moe_schedule(const MoeGroupedArgs& a, MoeSched& S) {
  const int n = a.T * a.top_k, n_exp = a.n_exp, ne = n_exp + 1, slots = a.top_k + 1;
  const int tid = threadIdx.x, bs = blockDim.x;
  const int nw = (n + 31) / 32;
  const bool masks = ne * nw <= MOE_SCHED_MASK_WORDS;
  if (masks)
    for (int i = tid; i < ne * nw; i += bs) S.mask[i] = 0u;
  else
    for (int i = tid; i < ne; i += bs) S.fill[i] = 0;
  for (int i = tid; i < n; i += bs) S.idx[i] = a.idx[i];
  __syncthreads();
  for (int i = tid; i < n; i += bs) {
    const int e = S.idx[i];
    if (e >= 0 && e < n_exp) {
      const int p = e + 1;
      if (masks) atomicOr(&S.mask[p * nw + (i >> 5)], 1u << (i & 31));
      else atomicAdd(&S.fill[p], 1);
    }
  }
  __syncthreads();
  // Jobs per position (the shared expert: T), then their exclusive sums.
  if (tid < 64) {
    const int lane = tid;
    int run = 0;
    for (int base = 0; base < ne; base += 64) {
      const int p = base + lane;
      int c = 0;
      if (p == 0) {
        c = a.T;
      } else if (p < ne) {
        if (masks)
          for (int w = 0; w < nw; ++w) c += __builtin_popcount(S.mask[p * nw + w]);
        else
          c = S.fill[p];
      }
      const int jc = wave_scan_add(c);  // inclusive
      if (p < ne) S.joff[p] = run + jc - c;
      run += __builtin_amdgcn_readlane(jc, 63);
    }
    if (lane == 0) S.joff[ne] = run;
  }
  __syncthreads();
  moe_chunk_offsets<JPW>(S, ne);
  for (int i = tid; i < n; i += bs) {
    const int e = S.idx[i];
    if (e >= 0 && e < n_exp) {
      const int p = e + 1;
      int rank = 0;
      if (masks) {
        const unsigned* m = &S.mask[p * nw];
        for (int w = 0; w < (i >> 5); ++w) rank += __builtin_popcount(m[w]);
        rank += __builtin_popcount(m[i >> 5] & ((1u << (i & 31)) - 1u));
      } else {
        for (int q = 0; q < i; ++q) rank += S.idx[q] == e;
      }
      S.jobs[S.joff[p] + rank] = (i / a.top_k) * slots + i % a.top_k;
    }
  }
  for (int t = tid; t < a.T; t += bs) S.jobs[t] = t * slots + a.top_k;  // position 0: joff[0] = 0
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int i = tid; i <= ne; i += bs) a.sched[i] = S.joff[i];
    for (int i = tid; i < a.T * slots; i += bs) a.sched[ne + 1 + i] = S.jobs[i];
  }
  return S.coff[ne];
}

// The down launch's copy of the schedule that the gate/up launch before it
// published (a.sched), chunked by this launch's JPW.
template <int JPW>
__device__ int moe_schedule_load(const MoeGroupedArgs& a, MoeSched& S) {
  const int ne = a.n_exp + 1, total = a.T * (a.top_k + 1);
  for (int i = threadIdx.x; i <= ne; i += blockDim.x) S.joff[i] = a.sched[i];
  for (int i = threadIdx.x; i < total; i += blockDim.x) S.jobs[i] = a.sched[ne + 1 + i];
  __syncthreads();
  moe_chunk_offsets<JPW>(S, ne);
  __syncthreads();
  return S.coff[ne];
}

struct MoeItem {
  int e, tile, j0, nj;  // expert, tile, first job (into S.jobs), job count
};

template <int JPW>
__device__ __forceinline__ MoeItem moe_item(const MoeSched& S, int ne, int tiles, int i) {
  int lo = 0, hi = ne - 1;  // the position p with coff[p] * tiles <= i < coff[p + 1] * tiles
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (S.coff[mid] * tiles <= i) lo = mid;
    else hi = mid - 1;
  }
  const int p = lo, ch = S.coff[p + 1] - S.coff[p], r = i - S.coff[p] * tiles;
  const int c = r % ch, cnt = S.joff[p + 1] - S.joff[p];
  MoeItem it;
  it.e = moe_expert_at(p, ne - 1);
  it.tile = r / ch;
  it.j0 = S.joff[p] + c * JPW;
  it.nj = cnt - c * JPW < JPW ? cnt - c * JPW : JPW;
  return it;
}

// Housekeeping for the down launch, done by the gate/up launch: zero its
// arrival counters (workgroup 0), and the shared-expert gate
// g_t = sigmoid(shared_gate_inp . x_t) (llm_moe.adb:285-293), one wave per
// token.
__device__ __forceinline__ void moe_gu_prologue(const MoeGroupedArgs& a, const float* __restrict__ x, int nw, int w,
                                                int lane) {
  if (blockIdx.x == 0)
    for (int i = threadIdx.x; i < a.T * a.blocks_dim; i += blockDim.x) a.count[(size_t)i * COUNTER_STRIDE] = 0u;
  for (int t = blockIdx.x * nw + w; t < a.T; t += gridDim.x * nw) {
    float s = 0.f;
    if (a.sgi) {
      // dim / 256 float4 per lane, loaded together (dim is a multiple of 256).
      const float4* g4 = reinterpret_cast<const float4*>(a.sgi) + lane;
      const float4* x4 = reinterpret_cast<const float4*>(x + (size_t)t * a.dim) + lane;
      for (int b = 0; b < a.dim / 4; b += 64 * 8) {
        float4 gv[8], xv[8];
#pragma unroll
        for (int r = 0; r < 8; ++r) {
          const int i = b + 64 * r < a.dim / 4 ? b + 64 * r : 0;
          gv[r] = g4[i];
          xv[r] = x4[i];
        }
#pragma unroll
        for (int r = 0; r < 8; ++r)
          if (b + 64 * r < a.dim / 4) {
            s = __builtin_fmaf(gv[r].x, xv[r].x, s);
            s = __builtin_fmaf(gv[r].y, xv[r].y, s);
            s = __builtin_fmaf(gv[r].z, xv[r].z, s);
            s = __builtin_fmaf(gv[r].w, xv[r].w, s);
          }
      }
      s = wave_total(s);
    }
    if (lane == 0) a.gsh[t] = a.sgi ? 1.0f / (1.0f + expf(-s)) : 1.0f;
  }
}

}  // namespace kq
