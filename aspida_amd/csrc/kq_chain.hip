// kq_chain.hip -- the resident decode chain: one persistent launch runs an
// ordered list of packed matvecs ("steps"), e.g. every weight matrix of a
// decoder pass, without a launch boundary between them.
//
// A step whose x lies inside an earlier step's y depends on that producer.
// Instead of a grid-wide barrier between steps, every 64-row tile of every
// step has a ready flag holding the epoch (launch number) in which its rows
// were last written; a wave that needs activation column c of a step waits
// only for the producer tiles covering rows [256 c, 256 c + 256) of its x.
// Weights never depend on earlier steps, so a wave issues the loads of its
// next column before it waits or computes, and the weight stream continues
// while a dependency resolves.
//
// Work: step s is cut into units of one 64-row tile x (8 waves x spw)
// super-block columns; workgroup g of the G resident ones takes units g,
// g + G, ... of the whole list in step order, so every unit of an earlier
// step belongs to a workgroup that reaches it before any later unit and the
// waits cannot form a cycle.  The 8 waves' partial dots meet in LDS at one
// barrier per unit; one wave -- a different one each unit -- finishes the
// unit (sums the 8 in order, stores y or the tile's partial, publishes) while
// the others already start the next unit.  A tile of more than one unit
// sums their partials in the last arriving workgroup, in ascending unit
// order (deterministic), which then writes y and the tile's flag.  Each dot is
// the arithmetic of the packed batch-1 matvec (kq_packed.hip) for the same
// super-block column.
//
// Cross-workgroup data (y, partials, flags, counters) moves through
// device-scope (sc1) atomic stores and loads, which bypass the per-XCD L2s;
// a wave retires its stores (s_waitcnt) before it publishes a flag or an
// arrival.  A wait gives up after CH_MAX_POLLS polls (G larger than what the
// device keeps resident, or a bug), records the failure and goes on, so a
// launch always terminates.
#include <math.h>

#include <algorithm>
#include <cstring>
#include <vector>

#include "kq_chain.h"
#include "kq_host.h"
#include "kq_kernels.h"
#include "kq_packed.h"

namespace kq {

constexpr int CH_NW = 8;            // waves per workgroup
constexpr int CH_EPOCH_CTRS = 16;   // launch-number counters (G / 16 arrivals each)
constexpr unsigned CH_MAX_POLLS = 1u << 17;  // about 0.1 s of polling

struct ChainStepDev {
  const uint8_t* W;
  const float* x;
  float* y;
  float* part;           // ks > 1: [ks][ntiles][64]
  unsigned* count;       // ks > 1: one counter per tile, COUNTER_STRIDE apart
  unsigned* flag;        // [ntiles]: epoch of the last write of the tile's rows
  const unsigned* dflag; // the producer's flags, or null when x is an input of the launch
  int kind, nsb, out_rows, ntiles, ks, spw, unit0, xoff;
};

// Rows [r0, r1] of the producer are written (flags == epoch) -- every lane
// returns once they are.  false: gave up, after CH_MAX_POLLS polls or as soon
// as any wave of the launch has (err set), so a failing launch ends quickly.
__device__ __forceinline__ bool wait_rows(const unsigned* __restrict__ dflag, int r0, int r1, unsigned epoch,
                                          int lane, const unsigned* __restrict__ err) {
  const int lo = r0 / 64, n = r1 / 64 - lo + 1;  // n <= 63 (r1 - r0 < 4096 - 64)
  for (unsigned polls = 0;; ++polls) {
    const unsigned f = lane < n ? __hip_atomic_load(dflag + lo + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                                : epoch;
    if (__ballot(f != epoch) == 0ull) return true;
    const unsigned e = lane == 63 ? __hip_atomic_load(err, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
    if (polls >= CH_MAX_POLLS || __builtin_amdgcn_readlane(e, 63) != 0u) return false;
    __builtin_amdgcn_s_sleep(2);
  }
}

// The wave's activation columns c0 .. c0 + n - 1 of unit step st: one float4
// per lane each (device-scope loads: a producer on another XCD wrote them).
__device__ __forceinline__ float4 load_x4(const float* __restrict__ p) {
  float4 v;
  v.x = __hip_atomic_load(p + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.y = __hip_atomic_load(p + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.z = __hip_atomic_load(p + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  v.w = __hip_atomic_load(p + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return v;
}

struct ChainShared {
  float red[2][CH_NW][64];  // partial dots of the unit, by unit parity
  __attribute__((aligned(16))) float xst[CH_NW][256];
  unsigned epoch;
};

// Finishing a unit (one wave): its 64 rows' sum t goes to y directly
// (ks == 1), or to the tile's partial; the wave completing the tile's last
// unit sums the ks partials in ascending order (eight loads in flight at a
// time).  The writer of the rows publishes the tile's flag.
__device__ __forceinline__ void chain_finish(const ChainStepDev& st, int tile, int cg, float t, int lane,
                                             unsigned epoch) {
  const int row = tile * 64 + lane;
  if (st.ks > 1) {
    __hip_atomic_store(&st.part[((size_t)cg * st.ntiles + tile) * 64 + lane], t, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the partial is out before the arrival counts
    unsigned old = 0;
    if (lane == 0)
      old = __hip_atomic_fetch_add(&st.count[(size_t)tile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
    if (__builtin_amdgcn_readfirstlane(old) != (unsigned)(st.ks - 1)) return;
    t = 0.f;
    for (int k0 = 0; k0 < st.ks; k0 += 8) {
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[k] = k0 + k < st.ks ? __hip_atomic_load(&st.part[((size_t)(k0 + k) * st.ntiles + tile) * 64 + lane],
                                                  __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                              : 0.f;
#pragma unroll
      for (int k = 0; k < 8; ++k)
        if (k0 + k < st.ks) t += v[k];
    }
    if (lane == 0)
      __hip_atomic_store(&st.count[(size_t)tile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (row < st.out_rows) __hip_atomic_store(&st.y[row], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);  // the rows are out before the flag says so
  if (lane == 0) __hip_atomic_store(&st.flag[tile], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// This workgroup's units [u, u_end) of step st (stride G), kind KIND; `seq`
// counts the workgroup's units (unit parity and the finishing wave).  The
// first column's weights are requested before anything waits; after that the
// column registers are double-buffered -- each column's loads are issued
// before the previous column's arithmetic, across unit boundaries too.
template <int KIND>
__device__ __forceinline__ void chain_step(const ChainStepDev& st, int u, int u_end, int G, ChainShared& S, int lane,
                                           int w, int& seq, unsigned epoch, unsigned* __restrict__ err) {
  using R = typename Packed<KIND>::R;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  // Q8_0's register image (68 VGPRs) is too large to double-buffer next to
  // the staged activations: its columns load just before use.
  constexpr bool DB = KIND != Q8_0;
  const int spw = st.spw;
  // Column j of this wave in unit v, clamped into the matrix (a wave without
  // a column there re-reads a valid one, so that loads need no branch).
  auto col = [&](int v, int j) -> const uint8_t* {
    const int ul = v - st.unit0, c = ((ul % st.ks) * CH_NW + w) * spw + j;
    return st.W + ((size_t)(ul / st.ks) * st.nsb + (c < st.nsb ? c : st.nsb - 1)) * GB;
  };
  R cur;
  // Ordinary loads (not the streaming hint of the per-matrix kernels): the
  // chain measured 542 tok/s with them and 518 without on the 8B decode.
  if (DB) cur = Packed<KIND>::template load<false>(col(u, 0), lane);
  while (u < u_end) {
    const int ul = u - st.unit0, tile = ul / st.ks, cg = ul % st.ks;
    const int c0 = (cg * CH_NW + w) * spw;
    const int nc = c0 >= st.nsb ? 0 : (st.nsb - c0 < spw ? st.nsb - c0 : spw);
    // Wait for the producer rows of this wave's columns, then fetch x.
    float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
    if (nc > 0) {
      if (st.dflag && !wait_rows(st.dflag, st.xoff + 256 * c0, st.xoff + 256 * (c0 + nc) - 1, epoch, lane, err)) {
        if (lane == 0) __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      x0 = load_x4(st.x + (size_t)c0 * 256 + 4 * lane);
      if (nc > 1) x1 = load_x4(st.x + (size_t)(c0 + 1) * 256 + 4 * lane);
    }
    const int un = u + G;
    float acc = 0.f;
    for (int j = 0; j < nc; ++j) {
      float s16[16];
      if (DB) {
        // The next column: this unit's, else this wave's first of its next
        // unit (or, at the end of the step, the current one again).
        const uint8_t* np = j + 1 < nc ? col(u, j + 1) : un < u_end ? col(un, 0) : col(u, j);
        const R nxt = Packed<KIND>::template load<false>(np, lane);
        asm volatile("" ::: "memory");  // keep those loads issued here
        stage_x256(j == 0 ? x0 : x1, S.xst[w], lane, s16);
        acc += staged_dot<KIND>(cur, S.xst[w], s16);
        cur = nxt;
      } else {
        const R r = Packed<KIND>::template load<false>(col(u, j), lane);
        stage_x256(j == 0 ? x0 : x1, S.xst[w], lane, s16);
        acc += staged_dot<KIND>(r, S.xst[w], s16);
      }
    }
    if (DB && nc == 0 && un < u_end) cur = Packed<KIND>::template load<false>(col(un, 0), lane);
    // The waves meet once per unit; the partial buffer alternates with the
    // unit's parity, so the finishing wave reads it before anyone can write
    // it again (two barriers later).
    const int p = seq & 1;
    S.red[p][w][lane] = acc;
    __syncthreads();
    if (w == seq % CH_NW) {
      float t = S.red[p][0][lane];
#pragma unroll
      for (int k = 1; k < CH_NW; ++k) t += S.red[p][k][lane];
      chain_finish(st, tile, cg, t, lane, epoch);
    }
    ++seq;
    u = un;
  }
}

__global__ __launch_bounds__(64 * CH_NW) void kq_chain(const ChainStepDev* __restrict__ steps, int nsteps,
                                                       unsigned* __restrict__ epoch_ctr, unsigned* __restrict__ err) {
  __shared__ ChainShared S;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.x, G = gridDim.x;
  // This launch's number: every counter gets G / CH_EPOCH_CTRS arrivals per
  // launch (G is a multiple of CH_EPOCH_CTRS), so old / that + 1 is the same
  // in every workgroup; flags start at 0.
  if (threadIdx.x == 0) {
    const unsigned old = __hip_atomic_fetch_add(&epoch_ctr[(g % CH_EPOCH_CTRS) * COUNTER_STRIDE], 1u,
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    S.epoch = old / (unsigned)(G / CH_EPOCH_CTRS) + 1u;
  }
  __syncthreads();
  const unsigned epoch = S.epoch;
  int u = g, seq = 0;
  for (int s = 0; s < nsteps; ++s) {
    const ChainStepDev& st = steps[s];
    const int u_end = st.unit0 + st.ntiles * st.ks;
    if (u >= u_end) continue;
    switch (st.kind) {
      case Q4_K: chain_step<Q4_K>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
      case Q6_K: chain_step<Q6_K>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
      case Q5_K: chain_step<Q5_K>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
      case Q3_K: chain_step<Q3_K>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
      case Q2_K: chain_step<Q2_K>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
      default: chain_step<Q8_0>(st, u, u_end, G, S, lane, w, seq, epoch, err); break;
    }
    while (u < u_end) u += G;
  }
}

// ---- host ---------------------------------------------------------------------------

struct Chain {
  ChainStepDev* d_steps = nullptr;
  void* d_mem = nullptr;      // flags | counters | epoch counters | err | partials
  unsigned* epoch_ctr = nullptr;
  unsigned* err = nullptr;
  int nsteps = 0, G = 0;
};

static bool overlaps(const void* a, size_t na, const void* b, size_t nb) {
  const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
  return x < y + nb && y < x + na;
}

static int chain_grid() {
  int dev = 0, cus = 256, per = 1;
  (void)query_clean([&] {
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, (const void*)kq_chain, 64 * CH_NW, 0) != hipSuccess ||
        per <= 0)
      per = 1;  // fewer workgroups than fit: still all resident
  });
  const int G = per * cus / CH_EPOCH_CTRS * CH_EPOCH_CTRS;
  return G > 0 ? G : CH_EPOCH_CTRS;
}

hipError_t chain_create(const ChainStepDesc* desc, int n, Chain** out, const char** why) {
  *out = nullptr;
  *why = "";
  if (!desc || n <= 0) { *why = "no steps"; return hipErrorInvalidValue; }
  const int G = chain_grid();
  std::vector<ChainStepDev> st(n);
  size_t nflags = 0, ncount = 0, npart = 0;
  int units = 0;
  std::vector<size_t> flag_off(n), count_off(n), part_off(n);
  std::vector<int> producer(n, -1);
  for (int j = 0; j < n; ++j) {
    const ChainStepDesc& d = desc[j];
    if (block_bytes(d.kind) <= 0 || !d.packed || !d.x || !d.y || d.in_dim <= 0 || d.in_dim % 256 || d.out_dim <= 0 ||
        ((uintptr_t)d.x & 15)) {
      *why = "bad step (kind, pointers, in_dim % 256, 16-byte aligned x)";
      return hipErrorInvalidValue;
    }
    const size_t xb = (size_t)d.in_dim * 4, yb = (size_t)d.out_dim * 4;
    if (overlaps(d.x, xb, d.y, yb)) { *why = "a step's x overlaps its y"; return hipErrorInvalidValue; }
    int dep = -1;
    for (int i = 0; i < j; ++i) {
      if (overlaps(d.y, yb, desc[i].y, (size_t)desc[i].out_dim * 4) ||
          overlaps(d.y, yb, desc[i].x, (size_t)desc[i].in_dim * 4)) {
        *why = "a step writes memory an earlier step reads or writes";
        return hipErrorInvalidValue;
      }
      if (overlaps(d.x, xb, desc[i].y, (size_t)desc[i].out_dim * 4)) dep = i;
    }
    ChainStepDev& s = st[j];
    s.W = (const uint8_t*)d.packed;
    s.x = d.x;
    s.y = d.y;
    s.kind = d.kind;
    s.nsb = d.in_dim / 256;
    s.out_rows = d.out_dim;
    s.ntiles = (d.out_dim + 63) / 64;
    s.xoff = 0;
    s.dflag = nullptr;
    if (dep >= 0) {
      const uintptr_t y0 = (uintptr_t)desc[dep].y, x0 = (uintptr_t)d.x;
      if (x0 < y0 || x0 + xb > y0 + (size_t)desc[dep].out_dim * 4) {
        *why = "a step's x must lie inside one earlier step's y";
        return hipErrorInvalidValue;
      }
      s.xoff = (int)((x0 - y0) / 4);
    }
    // Columns per wave: 2 when that divides the columns into whole units and
    // still gives every workgroup a unit, else 1.
    s.spw = s.nsb % (CH_NW * 2) == 0 && (long)s.ntiles * (s.nsb / (CH_NW * 2)) >= G ? 2 : 1;
    s.ks = (s.nsb + CH_NW * s.spw - 1) / (CH_NW * s.spw);
    s.unit0 = units;
    units += s.ntiles * s.ks;
    flag_off[j] = nflags;
    nflags += s.ntiles;
    count_off[j] = ncount;
    part_off[j] = npart;
    if (s.ks > 1) {
      ncount += (size_t)s.ntiles * COUNTER_STRIDE;
      npart += (size_t)s.ks * s.ntiles * 64;
    }
    s.flag = nullptr;
    s.count = nullptr;
    s.part = nullptr;
    producer[j] = dep;
  }
  // Device memory: flags | counters | epoch counters | err (256-byte parts) | partials.
  auto r256 = [](size_t b) { return (b + 255) / 256 * 256; };
  const size_t b_flags = r256(nflags * 4), b_count = r256(ncount * 4), b_epoch = r256(CH_EPOCH_CTRS * COUNTER_STRIDE * 4),
               b_err = 256, b_part = r256(npart * 4);
  Chain* c = new Chain();
  c->nsteps = n;
  c->G = G;
  hipError_t e = hipMalloc(&c->d_mem, b_flags + b_count + b_epoch + b_err + b_part);
  if (e == hipSuccess) e = hipMemset(c->d_mem, 0, b_flags + b_count + b_epoch + b_err);
  if (e == hipSuccess) e = hipMalloc(&c->d_steps, sizeof(ChainStepDev) * n);
  if (e != hipSuccess) {
    chain_destroy(c);
    *why = "device memory";
    return e;
  }
  uint8_t* base = (uint8_t*)c->d_mem;
  unsigned* flags = (unsigned*)base;
  unsigned* counts = (unsigned*)(base + b_flags);
  c->epoch_ctr = (unsigned*)(base + b_flags + b_count);
  c->err = (unsigned*)(base + b_flags + b_count + b_epoch);
  float* parts = (float*)(base + b_flags + b_count + b_epoch + b_err);
  for (int j = 0; j < n; ++j) {
    const int dep = producer[j];
    st[j].flag = flags + flag_off[j];
    st[j].dflag = dep >= 0 ? flags + flag_off[dep] : nullptr;
    if (st[j].ks > 1) {
      st[j].count = counts + count_off[j];
      st[j].part = parts + part_off[j];
    }
  }
  e = hipMemcpy(c->d_steps, st.data(), sizeof(ChainStepDev) * n, hipMemcpyHostToDevice);
  if (e != hipSuccess) {
    chain_destroy(c);
    *why = "upload";
    return e;
  }
  *out = c;
  return hipSuccess;
}

hipError_t chain_run(Chain* c, hipStream_t s) {
  hipLaunchKernelGGL(kq_chain, dim3(c->G), dim3(64 * CH_NW), 0, s, c->d_steps, c->nsteps, c->epoch_ctr, c->err);
  return hipGetLastError();
}

hipError_t chain_check(Chain* c, unsigned* failed) {
  unsigned v = 0;
  hipError_t e = hipMemcpy(&v, c->err, 4, hipMemcpyDeviceToHost);
  if (e == hipSuccess && v) e = hipMemset(c->err, 0, 4);
  *failed = v;
  return e;
}

void chain_destroy(Chain* c) {
  if (!c) return;
  if (c->d_steps) (void)hipFree(c->d_steps);
  if (c->d_mem) (void)hipFree(c->d_mem);
  delete c;
}

int chain_workgroups(const Chain* c) { return c->G; }

}  // namespace kq
