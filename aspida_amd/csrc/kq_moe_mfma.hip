// kq_moe_mfma.hip -- the grouped MoE experts on the matrix cores, for any
// number of tokens T >= 2 with Q4_K or Q6_K projections.  Three launches:
//
//   moe_gate_up_mf  every workgroup first derives the schedule
//                   (kq_moe_sched.h: jobs bucketed per expert, shared expert
//                   first) in LDS, cut into chunks of up to MR_J jobs, and
//                   keeps its own units' chunks; workgroup 0 publishes the
//                   chunk table for the down launch.  Then
//                   h[job][row] = silu(gate . x_t) * (up . x_t)
//                   (llm_moe.adb:124-132), then the shared-expert gate
//                   g_t = sigmoid(shared_gate_inp . x_t) (llm_moe.adb:285-293).
//   moe_down_mf     yk[job][row] = down . h[job].
//   moe_combine_mf  y = sum_k top_w[k] yk[k] (ascending k) + g_t yk[top_k]
//                   (llm_moe.adb:270-299).
//
// A unit of the two expert launches is (chunk, 64-row tile): a workgroup of
// four waves takes one unit at a time, wave w the tile's 16-row block w over every super-block
// column, so no wave waits for another's partial sums.  Each column is
// multiplied by the batch-1 matrix-core arithmetic of 16-row blocks
// (kq_mv_mfma.h: the column's compact activation image, MFMA on
// f16-subnormal codes, scales in f32); the images of the chunk's jobs are
// built once per workgroup in LDS and shared by the four waves.  A wave
// keeps two columns of weights in registers: the next column's loads -- at
// a unit's last column, the next unit's first and its activations -- are in
// flight while the current one is multiplied.  A one-job chunk repeats its job
// in the second slot (every load stays in bounds) and runs the one-job dots.
// Every sum is in a fixed order, so the results are deterministic.
#include <math.h>

#include <algorithm>
#include <map>
#include <mutex>

#include "kq_host.h"
#include "kq_kernels.h"
#include "kq_moe.h"
#include "kq_moe_sched.h"
#include "kq_mv_mfma.h"

namespace kq {

constexpr int MR_J = MOE_MFMA_JPW;  // jobs per chunk
constexpr int MR_GC = 8;            // super-block columns whose images sit in LDS at once
constexpr int MR_THREADS = 256;     // four waves: the 16-row blocks of a tile (HW = 1)

// One activation image: the compact A image of one job's super-block
// column, its sub-block sums, and 1/S.
struct MrImg {
  uint4 q[8][17];
  float xsum[16];
  float invS;
  float pad[3];
};

// ---- the schedule ---------------------------------------------------------------

// Chunk c of the schedule S (chunks are numbered position-major,
// kq_moe_sched.h): {expert, job, job or -1, 0}.
__device__ __forceinline__ int4 mr_chunk_entry(const MoeSched& S, int c, int n_exp) {
  int lo = 0, hi = n_exp;  // the position p with coff[p] <= c < coff[p + 1]
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (S.coff[mid] <= c) lo = mid;
    else hi = mid - 1;
  }
  const int j = S.joff[lo] + (c - S.coff[lo]) * MR_J;
  return make_int4(moe_expert_at(lo, n_exp), S.jobs[j], j + 1 < S.joff[lo + 1] ? S.jobs[j + 1] : -1, 0);
}

// Units a gate/up workgroup takes at most (its grid is sized for it): their
// chunks are kept in LDS once the schedule's tables are overwritten.
constexpr int MR_UNITS_MAX = 32;

// ---- shared pieces of the two expert launches -------------------------------------

// Clears every image once (slot 16 and the unused dwords stay zero: the
// builds rewrite only the data dwords).
__device__ __forceinline__ void mr_clear(MrImg (&img)[MR_J][MR_GC]) {
  uint4* p = &img[0][0].q[0][0];
  constexpr int n = (int)(sizeof(MrImg) * MR_J * MR_GC / 16);
  for (int i = threadIdx.x; i < n; i += blockDim.x) p[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Image (jj, c) of columns g0 .. g0 + gc - 1 is built by wave (jj gc + c) % 4;
// a wave builds at most MR_J * MR_GC / 4 of them.  The activations are
// loaded first (mr_xload), the images built after the workgroup barrier
// (mr_build).
// With NWV = 8 waves (two halves), image (jj, c) is built by wave
// (jj gc + c) % 8, at most MR_J * MR_GC / 8 per wave.
constexpr int MR_BPW = MR_J * MR_GC / 4;

template <int NWV = 4>
__device__ __forceinline__ void mr_xload(float4 (&xv)[MR_BPW], const float* const (&src)[MR_J], int g0, int gc, int w,
                                         int lane) {
#pragma unroll
  for (int k = 0; k < MR_J * MR_GC / NWV; ++k) {
    const int i = w + NWV * k;
    const int ii = i < MR_J * gc ? i : 0;  // past the group: a valid row, unused
    const int jj = ii / gc, c = ii - jj * gc;
    const float* row = jj == 0 ? src[0] : src[1];  // a select, not an indexed (scratch) array
    xv[k] = reinterpret_cast<const float4*>(row + (size_t)(g0 + c) * 256)[lane];
  }
}

template <int KIND, int NWV = 4>
__device__ __forceinline__ void mr_build(MrImg (&img)[MR_J][MR_GC], const float4 (&xv)[MR_BPW], int gc, int nj,
                                         int w, int lane) {
#pragma unroll
  for (int k = 0; k < MR_J * MR_GC / NWV; ++k) {
    const int i = w + NWV * k;
    if (i < nj * gc) {
      const int jj = i / gc, c = i - jj * gc;
      MrImg& m = img[jj][c];
      const MvLane L = mv_lane<KIND, 17>(m.q, lane);
      const float invS = build_image<KIND>(xv[k], L, m.xsum, wave_max_abs_bits(xv[k]));
      if (lane == 0) m.invS = invS;
    }
  }
}

// The dots of NJ jobs with one column of the wave's 16-row block: each
// weight operand is decoded once for all jobs, and the row's scales are
// extracted once (the arithmetic of mv_dot, kq_mv_mfma.h, 16-row case).
template <int KIND, int NJ> struct MrDot;

template <int NJ> struct MrDot<Q4_K, NJ> {
  __device__ static __forceinline__ void run(const MvCol<Q4_K, 1>& c, const MrImg (&img)[MR_J][MR_GC], int ci,
                                             const MvLane& L, int lane, float (&acc)[MR_J]) {
    const int g = lane >> 4;
    mf4 D[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) D[jj] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const uint32_t q = dword_of(j < 4 ? c.a[0] : c.b[0], j & 3);
      const uint32_t t = q >> 8;
      const uint4 B = make_uint4(q & 0x000F000Fu, t & 0x000F000Fu, q & 0x00F000F0u, t & 0x00F000F0u);
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) D[jj] = mfma_f16(img_frag(img[jj][ci].q, j, lane), B, D[jj]);
    }
    const uint4 h = c.h;
    const uint32_t psc = L.upper ? h.w : h.y, pm = L.upper ? h.w : h.z;
    const uint32_t scp = ((psc >> L.b0) & L.m1) | ((h.y >> (L.b0 + 2u)) & L.m2);
    const uint32_t mp = ((pm >> L.mshift) & L.m1) | ((h.z >> (L.b0 + 2u)) & L.m2);
    const float sca = (float)(scp & 0xFFu), scb = (float)((scp >> 8) & 0xFFu);
    const float ma = (float)(mp & 0xFFu), mb = (float)((mp >> 8) & 0xFFu);
    const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(h.x >> 16);
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const float2 X = *reinterpret_cast<const float2*>(&img[jj][ci].xsum[2 * g]);
      const float sa = __builtin_fmaf(D[jj][1], 1.f / 2048.f, D[jj][0]);
      const float sb = __builtin_fmaf(D[jj][3], 1.f / 2048.f, D[jj][2]);
      const float T = __builtin_fmaf(scb, sb, sca * sa);
      const float M = __builtin_fmaf(mb, X.y, ma * X.x);
      acc[jj] = __builtin_fmaf(__builtin_fmaf(d, T, -(dmin * M)), img[jj][ci].invS, acc[jj]);
    }
  }
};

template <int NJ> struct MrDot<Q6_K, NJ> {
  __device__ static __forceinline__ void run(const MvCol<Q6_K, 1>& c, const MrImg (&img)[MR_J][MR_GC], int ci,
                                             const MvLane& L, int lane, float (&acc)[MR_J]) {
    const int g = lane >> 4;
    mf4 D0[NJ], D1[NJ];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) D0[jj] = D1[jj] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t a = dword_of(c.a[0], j), b = dword_of(c.b[0], j), q = dword_of(c.q[0], j);
      // 6-bit codes of sub-blocks k = 0..3 as bytes (as Block<Q6_K>::dot).
      const uint32_t z0 = (a & 0x0F0F0F0Fu) | ((q << 4) & 0x30303030u);
      const uint32_t z1 = (b & 0x0F0F0F0Fu) | ((q << 2) & 0x30303030u);
      const uint32_t z2 = ((a >> 4) & 0x0F0F0F0Fu) | (q & 0x30303030u);
      const uint32_t z3 = ((b >> 4) & 0x0F0F0F0Fu) | ((q >> 2) & 0x30303030u);
      const uint4 B0 = make_uint4(bytes02(z0), bytes13(z0), bytes02(z1), bytes13(z1));
      const uint4 B1 = make_uint4(bytes02(z2), bytes13(z2), bytes02(z3), bytes13(z3));
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        D0[jj] = mfma_f16(img_frag(img[jj][ci].q, j, lane), B0, D0[jj]);
        D1[jj] = mfma_f16(img_frag(img[jj][ci].q, 4 + j, lane), B1, D1[jj]);
      }
    }
    const bool half1 = g >= 2;  // the scales of half 1 are dwords 2, 3 of the scale chunk
    const uint32_t sx = half1 ? c.sc.z : c.sc.x, sy = half1 ? c.sc.w : c.sc.y;
    const int tb = 8 * (g & 1);  // byte t of each scale dword
    const float c0 = (float)(int32_t)__builtin_amdgcn_sbfe(sx, tb, 8);
    const float c1 = (float)(int32_t)__builtin_amdgcn_sbfe(sx, tb + 16, 8);
    const float c2 = (float)(int32_t)__builtin_amdgcn_sbfe(sy, tb, 8);
    const float c3 = (float)(int32_t)__builtin_amdgcn_sbfe(sy, tb + 16, 8);
    const float d = f16_ada(c.d) * 16777216.f;
    constexpr float K32 = 32.f / 16777216.f;
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj) {
      const float4 X = *reinterpret_cast<const float4*>(&img[jj][ci].xsum[4 * g]);  // sub-blocks k = 0..3 of quarter g
      const float s0 = __builtin_fmaf(D0[jj][1], 1.f / 2048.f, D0[jj][0]);
      const float s1 = __builtin_fmaf(D0[jj][3], 1.f / 2048.f, D0[jj][2]);
      const float s2 = __builtin_fmaf(D1[jj][1], 1.f / 2048.f, D1[jj][0]);
      const float s3 = __builtin_fmaf(D1[jj][3], 1.f / 2048.f, D1[jj][2]);
      // The codes are stored offset by 32: sum (q - 32) x = sum q x - 32 sum x.
      float T = c0 * __builtin_fmaf(-K32, X.x, s0);
      T = __builtin_fmaf(c1, __builtin_fmaf(-K32, X.y, s1), T);
      T = __builtin_fmaf(c2, __builtin_fmaf(-K32, X.z, s2), T);
      T = __builtin_fmaf(c3, __builtin_fmaf(-K32, X.w, s3), T);
      acc[jj] = __builtin_fmaf(d * T, img[jj][ci].invS, acc[jj]);
    }
  }
};

// The column's dots for the unit's jobs (one or two).
template <int KIND>
__device__ __forceinline__ void mr_dot(const MvCol<KIND, 1>& c, const MrImg (&img)[MR_J][MR_GC], int ci,
                                       const MvLane& L, int lane, bool two, float (&acc)[MR_J]) {
  if (two) MrDot<KIND, 2>::run(c, img, ci, L, lane, acc);
  else MrDot<KIND, 1>::run(c, img, ci, L, lane, acc);
}

// Lane (n, g) holds quarter g of row n: every lane gets its row's total
// (quarters in ascending order).
__device__ __forceinline__ float mr_rows(float v, int lane) {
  const int n = lane & 15;
  const float q0 = __shfl(v, n), q1 = __shfl(v, n + 16), q2 = __shfl(v, n + 32), q3 = __shfl(v, n + 48);
  return ((q0 + q1) + q2) + q3;
}

// A chunk table entry, read through the scalar cache (the expert launches
// only read the table; scalar loads wait on their own counter, not on the
// weight loads in flight).
typedef const __attribute__((address_space(4))) int* MrTab;
__device__ __forceinline__ int4 mr_chunk(const MoeGroupedArgs& a, int i) {
  const MrTab p = (MrTab)a.units + 4 * i;
  return make_int4(p[0], p[1], p[2], p[3]);
}

// All int: a struct with padding bytes is copied as a byte array the
// compiler keeps in memory (promoted to LDS, whose indexing then reads the
// workgroup size from the dispatch packet -- microseconds at launch).
struct MrUnit {
  int e, tile, job[MR_J];
  int two;
};

__device__ __forceinline__ MrUnit mr_unit(const int4& C, int u, int tiles) {
  MrUnit r;
  r.e = C.x;
  r.tile = u % tiles;
  r.job[0] = C.y;
  r.two = C.z >= 0;
  r.job[1] = r.two ? C.z : C.y;
  return r;
}

// The unit's first column: units start at different columns (tile mod the
// column count) so that the launch's first loads spread over the whole of
// every expert matrix rather than all hitting its first column.  Only when
// every column's image fits at once (one group); otherwise column 0.
__device__ __forceinline__ int mr_rot(const MrUnit& U, int nsb) { return nsb <= MR_GC ? U.tile % nsb : 0; }
__device__ __forceinline__ int mr_col(int s, int rot, int nsb) { return s + rot < nsb ? s + rot : s + rot - nsb; }

// ---- gate/up ----------------------------------------------------------------------

// The combine launch's shared-expert gate g_t (one wave per token), spread
// over the grid.
template <int NWV>
__device__ __forceinline__ void mr_housekeeping(const MoeGroupedArgs& a, int w, int lane) {
  for (int t = blockIdx.x * NWV + w; t < a.T; t += gridDim.x * NWV) {
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

// The activation slices a step prefetches: the images of the group that
// starts at the next step (`real`), or a repeat of slice 0 (cached) that
// keeps every step's load count equal.
template <int NWV>
__device__ __forceinline__ void mr_xnext(float4 (&xv)[MR_BPW], const float* const (&src)[MR_J], bool real, int g0,
                                         int nsb, int w, int lane) {
  mr_xload<NWV>(xv, src, real ? g0 : 0, real ? std::min(MR_GC, nsb - g0) : 1, w, lane);
}

// The column after step s of this wave's half (mr_col order), or at the
// unit's last step the next unit's first column of that half.
template <int HW>
__device__ __forceinline__ int mr_next_col(int s, bool last, int rot, int rotN, int nsb) {
  const int hf = HW == 2 ? __builtin_amdgcn_readfirstlane(threadIdx.x >> 8) : 0;
  return last ? mr_col(2 * hf, rotN, nsb) : mr_col(s + 2 * HW, rot, nsb);
}

template <int KIND>
__global__ __launch_bounds__(MR_THREADS) void moe_gate_up_mf(MoeGroupedArgs a) {
  constexpr int NWV = 4;
  // The schedule's tables, then (once this workgroup's chunks are copied out)
  // the activation images.
  constexpr size_t LDS = sizeof(MrImg) * MR_J * MR_GC > sizeof(MoeSched) ? sizeof(MrImg) * MR_J * MR_GC
                                                                          : sizeof(MoeSched);
  __shared__ __attribute__((aligned(16))) unsigned char lds[LDS];
  __shared__ int4 mine[MR_UNITS_MAX];
  MoeSched& S = *reinterpret_cast<MoeSched*>(lds);
  MrImg(&img)[MR_J][MR_GC] = *reinterpret_cast<MrImg(*)[MR_J][MR_GC]>(lds);
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int slots = a.top_k + 1, nsb = a.dim / 256, tiles = a.I / 64;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  const int units = moe_schedule<MR_J>(a, S) * tiles;
  if (blockIdx.x == 0) {  // the chunk table of the down launch
    for (int c = threadIdx.x; c < units / tiles; c += blockDim.x) a.units[1 + c] = mr_chunk_entry(S, c, a.n_exp);
    if (threadIdx.x == 0) a.units[0] = make_int4(units / tiles, 0, 0, 0);
  }
  for (int k = threadIdx.x; k < MR_UNITS_MAX; k += blockDim.x) {
    const int uk = blockIdx.x + k * (int)gridDim.x;
    if (uk < units) mine[k] = mr_chunk_entry(S, uk / tiles, a.n_exp);
  }
  __syncthreads();  // the tables are no longer read: the LDS takes the images
  int u = blockIdx.x, k = 0;
  if (u >= units) {
    mr_housekeeping<NWV>(a, w, lane);
    return;
  }
  const int4 C = mine[0];
  const auto gbase = [&](const MrUnit& V, const uint8_t* routed, const uint8_t* sh) {
    return (V.e == a.n_exp ? sh : routed + (size_t)V.e * a.gu_stride) + (size_t)V.tile * nsb * GB;
  };
  const auto xrow = [&](const MrUnit& V, int jj) { return a.x + (size_t)(V.job[jj] / slots) * a.dim; };
  MrUnit U = mr_unit(C, u, tiles);
  const float* src[MR_J] = {xrow(U, 0), xrow(U, 1)};
  // First the activations of the first group, then the weights: loads return
  // in order, so the images need not wait for the weights.
  float4 xv[MR_BPW];
  mr_xload<NWV>(xv, src, 0, std::min(MR_GC, nsb), w, lane);
  const uint8_t* G = gbase(U, a.gate, a.sh_gate);
  const uint8_t* P = gbase(U, a.up, a.sh_up);
  int rot = mr_rot(U, nsb);
  MvCol<KIND, 1> g0, u0, g1, u1;
  g0.load(G + (size_t)rot * GB, lane, w);
  u0.load(P + (size_t)rot * GB, lane, w);
  mr_clear(img);
  const MvLane L = mv_lane<KIND, 17>(img[0][0].q, lane);  // the dots use only its scale fields
  for (;;) {
    // The next unit (this one again after the last: its loads go unused).
    const int un = u + (int)gridDim.x;
    const bool more = un < units;
    const int4 CN = mine[more ? k + 1 : k];
    MrUnit N = U;
    const float* srcN[MR_J] = {src[0], src[1]};
    const uint8_t *Gn = G, *Pn = P;
    int rotN = rot;
    float ag[MR_J] = {0.f, 0.f}, au[MR_J] = {0.f, 0.f};
    for (int s = 0; s < nsb; s += 2) {
      const bool group = s % MR_GC == 0;  // MR_GC is even: groups start at even columns
      const int c0 = mr_col(s, rot, nsb), c1 = mr_col(s + 1 < nsb ? s + 1 : s, rot, nsb);
      g1.load(G + (size_t)c1 * GB, lane, w);
      u1.load(P + (size_t)c1 * GB, lane, w);
      if (group) {
        __syncthreads();  // the previous group's images are no longer read
        mr_build<KIND>(img, xv, std::min(MR_GC, nsb - s), U.two ? 2 : 1, w, lane);
        __syncthreads();
      }
      mr_dot<KIND>(g0, img, c0 % MR_GC, L, lane, U.two, ag);
      mr_dot<KIND>(u0, img, c0 % MR_GC, L, lane, U.two, au);
      asm volatile("" ::: "memory");  // the next loads after this column's work
      const bool last = s + 2 >= nsb;
      if (last && more) {
        N = mr_unit(CN, un, tiles);
        srcN[0] = xrow(N, 0);
        srcN[1] = xrow(N, 1);
        Gn = gbase(N, a.gate, a.sh_gate);
        Pn = gbase(N, a.up, a.sh_up);
        rotN = mr_rot(N, nsb);
      }
      const float* const xs[MR_J] = {last ? srcN[0] : src[0], last ? srcN[1] : src[1]};
      mr_xnext<NWV>(xv, xs, last || (s + 2) % MR_GC == 0, last ? 0 : s + 2, nsb, w, lane);
      const size_t off2 = (size_t)(last ? rotN : mr_col(s + 2, rot, nsb)) * GB;
      g0.load((last ? Gn : G) + off2, lane, w);
      u0.load((last ? Pn : P) + off2, lane, w);
      if (s + 1 < nsb) {
        mr_dot<KIND>(g1, img, c1 % MR_GC, L, lane, U.two, ag);
        mr_dot<KIND>(u1, img, c1 % MR_GC, L, lane, U.two, au);
      }
    }
    const int row = U.tile * 64 + 16 * w + (lane & 15), q = lane >> 4;
#pragma unroll
    for (int jj = 0; jj < MR_J; ++jj) {
      const float g = mr_rows(ag[jj], lane), v = mr_rows(au[jj], lane);
      if (q == jj && (jj == 0 || U.two)) a.h[(size_t)U.job[jj] * a.I + row] = (g / (1.0f + expf(-g))) * v;
    }
    if (!more) break;
    u = un;
    ++k;
    U = N;
    src[0] = srcN[0];
    src[1] = srcN[1];
    G = Gn;
    P = Pn;
    rot = rotN;
  }
  mr_housekeeping<NWV>(a, w, lane);
}

// ---- down, then combine --------------------------------------------------------------

// HW = 2 (eight waves): the tile's four 16-row blocks are each walked by two
// waves, half hf taking the column steps s = 2 hf, 2 hf + 4, ... (two
// columns per step), so a unit's columns are in flight twice as wide; the
// halves meet in LDS (half 0's sum first) before yk is written.  Only for
// 3..MR_GC columns (every half has a step, every image fits at once, built at
// the unit's start); HW = 1 walks all columns in one wave per block.
// Measured (Qwen3-MoE layer, down Q6_K 2048x768, so 3 columns): T = 32
// 138.2/139.1 -> 134.7/136.8 us, T = 8 unchanged; the same split of the
// gate/up launch (8 columns) measured T = 8 62.2 -> 67.6 us and is not used.

template <int KIND, int HW>
__global__ __launch_bounds__(MR_THREADS * HW) void moe_down_mf(MoeGroupedArgs a) {
  constexpr int NWV = 4 * HW;
  __shared__ MrImg img[MR_J][MR_GC];
  __shared__ float red[HW == 2 ? 4 * MR_J * 64 : 1];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int wb = w & 3, hf = w >> 2;
  const int nsb = a.I / 256, tiles = a.tiles_dim;
  constexpr int GB = 64 * Block<KIND>::BYTES;
  int u = blockIdx.x;
  const int4 C = mr_chunk(a, 1 + u / tiles);
  const int units = mr_chunk(a, 0).x * tiles;
  if (u >= units) return;
  const auto dbase = [&](const MrUnit& V) {
    return (V.e == a.n_exp ? a.sh_down : a.down + (size_t)V.e * a.d_stride) + (size_t)V.tile * nsb * GB;
  };
  const auto hrow = [&](const MrUnit& V, int jj) { return a.h + (size_t)V.job[jj] * a.I; };
  MrUnit U = mr_unit(C, u, tiles);
  const float* src[MR_J] = {hrow(U, 0), hrow(U, 1)};
  float4 xv[MR_BPW];
  mr_xload<NWV>(xv, src, 0, std::min(MR_GC, nsb), w, lane);
  const uint8_t* D = dbase(U);
  int rot = mr_rot(U, nsb);
  MvCol<KIND, 1> d0, d1;
  d0.load(D + (size_t)mr_col(2 * hf, rot, nsb) * GB, lane, wb);
  mr_clear(img);
  const MvLane L = mv_lane<KIND, 17>(img[0][0].q, lane);
  for (;;) {
    // The next unit (this one again after the last: its loads go unused).
    const int un = u + (int)gridDim.x;
    const bool more = un < units;
    const int4 CN = mr_chunk(a, 1 + (more ? un : u) / tiles);
    MrUnit N = U;
    const float* srcN[MR_J] = {src[0], src[1]};
    const uint8_t* Dn = D;
    int rotN = rot;
    float ad[MR_J] = {0.f, 0.f};
    if (HW == 2) {
      __syncthreads();
      mr_build<KIND, NWV>(img, xv, nsb, U.two ? 2 : 1, w, lane);
      __syncthreads();
    }
    for (int s = 2 * hf; s < nsb; s += 2 * HW) {
      const bool group = HW == 1 && s % MR_GC == 0;
      const int c0 = mr_col(s, rot, nsb), c1 = mr_col(s + 1 < nsb ? s + 1 : s, rot, nsb);
      d1.load(D + (size_t)c1 * GB, lane, wb);
      if (group) {
        __syncthreads();
        mr_build<KIND>(img, xv, std::min(MR_GC, nsb - s), U.two ? 2 : 1, w, lane);
        __syncthreads();
      }
      mr_dot<KIND>(d0, img, c0 % MR_GC, L, lane, U.two, ad);
      asm volatile("" ::: "memory");
      const bool last = s + 2 * HW >= nsb;
      if (last && more) {
        N = mr_unit(CN, un, tiles);
        srcN[0] = hrow(N, 0);
        srcN[1] = hrow(N, 1);
        Dn = dbase(N);
        rotN = mr_rot(N, nsb);
      }
      const float* const xs[MR_J] = {last ? srcN[0] : src[0], last ? srcN[1] : src[1]};
      mr_xnext<NWV>(xv, xs, last || (HW == 1 && (s + 2) % MR_GC == 0), last ? 0 : s + 2, nsb, w, lane);
      d0.load((last ? Dn : D) + (size_t)mr_next_col<HW>(s, last, rot, rotN, nsb) * GB, lane, wb);
      if (s + 1 < nsb) mr_dot<KIND>(d1, img, c1 % MR_GC, L, lane, U.two, ad);
    }
    // yk of the unit's jobs; the combine launch after this one reads them.
    const int row = U.tile * 64 + 16 * wb + (lane & 15), q = lane >> 4;
#pragma unroll
    for (int jj = 0; jj < MR_J; ++jj) {
      float v = mr_rows(ad[jj], lane);
      if (HW == 2) {
        float* r = red + (wb * MR_J + jj) * 64;
        if (hf == 1) r[lane] = v;
        __syncthreads();
        if (hf == 0) v += r[lane];
      }
      if (hf == 0 && q == jj && (jj == 0 || U.two) && row < a.dim) a.yk[(size_t)U.job[jj] * a.dim + row] = v;
    }
    if (!more) break;
    u = un;
    U = N;
    src[0] = srcN[0];
    src[1] = srcN[1];
    D = Dn;
    rot = rotN;
  }
}

// y[t][row] = sum_k top_w[t][k] yk[t slots + k][row] (ascending k) +
// g_t yk[t slots + top_k][row] (llm_moe.adb:270-299); one thread per
// (token, row), yk loads batched eight at a time.  A token with an expert id
// outside [0, n_exp) had a job the schedule dropped: its y is not written.
__global__ __launch_bounds__(256) void moe_combine_mf(MoeGroupedArgs a) {
  const int row = blockIdx.x * 256 + threadIdx.x, t = blockIdx.y;
  if (row >= a.dim) return;
  const int slots = a.top_k + 1;
  const float* yt = a.yk + (size_t)t * slots * a.dim + row;
  const float vs = yt[(size_t)a.top_k * a.dim], gs = a.gsh[t];
  float acc = 0.f;
  bool valid = true;
  for (int k0 = 0; k0 < a.top_k; k0 += 8) {
    float v[8], wk[8];
    int e[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int k = k0 + i < a.top_k ? k0 + i : k0;
      v[i] = yt[(size_t)k * a.dim];
      wk[i] = a.top_w[t * a.top_k + k];
      e[i] = a.idx[t * a.top_k + k];
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      if (k0 + i < a.top_k) acc = acc + wk[i] * v[i];
      valid = valid && e[i] >= 0 && e[i] < a.n_exp;
    }
  }
  if (valid) a.y[(size_t)t * a.dim + row] = acc + gs * vs;
}

// The combine of token t (blockIdx.x), then H[t] += y[t] and
// nx[t] = (H[t] / rms) * w with rms = sqrt(mean(H[t]^2) + 1e-6)
// (LLM_RMSNorm.Forward, src/llm/llm_rmsnorm.adb:10-41): moe_combine_mf's
// arithmetic per element and the one-workgroup norm of the model chain's
// chain_add_norm (256 threads, float4 per thread and step, the same order of
// the sum of squares), so the results are those of the two launches it
// replaces.  A token with an invalid expert id keeps its y, which is still
// added, as the two launches would.
constexpr int MR_NORM_THREADS = 256;
constexpr int MR_NORM_HELD = 4;  // float4 per thread held in registers: rows of up to 4096
__global__ __launch_bounds__(MR_NORM_THREADS) void moe_combine_norm_mf(MoeGroupedArgs a) {
  __shared__ float part[MR_NORM_THREADS / 64];
  __shared__ float wk[MOE_MAX_TOPK];
  const int t = blockIdx.x, slots = a.top_k + 1, n4 = a.dim / 4;
  if ((int)threadIdx.x < a.top_k) wk[threadIdx.x] = a.top_w[t * a.top_k + threadIdx.x];
  const float gs = a.gsh[t];
  bool valid = true;
  for (int k = 0; k < a.top_k; ++k) {
    const int e = a.idx[t * a.top_k + k];
    valid = valid && e >= 0 && e < a.n_exp;
  }
  __syncthreads();
  float4* __restrict__ h = reinterpret_cast<float4*>(a.norm_h + (size_t)t * a.dim);
  float4* __restrict__ y4 = reinterpret_cast<float4*>(a.y + (size_t)t * a.dim);
  const float4* __restrict__ yt = reinterpret_cast<const float4*>(a.yk + (size_t)t * slots * a.dim);
  const float4* __restrict__ w4 = reinterpret_cast<const float4*>(a.norm_w);
  float4* __restrict__ nx = reinterpret_cast<float4*>(a.norm_nx + (size_t)t * a.dim);
  // y = sum_k top_w[k] yk[k] (ascending k) + g_t yk[top_k], then v = H + y.
  const auto sum_row = [&](int i) {
    float4 yv;
    if (valid) {
      float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
      for (int k = 0; k < a.top_k; ++k) {
        const float4 v = yt[(size_t)k * n4 + i];
        const float w = wk[k];
        acc = make_float4(acc.x + w * v.x, acc.y + w * v.y, acc.z + w * v.z, acc.w + w * v.w);
      }
      const float4 vs = yt[(size_t)a.top_k * n4 + i];
      yv = make_float4(acc.x + gs * vs.x, acc.y + gs * vs.y, acc.z + gs * vs.z, acc.w + gs * vs.w);
      y4[i] = yv;
    } else {
      yv = y4[i];
    }
    const float4 hv = h[i];
    const float4 v = make_float4(hv.x + yv.x, hv.y + yv.y, hv.z + yv.z, hv.w + yv.w);
    h[i] = v;
    return v;
  };
  float ss = 0.f;
  const auto square = [&](const float4& v) {
    ss += v.x * v.x;
    ss += v.y * v.y;
    ss += v.z * v.z;
    ss += v.w * v.w;
  };
  float4 held[MR_NORM_HELD];
#pragma unroll
  for (int q = 0; q < MR_NORM_HELD; ++q) {
    const int i = (int)threadIdx.x + q * MR_NORM_THREADS;
    if (i < n4) {
      held[q] = sum_row(i);
      square(held[q]);
    }
  }
  for (int i = (int)threadIdx.x + MR_NORM_HELD * MR_NORM_THREADS; i < n4; i += MR_NORM_THREADS) square(sum_row(i));
  ss = wave_total(ss);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.f;
#pragma unroll
  for (int k = 0; k < MR_NORM_THREADS / 64; ++k) tot += part[k];
  const float rms = sqrtf(tot / (float)a.dim + 1e-6f);
  const auto norm = [&](int i, const float4& v) {
    const float4 g = w4[i];
    nx[i] = make_float4((v.x / rms) * g.x, (v.y / rms) * g.y, (v.z / rms) * g.z, (v.w / rms) * g.w);
  };
#pragma unroll
  for (int q = 0; q < MR_NORM_HELD; ++q) {
    const int i = (int)threadIdx.x + q * MR_NORM_THREADS;
    if (i < n4) norm(i, held[q]);
  }
  for (int i = (int)threadIdx.x + MR_NORM_HELD * MR_NORM_THREADS; i < n4; i += MR_NORM_THREADS) norm(i, h[i]);
}

// ---- launchers ------------------------------------------------------------------

// Resident workgroups of a kernel on the current device (per CU times CUs),
// cached per (kernel, device) once the queries ran cleanly (kq_host.h); 256
// while an error from earlier work on this thread is pending.
static int mmoe_resident(const void* kernel, int threads) {
  static std::mutex mu;
  static std::map<std::pair<const void*, int>, int> cache;
  int dev = 0;
  if (hipPeekAtLastError() != hipSuccess || hipGetDevice(&dev) != hipSuccess) return 256;
  std::lock_guard<std::mutex> lk(mu);
  auto it = cache.find({kernel, dev});
  if (it != cache.end()) return it->second;
  int cus = 0, per = 0;
  if (!query_clean([&] {
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
          cus = 256;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per, kernel, threads, 0) != hipSuccess || per <= 0) per = 1;
      }))
    return 256;
  return cache[{kernel, dev}] = per * cus;
}

// Enough workgroups for every unit the schedule can produce (the chunk
// bound times the tiles), at most what the device keeps resident at once.
static int mr_grid(const MoeGroupedArgs& a, int tiles, const void* kernel, int threads) {
  const long bound = (long)tiles * moe_max_chunks(a.T, a.top_k, std::min(a.n_exp, a.T * a.top_k), MR_J);
  return (int)std::max<long>(1, std::min<long>(bound, mmoe_resident(kernel, threads)));
}

// Two halves per 16-row block of the down launch where every half has a
// column step and the images fit at once (moe_down_mf).
static bool mr_halves(int nsb) { return nsb >= 3 && nsb <= MR_GC; }

// The gate/up launch: also enough workgroups that none takes more than
// MR_UNITS_MAX units.
template <int KIND>
static void launch_gate_up_mf(const MoeGroupedArgs& a, hipStream_t s) {
  const int tiles = a.I / 64;
  const long bound = (long)tiles * moe_max_chunks(a.T, a.top_k, std::min(a.n_exp, a.T * a.top_k), MR_J);
  const int grid = (int)std::max<long>(mr_grid(a, tiles, (const void*)moe_gate_up_mf<KIND>, MR_THREADS),
                                       (bound + MR_UNITS_MAX - 1) / MR_UNITS_MAX);
  hipLaunchKernelGGL(moe_gate_up_mf<KIND>, dim3(grid), dim3(MR_THREADS), 0, s, a);
}

template <int KIND>
static void launch_down_mf(const MoeGroupedArgs& a, hipStream_t s) {
  const int tiles = a.tiles_dim;
  if (mr_halves(a.I / 256))
    hipLaunchKernelGGL((moe_down_mf<KIND, 2>), dim3(mr_grid(a, tiles, (const void*)moe_down_mf<KIND, 2>, 512)),
                       dim3(512), 0, s, a);
  else
    hipLaunchKernelGGL((moe_down_mf<KIND, 1>), dim3(mr_grid(a, tiles, (const void*)moe_down_mf<KIND, 1>, 256)),
                       dim3(256), 0, s, a);
}

bool moe_mfma_kind(int kind) { return kind == Q4_K || kind == Q6_K; }

template <int GK, int DK>
static hipError_t launch_mr(const MoeGroupedArgs& a, hipStream_t s) {
  launch_gate_up_mf<GK>(a, s);
  launch_down_mf<DK>(a, s);
  if (a.norm_h && a.norm_w && a.norm_nx && a.dim % 4 == 0) {
    hipLaunchKernelGGL(moe_combine_norm_mf, dim3(a.T), dim3(MR_NORM_THREADS), 0, s, a);
    if (a.norm_done) *a.norm_done = true;
  } else {
    hipLaunchKernelGGL(moe_combine_mf, dim3((a.dim + 255) / 256, a.T), dim3(256), 0, s, a);
  }
  return hipGetLastError();
}

hipError_t launch_moe_grouped_mfma(const MoeGroupedArgs& a, int gu_kind, int down_kind, hipStream_t s) {
  if (!moe_mfma_kind(gu_kind) || !moe_mfma_kind(down_kind)) return hipErrorNotSupported;
  if (gu_kind == Q4_K) return down_kind == Q4_K ? launch_mr<Q4_K, Q4_K>(a, s) : launch_mr<Q4_K, Q6_K>(a, s);
  return down_kind == Q4_K ? launch_mr<Q6_K, Q4_K>(a, s) : launch_mr<Q6_K, Q6_K>(a, s);
}

}  // namespace kq
