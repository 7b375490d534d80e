// kq_mmw.hip -- small-batch (B = 2..64) Q4_K / Q6_K products over the packed
// layout of kq_packed.h with one wave per (64-row tile, super-block column):
// Y[b][out] = sum_k W[out][k] X[b][k].
//
// A pre-pass (kq_xsplit_cols) splits the activations column by column: per
// (row, super-block column) a power of two S brings the column's largest |x|
// just below 2^14, and x S is stored as f16 hi + lo parts, the column's rows
// contiguous.  Each wave then multiplies all 64 rows of its column (four
// 16-row blocks) against the 16 MB activation rows: a 16-row block's decoded
// codes feed every activation block, and each activation fragment, loaded
// from L2 straight into registers, feeds all four row blocks.  The main loop
// has no LDS traffic and no barrier.  The four waves of a workgroup take
// consecutive columns of one tile and add their results in LDS in wave order;
// a tile's column groups (gridDim.y > 1) add theirs through device-scope
// partial sums, the last workgroup to arrive summing them in ascending order.
// Numerics and MFMA lane layouts otherwise follow kq_mmq.hip: codes as f16
// subnormals, exact f16 products, f32 accumulation.
#include <algorithm>

#include "kq_kernels.h"
#include "kq_mmq.h"

namespace kq {

// Split activations, column by column (bp = 16 MB rows, zero past B):
//   xc[s][b][512]  f16 hi (256) then lo (256) of x[b][256 s + i] S_bs, each
//                  quad of elements stored as (0, 2, 1, 3);
//   sc[s][b][32]   f16 hi (16) then lo (16) of XSUM_UNIT times the SUB-element
//                  sums of x S_bs (Q4_K: 8 sums and 8 zeros);
//   ic[s][b]       1 / S_bs.
struct MmwArgs {
  const uint8_t* P;  // packed weights
  int nsb, out_dim, B, bp, spw;  // spw: columns per wave
  const _Float16 *xc, *sc;
  const float* ic;
  float* Y;          // [B][out_dim]
  float* part;       // [ks][ntiles][16 MB][64] partial sums (ks > 1)
  unsigned* count;   // [ntiles] arrival counters
};

// One wave per (row, column): grid (nsb, bp / 4), four rows per workgroup,
// lane l holding elements 4l .. 4l+3 of the column.  S = 2^se with se = 140
// minus the biased exponent of the column's largest |x| (so max |x S| <
// 2^14), at most 120; 0 for an all-zero or non-finite column.
template <int SUB>
__global__ __launch_bounds__(256) void kq_xsplit_cols(const float* __restrict__ X, int B, int bp, int in_dim,
                                                      _Float16* __restrict__ xc, _Float16* __restrict__ sc,
                                                      float* __restrict__ ic) {
  constexpr int QPS = SUB / 4;  // lanes per sub-block
  const int s = blockIdx.x, lane = threadIdx.x & 63;
  const int b = 4 * blockIdx.y + (threadIdx.x >> 6);
  float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
  if (b < B) v = *reinterpret_cast<const float4*>(X + (size_t)b * in_dim + 256 * s + 4 * lane);
  const uint32_t mx = wave_max_abs_bits(v);
  const int se = (mx == 0u || mx >= 0x7F800000u) ? 0 : std::min(140 - (int)(mx >> 23), 120);
  const float S = __builtin_bit_cast(float, (uint32_t)(se + 127) << 23);
  v.x *= S; v.y *= S; v.z *= S; v.w *= S;
  const _Float16 h0 = (_Float16)v.x, h1 = (_Float16)v.y, h2 = (_Float16)v.z, h3 = (_Float16)v.w;
  const _Float16 l0 = (_Float16)(v.x - (float)h0), l1 = (_Float16)(v.y - (float)h1);
  const _Float16 l2 = (_Float16)(v.z - (float)h2), l3 = (_Float16)(v.w - (float)h3);
  _Float16* row = xc + ((size_t)s * bp + b) * 512 + 4 * lane;
  const uint2 ph = make_uint2(pack_h(h0, h2), pack_h(h1, h3)), pl = make_uint2(pack_h(l0, l2), pack_h(l1, l3));
  __builtin_memcpy(row, &ph, 8);
  __builtin_memcpy(row + 256, &pl, 8);
  float sum = (v.x + v.y) + (v.z + v.w);
#pragma unroll
  for (int o = 1; o < QPS; o <<= 1) sum += __shfl_xor(sum, o, 64);
  _Float16* srow = sc + ((size_t)s * bp + b) * 32;
  if (lane % QPS == 0) {
    sum *= XSUM_UNIT;  // |sum| < 32 * 2^14 before this: keep it inside f16's range
    const _Float16 shi = (_Float16)sum;
    srow[lane / QPS] = shi;
    srow[16 + lane / QPS] = (_Float16)(sum - (float)shi);
  }
  // Q4_K: slots 8..15 of each half are zero padding (lanes 32..39: hi, 40..47: lo).
  if (SUB == 32 && lane >= 32 && lane < 48) srow[(lane < 40 ? 8 : 24) + (lane & 7)] = (_Float16)0.f;
  if (lane == 0) ic[(size_t)s * bp + b] = __builtin_bit_cast(float, (uint32_t)(127 - se) << 23);
}

// Floats per activation row of the LDS sum: 64 rows plus 4, so the four lane
// groups of a store land on different banks.
constexpr int MMW_PAD = 68;

// Buffer loads: a wave-uniform base in a buffer resource (scalar registers)
// and 32-bit lane offsets, so the many loads of a column share one base
// instead of each holding a 64-bit address in vector registers.  aux 2 is
// the non-temporal policy (weights, read once).
typedef __amdgpu_buffer_rsrc_t rsrc_t;
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ rsrc_t mmw_rsrc(const void* base) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, -1, 0x00020000);
}
template <int AUX = 0>
__device__ __forceinline__ uint4 bld16(rsrc_t r, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, AUX);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
template <int AUX = 0>
__device__ __forceinline__ uint2 bld8(rsrc_t r, uint32_t vo, uint32_t so) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, AUX);
  return make_uint2(v[0], v[1]);
}
template <int AUX = 0>
__device__ __forceinline__ uint32_t bld4(rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, vo, so, AUX);
}
__device__ __forceinline__ h8 bldh8(rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_bit_cast(h8, __builtin_amdgcn_raw_buffer_load_b128(r, vo, so, 0));
}
__device__ __forceinline__ h4 bldh4(rsrc_t r, uint32_t vo, uint32_t so) {
  return __builtin_bit_cast(h4, __builtin_amdgcn_raw_buffer_load_b64(r, vo, so, 0));
}

// R[rb][mb][r] is this wave's sum for weight row 16 rb + (lane % 16) and
// activation row 16 mb + 4 (lane / 16) + r.  The workgroup adds its four
// waves' sums in wave order; with gridDim.y column groups per tile the
// groups' sums meet as partials, added in ascending group order by the last
// workgroup to arrive.
template <int MB>
__device__ __forceinline__ void mmw_epilogue(const MmwArgs& a, const f4 (&R)[4][MB], float* red) {
  __shared__ unsigned is_last;
  constexpr int BP = 16 * MB, PER = BP * 64 / 256;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, j = lane & 15, q = lane >> 4;
  float* mine = red + w * BP * MMW_PAD;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
      for (int r = 0; r < 4; ++r) mine[(16 * mb + 4 * q + r) * MMW_PAD + 16 * rb + j] = R[rb][mb][r];
  __syncthreads();
  // Thread t owns outputs o = t + 256 i: activation row o / 64, tile row o % 64.
  const int t = threadIdx.x, tile = blockIdx.x, ks = gridDim.y;
  float sum[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = t + 256 * i, at = (o >> 6) * MMW_PAD + (o & 63);
    sum[i] = ((red[at] + red[BP * MMW_PAD + at]) + red[2 * BP * MMW_PAD + at]) + red[3 * BP * MMW_PAD + at];
  }
  if (ks == 1) {
#pragma unroll
    for (int i = 0; i < PER; ++i) {
      const int o = t + 256 * i, b = o >> 6, row = 64 * tile + (o & 63);
      if (b < a.B && row < a.out_dim) a.Y[(size_t)b * a.out_dim + row] = sum[i];
    }
    return;
  }
  const size_t ntiles = gridDim.x;
  float* pp = a.part + ((size_t)blockIdx.y * ntiles + tile) * BP * 64;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    __hip_atomic_store(pp + t + 256 * i, sum[i], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (t == 0)
    is_last = __hip_atomic_fetch_add(&a.count[(size_t)tile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ks - 1)
                  ? 1u
                  : 0u;
  __syncthreads();
  if (!is_last) return;
#pragma unroll
  for (int i = 0; i < PER; ++i)
    sum[i] = __hip_atomic_load(a.part + (size_t)tile * BP * 64 + t + 256 * i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
  for (int k = 1; k < ks; ++k) {
    float v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i)
      v[i] = __hip_atomic_load(a.part + ((size_t)k * ntiles + tile) * BP * 64 + t + 256 * i, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
    for (int i = 0; i < PER; ++i) sum[i] += v[i];
  }
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int o = t + 256 * i, b = o >> 6, row = 64 * tile + (o & 63);
    if (b < a.B && row < a.out_dim) a.Y[(size_t)b * a.out_dim + row] = sum[i];
  }
  if (t == 0) __hip_atomic_store(&a.count[(size_t)tile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Load schedule.  Every load of a column is issued before its first product
// (weights, sums, scales and the activation fragments of all four 64-element
// groups), so the wave waits out the memory latency once per column.
// Scheduling barriers keep the loads there: the scheduler otherwise moves
// each group's loads next to their first use, and the latency (about 2.5 us
// with every wave of the launch loading at once) is paid once per group.
// Activation rows past B are not loaded (their lanes' fragments are zero).
// A wave over several columns keeps a running total besides the column's
// sums and has fewer registers to spare: it loads MMW_AHEAD groups ahead.
template <int KIND, int MB, bool ONE>
constexpr int MMW_AHEAD = ONE ? 4 : MB == 1 ? 3 : (MB == 2 && KIND == Q4_K) ? 2 : 1;

// Q4_K.  Per column: the sub-block scales go into the codes (sc q, exact f16
// subnormals), so each (row block, activation block) pair
// is one MFMA chain over the column's 256 elements, scaled by d once; the
// mins enter through two K=16 MFMAs against the sub-block sums.
template <int MB, bool ONE>
__global__ __launch_bounds__(256) void kq_mmw_q4k(MmwArgs a) {
  constexpr int GB = 64 * 144, BP = 16 * MB, AHEAD = MMW_AHEAD<Q4_K, MB, ONE>;
  __shared__ __attribute__((aligned(16))) float red[4 * BP * MMW_PAD];
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = (4 * blockIdx.y + w) * a.spw;
  const uint8_t* g = a.P + ((size_t)blockIdx.x * a.nsb + c0) * GB;
  // Lane offsets: codes of row j, lane group q (bytes 8q .. 8q+7 of each
  // 32-byte group); activation row j, elements 8q ..; sums 4q .. of row j;
  // scales of rows 4q .. 4q+3.
  const uint32_t vh = 16 * j, vc = 16 * j + 8 * (q & 1) + 1024 * (q >> 1);
  const uint32_t vx = 1024 * j + 16 * q, vs = 64 * j + 8 * q, vi = 16 * q;
  f4 acc[4][MB];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = f4{0.f, 0.f, 0.f, 0.f};
  const int ncol = ONE ? 1 : a.spw;  // one column: the sum is the column's, no running total
  for (int c = 0; c < ncol; ++c, g += GB) {
    const int col = c0 + c;
    const rsrc_t rw = mmw_rsrc(g), rx = mmw_rsrc(a.xc + (size_t)col * a.bp * 512);
    const rsrc_t rs = mmw_rsrc(a.sc + (size_t)col * a.bp * 32), ri = mmw_rsrc(a.ic + (size_t)col * a.bp);
    Q4Regs r[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      r[rb].h = bld16<2>(rw, vh + 256 * rb, 0);
#pragma unroll
      for (int gq = 0; gq < 4; ++gq) r[rb].wc[gq] = bld8<2>(rw, vc + 256 * rb, (1 + 2 * gq) * 1024);
    }
    h4 xs[MB][2];
    f4 inv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xs[mb][0] = bldh4(rs, vs, 1024 * mb);
      xs[mb][1] = bldh4(rs, vs + 32, 1024 * mb);
      inv[mb] = __builtin_bit_cast(f4, bld16(ri, vi, 64 * mb));
    }
    // A[gq][mb]: hi elements 64 gq + 8q .., 64 gq + 32 + 8q .., then lo.
    h8 A[4][MB][4];
    auto load_a = [&](int gq) {
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        const uint32_t so = 16384 * mb;
        if (16 * mb + j < a.B) {
          A[gq][mb][0] = bldh8(rx, vx + 128 * gq, so);
          A[gq][mb][1] = bldh8(rx, vx + 128 * gq + 64, so);
          A[gq][mb][2] = bldh8(rx, vx + 512 + 128 * gq, so);
          A[gq][mb][3] = bldh8(rx, vx + 512 + 128 * gq + 64, so);
        } else {
#pragma unroll
          for (int p = 0; p < 4; ++p) A[gq][mb][p] = h8{};
        }
      }
    };
#pragma unroll
    for (int gq = 0; gq < AHEAD; ++gq) load_a(gq);
    f4 D[4][MB];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) D[rb][mb] = f4{0.f, 0.f, 0.f, 0.f};
    // Scales and mins as bytes (get_scale_min_k4): sub-blocks 0-3 in scl /
    // mnl, 4-7 in sch / mnh.
    uint32_t scl[4], sch[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      scl[rb] = r[rb].h.y & 0x3F3F3F3Fu;
      sch[rb] = (r[rb].h.w & 0x0F0F0F0Fu) | ((r[rb].h.y >> 2) & 0x30303030u);
    }
#pragma unroll
    for (int gq = 0; gq < 4; ++gq) {
      if (gq + AHEAD < 4) load_a(gq + AHEAD);
      __builtin_amdgcn_sched_barrier(0);
      // Codes times their sub-block scale, sc q <= 945: the f16 subnormal
      // bit patterns of sc q 2^-24, from one packed 16-bit multiply per pair
      // (low nibbles: sub-block 2 gq, high: 2 gq + 1).
      const uint32_t sel0 = (gq & 1) ? 0x0C020C02u : 0x0C000C00u, sel1 = sel0 + 0x00010001u;
      h8 bw[4][2];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const uint32_t sc = gq < 2 ? scl[rb] : sch[rb];
        const u16x2 p0 = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, sc, sel0));
        const u16x2 p1 = __builtin_bit_cast(u16x2, __builtin_amdgcn_perm(0u, sc, sel1));
        const uint32_t w0 = r[rb].wc[gq].x, w1 = r[rb].wc[gq].y;
        const uint32_t nib[8] = {w0, w0 >> 8, w1, w1 >> 8, w0 >> 4, w0 >> 12, w1 >> 4, w1 >> 12};
        uint32_t bq[8];
#pragma unroll
        for (int k = 0; k < 8; ++k)
          bq[k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, nib[k] & 0x000F000Fu) * (k < 4 ? p0 : p1));
        bw[rb][0] = as_h8(bq[0], bq[1], bq[2], bq[3]);
        bw[rb][1] = as_h8(bq[4], bq[5], bq[6], bq[7]);
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int p = 0; p < 4; ++p)
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) D[rb][mb] = mfma32(A[gq][mb][p], bw[rb][p & 1], D[rb][mb]);
    }
    __builtin_amdgcn_sched_barrier(0);
    // Min terms: lane group q gives the mins of sub-blocks 4 (q % 2) .. + 3
    // as f16 subnormals m 2^-24 (the sums operand is zero for q >= 2).
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint4 h = r[rb].h;
      const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f;
      const float dmin = f16_ada(h.x >> 16) * (16777216.f / XSUM_UNIT);
      const uint32_t m4 = (q & 1) ? ((h.w >> 4) & 0x0F0F0F0Fu) | ((h.z >> 2) & 0x30303030u) : h.z & 0x3F3F3F3Fu;
      const h4 mins = as_h4(__builtin_amdgcn_perm(0u, m4, 0x0C010C00u), __builtin_amdgcn_perm(0u, m4, 0x0C030C02u));
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f4 Dm = mfma16(xs[mb][0], mins, f4{0.f, 0.f, 0.f, 0.f});
        Dm = mfma16(xs[mb][1], mins, Dm);
        acc[rb][mb] += (d * inv[mb]) * D[rb][mb];
        acc[rb][mb] -= (dmin * inv[mb]) * Dm;
      }
    }
  }
  mmw_epilogue<MB>(a, acc, red);
}

// Q6_K.  16-element sub-blocks with signed 8-bit scales: each sub-block's
// dot (codes 0..63 as f16 subnormals, K = 16 MFMAs) gets a fresh
// accumulator and its scale in f32; the code offset, 32 d sum_s sc_s
// sum_s x, is two K=16 MFMAs of the scales against the sub-block sums.
template <int MB, bool ONE>
__global__ __launch_bounds__(256) void kq_mmw_q6k(MmwArgs a) {
  constexpr int GB = 64 * 210, BP = 16 * MB, AHEAD = MMW_AHEAD<Q6_K, MB, ONE>;
  __shared__ __attribute__((aligned(16))) float red[4 * BP * MMW_PAD];
  const int lane = threadIdx.x & 63, j = lane & 15, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c0 = (4 * blockIdx.y + w) * a.spw;
  const uint8_t* g = a.P + ((size_t)blockIdx.x * a.nsb + c0) * GB;
  // Lane offsets: bytes 4q .. 4q+3 of row j in each code plane; activation
  // row j, elements 4q ..; sums 4q .. of row j; scales of rows 4q .. 4q+3.
  const uint32_t vw = 16 * j + 4 * q, vx = 1024 * j + 8 * q, vs = 64 * j + 8 * q, vi = 16 * q;
  f4 acc[4][MB];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb)
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[rb][mb] = f4{0.f, 0.f, 0.f, 0.f};
  const int ncol = ONE ? 1 : a.spw;  // one column: the sum is the column's, no running total
  for (int c = 0; c < ncol; ++c, g += GB) {
    const int col = c0 + c;
    const rsrc_t rw = mmw_rsrc(g), rx = mmw_rsrc(a.xc + (size_t)col * a.bp * 512);
    const rsrc_t rs = mmw_rsrc(a.sc + (size_t)col * a.bp * 32), ri = mmw_rsrc(a.ic + (size_t)col * a.bp);
    Q6Regs r[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint32_t row = 16 * rb + j;
      r[rb].d = __builtin_amdgcn_raw_buffer_load_b16(rw, 2 * row, 13 * 1024, 2);
      r[rb].sc = bld16<2>(rw, 16 * row, 12 * 1024);
#pragma unroll
      for (int ht = 0; ht < 4; ++ht) {
        const int hh = ht >> 1, t = ht & 1;
        r[rb].wa[ht] = bld4<2>(rw, vw + 256 * rb, (4 * hh + t) * 1024);
        r[rb].wb[ht] = bld4<2>(rw, vw + 256 * rb, (4 * hh + 2 + t) * 1024);
        r[rb].wq[ht] = bld4<2>(rw, vw + 256 * rb, (8 + 2 * hh + t) * 1024);
      }
    }
    h4 xs[MB][2];
    f4 inv[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
      xs[mb][0] = bldh4(rs, vs, 1024 * mb);
      xs[mb][1] = bldh4(rs, vs + 32, 1024 * mb);
      inv[mb] = __builtin_bit_cast(f4, bld16(ri, vi, 64 * mb));
    }
    // X[ht][mb][k], k < 4 hi, k >= 4 lo: elements 128 hh + 16 t + 32 k + 4q ..
    h4 X[4][MB][8];
    auto load_x = [&](int ht) {
      const int xo = 128 * (ht >> 1) + 16 * (ht & 1);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          if (16 * mb + j < a.B) {
            X[ht][mb][k] = bldh4(rx, vx + 2 * (xo + 32 * k), 16384 * mb);
            X[ht][mb][4 + k] = bldh4(rx, vx + 512 + 2 * (xo + 32 * k), 16384 * mb);
          } else {
            X[ht][mb][k] = X[ht][mb][4 + k] = h4{};
          }
        }
    };
#pragma unroll
    for (int ht = 0; ht < AHEAD; ++ht) load_x(ht);
    __builtin_amdgcn_sched_barrier(0);
    f4 cacc[4][MB];  // the column's sum, in units of 1 / S
    // Code offset, -32 d sum_s sc_s xsum_s (lane group q: scales
    // 4q .. 4q+3), before the products: placed after them, it kept every
    // product's result live and spilled.
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
      const uint4 scw = r[rb].sc;
      const uint32_t w4 = q == 0 ? scw.x : q == 1 ? scw.y : q == 2 ? scw.z : scw.w;
      const h4 scb = as_h4(pack_h2((float)(int8_t)(w4 & 0xFF), (float)(int8_t)((w4 >> 8) & 0xFF)),
                           pack_h2((float)(int8_t)((w4 >> 16) & 0xFF), (float)(int8_t)(w4 >> 24)));
      const float off = 32.f * f16_ada(r[rb].d) * (1.f / XSUM_UNIT);
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) {
        f4 Do = mfma16(xs[mb][0], scb, f4{0.f, 0.f, 0.f, 0.f});
        Do = mfma16(xs[mb][1], scb, Do);
        cacc[rb][mb] = -off * Do;
      }
    }
    float d24[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) d24[rb] = f16_ada(r[rb].d) * 16777216.f;
#pragma unroll
    for (int ht = 0; ht < 4; ++ht) {
      if (ht + AHEAD < 4) load_x(ht + AHEAD);
      __builtin_amdgcn_sched_barrier(0);
      const int hh = ht >> 1, t = ht & 1;
      h4 bq[4][4];
      float sc[4][4];
#pragma unroll
      for (int rb = 0; rb < 4; ++rb) {
        const uint32_t A = r[rb].wa[ht], Bw = r[rb].wb[ht], Qw = r[rb].wq[ht];
        const uint32_t z[4] = {(A & 0x0F0F0F0Fu) | ((Qw << 4) & 0x30303030u),
                               (Bw & 0x0F0F0F0Fu) | ((Qw << 2) & 0x30303030u),
                               ((A >> 4) & 0x0F0F0F0Fu) | (Qw & 0x30303030u),
                               ((Bw >> 4) & 0x0F0F0F0Fu) | ((Qw >> 2) & 0x30303030u)};
        const uint32_t sw0 = hh ? r[rb].sc.z : r[rb].sc.x, sw1 = hh ? r[rb].sc.w : r[rb].sc.y;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          bq[rb][k] = as_h4(z[k] & 0x003F003Fu, (z[k] >> 8) & 0x003F003Fu);
          // sub-block 8 hh + 2 k + t: int8 scale byte (2 k + t) of the dword pair (sw0, sw1)
          const uint32_t sw = k < 2 ? sw0 : sw1;
          sc[rb][k] = d24[rb] * (float)(int32_t)__builtin_amdgcn_sbfe(sw, 8 * t + 16 * (k & 1), 8);
        }
      }
#pragma unroll
      for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          f4 Dk[4];
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) Dk[rb] = mfma16(X[ht][mb][k], bq[rb][k], f4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) Dk[rb] = mfma16(X[ht][mb][4 + k], bq[rb][k], Dk[rb]);
#pragma unroll
          for (int rb = 0; rb < 4; ++rb) cacc[rb][mb] += sc[rb][k] * Dk[rb];
        }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int rb = 0; rb < 4; ++rb)
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) acc[rb][mb] += inv[mb] * cacc[rb][mb];
  }
  mmw_epilogue<MB>(a, acc, red);
}

// ---- host side --------------------------------------------------------------

bool mmw_takes(int kind, int in_dim) { return mfma_kind(kind) && in_dim > 0 && in_dim % 1024 == 0; }

// Column groups per tile: the fewest (the most columns per wave, so the
// fewest partial sums) that still give at least MMW_MIN_GROUPS workgroups.
constexpr long MMW_MIN_GROUPS = 512;

int mmw_ks(int in_dim, int out_dim) {
  const int groups = in_dim / 1024, ntiles = (out_dim + 63) / 64;
  const int oks = packed_plan_override_ks();
  if (oks > 0 && groups % oks == 0) return oks;
  for (int ks = 1; ks <= groups; ++ks)
    if (groups % ks == 0 && (long)ntiles * ks >= MMW_MIN_GROUPS) return ks;
  return groups;
}

static int mmw_bpad(int batch) { return 16 * ((std::min(std::max(batch, 1), 64) + 15) / 16); }

// Workspace: xc [nsb][bp][512] and sc [nsb][bp][32] f16, ic [nsb][bp] f32,
// then partials [ks][ntiles][bp][64] f32 when ks > 1.
static size_t mmw_split_bytes(int in_dim, int bp) {
  const size_t nsb = in_dim / 256;
  return (nsb * bp * (512 + 32) * 2 + nsb * bp * 4 + 255) / 256 * 256;
}

size_t mmw_workspace_bytes(int in_dim, int out_dim, int batch) {
  const int bp = mmw_bpad(batch), ks = mmw_ks(in_dim, out_dim), ntiles = (out_dim + 63) / 64;
  size_t n = mmw_split_bytes(in_dim, bp);
  if (ks > 1) n += (size_t)ks * ntiles * bp * 64 * 4;
  return n;
}

hipError_t launch_matmul_mmw(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                             void* work, unsigned* count, hipStream_t s) {
  if (!mmw_takes(kind, in_dim)) return hipErrorNotSupported;
  if (batch < 1 || batch > 64 || out_dim <= 0) return hipErrorInvalidValue;
  const int bp = mmw_bpad(batch), nsb = in_dim / 256, ntiles = (out_dim + 63) / 64;
  const int ks = mmw_ks(in_dim, out_dim), spw = nsb / (4 * ks);
  uint8_t* w = (uint8_t*)work;
  _Float16* xc = (_Float16*)w;
  _Float16* sc = xc + (size_t)nsb * bp * 512;
  float* ic = (float*)(sc + (size_t)nsb * bp * 32);
  float* part = (float*)(w + mmw_split_bytes(in_dim, bp));
  const dim3 sgrid(nsb, bp / 4);
  if (kind == Q4_K)
    hipLaunchKernelGGL(kq_xsplit_cols<32>, sgrid, dim3(256), 0, s, X, batch, bp, in_dim, xc, sc, ic);
  else
    hipLaunchKernelGGL(kq_xsplit_cols<16>, sgrid, dim3(256), 0, s, X, batch, bp, in_dim, xc, sc, ic);
  const MmwArgs a{(const uint8_t*)P, nsb, out_dim, batch, bp, spw, xc, sc, ic, Y, part, count};
  const dim3 grid(ntiles, ks);
#define KQ_MMW(MB)                                                                               \
  case MB:                                                                                       \
    if (kind == Q4_K) {                                                                          \
      if (spw == 1) hipLaunchKernelGGL((kq_mmw_q4k<MB, true>), grid, dim3(256), 0, s, a);         \
      else hipLaunchKernelGGL((kq_mmw_q4k<MB, false>), grid, dim3(256), 0, s, a);                 \
    } else {                                                                                     \
      if (spw == 1) hipLaunchKernelGGL((kq_mmw_q6k<MB, true>), grid, dim3(256), 0, s, a);         \
      else hipLaunchKernelGGL((kq_mmw_q6k<MB, false>), grid, dim3(256), 0, s, a);                 \
    }                                                                                            \
    break;
  switch (bp / 16) {
    KQ_MMW(1) KQ_MMW(2) KQ_MMW(3) KQ_MMW(4)
    default: return hipErrorInvalidValue;
  }
#undef KQ_MMW
  return hipGetLastError();
}

}  // namespace kq
