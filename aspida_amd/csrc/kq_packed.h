// kq_packed.h -- the lane-interleaved ("packed") HBM layout of K-quant
// weights used by the batch-1 decode kernels, and the per-lane register
// image of one super-block in that layout.
//
// A ggml row-major matrix [out][in/256 super-blocks] is regrouped into tiles
// of 64 consecutive rows.  Tile t, super-block column s occupies 64 * BYTES
// contiguous bytes at ((t * nsb) + s) * 64 * BYTES, holding the 64 rows'
// super-blocks of that column:
//   * chunk planes: byte b < 16 * C of row r (0..63) sits at
//       (b / 16) * 1024 + r * 16 + (b % 16),
//     so one 16-byte load per lane reads 1 KB contiguous for the wave;
//   * tail planes: the few bytes past the last whole chunk (the f16 d of
//     Q6_K, the scales and d of Q3_K, d/dmin of Q2_K) are stored as arrays
//     [64][field bytes] after the chunk planes, one plane per field;
//   * Q8_0 (eight 34-byte blocks per 256 elements) places the 32 codes of
//     block j in chunks 2j and 2j+1 and the eight f16 scales in chunk 16.
// The regrouping only moves bytes: every tile holds exactly 64 * BYTES bytes,
// and rows past out_rows in the last tile are zero.  Each lane of a wave then
// owns one row and holds its whole super-block in registers, and every lane
// multiplies the same activations, which the kernels keep in scalar
// registers.
#pragma once
#include "kq_blocks.h"

namespace kq {

template <int KIND> struct Packed;

// Arrival counters of the cross-workgroup sums sit COUNTER_STRIDE unsigned
// apart (256 bytes): device-scope atomics on one cache line serialize
// (about 12 ns each on MI355X), so tiles must not share a line.
constexpr int COUNTER_STRIDE = 64;

// Offset of byte b (0..BYTES-1) of row r's super-block inside its
// (tile, column) group, for the formats whose only irregularity is a tail.
// Returns -1 for bytes a format maps separately.
__host__ __device__ constexpr int packed_offset(int kind, int r, int b) {
  switch (kind) {
    case Q4_K: return (b / 16) * 1024 + r * 16 + (b % 16);
    case Q5_K: return (b / 16) * 1024 + r * 16 + (b % 16);
    case Q6_K:
      return b < 208 ? (b / 16) * 1024 + r * 16 + (b % 16) : 13 * 1024 + r * 2 + (b - 208);
    case Q3_K:
      return b < 96 ? (b / 16) * 1024 + r * 16 + (b % 16)
                    : (b < 108 ? 6 * 1024 + r * 12 + (b - 96) : 6 * 1024 + 768 + r * 2 + (b - 108));
    case Q2_K: return b < 80 ? (b / 16) * 1024 + r * 16 + (b % 16) : 5 * 1024 + r * 4 + (b - 80);
    case Q8_0: {
      const int j = b / 34, o = b % 34;
      return o < 2 ? 16 * 1024 + r * 16 + 2 * j + o : (2 * j + (o - 2) / 16) * 1024 + r * 16 + (o - 2) % 16;
    }
    default: return -1;
  }
}

// The 16-row block a workgroup takes.  Workgroups go to the 8 XCDs round
// robin (workgroup p to XCD p % 8), each XCD with its own L2, and the four
// 16-row blocks of a 64-row tile share the 128-byte lines of the packed
// group's narrow tail planes (Q2_K's 4-byte, Q3_K's 12- and 2-byte, Q6_K's
// 2-byte planes: a quarter or half line per block).  So each whole round of
// 32 workgroups takes 8 tiles, a tile's four blocks on one XCD: p takes tile
// 8 (p / 32) + p % 8, block (p / 8) % 4.  A last partial round keeps p.  A
// permutation of [0, n) whatever the dispatch order (which only decides the
// cache sharing).
__host__ __device__ constexpr int mv16_block(int p, int n) {
  const int full = n & ~31;
  return p < full ? (((p >> 5) << 3) + (p & 7)) * 4 + ((p >> 3) & 3) : p;
}

// Whole-chunk loads of row `lane`'s super-block from the group at g;
// non-temporal (NT) when the launch reads the group once.
template <int C, bool NT = true>
__device__ __forceinline__ void load_chunks(const uint8_t* g, int lane, uint4 (&ch)[C]) {
  const uint8_t* p = g + lane * 16;
#pragma unroll
  for (int k = 0; k < C; ++k) ch[k] = NT ? ld16nt(p + k * 1024) : ld16(p + k * 1024);
}

// Make the compiler treat a register image as changed (it is not): a loop
// that multiplies one super-block by several activation vectors then decodes
// it per use instead of hoisting the whole decoded block (256 floats per
// lane) out of the loop.
template <class R>
__device__ __forceinline__ void opaque_regs(R& r) {
  static_assert(sizeof(R) % 4 == 0, "register image of whole dwords");
  uint32_t w[sizeof(R) / 4];
  __builtin_memcpy(w, &r, sizeof(R));
#pragma unroll
  for (int i = 0; i < (int)(sizeof(R) / 4); ++i) asm volatile("" : "+v"(w[i]));
  __builtin_memcpy(&r, w, sizeof(R));
}

template <> struct Packed<Q4_K> {
  struct R { uint4 ch[9]; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<9, NT>(g, lane, r.ch);
    return r;
  }
  __device__ static __forceinline__ Block<Q4_K>::W quarter(const R& r, int q) {
    return {r.ch[0], r.ch[1 + 2 * q], r.ch[2 + 2 * q]};
  }
};

template <> struct Packed<Q5_K> {
  struct R { uint4 ch[11]; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<11, NT>(g, lane, r.ch);
    return r;
  }
  __device__ static __forceinline__ Block<Q5_K>::W quarter(const R& r, int q) {
    return {r.ch[0], r.ch[1], r.ch[2], r.ch[3 + 2 * q], r.ch[4 + 2 * q]};
  }
};

template <> struct Packed<Q6_K> {
  struct R { uint4 ch[13]; uint32_t d; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<13, NT>(g, lane, r.ch);
    r.d = ld2(g + 13 * 1024 + 2 * lane);
    return r;
  }
  // Quarter c = 2h + t: ql bytes 64h+16t.. and 64h+32+16t.., qh bytes
  // 128+32h+16t.., the 16 scales, d (the ggml offsets of Block<Q6_K>::load_w).
  __device__ static __forceinline__ Block<Q6_K>::W quarter(const R& r, int c) {
    const int h = c >> 1, t = c & 1;
    return {r.ch[4 * h + t], r.ch[4 * h + 2 + t], r.ch[8 + 2 * h + t], r.ch[12], r.d};
  }
};

template <> struct Packed<Q3_K> {
  struct R { uint4 ch[6]; uint4 s; uint32_t d; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<6, NT>(g, lane, r.ch);
    const uint8_t* sp = g + 6 * 1024 + 12 * lane;
    r.s = make_uint4(ld4(sp), ld4(sp + 4), ld4(sp + 8), 0u);
    r.d = ld2(g + 6 * 1024 + 768 + 2 * lane);
    return r;
  }
  // Quarter c = 2nh + g: qs bytes 32+32nh+16g.., hmask bytes 16g.. (ggml offsets).
  __device__ static __forceinline__ Block<Q3_K>::W quarter(const R& r, int c) {
    const int nh = c >> 1, g = c & 1;
    return {r.ch[2 + 2 * nh + g], r.ch[g], r.s, r.d};
  }
};

template <> struct Packed<Q2_K> {
  struct R { uint4 ch[5]; uint32_t d; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<5, NT>(g, lane, r.ch);
    r.d = ld4(g + 5 * 1024 + 4 * lane);
    return r;
  }
  // Quarter c = 2nh + g: qs bytes 16+32nh+16g.., scale bytes 8nh..8nh+7.
  __device__ static __forceinline__ Block<Q2_K>::W quarter(const R& r, int c) {
    const int nh = c >> 1, g = c & 1;
    return {r.ch[1 + 2 * nh + g], nh ? make_uint2(r.ch[0].z, r.ch[0].w) : make_uint2(r.ch[0].x, r.ch[0].y), r.d};
  }
};

template <> struct Packed<Q8_0> {
  struct R { uint4 ch[17]; };
  template <bool NT = true>
  __device__ static __forceinline__ R load(const uint8_t* g, int lane) {
    R r;
    load_chunks<17, NT>(g, lane, r.ch);
    return r;
  }
  // Quarter c owns blocks 2c and 2c+1: codes in chunks 4c..4c+3, scales in
  // dword c of chunk 16.
  __device__ static __forceinline__ Block<Q8_0>::W quarter(const R& r, int c) {
    const uint32_t dw = c == 0 ? r.ch[16].x : c == 1 ? r.ch[16].y : c == 2 ? r.ch[16].z : r.ch[16].w;
    return {r.ch[4 * c], r.ch[4 * c + 1], r.ch[4 * c + 2], r.ch[4 * c + 3], dw & 0xFFFFu, dw >> 16};
  }
};

#ifndef KQ_HOST_EMULATION
// s16[j] = sum of xs[16j .. 16j+15] for the 256 activations at xs (16-byte
// aligned), as wave-uniform values.
__device__ __forceinline__ void sb_sums(const float* __restrict__ xs, int lane, float (&s16)[16]) {
  float4 v;
  __builtin_memcpy(&v, __builtin_assume_aligned(xs + 4 * lane, 16), 16);
  float t = (v.x + v.y) + (v.z + v.w);
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0xB1, 0xF, 0xF, false));
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x4E, 0xF, 0xF, false));
#pragma unroll
  for (int j = 0; j < 16; ++j) s16[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), 4 * j));
}

// One super-block column of row `lane`: sum_i w_i x_i over its 256 elements.
template <int KIND>
__device__ __forceinline__ float sb_dot(const typename Packed<KIND>::R& r, const float* __restrict__ xs, int lane) {
  using B = Block<KIND>;
  float s16[16];
  sb_sums(xs, lane, s16);
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    XQuarter X;
    B::load_x(xs, s16, q, X);
    acc += B::dot(Packed<KIND>::quarter(r, q), q, X);
  }
  return acc;
}

// Activations staged through LDS: a wave that multiplies its super-block
// column by a 256-element activation slice loads the slice as one float4 per
// lane (a single coalesced 1 KB load, which can be issued well ahead), writes
// it to the wave's own LDS slot and reads it back in every lane (broadcast),
// instead of a chain of dependent scalar loads.  Within a wave, LDS
// operations complete in program order, so the slot needs no workgroup
// barrier; wave_barrier keeps the compiler from moving the reads above the
// write.  The per-16 sums the K-quant dots take come from the same float4s.
__device__ __forceinline__ void stage_x256(float4 v, float* __restrict__ slot, int lane, float (&s16)[16]) {
  __builtin_amdgcn_wave_barrier();
  *reinterpret_cast<float4*>(slot + 4 * lane) = v;
  float t = (v.x + v.y) + (v.z + v.w);
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0xB1, 0xF, 0xF, false));
  t += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, t), 0x4E, 0xF, 0xF, false));
#pragma unroll
  for (int j = 0; j < 16; ++j)
    s16[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, t), 4 * j));
  __builtin_amdgcn_wave_barrier();
}

template <int KIND>
__device__ __forceinline__ float staged_dot(const typename Packed<KIND>::R& r, const float* __restrict__ xs,
                                         const float (&s16)[16]) {
  using B = Block<KIND>;
  float acc = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    XQuarter X;
    B::load_x(xs, s16, q, X);
    acc += B::dot(Packed<KIND>::quarter(r, q), q, X);
  }
  return acc;
}

// The gate and up dots over the same staged activations.
template <int KIND>
__device__ __forceinline__ float2 staged_dot2(const typename Packed<KIND>::R& rg, const typename Packed<KIND>::R& ru,
                                           const float* __restrict__ xs, const float (&s16)[16]) {
  using B = Block<KIND>;
  float g = 0.f, u = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    XQuarter X;
    B::load_x(xs, s16, q, X);
    g += B::dot(Packed<KIND>::quarter(rg, q), q, X);
    u += B::dot(Packed<KIND>::quarter(ru, q), q, X);
  }
  return make_float2(g, u);
}
// Sum of the NW waves' partial dots (LDS) and of the tile's ks = gridDim.y
// workgroups (workspace), then y.  `gtile` indexes the workspace and
// counters (tiles of every segment of a launch), `tile` the rows of y.
//
// Cross-workgroup sum ("last arrival"), and why it needs no fence.  Every
// cross-workgroup handoff in this library (partial sums here and in the
// small-batch and resident-chain kernels, router logits, MoE slot outputs)
// follows the same three steps, and rests on the gfx942/gfx950 memory model
// as LLVM's AMDGPU backend implements it (AMDGPUUsage, "Memory Model GFX942"):
//  1. The data are written with agent-scope atomic stores.  At agent scope
//     these are global_store ... sc1: the store is made coherent across the
//     XCDs' separate L2s (written through to memory-side coherence), unlike
//     a plain store, which may stay in one XCD's L2.
//  2. s_waitcnt vmcnt(0): the wave's stores are acknowledged -- for sc1
//     stores that is after they reached the coherence point -- before it
//     issues the agent-scope fetch_add that counts its arrival.
//  3. The workgroup that sees count == ks - 1 reads the data with
//     agent-scope atomic loads (global_load ... sc1, which do not return a
//     stale L2 line).  They are issued only after that fetch_add returned
//     (control dependence through its result), and every other arrival was
//     counted only after its stores were acknowledged in step 2.
// An agent-scope release / acquire pair would add what the backend emits for
// non-atomic data: buffer_wbl2 (write back the whole L2) before the counter
// update and buffer_inv (invalidate it) after -- about ten times this
// epilogue's cost in a first version.  Here no non-atomic data cross
// workgroups, so those are not needed.  The last arrival adds the partials
// in ascending order and re-arms the counter for the next launch.
template <int NW>
__device__ __forceinline__ void mv_epilogue(float acc, int gtile, int tile, int out_rows, float* __restrict__ y,
                                            float* __restrict__ part, unsigned* __restrict__ count) {
  __shared__ float red[NW > 1 ? NW * 64 : 1];
  __shared__ unsigned is_last;
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int ks = gridDim.y;
  if (NW > 1) {
    red[w * 64 + lane] = acc;
    __syncthreads();
    if (w == 0) {
      float t = red[lane];
#pragma unroll
      for (int k = 1; k < NW; ++k) t += red[k * 64 + lane];
      acc = t;
    }
  }
  const int row = tile * 64 + lane;
  if (ks == 1) {
    if (w == 0 && row < out_rows) y[row] = acc;
    return;
  }
  const size_t ntiles = gridDim.x;
  if (w == 0)
    __hip_atomic_store(&part[((size_t)blockIdx.y * ntiles + gtile) * 64 + lane], acc, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0)
    is_last = __hip_atomic_fetch_add(&count[(size_t)gtile * COUNTER_STRIDE], 1u, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT) == (unsigned)(ks - 1)
                  ? 1u
                  : 0u;
  __syncthreads();
  if (is_last && w == 0) {
    // Eight partials in flight at a time, added in ascending k.
    float t = 0.f;
    for (int k0 = 0; k0 < ks; k0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        v[u] = k0 + u < ks ? __hip_atomic_load(&part[((size_t)(k0 + u) * ntiles + gtile) * 64 + lane],
                                                __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : 0.f;
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (k0 + u < ks) t += v[u];
    }
    if (row < out_rows) y[row] = t;
    if (lane == 0)
      __hip_atomic_store(&count[(size_t)gtile * COUNTER_STRIDE], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
#endif  // KQ_HOST_EMULATION

}  // namespace kq
