// kq_common.h -- block layouts and device helpers shared by the K-quant kernels.
//
// Super-block byte layouts (256 elements each; ggml block_q*_K, restated from
// src/llm/llm_dequant.adb:110-121, 199-206, 277-289, 329-343, 419-425):
//   Q4_K 144 B: d f16 | dmin f16 | scales[12] | qs[128]
//   Q5_K 176 B: d f16 | dmin f16 | scales[12] | qh[32] | qs[128]
//   Q6_K 210 B: ql[128] | qh[64] | int8 scales[16] | d f16
//   Q3_K 110 B: hmask[32] | qs[64] | scales[12] | d f16
//   Q2_K  84 B: scales[16] | qs[64] | d f16 | dmin f16
//   Q8_0  34 B per 32 elements: d f16 | int8 qs[32]
// Kind codes are LLM_Weight.Kind_Code's (src/llm/llm_weight.adb:277-292).
#pragma once
#ifndef KQ_HOST_EMULATION
#include <hip/hip_runtime.h>
#endif
#include <stdint.h>

namespace kq {

enum Kind : int { Q4_K = 0, Q6_K = 1, Q5_K = 2, Q3_K = 3, Q2_K = 4, Q8_0 = 5 };

__host__ __device__ constexpr int block_bytes(int kind) {
  return kind == Q4_K ? 144 : kind == Q6_K ? 210 : kind == Q5_K ? 176
       : kind == Q3_K ? 110 : kind == Q2_K ? 84 : kind == Q8_0 ? 272 : -1;
}

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Two f16 lanes packed in one dword, reinterpreted.  The K-quant kernels put
// small unsigned codes q into the mantissa of an f16 whose exponent field is
// zero: that half is the subnormal q * 2^-24 (or q * 2^(s-24) when the code
// sits s bits up), exact for q < 1024.  v_fma_mix_f32 then multiplies it by an
// f32 activation with no separate int->float conversion.
__device__ __forceinline__ half2_t as_h2(uint32_t v) { return __builtin_bit_cast(half2_t, v); }

// acc += lo(p) * xa + hi(p) * xb  (two v_fma_mix_f32).
__device__ __forceinline__ float fma_pair(uint32_t p, float xa, float xb, float acc) {
  const half2_t h = as_h2(p);
  acc = __builtin_fmaf((float)h.x, xa, acc);
  return __builtin_fmaf((float)h.y, xb, acc);
}

// IEEE half -> f32 with Aspida's rule that exponent 31 (Inf/NaN) reads as
// +0.0 (F16_To_F32, src/llm/llm_dequant.adb:46-48).  Subnormal and normal
// halves convert exactly.
__device__ __forceinline__ float f16_ada(uint32_t bits16) {
  const float f = (float)__builtin_bit_cast(_Float16, (uint16_t)bits16);
  return __builtin_isfinite(f) ? f : 0.0f;
}

// Unaligned little-endian loads.  Super-blocks of 84/110/210 bytes leave
// fields only 2- or 4-byte aligned; gfx950 serves dword loads at any such
// alignment and the compiler emits global_load_dwordx{1,2,4} for these.
__device__ __forceinline__ uint4 ld16(const uint8_t* p) { uint4 v; __builtin_memcpy(&v, p, 16); return v; }
// A 16-byte-aligned load marked non-temporal: weights streamed once per
// launch need not displace reusable lines in L2 and the Infinity Cache.
typedef unsigned int kq_v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld16nt(const uint8_t* p) {
  const kq_v4u v = __builtin_nontemporal_load(reinterpret_cast<const kq_v4u*>(__builtin_assume_aligned(p, 16)));
  return make_uint4(v.x, v.y, v.z, v.w);
}
typedef unsigned int kq_v2u __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld8nt(const uint8_t* p) {
  const kq_v2u v = __builtin_nontemporal_load(reinterpret_cast<const kq_v2u*>(__builtin_assume_aligned(p, 8)));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint32_t ld4nt(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(__builtin_assume_aligned(p, 4)));
}
__device__ __forceinline__ uint2 ld8(const uint8_t* p) { uint2 v; __builtin_memcpy(&v, p, 8); return v; }
__device__ __forceinline__ uint32_t ld4(const uint8_t* p) { uint32_t v; __builtin_memcpy(&v, p, 4); return v; }
__device__ __forceinline__ uint32_t ld2(const uint8_t* p) { uint16_t v; __builtin_memcpy(&v, p, 2); return v; }

__device__ __forceinline__ uint32_t bfe(uint32_t v, uint32_t off, uint32_t w) {
  return __builtin_amdgcn_ubfe(v, off, w);
}
__device__ __forceinline__ uint32_t rotr(uint32_t v, uint32_t s) {
  return __builtin_amdgcn_alignbit(v, v, s);
}

#ifndef KQ_HOST_EMULATION
// Sum over a wavefront (64 lanes); every lane receives the total.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// DPP lane moves within a wave (no LDS round trip).  dpp_from(v, ctrl, old):
// the value of the source lane that ctrl names, or `old` where there is none.
// Controls: row_shr:n = 0x110 + n (from lane - n within a row of 16),
// row_bcast:15 = 0x142 (lane 15 of the previous row, rows 1 and 3),
// row_bcast:31 = 0x143 (lane 31, rows 2 and 3).
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_from(int v, int old) {
  return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_from(float v, float old) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old), __builtin_bit_cast(int, v),
                                                               CTRL, ROW_MASK, 0xF, false));
}

// Inclusive scan over the 64 lanes (lane l gets v_0 + ... + v_l, added in a
// fixed order); lane 63 holds the total.
template <class T>
__device__ __forceinline__ T wave_scan_add(T v) {
  v += dpp_from<0x111>(v, T(0));
  v += dpp_from<0x112>(v, T(0));
  v += dpp_from<0x114>(v, T(0));
  v += dpp_from<0x118>(v, T(0));
  v += dpp_from<0x142, 0xA>(v, T(0));
  v += dpp_from<0x143, 0xC>(v, T(0));
  return v;
}

// The wave total, in every lane.
__device__ __forceinline__ float wave_total(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wave_scan_add(v)), 63));
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_from<0x111>(v, v));
  v = fmaxf(v, dpp_from<0x112>(v, v));
  v = fmaxf(v, dpp_from<0x114>(v, v));
  v = fmaxf(v, dpp_from<0x118>(v, v));
  v = fmaxf(v, dpp_from<0x142, 0xA>(v, v));
  v = fmaxf(v, dpp_from<0x143, 0xC>(v, v));
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Arg-max over the wave: the largest v, the lowest index among equals
// (NaN never wins; with only NaN left the index stays 0x7fffffff).  Result in
// every lane.
__device__ __forceinline__ void wave_argmax(float& v, int& i) {
#define KQ_ARGMAX_STEP(CTRL, RM)                                   \
  {                                                                \
    const float ov = dpp_from<CTRL, RM>(v, v);                     \
    const int oi = dpp_from<CTRL, RM>(i, i);                       \
    if (ov > v || (ov == v && oi < i)) { v = ov; i = oi; }         \
  }
  KQ_ARGMAX_STEP(0x111, 0xF)
  KQ_ARGMAX_STEP(0x112, 0xF)
  KQ_ARGMAX_STEP(0x114, 0xF)
  KQ_ARGMAX_STEP(0x118, 0xF)
  KQ_ARGMAX_STEP(0x142, 0xA)
  KQ_ARGMAX_STEP(0x143, 0xC)
#undef KQ_ARGMAX_STEP
  v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
  i = __builtin_amdgcn_readlane(i, 63);
}

// The bits of the largest |x| over the wave's float4s, in every lane.
// Non-negative floats order as their bit patterns do, so the reduction is an
// unsigned max on DPP-fused instructions; a NaN sorts above every finite
// value (its column then takes S = 1; its outputs are NaN either way).
__device__ __forceinline__ uint32_t wave_max_abs_bits(float4 v) {
  uint32_t m = max(max(__builtin_bit_cast(uint32_t, v.x) & 0x7FFFFFFFu, __builtin_bit_cast(uint32_t, v.y) & 0x7FFFFFFFu),
                   max(__builtin_bit_cast(uint32_t, v.z) & 0x7FFFFFFFu, __builtin_bit_cast(uint32_t, v.w) & 0x7FFFFFFFu));
  auto step = [](uint32_t a, uint32_t b) { return a > b ? a : b; };
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x111, 0xF, 0xF, true));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x112, 0xF, 0xF, true));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x114, 0xF, 0xF, true));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x118, 0xF, 0xF, true));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x142, 0xA, 0xF, true));
  m = step(m, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)m, 0x143, 0xC, 0xF, true));
  return (uint32_t)__builtin_amdgcn_readlane((int)m, 63);
}
#endif


}  // namespace kq
