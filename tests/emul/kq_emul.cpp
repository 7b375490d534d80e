// Host (x86) build of the device block math in aspida_amd/csrc/kq_blocks.h,
// for CPU tests of the kernels' arithmetic against the oracle.  The few AMDGPU
// builtins the block functions use are given their documented semantics here;
// everything else (the f16-subnormal codes, the factorized sums) is the same
// source the GPU compiles.
#include <cmath>
#include <cstdint>
#include <cstring>

#define KQ_HOST_EMULATION 1
#define __device__
#define __host__
#define __forceinline__ inline
#define __shared__

static inline uint32_t __builtin_amdgcn_ubfe(uint32_t v, uint32_t off, uint32_t w) {
  off &= 31; w &= 31;
  return w == 0 ? 0u : (v >> off) & ((1u << w) - 1u);
}
// Result type as the device builtin declares it (unsigned), so a missing
// signed conversion in the kernel source shows up here too.
static inline uint32_t __builtin_amdgcn_sbfe(uint32_t v, uint32_t off, uint32_t w) {
  off &= 31; w &= 31;
  if (w == 0) return 0;
  uint32_t u = (v >> off) & ((1u << w) - 1u);
  return (u >> (w - 1)) ? (u | ~((1u << w) - 1u)) : u;
}
static inline uint32_t __builtin_amdgcn_alignbit(uint32_t a, uint32_t b, uint32_t s) {
  return (uint32_t)((((uint64_t)a << 32) | b) >> (s & 31));
}
struct uint2 { uint32_t x, y; };
struct uint4 { uint32_t x, y, z, w; };
static inline uint2 make_uint2(uint32_t x, uint32_t y) { return {x, y}; }
static inline uint4 make_uint4(uint32_t x, uint32_t y, uint32_t z, uint32_t w) { return {x, y, z, w}; }
using std::max;
using std::min;

#include "../../aspida_amd/csrc/kq_blocks.h"
#include "../../aspida_amd/csrc/kq_packed.h"

extern "C" float kq_emul_quarter(int kind, const uint8_t* sb, int c, const float* xs, const float* xq) {
  switch (kind) {
    case kq::Q4_K: return kq::quarter<kq::Q4_K>(sb, c, xs, xq);
    case kq::Q6_K: return kq::quarter<kq::Q6_K>(sb, c, xs, xq);
    case kq::Q5_K: return kq::quarter<kq::Q5_K>(sb, c, xs, xq);
    case kq::Q3_K: return kq::quarter<kq::Q3_K>(sb, c, xs, xq);
    case kq::Q2_K: return kq::quarter<kq::Q2_K>(sb, c, xs, xq);
    case kq::Q8_0: return kq::quarter<kq::Q8_0>(sb, c, xs, xq);
  }
  return NAN;
}

// The aligned-load helpers on their own: 16 / 12 bytes at p.
extern "C" void kq_emul_ld16e(const uint8_t* p, uint8_t* out) {
  const uint4 v = kq::ld16e(p);
  std::memcpy(out, &v, 16);
}
extern "C" void kq_emul_ld12e(const uint8_t* p, uint8_t* out) {
  const uint4 v = kq::ld12e(p);
  std::memcpy(out, &v, 12);
}

// Packed layout (kq_packed.h): where byte b of row r's super-block lands in
// its 64-row group.
extern "C" int kq_emul_packed_offset(int kind, int r, int b) { return kq::packed_offset(kind, r, b); }

// The 16-row block physical workgroup p of n takes (kq_packed.h).
extern "C" int kq_emul_mv16_block(int p, int n) { return kq::mv16_block(p, n); }

// Row `lane`'s dot over one super-block column of a packed 64-row group, as
// kq_mv_packed forms it: the lane's registers from Packed<K>::load, the four
// quarters from Packed<K>::quarter, activations xs and per-16 sums s16.
template <int K>
static float packed_row(const uint8_t* g, int lane, const float* xs, const float* s16) {
  const typename kq::Packed<K>::R r = kq::Packed<K>::load(g, lane);
  float acc = 0.f;
  for (int q = 0; q < 4; ++q) {
    kq::XQuarter X;
    kq::Block<K>::load_x(xs, s16, q, X);
    acc += kq::Block<K>::dot(kq::Packed<K>::quarter(r, q), q, X);
  }
  return acc;
}

extern "C" float kq_emul_packed_row(int kind, const uint8_t* g, int lane, const float* xs, const float* s16) {
  switch (kind) {
    case kq::Q4_K: return packed_row<kq::Q4_K>(g, lane, xs, s16);
    case kq::Q6_K: return packed_row<kq::Q6_K>(g, lane, xs, s16);
    case kq::Q5_K: return packed_row<kq::Q5_K>(g, lane, xs, s16);
    case kq::Q3_K: return packed_row<kq::Q3_K>(g, lane, xs, s16);
    case kq::Q2_K: return packed_row<kq::Q2_K>(g, lane, xs, s16);
    case kq::Q8_0: return packed_row<kq::Q8_0>(g, lane, xs, s16);
  }
  return NAN;
}
