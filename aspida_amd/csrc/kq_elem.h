// kq_elem.h -- one dequantized weight: element P of a K-quant super-block,
// computed with the CPU decoder's own operation order and roundings, so the
// f32 bits equal Decode_Q*K_Block's (llm_dequant.adb:122-554).  The block's
// bytes come from a byte source: a row-major ggml block (RowMajorBytes) or
// one row of a packed (tile, column) group (PackedBytes, kq_packed.h).
#pragma once
#include "kq_packed.h"

namespace kq {

struct RowMajorBytes {
  const uint8_t* b;
  __device__ __forceinline__ uint32_t operator()(int i) const { return b[i]; }
};

// Row r of a packed (tile, column) group at g, read through a buffer
// resource (the group's base in scalar registers, 32-bit offsets).
template <int KIND> struct PackedBytes {
  __amdgpu_buffer_rsrc_t g;
  int r;  // row within the tile
  __device__ __forceinline__ PackedBytes(const uint8_t* base, int row)
      : g(__builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(base), (short)0, 64 * Block<KIND>::BYTES, 0x00020000)),
        r(row) {}
  __device__ __forceinline__ uint32_t operator()(int i) const {
    return __builtin_amdgcn_raw_buffer_load_b8(g, packed_offset(KIND, r, i), 0, 0);
  }
};

// Little-endian 16-bit field at byte i.
template <class BY>
__device__ __forceinline__ uint32_t by16(const BY& b, int i) { return b(i) | (b(i + 1) << 8); }

// Q4_K/Q5_K (scale, min) pair j of the 12 scale bytes at byte o (get_scale_min_k4).
template <class BY>
__device__ __forceinline__ void get_sm(const BY& b, int o, int j, int& s, int& m) {
  if (j < 4) {
    s = b(o + j) & 63;
    m = b(o + j + 4) & 63;
  } else {
    s = (b(o + j + 4) & 0x0F) | ((b(o + j - 4) >> 6) << 4);
    m = (b(o + j + 4) >> 4) | ((b(o + j) >> 6) << 4);
  }
}

template <int KIND> struct Elem;

template <> struct Elem<Q4_K> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int g = P / 64, hi = (P % 64) / 32, l = P % 32;
    int s, m;
    get_sm(b, 4, 2 * g + hi, s, m);
    const float d = f16_ada(by16(b, 0)), dmin = f16_ada(by16(b, 2));
    const uint32_t q = b(16 + 32 * g + l);
    const float D = d * (float)s, M = dmin * (float)m;
    return __fsub_rn(__fmul_rn(D, (float)(hi ? (q >> 4) : (q & 15))), M);
  }
};
template <> struct Elem<Q5_K> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int g = P / 64, hi = (P % 64) / 32, l = P % 32;
    int s, m;
    get_sm(b, 4, 2 * g + hi, s, m);
    const float d = f16_ada(by16(b, 0)), dmin = f16_ada(by16(b, 2));
    const uint32_t q = b(48 + 32 * g + l), h = b(16 + l);
    const uint32_t v = (hi ? (q >> 4) : (q & 15)) + (((h >> (2 * g + hi)) & 1u) << 4);
    return __fsub_rn(__fmul_rn(d * (float)s, (float)v), dmin * (float)m);
  }
};
template <> struct Elem<Q6_K> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int h = P / 128, k = (P % 128) / 32, l = P % 32;
    const uint32_t ql = b(64 * h + l + (k & 1) * 32), qh = b(128 + 32 * h + l);
    const uint32_t lo = (k & 2) ? (ql >> 4) : (ql & 15);
    const int q = (int)(lo | (((qh >> (2 * k)) & 3u) << 4)) - 32;
    const int sc = (int8_t)b(192 + 8 * h + l / 16 + 2 * k);
    const float d = f16_ada(by16(b, 208));
    return __fmul_rn(d * (float)sc, (float)q);
  }
};
template <> struct Elem<Q3_K> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int nh = P / 128, j = (P % 128) / 32, g = (P % 32) / 16, l = P % 16;
    const int low2 = (b(32 + 32 * nh + 16 * g + l) >> (2 * j)) & 3;
    const int hbit = (b(16 * g + l) >> (4 * nh + j)) & 1;
    const int is = 8 * nh + 2 * j + g;
    // 6-bit scale is: low nibble from byte is%8 of scales[0..7] (shifted by 4
    // for is >= 8), high two bits from scales[8 + is%4] at bit 2*(is/4).
    const uint32_t lo4 = (b(96 + (is % 8)) >> (4 * (is / 8))) & 15u;
    const uint32_t hi2 = (b(104 + (is % 4)) >> (2 * (is / 4))) & 3u;
    const int sc = (int)(lo4 | (hi2 << 4)) - 32;
    const float d = f16_ada(by16(b, 108));
    return __fmul_rn(__fmul_rn(d, (float)sc), (float)(low2 + 4 * hbit - 4));
  }
};
template <> struct Elem<Q2_K> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int nh = P / 128, j = (P % 128) / 32, g = (P % 32) / 16, l = P % 16;
    const uint32_t sc = b(8 * nh + 2 * j + g);
    const float q = (float)((b(16 + 32 * nh + 16 * g + l) >> (2 * j)) & 3);
    const float d = f16_ada(by16(b, 80)), dmin = f16_ada(by16(b, 82));
    return __fsub_rn(__fmul_rn(d * (float)(sc & 15), q), dmin * (float)(sc >> 4));
  }
};
template <> struct Elem<Q8_0> {
  template <class BY> __device__ static __forceinline__ float at(const BY& b, int P) {
    const int o = 34 * (P / 32);
    return __fmul_rn(f16_ada(by16(b, o)), (float)(int8_t)b(o + 2 + P % 32));
  }
};

template <int KIND, class BY>
__device__ __forceinline__ float dequant_elem(const BY& b, int P) { return Elem<KIND>::at(b, P); }

}  // namespace kq
