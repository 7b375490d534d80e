// kq_matvec.hip -- batch-1 K-quant matvec kernels for gfx950, plus the dense
// f32 matvec, the bit-exact dequantizer and the small-batch fallback.
//
// Batch-1 decode is HBM-bound (0.3-0.8 weight bytes per multiply-add), so the
// kernels stream each weight byte exactly once with 16-byte loads and spend
// as few VALU instructions per element as possible (v_fma_mix_f32 on f16
// subnormal codes, see kq_blocks.h).  Two lane layouts are provided:
//
//  * kq_mv_coal<K, R>: four lanes per super-block, 16 super-blocks per wave
//    step, R rows per wave.  Every load instruction reads contiguous bytes;
//    each lane keeps its 64 activations in registers and reuses them for the
//    R rows.
//  * kq_mv_lanes<K>: one row per lane, 64 rows per wave, all lanes at the same
//    super-block.  The activations are wave-uniform and arrive by scalar
//    loads; the super-block range is split over blockIdx.y and the partial sums
//    are added in a fixed order by kq_mv_reduce.
#include "kq_blocks.h"
#include "kq_kernels.h"

namespace kq {

// xq[i] = x[16i] + x[16i+1] + ... + x[16i+15] (ascending) for i < n16, over
// `rows` activation rows of n16 * 16 elements: the per-group activation sums
// the kernels use for the min / offset terms of each scale sub-block.
__global__ void xsum16(const float* __restrict__ x, int n16, int rows, float* __restrict__ xq) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n16 * rows) return;
  const float4* p = (const float4*)(x + (size_t)i * 16);
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const float4 v = p[k];
    s += v.x; s += v.y; s += v.z; s += v.w;
  }
  xq[i] = s;
}

template <int KIND, int R>
__global__ __launch_bounds__(256) void kq_mv_coal(const uint8_t* __restrict__ W, size_t row_bytes,
                                                  int nsb, int out_rows,
                                                  const float* __restrict__ x,
                                                  const float* __restrict__ xq,
                                                  float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave * R;
  if (row0 >= out_rows) return;
  const int c = lane & 3, slot = lane >> 2;
  const uint8_t* rp[R];
#pragma unroll
  for (int r = 0; r < R; ++r) rp[r] = W + (size_t)min(row0 + r, out_rows - 1) * row_bytes;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  for (int sb = slot; sb < nsb; sb += 16) {
    const float* xs = x + (size_t)sb * 256;
    const float* qs = xq + (size_t)sb * 16;
#pragma unroll
    for (int r = 0; r < R; ++r)
      acc[r] += Block<KIND>::quarter(rp[r] + (size_t)sb * Block<KIND>::BYTES, c, xs, qs);
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < out_rows) y[row0 + r] = v;
  }
}

template <int KIND>
__global__ __launch_bounds__(256) void kq_mv_lanes(const uint8_t* __restrict__ W, size_t row_bytes,
                                                   int nsb, int out_rows, int sb_per_split,
                                                   const float* __restrict__ x,
                                                   const float* __restrict__ xq,
                                                   float* __restrict__ part) {
  const int lane = threadIdx.x & 63;
  const int row = (blockIdx.x * 4 + (threadIdx.x >> 6)) * 64 + lane;
  const int split = blockIdx.y;
  const uint8_t* rp = W + (size_t)min(row, out_rows - 1) * row_bytes;
  const int sb0 = split * sb_per_split;
  const int sb1 = min(nsb, sb0 + sb_per_split);
  float acc = 0.f;
  for (int sb = sb0; sb < sb1; ++sb) {
    const uint8_t* blk = rp + (size_t)sb * Block<KIND>::BYTES;
    const float* xs = x + (size_t)sb * 256;
    const float* qs = xq + (size_t)sb * 16;
#pragma unroll
    for (int c = 0; c < 4; ++c) acc += Block<KIND>::quarter(blk, c, xs, qs);
  }
  if (row < out_rows) part[(size_t)split * out_rows + row] = acc;
}

// y[o] = sum over splits s = 0..nsplit-1 (ascending) of part[s][o].
__global__ void kq_mv_reduce(const float* __restrict__ part, int nsplit, int out_rows,
                             float* __restrict__ y) {
  const int o = blockIdx.x * blockDim.x + threadIdx.x;
  if (o >= out_rows) return;
  float s = 0.f;
  for (int k = 0; k < nsplit; ++k) s += part[(size_t)k * out_rows + o];
  y[o] = s;
}

// Small-batch fallback on the vector ALUs: the weights are read once per
// row-step and applied to every activation row (used when MFMA tiles do not
// pay, and as the reference path for the MFMA kernels).
template <int KIND, int R>
__global__ __launch_bounds__(256) void kq_mm_coal(const uint8_t* __restrict__ W, size_t row_bytes,
                                                  int nsb, int in_dim, int out_rows, int batch,
                                                  const float* __restrict__ X,
                                                  const float* __restrict__ XQ,
                                                  float* __restrict__ Y) {
  const int lane = threadIdx.x & 63;
  const int wave = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int row0 = wave * R;
  if (row0 >= out_rows) return;
  const int c = lane & 3, slot = lane >> 2;
  for (int b = 0; b < batch; ++b) {
    const float* x = X + (size_t)b * in_dim;
    const float* xq = XQ + (size_t)b * (in_dim / 16);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int sb = slot; sb < nsb; sb += 16) {
      const float* xs = x + (size_t)sb * 256;
      const float* qs = xq + (size_t)sb * 16;
#pragma unroll
      for (int r = 0; r < R; ++r)
        acc[r] += Block<KIND>::quarter(W + (size_t)min(row0 + r, out_rows - 1) * row_bytes +
                                           (size_t)sb * Block<KIND>::BYTES, c, xs, qs);
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float v = wave_sum(acc[r]);
      if (lane == 0 && row0 + r < out_rows) Y[(size_t)b * out_rows + row0 + r] = v;
    }
  }
}

// ---- dense f32: y = W x, W row-major [out][in]; one wave per row, float4
// loads when the row is 16-byte aligned (gpu_matvec.cu:903-924 computes the
// same product).
__global__ __launch_bounds__(256) void dense_mv(const float* __restrict__ W, int in_dim, int out_rows,
                                                const float* __restrict__ x, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= out_rows) return;
  const float* r = W + (size_t)row * in_dim;
  float acc = 0.f;
  if ((in_dim & 3) == 0 && (((uintptr_t)r) & 15) == 0 && (((uintptr_t)x) & 15) == 0) {
    const float4* r4 = (const float4*)r;
    const float4* x4 = (const float4*)x;
    const int n4 = in_dim >> 2;
    for (int i = lane; i < n4; i += 64) {
      const float4 a = r4[i], b = x4[i];
      acc = __builtin_fmaf(a.x, b.x, acc);
      acc = __builtin_fmaf(a.y, b.y, acc);
      acc = __builtin_fmaf(a.z, b.z, acc);
      acc = __builtin_fmaf(a.w, b.w, acc);
    }
  } else {
    for (int i = lane; i < in_dim; i += 64) acc = __builtin_fmaf(r[i], x[i], acc);
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// ---- bit-exact dequantization (test export).  Element P of a super-block is
// computed with the CPU decoder's own operation order, one rounding, so the
// f32 bits equal Decode_Q*K_Block's (llm_dequant.adb:122-554).
__device__ __forceinline__ uint32_t byte_at(const uint8_t* p, int i) { return p[i]; }

template <int KIND>
__device__ float dequant_elem(const uint8_t* b, int P);

__device__ __forceinline__ void get_sm(const uint8_t* sc, int j, int& s, int& m) {
  if (j < 4) { s = sc[j] & 63; m = sc[j + 4] & 63; }
  else { s = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4); m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4); }
}

template <> __device__ float dequant_elem<Q4_K>(const uint8_t* b, int P) {
  const int g = P / 64, hi = (P % 64) / 32, l = P % 32;
  int s, m;
  get_sm(b + 4, 2 * g + hi, s, m);
  const float d = f16_ada(ld2(b)), dmin = f16_ada(ld2(b + 2));
  const uint32_t q = b[16 + 32 * g + l];
  const float D = d * (float)s, M = dmin * (float)m;
  return __fsub_rn(__fmul_rn(D, (float)(hi ? (q >> 4) : (q & 15))), M);
}
template <> __device__ float dequant_elem<Q5_K>(const uint8_t* b, int P) {
  const int g = P / 64, hi = (P % 64) / 32, l = P % 32;
  int s, m;
  get_sm(b + 4, 2 * g + hi, s, m);
  const float d = f16_ada(ld2(b)), dmin = f16_ada(ld2(b + 2));
  const uint32_t q = b[48 + 32 * g + l], h = b[16 + l];
  const uint32_t v = (hi ? (q >> 4) : (q & 15)) + (((h >> (2 * g + hi)) & 1u) << 4);
  return __fsub_rn(__fmul_rn(d * (float)s, (float)v), dmin * (float)m);
}
template <> __device__ float dequant_elem<Q6_K>(const uint8_t* b, int P) {
  const int h = P / 128, k = (P % 128) / 32, l = P % 32;
  const uint32_t ql = b[64 * h + l + (k & 1) * 32], qh = b[128 + 32 * h + l];
  const uint32_t lo = (k & 2) ? (ql >> 4) : (ql & 15);
  const int q = (int)(lo | (((qh >> (2 * k)) & 3u) << 4)) - 32;
  const int sc = (int8_t)b[192 + 8 * h + l / 16 + 2 * k];
  const float d = f16_ada(ld2(b + 208));
  return __fmul_rn(d * (float)sc, (float)q);
}
template <> __device__ float dequant_elem<Q3_K>(const uint8_t* b, int P) {
  const int nh = P / 128, j = (P % 128) / 32, g = (P % 32) / 16, l = P % 16;
  const int low2 = (b[32 + 32 * nh + 16 * g + l] >> (2 * j)) & 3;
  const int hbit = (b[16 * g + l] >> (4 * nh + j)) & 1;
  const int is = 8 * nh + 2 * j + g;
  // 6-bit scale is: low nibble from byte is%8 of scales[0..7] (shifted by 4
  // for is >= 8), high two bits from scales[8 + is%4] at bit 2*(is/4).
  const uint32_t lo4 = (b[96 + (is % 8)] >> (4 * (is / 8))) & 15u;
  const uint32_t hi2 = (b[104 + (is % 4)] >> (2 * (is / 4))) & 3u;
  const int sc = (int)(lo4 | (hi2 << 4)) - 32;
  const float d = f16_ada(ld2(b + 108));
  return __fmul_rn(__fmul_rn(d, (float)sc), (float)(low2 + 4 * hbit - 4));
}
template <> __device__ float dequant_elem<Q2_K>(const uint8_t* b, int P) {
  const int nh = P / 128, j = (P % 128) / 32, g = (P % 32) / 16, l = P % 16;
  const uint32_t sc = b[8 * nh + 2 * j + g];
  const float q = (float)((b[16 + 32 * nh + 16 * g + l] >> (2 * j)) & 3);
  const float d = f16_ada(ld2(b + 80)), dmin = f16_ada(ld2(b + 82));
  return __fsub_rn(__fmul_rn(d * (float)(sc & 15), q), dmin * (float)(sc >> 4));
}
template <> __device__ float dequant_elem<Q8_0>(const uint8_t* b, int P) {
  const uint8_t* blk = b + 34 * (P / 32);
  return __fmul_rn(f16_ada(ld2(blk)), (float)(int8_t)blk[2 + P % 32]);
}

template <int KIND>
__global__ void kq_dequant(const uint8_t* __restrict__ W, size_t row_bytes, int nsb, int out_rows,
                           float* __restrict__ dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t per_row = (size_t)nsb * 256;
  if (i >= per_row * (size_t)out_rows) return;
  const size_t o = i / per_row, e = i % per_row;
  const uint8_t* sb = W + o * row_bytes + (e / 256) * Block<KIND>::BYTES;
  dst[i] = dequant_elem<KIND>(sb, (int)(e % 256));
}

// ---- launchers --------------------------------------------------------------

MvConfig default_mv_config(int kind, int in_dim, int out_dim) {
  (void)kind;
  (void)in_dim;
  MvConfig c;
  c.layout = MvLayout::Coalesced;
  // Enough waves to cover 256 CUs several times over, with the largest row
  // reuse that allows it.
  c.rows_per_wave = out_dim >= 8192 ? 4 : 2;
  c.splits = 1;
  return c;
}

size_t mv_part_floats(const MvConfig& cfg, int in_dim, int out_dim) {
  if (cfg.layout != MvLayout::Lanes || cfg.splits <= 1) return 0;
  const int nsb = in_dim / 256;
  const int per = (nsb + cfg.splits - 1) / cfg.splits;
  const int real_splits = (nsb + per - 1) / per;
  return real_splits > 1 ? (size_t)real_splits * out_dim : 0;
}

template <int KIND>
static hipError_t launch_mv_kind(const uint8_t* W, int in_dim, int out_dim, const float* x, const float* xq,
                                 float* y, hipStream_t s, const MvConfig& cfg, float* part) {
  const int nsb = in_dim / 256;
  const size_t row_bytes = (size_t)nsb * Block<KIND>::BYTES;
  if (cfg.layout == MvLayout::Lanes) {
    const int nsplit = cfg.splits > 0 ? cfg.splits : 1;
    const int per = (nsb + nsplit - 1) / nsplit;
    const int real_splits = (nsb + per - 1) / per;
    const int waves = (out_dim + 63) / 64;
    dim3 grid((waves + 3) / 4, real_splits);
    float* dst = real_splits == 1 ? y : part;
    hipLaunchKernelGGL(kq_mv_lanes<KIND>, grid, dim3(256), 0, s, W, row_bytes, nsb, out_dim, per, x, xq, dst);
    if (real_splits > 1)
      hipLaunchKernelGGL(kq_mv_reduce, dim3((out_dim + 255) / 256), dim3(256), 0, s, part, real_splits,
                         out_dim, y);
    return hipGetLastError();
  }
  const int R = cfg.rows_per_wave;
#define KQ_LAUNCH_R(RR)                                                                         \
  if (R == RR) {                                                                                \
    const int waves = (out_dim + RR - 1) / RR;                                                  \
    hipLaunchKernelGGL((kq_mv_coal<KIND, RR>), dim3((waves + 3) / 4), dim3(256), 0, s, W,       \
                       row_bytes, nsb, out_dim, x, xq, y);                                      \
    return hipGetLastError();                                                                   \
  }
  KQ_LAUNCH_R(1) KQ_LAUNCH_R(2) KQ_LAUNCH_R(4) KQ_LAUNCH_R(8)
#undef KQ_LAUNCH_R
  return hipErrorInvalidValue;
}

hipError_t launch_xsum(const float* x, int in_dim, int rows, float* xq, hipStream_t s) {
  const int n = (in_dim / 16) * rows;
  hipLaunchKernelGGL(xsum16, dim3((n + 255) / 256), dim3(256), 0, s, x, in_dim / 16, rows, xq);
  return hipGetLastError();
}

hipError_t launch_matvec(int kind, const void* W, int in_dim, int out_dim, const float* x, const float* xq,
                         float* y, hipStream_t s, const MvConfig& cfg, float* part) {
  const uint8_t* w = (const uint8_t*)W;
  switch (kind) {
    case Q4_K: return launch_mv_kind<Q4_K>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    case Q6_K: return launch_mv_kind<Q6_K>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    case Q5_K: return launch_mv_kind<Q5_K>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    case Q3_K: return launch_mv_kind<Q3_K>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    case Q2_K: return launch_mv_kind<Q2_K>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    case Q8_0: return launch_mv_kind<Q8_0>(w, in_dim, out_dim, x, xq, y, s, cfg, part);
    default: return hipErrorInvalidValue;
  }
}

template <int KIND>
static hipError_t launch_mm_kind(const uint8_t* W, int in_dim, int out_dim, int batch, const float* X,
                                 const float* XQ, float* Y, hipStream_t s) {
  const int nsb = in_dim / 256;
  const size_t row_bytes = (size_t)nsb * Block<KIND>::BYTES;
  const int waves = (out_dim + 3) / 4;
  hipLaunchKernelGGL((kq_mm_coal<KIND, 4>), dim3((waves + 3) / 4), dim3(256), 0, s, W, row_bytes, nsb,
                     in_dim, out_dim, batch, X, XQ, Y);
  return hipGetLastError();
}

hipError_t launch_matmul_valu(int kind, const void* W, int in_dim, int out_dim, int batch, const float* X,
                              const float* XQ, float* Y, hipStream_t s) {
  const uint8_t* w = (const uint8_t*)W;
  switch (kind) {
    case Q4_K: return launch_mm_kind<Q4_K>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    case Q6_K: return launch_mm_kind<Q6_K>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    case Q5_K: return launch_mm_kind<Q5_K>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    case Q3_K: return launch_mm_kind<Q3_K>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    case Q2_K: return launch_mm_kind<Q2_K>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    case Q8_0: return launch_mm_kind<Q8_0>(w, in_dim, out_dim, batch, X, XQ, Y, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_dense(const float* W, int in_dim, int out_dim, const float* x, float* y, hipStream_t s) {
  hipLaunchKernelGGL(dense_mv, dim3((out_dim + 3) / 4), dim3(256), 0, s, W, in_dim, out_dim, x, y);
  return hipGetLastError();
}

hipError_t launch_dequant(int kind, const void* W, int in_dim, int out_dim, float* dst, hipStream_t s) {
  const uint8_t* w = (const uint8_t*)W;
  const int nsb = in_dim / 256;
  const size_t n = (size_t)out_dim * in_dim;
  const dim3 grid((unsigned)((n + 255) / 256));
#define KQ_DQ(K)                                                                                   \
  case K:                                                                                          \
    hipLaunchKernelGGL(kq_dequant<K>, grid, dim3(256), 0, s, w, (size_t)nsb * block_bytes(K), nsb, \
                       out_dim, dst);                                                              \
    return hipGetLastError();
  switch (kind) {
    KQ_DQ(Q4_K) KQ_DQ(Q6_K) KQ_DQ(Q5_K) KQ_DQ(Q3_K) KQ_DQ(Q2_K) KQ_DQ(Q8_0)
    default: return hipErrorInvalidValue;
  }
#undef KQ_DQ
}

}  // namespace kq
