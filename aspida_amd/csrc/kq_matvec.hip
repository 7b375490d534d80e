// kq_matvec.hip -- batch-1 K-quant matvec kernels for gfx950, plus the dense
// f32 matvec, the bit-exact dequantizer and the small-batch vector-ALU path.
//
// Batch-1 decode is HBM-bound (0.3-0.8 weight bytes per multiply-add), so the
// kernels stream each weight byte exactly once and spend as few VALU
// instructions per element as possible (v_fma_mix_f32 on f16 subnormal codes,
// see kq_blocks.h).  kq_mv_stream keeps every wave resident for the whole
// launch with its activations in registers, and overlaps the next row
// block's loads with the current block's arithmetic.
#include "kq_blocks.h"
#include "kq_elem.h"
#include "kq_kernels.h"

namespace kq {

// xq[i] = x[16i] + x[16i+1] + ... + x[16i+15] (ascending) for i < n16, over
// `rows` activation rows of n16 * 16 elements: the per-group activation sums
// the kernels use for the min / offset terms of each scale sub-block.
__global__ void xsum16(const float* __restrict__ x, int n16, int rows, float* __restrict__ xq) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n16 * rows) return;
  const float* p = x + (size_t)i * 16;
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 16; ++k) s += p[k];
  xq[i] = s;
}

// Row-streaming batch-1 matvec.  A team of nw waves covers one row at a time
// in chunks: wave w of the team owns super-blocks [w*spl, (w+1)*spl) of every
// row (spl a power of two <= 16), four lanes per super-block, so a wave
// covers 64 / (4*spl) rows per step.  Each lane loads the 64 activations of
// its (super-block, quarter) once and keeps them in registers for the whole
// launch; the team then walks row blocks blk = team, team + nteams, ... with
// R rows per lane-group per step, prefetching the next block's weights before
// computing the current one.  The lanes of a row are reduced with xor
// shuffles; with nw > 1 (MULTI) the team's partial sums meet in LDS, one team
// per workgroup so the barriers see identical trip counts.
//
// Every load is issued unconditionally (indices are clamped to valid rows and
// the last prefetch repeats the final block), so the compiler's memory
// wait counts stay static and a step waits only for its own block's bytes.
constexpr int STREAM_MAX_ROWS_STEP = 64;
constexpr int STREAM_MAX_TEAM = 8;  // waves per team (workgroup <= 512 threads)

// Workgroup barrier ordering LDS only: it does not wait for outstanding
// global loads, so prefetched weights stay in flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <int L>
__device__ __forceinline__ float row_sum_pow2(float v) {
#pragma unroll
  for (int o = 1; o < (1 << L); o <<= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// Sum over the 2^lpr_log2 lanes of an aligned group; lpr_log2 is wave-uniform.
__device__ __forceinline__ float row_sum(float v, int lpr_log2) {
  switch (lpr_log2) {
    case 2: return row_sum_pow2<2>(v);
    case 3: return row_sum_pow2<3>(v);
    case 4: return row_sum_pow2<4>(v);
    case 5: return row_sum_pow2<5>(v);
    default: return row_sum_pow2<6>(v);
  }
}

template <int KIND, int R, bool MULTI>
__global__ __launch_bounds__(512) void kq_mv_stream(const uint8_t* __restrict__ W, size_t row_bytes,
                                                    int nsb, int out_rows, const float* __restrict__ x,
                                                    const float* __restrict__ xq, float* __restrict__ y,
                                                    int spl_log2, int nw, int nteams) {
  using B = Block<KIND>;
  __shared__ float red[MULTI ? STREAM_MAX_TEAM * STREAM_MAX_ROWS_STEP : 1];
  const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
  const int tpw = (int)(blockDim.x >> 6) / nw;
  const int w = wv % nw;
  const int team = blockIdx.x * tpw + wv / nw;
  const int lpr_log2 = spl_log2 + 2;  // lanes per row
  const int rslot = lane >> lpr_log2;
  const int within = lane & ((1 << lpr_log2) - 1);
  const int c = within & 3;
  const int sb = (w << spl_log2) + (within >> 2);
  const float live = sb < nsb ? 1.f : 0.f;
  const int sbc = sb < nsb ? sb : nsb - 1;
  const int rows_step = (64 >> lpr_log2) * R;
  const int nblk = (out_rows + rows_step - 1) / rows_step;
  const int nsteps = team < nblk ? (nblk - team + nteams - 1) / nteams : 0;
  if (nsteps == 0) return;  // uniform over the team

  XQuarter xf;
  B::load_x(x + (size_t)sbc * 256, xq + (size_t)sbc * 16, c, xf);
  const uint8_t* wcol = W + (size_t)sbc * B::BYTES;

  typename B::W buf0[R], buf1[R];
  auto load = [&](int i, typename B::W* dst) {
    const int blk = team + min(i, nsteps - 1) * nteams;
    const int r0 = blk * rows_step + rslot * R;
#pragma unroll
    for (int j = 0; j < R; ++j) dst[j] = B::load_w(wcol + (size_t)min(r0 + j, out_rows - 1) * row_bytes, c);
  };
  auto compute = [&](int i, const typename B::W* cur) {
    const int blk = team + i * nteams;
    float acc[R];
#pragma unroll
    for (int j = 0; j < R; ++j) acc[j] = row_sum(live * B::dot(cur[j], c, xf), lpr_log2);
    if (!MULTI) {
      const int r0 = blk * rows_step + rslot * R;
      if (within == 0) {
#pragma unroll
        for (int j = 0; j < R; ++j)
          if (r0 + j < out_rows) y[r0 + j] = acc[j];
      }
    } else {
      if (within == 0) {
#pragma unroll
        for (int j = 0; j < R; ++j) red[w * rows_step + rslot * R + j] = acc[j];
      }
      lds_barrier();
      if ((int)threadIdx.x < rows_step) {
        float s = 0.f;
        for (int k = 0; k < nw; ++k) s += red[k * rows_step + threadIdx.x];
        const int r = blk * rows_step + threadIdx.x;
        if (r < out_rows) y[r] = s;
      }
      lds_barrier();
    }
  };
  load(0, buf0);
  for (int i = 0;; i += 2) {
    load(i + 1, buf1);
    compute(i, buf0);
    if (i + 1 >= nsteps) break;
    load(i + 2, buf0);
    compute(i + 1, buf1);
    if (i + 2 >= nsteps) break;
  }
}

// Small-batch product on the vector ALUs: four lanes per super-block, R rows
// per wave, the weights re-read (from cache) for each activation row.  The
// MFMA kernels cover the shapes where this is slow.
template <int KIND, int R>
__global__ __launch_bounds__(256) void kq_mm_valu(const uint8_t* __restrict__ W, size_t row_bytes,
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
        acc[r] += quarter<KIND>(W + (size_t)min(row0 + r, out_rows - 1) * row_bytes +
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

// ---- bit-exact dequantization (test export): dequant_elem, kq_elem.h.

template <int KIND>
__global__ void kq_dequant(const uint8_t* __restrict__ W, size_t row_bytes, int nsb, int out_rows,
                           float* __restrict__ dst) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  const size_t per_row = (size_t)nsb * 256;
  if (i >= per_row * (size_t)out_rows) return;
  const size_t o = i / per_row, e = i % per_row;
  const uint8_t* sb = W + o * row_bytes + (e / 256) * Block<KIND>::BYTES;
  dst[i] = dequant_elem<KIND>(RowMajorBytes{sb}, (int)(e % 256));
}

// ---- launchers --------------------------------------------------------------

static int num_cus() {
  static int n = [] {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      cus = 256;
    return cus;
  }();
  return n;
}

// Chunk of super-blocks per wave (a power of two <= 16) and waves per team
// for rows of nsb super-blocks: the chunk that leaves the fewest lanes idle,
// the larger one on ties, with at most STREAM_MAX_TEAM waves per team.
// Returns false when nsb exceeds 16 * STREAM_MAX_TEAM.
bool stream_shape(int nsb, int& spl_log2, int& nw) {
  double best = -1.0;
  spl_log2 = 0;
  nw = 0;
  for (int l = 4; l >= 0; --l) {
    const int spl = 1 << l;
    const int n = (nsb + spl - 1) / spl;
    if (n > STREAM_MAX_TEAM) continue;
    const double eff = (double)nsb / (double)(n * spl);
    if (eff > best + 1e-9) { best = eff; spl_log2 = l; nw = n; }
  }
  return nw > 0;
}

MvConfig default_mv_config(int kind, int in_dim, int out_dim) {
  (void)kind;
  (void)in_dim;
  (void)out_dim;
  MvConfig c;
  c.rows_per_wave = 2;
  c.waves_per_cu = 16;
  return c;
}

template <int KIND>
static hipError_t launch_mv_kind(const uint8_t* W, int in_dim, int out_dim, const float* x, const float* xq,
                                 float* y, hipStream_t s, const MvConfig& cfg) {
  const int nsb = in_dim / 256;
  const size_t row_bytes = (size_t)nsb * Block<KIND>::BYTES;
  int spl_log2, nw;
  if (nsb < 1) return hipErrorInvalidValue;
  if (!stream_shape(nsb, spl_log2, nw)) {
    // Rows longer than 32768 elements: the vector-ALU product with one row.
    const int waves = (out_dim + 3) / 4;
    hipLaunchKernelGGL((kq_mm_valu<KIND, 4>), dim3((waves + 3) / 4), dim3(256), 0, s, W, row_bytes, nsb,
                       in_dim, out_dim, 1, x, xq, y);
    return hipGetLastError();
  }
  const int R = cfg.rows_per_wave;
  const int rows_step = (64 >> (spl_log2 + 2)) * R;
  const int nblk = (out_dim + rows_step - 1) / rows_step;
  // One-wave teams share 256-thread workgroups; a multi-wave team has a
  // workgroup to itself, so its barriers only ever wait for its own waves.
  const int tpw = nw == 1 ? 4 : 1;
  const int threads = 64 * nw * tpw;
  int nteams = num_cus() * max(1, cfg.waves_per_cu / nw);
  nteams = min(nteams, nblk);
  nteams = (nteams + tpw - 1) / tpw * tpw;
  const int grid = nteams / tpw;
#define KQ_STREAM_R(RR)                                                                             \
  if (R == RR) {                                                                                    \
    if (nw == 1)                                                                                    \
      hipLaunchKernelGGL((kq_mv_stream<KIND, RR, false>), dim3(grid), dim3(threads), 0, s, W,       \
                         row_bytes, nsb, out_dim, x, xq, y, spl_log2, nw, nteams);                  \
    else                                                                                            \
      hipLaunchKernelGGL((kq_mv_stream<KIND, RR, true>), dim3(grid), dim3(threads), 0, s, W,        \
                         row_bytes, nsb, out_dim, x, xq, y, spl_log2, nw, nteams);                  \
    return hipGetLastError();                                                                       \
  }
  KQ_STREAM_R(1) KQ_STREAM_R(2) KQ_STREAM_R(4)
#undef KQ_STREAM_R
  return hipErrorInvalidValue;
}

hipError_t launch_xsum(const float* x, int in_dim, int rows, float* xq, hipStream_t s) {
  const int n = (in_dim / 16) * rows;
  hipLaunchKernelGGL(xsum16, dim3((n + 255) / 256), dim3(256), 0, s, x, in_dim / 16, rows, xq);
  return hipGetLastError();
}

hipError_t launch_matvec(int kind, const void* W, int in_dim, int out_dim, const float* x, const float* xq,
                         float* y, hipStream_t s, const MvConfig& cfg) {
  const uint8_t* w = (const uint8_t*)W;
  switch (kind) {
    case Q4_K: return launch_mv_kind<Q4_K>(w, in_dim, out_dim, x, xq, y, s, cfg);
    case Q6_K: return launch_mv_kind<Q6_K>(w, in_dim, out_dim, x, xq, y, s, cfg);
    case Q5_K: return launch_mv_kind<Q5_K>(w, in_dim, out_dim, x, xq, y, s, cfg);
    case Q3_K: return launch_mv_kind<Q3_K>(w, in_dim, out_dim, x, xq, y, s, cfg);
    case Q2_K: return launch_mv_kind<Q2_K>(w, in_dim, out_dim, x, xq, y, s, cfg);
    case Q8_0: return launch_mv_kind<Q8_0>(w, in_dim, out_dim, x, xq, y, s, cfg);
    default: return hipErrorInvalidValue;
  }
}

template <int KIND>
static hipError_t launch_mm_kind(const uint8_t* W, int in_dim, int out_dim, int batch, const float* X,
                                 const float* XQ, float* Y, hipStream_t s) {
  const int nsb = in_dim / 256;
  const size_t row_bytes = (size_t)nsb * Block<KIND>::BYTES;
  const int waves = (out_dim + 3) / 4;
  hipLaunchKernelGGL((kq_mm_valu<KIND, 4>), dim3((waves + 3) / 4), dim3(256), 0, s, W, row_bytes, nsb,
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
