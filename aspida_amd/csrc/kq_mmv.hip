// kq_mmv.hip -- small-batch products Y[b][out] = W X[b], 2 <= B <= 64, over
// packed Q4_K and Q6_K weights on the matrix cores, with the batch-1
// kernels' work split (kq_mv_mfma.hip): a workgroup takes RB 16-row blocks
// (a 16-row block, or a whole 64-row tile) over every super-block column,
// its NW waves split the columns, and the waves meet in LDS only -- no
// partial sums through memory and no activation pre-pass.  Each weight byte
// is read once per launch for up to 64 vectors.
//
// One v_mfma_f32_16x16x32_f16 (Q4_K) or v_mfma_f32_16x16x16_f16 (Q6_K) per
// scale sub-block is dense in both dimensions: A = the 16 vectors of a
// group's activations of that sub-block (rows = vectors), B = the codes of
// the 16 weight rows of a block (as in kq_mm16.hip).  Each wave converts its
// column's activations itself, per group of 16 vectors: x S (S a power of two
// putting the vector's largest |x| in the column just below 2^14) split into
// f16 hi (round toward zero) and lo = (x S - hi) 2^11 -- x to about 2^-22
// relative, as in every matrix-core kernel of this library -- laid out as
// the MFMA's A operands in registers.
//
// Q4_K: B = code x sub-block scale as f16 subnormals (q sc 2^-24, q sc <=
// 945, exact); the minimum term dmin sum_t m_t X_t is one more MFMA per
// sub-block of the same A against B = m_t (all k).  Q6_K: B = the signed
// code q - 32 as the f16 subnormal (q - 32) 2^-24 (exact), so no offset
// term; each sub-block's sum is scaled by its int8 scale in f32.
//
// Result per row: Decode_Q4K_Block (src/llm/llm_dequant.adb:536-553) or
// Decode_Q6K_Block (122-184) dotted with each vector (QMatVec,
// llm_dequant.adb:808-932, once per vector); the products are exact, the
// sums are the matrix cores' f32 sums in another order than the CPU's.
#include <algorithm>

#include "kq_host.h"
#include "kq_kernels.h"
#include "kq_mv_mfma.h"

namespace kq {

typedef _Float16 mmv_h4 __attribute__((ext_vector_type(4)));
typedef unsigned short mmv_u2 __attribute__((ext_vector_type(2)));

struct MmvArgs {
  const uint8_t* P;  // packed weights
  int nsb, out_rows, B, spw;
  const float* X;    // [B][nsb * 256]
  float* Y;          // [B][out_rows]
};

__device__ __forceinline__ mf4 mfma_k16(uint2 a, uint2 b, mf4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(mmv_h4, a), __builtin_bit_cast(mmv_h4, b), c, 0, 0,
                                               0);
}

// The pair (hi, lo) of two scaled activations: hi = f16(a S) and f16(b S)
// rounded toward zero, lo = f16 of the exact remainders times 2^11.
__device__ __forceinline__ void mmv_split(float a, float b, float S, float S11, uint32_t& hi, uint32_t& lo) {
  const auto h = __builtin_amdgcn_cvt_pkrtz(a * S, b * S);
  const float ra = __builtin_fmaf((float)h.x, -2048.f, a * S11);
  const float rb = __builtin_fmaf((float)h.y, -2048.f, b * S11);
  hi = __builtin_bit_cast(uint32_t, h);
  lo = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(ra, rb));
}

// Column activations of one group of 16 vectors as A operands.  Lane (b, kg)
// (b = lane % 16, kg = lane / 16) reads vector v0 + b (zero when v0 + b >= B).
//   Q4_K: sub-block t (elements 32 t .. 32 t + 31): elements 32 t + 8 kg +
//         {0, 2, 1, 3, 4, 6, 5, 7}, hi in ah[t], lo in al[t].
//   Q6_K: sub-block s (elements 16 s .. + 15): elements 16 s + 4 kq +
//         {0, 2, 1, 3} (kq = kg), hi in .x .y, lo in .z .w of a6[s].
// Returns 1/S of vector v0 + b (every lane of that vector).
template <int KIND> struct MmvX;

// Sum over the four lane rows (lanes l, l ^ 16, l ^ 32, l ^ 48) with the
// gfx950 row swaps, no LDS.
__device__ __forceinline__ float mmv_rows_sum(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

// Sub-block sums of x S (|.| <= 32 2^14) times this fit f16.
constexpr float MMV_XSUM = 1.f / 64.f;
// Largest scale exponent: S 2^11 = 2^(se + 11) must stay a finite f32 (a
// column whose largest |x| is below 2^-102 takes S = 2^116, its values then
// at most 2^10 after scaling, still far inside f16's range).
constexpr int MMV_SE_MAX = 116;

template <> struct MmvX<Q4_K> {
  uint4 ah[8], al[8];
  // The K = 16 A operand of the minimum term: lane (b, kq < 2) holds the
  // sums of sub-blocks 4 kq .. + 3 of vector b (times MMV_XSUM), hi in .x .y,
  // lo (times 2^11) in .z .w; zero for kq >= 2.
  uint4 as;
  __device__ __forceinline__ float build(const float* __restrict__ X, int in_dim, int B, int v0, int col, int lane) {
    const int b = lane & 15, kg = lane >> 4, v = v0 + b;
    float4 x[16];
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)(v < B ? v : 0) * in_dim + (size_t)col * 256 + 8 * kg);
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      x[2 * t] = v < B ? p[8 * t] : make_float4(0.f, 0.f, 0.f, 0.f);
      x[2 * t + 1] = v < B ? p[8 * t + 1] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[i].x), fabsf(x[i].y)), fmaxf(fabsf(x[i].z), fabsf(x[i].w))));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    int e = 0;
    const bool scaled = mx > 0.f && __builtin_isfinite(mx);
    if (scaled) (void)frexpf(mx, &e);
    const int se = scaled ? std::min(std::max(14 - e, -120), MMV_SE_MAX) : 0;
    const float S = ldexpf(1.f, se), S11 = ldexpf(1.f, se + 11);
    float su[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const float4 a = x[2 * t], c = x[2 * t + 1];
      uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
      mmv_split(a.x, a.z, S, S11, h0, l0);  // elements 0, 2
      mmv_split(a.y, a.w, S, S11, h1, l1);  // 1, 3
      mmv_split(c.x, c.z, S, S11, h2, l2);  // 4, 6
      mmv_split(c.y, c.w, S, S11, h3, l3);  // 5, 7
      ah[t] = make_uint4(h0, h1, h2, h3);
      al[t] = make_uint4(l0, l1, l2, l3);
      su[t] = (((a.x + a.y) + (a.z + a.w)) + ((c.x + c.y) + (c.z + c.w))) * S;
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) su[t] = mmv_rows_sum(su[t]) * MMV_XSUM;
    const int t0 = 4 * (kg & 1);
    _Float16 h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float v = kg < 2 ? (t0 ? su[4 + i] : su[i]) : 0.f;
      h[i] = (_Float16)v;
      l[i] = (_Float16)((v - (float)h[i]) * 2048.f);
    }
    as = make_uint4(pack_f16x2(h[0], h[1]), pack_f16x2(h[2], h[3]), pack_f16x2(l[0], l[1]), pack_f16x2(l[2], l[3]));
    return ldexpf(1.f, -se);
  }
};

template <> struct MmvX<Q6_K> {
  uint4 a6[16];
  __device__ __forceinline__ float build(const float* __restrict__ X, int in_dim, int B, int v0, int col, int lane) {
    const int b = lane & 15, kq = lane >> 4, v = v0 + b;
    float4 x[16];
    const float4* p = reinterpret_cast<const float4*>(X + (size_t)(v < B ? v : 0) * in_dim + (size_t)col * 256 + 4 * kq);
#pragma unroll
    for (int s = 0; s < 16; ++s) x[s] = v < B ? p[4 * s] : make_float4(0.f, 0.f, 0.f, 0.f);
    float mx = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[i].x), fabsf(x[i].y)), fmaxf(fabsf(x[i].z), fabsf(x[i].w))));
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    int e = 0;
    const bool scaled = mx > 0.f && __builtin_isfinite(mx);
    if (scaled) (void)frexpf(mx, &e);
    const int se = scaled ? std::min(std::max(14 - e, -120), MMV_SE_MAX) : 0;
    const float S = ldexpf(1.f, se), S11 = ldexpf(1.f, se + 11);
#pragma unroll
    for (int s = 0; s < 16; ++s) {
      uint32_t h0, l0, h1, l1;
      mmv_split(x[s].x, x[s].z, S, S11, h0, l0);  // elements 0, 2
      mmv_split(x[s].y, x[s].w, S, S11, h1, l1);  // 1, 3
      a6[s] = make_uint4(h0, h1, l0, l1);
    }
    return ldexpf(1.f, -se);
  }
};

// Staged conversion of a group of GV <= 4 vectors (GV = 8 also works): lane l converts vector
// v0 + l / (64 / GV), elements E c .. E c + E - 1 (E = 4 GV, c = l % (64 / GV))
// -- every lane busy, E elements each instead of 64 -- into the wave's LDS
// planes in A order (position 8 m + j holds element 8 m + ord[j], ord =
// 0 2 1 3 4 6 5 7, the pair order of the codes), then each lane reads its A
// operands (rows b >= GV are zero).  Same scale S per (vector, column), the
// same hi / lo split and, for Q4_K, the same sub-block sums as the direct
// build above.
// A vector's planes are 33 chunks of 16 bytes apart, so the 16 vectors a
// quarter-wave reads sit in distinct banks.
template <int GV>
struct MmvStage {
  uint4 hi[GV][33], lo[GV][33];  // 256 f16 per vector and plane (+ 1 pad)
  float sum[GV][8];              // sub-block sums of x S (Q4_K)
  float inv[16];                 // 1/S per vector of the group (zero past GV)
};

template <int LPV>
__device__ __forceinline__ float mmv_group_max(float v) {
#pragma unroll
  for (int o = 1; o < LPV; o <<= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

template <int KIND, int GV>
__device__ __forceinline__ void mmv_build_staged(MmvX<KIND>& A, MmvStage<GV>& st, const float* __restrict__ X,
                                                 int in_dim, int B, int v0, int col, int lane) {
  constexpr int LPV = 64 / GV, E = 4 * GV;
  const int vw = lane / LPV, c = lane % LPV, v = v0 + vw;
  float4 x[E / 4];
  const float4* p = reinterpret_cast<const float4*>(X + (size_t)(v < B ? v : 0) * in_dim + (size_t)col * 256 + E * c);
#pragma unroll
  for (int i = 0; i < E / 4; ++i) x[i] = v < B ? p[i] : make_float4(0.f, 0.f, 0.f, 0.f);
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < E / 4; ++i) mx = fmaxf(mx, fmaxf(fmaxf(fabsf(x[i].x), fabsf(x[i].y)), fmaxf(fabsf(x[i].z), fabsf(x[i].w))));
  mx = mmv_group_max<LPV>(mx);
  int e = 0;
  const bool scaled = mx > 0.f && __builtin_isfinite(mx);
  if (scaled) (void)frexpf(mx, &e);
  const int se = scaled ? std::min(std::max(14 - e, -120), MMV_SE_MAX) : 0;
  const float S = ldexpf(1.f, se), S11 = ldexpf(1.f, se + 11);
  float su = 0.f;
#pragma unroll
  for (int k = 0; k < E / 8; ++k) {
    const float4 a = x[2 * k], b = x[2 * k + 1];
    uint32_t h0, l0, h1, l1, h2, l2, h3, l3;
    mmv_split(a.x, a.z, S, S11, h0, l0);  // elements 0, 2
    mmv_split(a.y, a.w, S, S11, h1, l1);  // 1, 3
    mmv_split(b.x, b.z, S, S11, h2, l2);  // 4, 6
    mmv_split(b.y, b.w, S, S11, h3, l3);  // 5, 7
    st.hi[vw][E / 8 * c + k] = make_uint4(h0, h1, h2, h3);
    st.lo[vw][E / 8 * c + k] = make_uint4(l0, l1, l2, l3);
    if constexpr (KIND == Q4_K) su += (((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w))) * S;
  }
  if constexpr (KIND == Q4_K) {
    // Sub-block t = elements 32 t .. + 31: 32 / E lanes of the vector.
#pragma unroll
    for (int o = 1; o < 32 / E; o <<= 1) su += __shfl_xor(su, o, 64);
    if (c % (32 / E) == 0) st.sum[vw][c / (32 / E)] = su;
  }
  if (c == 0) st.inv[vw] = ldexpf(1.f, -se);
  if (lane >= GV && lane < 16) st.inv[lane] = 0.f;
  __builtin_amdgcn_wave_barrier();
  const int b = lane & 15, kg = lane >> 4;
  const bool has = b < GV;
  const int bb = has ? b : 0;
  if constexpr (KIND == Q4_K) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const uint4 h = st.hi[bb][4 * t + kg], l = st.lo[bb][4 * t + kg];
      A.ah[t] = has ? h : make_uint4(0u, 0u, 0u, 0u);
      A.al[t] = has ? l : make_uint4(0u, 0u, 0u, 0u);
    }
    const int t0 = 4 * (kg & 1);
    _Float16 h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float u = has && kg < 2 ? st.sum[bb][t0 + i] * MMV_XSUM : 0.f;
      h[i] = (_Float16)u;
      l[i] = (_Float16)((u - (float)h[i]) * 2048.f);
    }
    A.as = make_uint4(pack_f16x2(h[0], h[1]), pack_f16x2(h[2], h[3]), pack_f16x2(l[0], l[1]), pack_f16x2(l[2], l[3]));
  } else {
    const uint2* h2 = reinterpret_cast<const uint2*>(&st.hi[bb][0]);
    const uint2* l2 = reinterpret_cast<const uint2*>(&st.lo[bb][0]);
#pragma unroll
    for (int sb = 0; sb < 16; ++sb) {
      const uint2 h = h2[4 * sb + kg], l = l2[4 * sb + kg];
      A.a6[sb] = has ? make_uint4(h.x, h.y, l.x, l.y) : make_uint4(0u, 0u, 0u, 0u);
    }
  }
}

// One 16-row block's weights of a column as lane (n, kg) loads them (row r =
// 16 rbb + n of the 64-row group at grp).
template <int KIND> struct MmvW;

template <> struct MmvW<Q4_K> {
  uint4 h;      // d, dmin, the 12 scale bytes of row r
  uint2 wq[4];  // qs bytes 32 g + 8 kg .. + 7 of row r, g = 0..3
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int rbb, int lane) {
    const int n = lane & 15, kg = lane >> 4, r = 16 * rbb + n;
    h = ld16(grp + r * 16);
#pragma unroll
    for (int g = 0; g < 4; ++g) wq[g] = ld8nt(grp + (1 + 2 * g + (kg >> 1)) * 1024 + r * 16 + 8 * (kg & 1));
  }
};

template <> struct MmvW<Q6_K> {
  uint32_t ql[8], qh[4];  // bytes 4 kq .. + 3 of chunks 0..7 and 8..11 of row r
  uint4 sc;               // the 16 int8 scales of row r
  uint32_t d;             // d of row r (low 16 bits)
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int rbb, int lane) {
    const int n = lane & 15, kq = lane >> 4, r = 16 * rbb + n;
    const uint8_t* p = grp + r * 16 + 4 * kq;
#pragma unroll
    for (int c = 0; c < 8; ++c) ql[c] = ld4nt(p + c * 1024);
#pragma unroll
    for (int c = 0; c < 4; ++c) qh[c] = ld4nt(p + (8 + c) * 1024);
    sc = ld16(grp + 12 * 1024 + r * 16);
    d = ld2(grp + 13 * 1024 + 2 * r);
  }
};

// acc[i] (vector 4 (lane / 16) + i of the group, row lane % 16 of the block)
// += this column's dots times 1/S of those vectors.
__device__ __forceinline__ void mmv_dot(const MmvW<Q4_K>& W, const MmvX<Q4_K>& A, const float4& iv, float (&acc)[4]) {
  const uint4 hh = W.h;
  // Scales and mins as bytes (get_scale_min_k4, llm_dequant.adb:514-525):
  // sub-blocks 0-3 in scl/mnl, 4-7 in sch/mnh.
  const uint32_t scl = hh.y & 0x3F3F3F3Fu, mnl = hh.z & 0x3F3F3F3Fu;
  const uint32_t sch = (hh.w & 0x0F0F0F0Fu) | ((hh.y >> 2) & 0x30303030u);
  const uint32_t mnh = ((hh.w >> 4) & 0x0F0F0F0Fu) | ((hh.z >> 2) & 0x30303030u);
  mf4 dh = {0.f, 0.f, 0.f, 0.f}, dl = dh;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t sc = g < 2 ? scl : sch;
    const uint32_t sel0 = (g & 1) ? 0x0C020C02u : 0x0C000C00u, sel1 = sel0 + 0x00010001u;
    const mmv_u2 p0 = __builtin_bit_cast(mmv_u2, __builtin_amdgcn_perm(0u, sc, sel0));
    const mmv_u2 p1 = __builtin_bit_cast(mmv_u2, __builtin_amdgcn_perm(0u, sc, sel1));
    const uint32_t w0 = W.wq[g].x, w1 = W.wq[g].y;
    const uint32_t nib[8] = {w0, w0 >> 8, w1, w1 >> 8, w0 >> 4, w0 >> 12, w1 >> 4, w1 >> 12};
    uint32_t bq[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      bq[k] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(mmv_u2, nib[k] & 0x000F000Fu) * (k < 4 ? p0 : p1));
    const uint4 blo = make_uint4(bq[0], bq[1], bq[2], bq[3]), bhi = make_uint4(bq[4], bq[5], bq[6], bq[7]);
    dh = mfma_f16(A.ah[2 * g], blo, dh);
    dl = mfma_f16(A.al[2 * g], blo, dl);
    dh = mfma_f16(A.ah[2 * g + 1], bhi, dh);
    dl = mfma_f16(A.al[2 * g + 1], bhi, dl);
  }
  // Minimum terms sum_t m_t X_t: lane (n, kq) gives the mins of sub-blocks
  // 4 (kq % 2) .. + 3 as f16 subnormals m 2^-24 (the sums operand is zero for
  // kq >= 2, so those lanes' values drop out).
  const int kq = (threadIdx.x & 63) >> 4;
  const uint32_t m4 = (kq & 1) ? mnh : mnl;
  const uint2 bm = make_uint2(__builtin_amdgcn_perm(0u, m4, 0x0c010c00u), __builtin_amdgcn_perm(0u, m4, 0x0c030c02u));
  const mf4 z4 = {0.f, 0.f, 0.f, 0.f};
  const mf4 mh = mfma_k16(make_uint2(A.as.x, A.as.y), bm, z4), ml = mfma_k16(make_uint2(A.as.z, A.as.w), bm, z4);
  const float d = f16_ada(hh.x & 0xFFFFu) * 16777216.f;
  const float dmin = f16_ada(hh.x >> 16) * (16777216.f / MMV_XSUM);
  const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float dt = __builtin_fmaf(dl[i], 1.f / 2048.f, dh[i]);
    const float mt = __builtin_fmaf(ml[i], 1.f / 2048.f, mh[i]);
    acc[i] = __builtin_fmaf(__builtin_fmaf(-dmin, mt, d * dt), ivs[i], acc[i]);
  }
}

__device__ __forceinline__ void mmv_dot(const MmvW<Q6_K>& W, const MmvX<Q6_K>& A, const float4& iv, float (&acc)[4]) {
  const uint32_t hs[4] = {W.sc.x, W.sc.y, W.sc.z, W.sc.w};
  const mf4 z4 = {0.f, 0.f, 0.f, 0.f};
  // (q - 32) 2^-24 from q 2^-24: one packed f16 subtraction, exact.
  const _Float16 k32 = (_Float16)(32.f / 16777216.f);
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 off = {k32, k32};
  float th[4] = {0.f, 0.f, 0.f, 0.f}, tl[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sb = 0; sb < 16; ++sb) {
    const int hh = sb >> 3, k = (sb >> 1) & 3, t = sb & 1;
    const uint32_t lw = W.ql[4 * hh + 2 * (k & 1) + t], hw = W.qh[2 * hh + t];
    // 6-bit codes of elements 4 kq .. + 3 as bytes, then f16 pairs {0, 2}, {1, 3}.
    const uint32_t zc = (((k >> 1) ? (lw >> 4) : lw) & 0x0F0F0F0Fu) | (((hw >> (2 * k)) & 0x03030303u) << 4);
    const h2 q02 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(zc, zc, 0x0C020C00u)) - off;
    const h2 q13 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(zc, zc, 0x0C030C01u)) - off;
    const uint2 bq = make_uint2(__builtin_bit_cast(uint32_t, q02), __builtin_bit_cast(uint32_t, q13));
    const mf4 dh = mfma_k16(make_uint2(A.a6[sb].x, A.a6[sb].y), bq, z4);
    const mf4 dl = mfma_k16(make_uint2(A.a6[sb].z, A.a6[sb].w), bq, z4);
    const float sc = (float)(int)__builtin_amdgcn_sbfe(hs[sb >> 2], 8 * (sb & 3), 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      th[i] = __builtin_fmaf(sc, dh[i], th[i]);
      tl[i] = __builtin_fmaf(sc, dl[i], tl[i]);
    }
  }
  const float d = f16_ada(W.d) * 16777216.f;
  const float ivs[4] = {iv.x, iv.y, iv.z, iv.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) acc[i] = __builtin_fmaf(d * __builtin_fmaf(tl[i], 1.f / 2048.f, th[i]), ivs[i], acc[i]);
}

// Workgroup: RB 16-row blocks (RB = 1: block b = mv16_block(blockIdx.x),
// block b % 4 of tile b / 4; RB = 4: tile blockIdx.x) over every column, NW waves each
// taking columns w spw .. + spw - 1 one after another, NG groups of GV
// vectors per column (weights loaded once for all of them).  GV = 16 builds
// the A operands directly in registers; GV = 2 and 4 (batches of up to 4 on
// at most 8 waves) stage them through LDS: measured on MI355X, 14336x4096
// at 2 vectors 15.2 -> 12.5 us (Q4_K), 4 vectors 27.6 -> 19.9 us (Q6_K);
// at 8 vectors the staged build was slower than the direct one.
template <int KIND, int RB, int NW, int NG, int GV>
__global__ __launch_bounds__(64 * NW) void kq_mmv(MmvArgs a) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
  __shared__ float red[NW][256];
  __shared__ float sinv[NW][16];
  __shared__ MmvStage<GV < 16 ? GV : 1> stage[GV < 16 ? NW : 1];
  const int lane = threadIdx.x & 63, q = lane >> 4;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int b16 = RB == 4 ? 0 : mv16_block(blockIdx.x, gridDim.x);
  const int tile = RB == 4 ? blockIdx.x : b16 >> 2, rb0 = RB == 4 ? 0 : b16 & 3;
  const int in_dim = a.nsb * 256;
  float acc[RB][NG][4];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int g = 0; g < NG; ++g)
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[rb][g][i] = 0.f;
  for (int s = 0; s < a.spw; ++s) {
    const int col = w * a.spw + s;
    const uint8_t* grp = a.P + ((size_t)tile * a.nsb + col) * GB;
    asm volatile("" ::: "memory");  // this column's loads after the previous column's work
    MmvW<KIND> W[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) W[rb].load(grp, rb0 + rb, lane);
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (GV * g < a.B) {
        MmvX<KIND> A;
        float4 iv;
        __builtin_amdgcn_wave_barrier();
        if constexpr (GV < 16) {
          mmv_build_staged<KIND, GV>(A, stage[w], a.X, in_dim, a.B, GV * g, col, lane);
          iv = *reinterpret_cast<const float4*>(&stage[w].inv[4 * q]);
        } else {
          const float inv = A.build(a.X, in_dim, a.B, 16 * g, col, lane);
          if (lane < 16) sinv[w][lane] = inv;
          __builtin_amdgcn_wave_barrier();
          iv = *reinterpret_cast<const float4*>(&sinv[w][4 * q]);
        }
        __builtin_amdgcn_wave_barrier();
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) mmv_dot(W[rb], A, iv, acc[rb][g]);
      }
    }
  }
  // The waves' sums, ascending w: per (block, group), thread t < 256 owns
  // vector GV g + 4 (t % 64 / 16) + t / 64 of row t % 16 of the block.
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int g = 0; g < NG; ++g) {
      if (GV * g >= a.B) continue;
#pragma unroll
      for (int i = 0; i < 4; ++i) red[w][i * 64 + lane] = acc[rb][g][i];
      __syncthreads();
      for (int t = threadIdx.x; t < 256; t += 64 * NW) {
        float sum = red[0][t];
#pragma unroll
        for (int k = 1; k < NW; ++k) sum += red[k][t];
        const int l = t & 63, vi = 4 * (l >> 4) + (t >> 6), v = GV * g + vi;
        const int row = tile * 64 + 16 * (rb0 + rb) + (l & 15);
        if (vi < GV && v < a.B && row < a.out_rows) a.Y[(size_t)v * a.out_rows + row] = sum;
      }
      __syncthreads();
    }
}

// ---- host ---------------------------------------------------------------------

bool mmv_kind(int kind) { return kind == Q4_K || kind == Q6_K; }

// Whole 64-row tiles per workgroup when they nearly fill the device (the
// activations are then converted once per 64 rows), else 16-row blocks;
// waves: the largest of 8, 4, 2, 1 dividing the columns (16 waves would cap
// a wave at 128 registers).
struct MmvPlan {
  int rb, nw, spw;
};
static int mmv_cus() {
  static OnceQuery<int> q;
  return q.get(
      [] {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0)
          c = 256;
        return c;
      },
      256);
}
static MmvPlan mmv_plan(int kind, int in_dim, int out_dim, int ng) {
  const int nsb = in_dim / 256, tiles = (out_dim + 63) / 64;
  MmvPlan p{tiles * 4 >= 3 * mmv_cus() ? 4 : 1, 1, nsb};
  for (int nw : {16, 8, 4, 2}) {
    // 16 waves cap a wave at 128 registers: only Q4_K, 16-row blocks, one group fit.
    if (nw == 16 && (kind != Q4_K || p.rb != 1 || ng != 1)) continue;
    if (nsb % nw == 0) {
      p.nw = nw;
      break;
    }
  }
  p.spw = nsb / p.nw;
  return p;
}

// Q6_K 14336x4096 on MI355X: 64 vectors in one 4-wave launch 124.7 us, in
// two 8-wave launches of 32 2 x 44.5 us.
int mmv_step(int kind, int in_dim, int out_dim) {
  return kind == Q6_K && mmv_plan(kind, in_dim, out_dim, 4).rb == 4 ? 32 : 64;
}

hipError_t launch_matmul_mmv(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                             hipStream_t s) {
  if (!mmv_kind(kind)) return hipErrorNotSupported;
  if (batch < 1 || batch > 64 || in_dim <= 0 || in_dim % 256 || out_dim <= 0 || ((uintptr_t)X & 15))
    return hipErrorInvalidValue;
  const int ng = (batch + 15) / 16;
  MmvPlan p = mmv_plan(kind, in_dim, out_dim, ng);
  const int tiles = (out_dim + 63) / 64;
  const dim3 grid(p.rb == 4 ? tiles : (out_dim + 15) / 16);
  // Q6_K on 64-row tiles with four groups: 4 waves (8 spill registers).
  if (kind == Q6_K && p.rb == 4 && ng == 4 && p.nw == 8) {
    p.nw = 4;
    p.spw *= 2;
  }
  const MmvArgs a{(const uint8_t*)P, in_dim / 256, out_dim, batch, p.spw, X, Y};
#define KQ_MMV(K, RB, NW, NG, GV) hipLaunchKernelGGL((kq_mmv<K, RB, NW, NG, GV>), grid, dim3(64 * NW), 0, s, a)
#define KQ_MMV_NG(K, RB, NW)                    \
  if (batch <= 2) KQ_MMV(K, RB, NW, 1, 2);      \
  else if (batch <= 4) KQ_MMV(K, RB, NW, 1, 4); \
  else switch (ng) {                            \
      case 1: KQ_MMV(K, RB, NW, 1, 16); break;  \
      case 2: KQ_MMV(K, RB, NW, 2, 16); break;  \
      case 3: KQ_MMV(K, RB, NW, 3, 16); break;  \
      default: KQ_MMV(K, RB, NW, 4, 16); break; \
    }
#define KQ_MMV_NW(K, RB)                             \
  switch (p.nw) {                                    \
    case 8: KQ_MMV_NG(K, RB, 8) break;               \
    case 4: KQ_MMV_NG(K, RB, 4) break;               \
    case 2: KQ_MMV_NG(K, RB, 2) break;               \
    default: KQ_MMV_NG(K, RB, 1) break;              \
  }
  if (kind == Q4_K) {
    if (p.nw == 16) KQ_MMV(Q4_K, 1, 16, 1, 16);
    else if (p.rb == 4) KQ_MMV_NW(Q4_K, 4) else KQ_MMV_NW(Q4_K, 1)
  } else {
    if (p.rb == 4) KQ_MMV_NW(Q6_K, 4) else KQ_MMV_NW(Q6_K, 1)
  }
#undef KQ_MMV_NW
#undef KQ_MMV_NG
#undef KQ_MMV
  return hipGetLastError();
}

}  // namespace kq
