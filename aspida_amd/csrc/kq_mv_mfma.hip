// kq_mv_mfma.hip -- batch-1 matvec of Q4_K and Q6_K weights on the matrix
// cores, over the packed layout (kq_packed.h).
//
// The VALU decode kernel (kq_packed.hip) spends one v_fma_mix_f32 per weight
// plus 0.6-1.5 instructions of unpacking and scaling, which keeps the vector
// ALUs too busy for weight loads and arithmetic to overlap.  Here the
// multiply-adds run on v_mfma_f32_16x16x32_f16 and the vector ALUs only unpack
// codes and apply the per-sub-block scales.
//
// One MFMA (A 16x32, B 32x16, D 16x16; lane layouts as in kq_mmq.hip):
//   B[k][n]  n = a weight row of a 16-row block; k = 8 g + t: 8 codes of
//            "quarter" g of that row, as f16 subnormals (q 2^-24, or 16 q
//            2^-24 for a high nibble left in place).  Lane (n, g) loads
//            exactly the packed bytes its codes come from.
//   A[m][k]  m = 4 g + 2 kappa + p: plane p (hi, lo) of the scaled activation
//            at k when k lies in sub-block kappa of lane group g's pair of
//            sub-blocks, zero otherwise (only lanes 20 g + r hold data).
//   D[m][n]  sum over that sub-block of q x (plane p) for row n; it sits in
//            lane n + 16 (m / 4) element m % 4, so lane (n, g) ends up with
//            both planes of the two sub-blocks whose codes and scales it read.
// Q4_K: quarter g = qs bytes 32 g .. 32 g + 31, sub-blocks 2g (low nibbles)
// and 2g + 1 (high nibbles); MFMA j takes qs dword j (elements 4j + {0,2,1,3}
// of both).  Eight MFMAs per 16-row block and super-block, one accumulator.
// Q6_K: quarter g = 2h + t holds sub-blocks 8h + t + 2k (k = 0..3) -- the
// quarter split of Block<Q6_K>; MFMA (T, j) takes 4 elements of sub-blocks
// k = 2T, 2T + 1, built from ql/qh dword j; two accumulators (T = 0, 1).
// A wave takes a 64-row tile (four blocks) and a range of super-block columns.
//
// A depends on x only.  Per column each wave builds it in its own 8 KB LDS
// image (one float4 of x per lane; the zero part is written once) and reads it
// back as 8 16-byte fragments per lane, shared by the tile's four row blocks.
// Activations are scaled per column: x' = x S, with S a power of two that puts
// the column's largest |x| just below 2^14 (Q4_K's high-nibble sub-blocks take
// S / 16, which absorbs their codes' factor 16), hi = f16(x'), lo = f16(x' - hi)
// -- x to about 2^-22 relative.  The minimum / code-offset terms use the f32
// sub-block sums of x S.  Row headers (Q4_K d, dmin, scales; Q6_K scales, d)
// are loaded once per row and shared through LDS by the row's four quarters.
//
// Accuracy.  The matrix cores do not round each addition as IEEE f32 does:
// measured on MI355X, a product much smaller than the largest one in the same
// sum (and, in a chain of MFMAs, than the accumulator) keeps fewer bits.  So
// the result is within about 1e-6 of sum |w x| for ordinary activations, but
// within only ~1e-4 when a column holds outliers 10^4 times its other values
// (the VALU kernel: ~1e-7).  The lo plane is stored times 2^11 so that its
// products are as large as hi's.
//
// Result per row: the decodes of Decode_Q4K_Block / Decode_Q6K_Block
// (src/llm/llm_dequant.adb:536-553, 140-181) dotted with x, in a different
// summation order from the CPU's (QMatVec, llm_dequant.adb:808-932).
#include <algorithm>
#include <atomic>

#include "kq_packed.h"
#include "kq_kernels.h"

namespace kq {

typedef _Float16 mh8 __attribute__((ext_vector_type(8)));
typedef float mf4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_f16x2(_Float16 a, _Float16 b) {
  return (uint32_t)__builtin_bit_cast(uint16_t, a) | ((uint32_t)__builtin_bit_cast(uint16_t, b) << 16);
}

__device__ __forceinline__ mf4 mfma_f16(uint4 a, uint4 b, mf4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(mh8, a), __builtin_bit_cast(mh8, b), c, 0, 0, 0);
}

// Per-lane constants of one wave.
struct MvLane {
  uint32_t* wr_hi;  // this lane's image writes (plane hi; plane lo is the next lane's slot)
  float odd;        // activation factor of this lane's elements (Q4_K high nibbles: 1/16)
  bool xs_writer;   // this lane stores a sub-block sum ...
  int xs_pos;       // ... at this index of the wave's sum array
  // Q4_K scale extraction for sub-blocks 2g, 2g+1 (get_scale_min_k4,
  // llm_dequant.adb:514-525): both pairs sit in bytes b0, b0 + 1 of the scale
  // dwords; g >= 2 takes the low/high nibbles of the third dword plus two bits
  // from the first/second.
  bool upper;
  uint32_t b0, m1, m2, mshift;
};

// Image slot of A row m = 4 grp + r in lane group grp (the MFMA's lane
// 16 grp + m = 20 grp + r): the full 64-lane image, or the compact one that
// keeps only these 16 data lanes (4 grp + r) plus slot 16, always zero, which
// every other lane reads.
template <int IL>
__device__ __forceinline__ constexpr int img_slot(int grp, int r) {
  return IL == 64 ? 20 * grp + r : 4 * grp + r;
}

template <int KIND, int IL>
__device__ __forceinline__ MvLane mv_lane(uint4 (&img)[8][IL], int lane) {
  MvLane L;
  const int g = lane >> 4;
  L.upper = g >= 2;
  L.b0 = 16u * (uint32_t)(g & 1);
  L.m1 = L.upper ? 0x0F0Fu : 0x3F3Fu;
  L.m2 = L.upper ? 0x3030u : 0u;
  L.mshift = L.b0 + (L.upper ? 4u : 0u);
  if (KIND == Q4_K) {
    // Elements 4 lane .. +3 = elements 4 bj .. of sub-block bs: MFMA bj, rows
    // m = 2 bs (+1) of k-group bs / 2, dwords 2 (bs % 2) + {0, 1}.
    const int bs = lane >> 3, bj = lane & 7;
    L.wr_hi = reinterpret_cast<uint32_t*>(&img[bj][img_slot<IL>(bs >> 1, 2 * (bs & 1))]) + 2 * (bs & 1);
    L.odd = (bs & 1) ? 0.0625f : 1.f;
    L.xs_writer = bj == 4;  // after the quad sums and row_shr:4
    L.xs_pos = bs;
  } else {
    // Element E = 4 lane = 128 h + 32 k + 16 t + 4 j: quarter c = 2h + t,
    // MFMA (T = k / 2, j) = image slot 4T + j, rows m = 4c + 2 (k % 2) (+1),
    // dwords 2 (k % 2) + {0, 1}.  Sub-block E / 16 = 8h + 2k + t, stored at
    // 4c + k so that lane group c reads its four sums as one float4.
    const int E = 4 * lane, h = E >> 7, k = (E >> 5) & 3, t = (E >> 4) & 1, j = (E >> 2) & 3;
    const int c = 2 * h + t;
    L.wr_hi = reinterpret_cast<uint32_t*>(&img[4 * (k >> 1) + j][img_slot<IL>(c, 2 * (k & 1))]) + 2 * (k & 1);
    L.odd = 1.f;
    L.xs_writer = (lane & 3) == 0;  // after the quad sums
    L.xs_pos = 4 * c + k;
  }
  return L;
}

// Builds the column's A image and sub-block sums of x S from the lane's
// float4 of x; returns 1/S.
template <int KIND>
__device__ __forceinline__ float build_image(float4 xv, const MvLane& L, float* xsum) {
  float mx = fmaxf(fmaxf(fabsf(xv.x), fabsf(xv.y)), fmaxf(fabsf(xv.z), fabsf(xv.w)));
  mx = wave_max(mx);
  int e = 0;
  const bool scaled = mx > 0.f && __builtin_isfinite(mx);
  if (scaled) (void)frexpf(mx, &e);
  const int se = scaled ? std::min(std::max(14 - e, -120), 120) : 0;
  const float S = ldexpf(1.f, se);
  const float sl = S * L.odd;
  const float v0 = xv.x * sl, v1 = xv.y * sl, v2 = xv.z * sl, v3 = xv.w * sl;
  const _Float16 h0 = (_Float16)v0, h1 = (_Float16)v1, h2 = (_Float16)v2, h3 = (_Float16)v3;
  // lo is stored times 2^11 (exact: a power of two), so that its products
  // stay as large as hi's inside the matrix cores' sums.
  const _Float16 l0 = (_Float16)((v0 - (float)h0) * 2048.f), l1 = (_Float16)((v1 - (float)h1) * 2048.f);
  const _Float16 l2 = (_Float16)((v2 - (float)h2) * 2048.f), l3 = (_Float16)((v3 - (float)h3) * 2048.f);
  float su = (xv.x + xv.y) + (xv.z + xv.w);
  su += dpp_from<0xB1>(su, 0.f);
  su += dpp_from<0x4E>(su, 0.f);
  if (KIND == Q4_K) su += dpp_from<0x114>(su, 0.f);  // 32-element sub-blocks: two quads
  *reinterpret_cast<uint2*>(L.wr_hi) = make_uint2(pack_f16x2(h0, h2), pack_f16x2(h1, h3));
  *reinterpret_cast<uint2*>(L.wr_hi + 4) = make_uint2(pack_f16x2(l0, l2), pack_f16x2(l1, l3));
  if (L.xs_writer) xsum[L.xs_pos] = su * S;
  return ldexpf(1.f, -se);
}

// One super-block column of RB 16-row blocks (RB = 4: the whole 64-row tile;
// RB = 1: block rb0 of it) as lane (n, g) loads it.
template <int KIND, int RB> struct MvCol;

// Q4_K: the header (d, dmin, scales) -- with RB = 4 of row `lane`, one
// coalesced 1 KB load shared through LDS; with RB = 1 of the lane's own row
// 16 rb0 + n -- and the qs chunks 1 + 2g, 2 + 2g of rows 16 rb + n.
template <int RB> struct MvCol<Q4_K, RB> {
  uint4 h, a[RB], b[RB];
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, g = lane >> 4;
    h = ld16(grp + (RB == 4 ? lane : 16 * rb0 + n) * 16);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      a[rb] = ld16(r + (1 + 2 * g) * 1024);
      b[rb] = ld16(r + (2 + 2 * g) * 1024);
    }
  }
};

// Q6_K (g = 2h + t): ql chunks 4h + t (codes k = 0, 2), 4h + 2 + t (k = 1, 3)
// and qh chunk 8 + 2h + t of rows 16 rb + n; the scale chunk 12 and d of row
// `lane` (RB = 4) or of the lane's own row (RB = 1).
template <int RB> struct MvCol<Q6_K, RB> {
  uint4 a[RB], b[RB], q[RB], sc;
  uint32_t d;
  __device__ __forceinline__ void load(const uint8_t* __restrict__ grp, int lane, int rb0) {
    const int n = lane & 15, g = lane >> 4, h = g >> 1, t = g & 1;
    const int hr = RB == 4 ? lane : 16 * rb0 + n;
    sc = ld16(grp + 12 * 1024 + hr * 16);
    d = ld2(grp + 13 * 1024 + hr * 2);
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint8_t* r = grp + (16 * (rb0 + rb) + n) * 16;
      a[rb] = ld16(r + (4 * h + t) * 1024);
      b[rb] = ld16(r + (4 * h + 2 + t) * 1024);
      q[rb] = ld16(r + (8 + 2 * h + t) * 1024);
    }
  }
};

// Bytes 0 and 2 of z as two f16 halves, and bytes 1 and 3.
__device__ __forceinline__ uint32_t bytes02(uint32_t z) { return __builtin_amdgcn_perm(z, z, 0x0C020C00u); }
__device__ __forceinline__ uint32_t bytes13(uint32_t z) { return __builtin_amdgcn_perm(z, z, 0x0C030C01u); }

// The per-row header words of a column, shared through LDS.
template <int KIND> struct MvHdr;
template <> struct MvHdr<Q4_K> {
  uint4 h[64];
};
template <> struct MvHdr<Q6_K> {
  uint4 sc[64];
  uint32_t d[64];
};

// Lane `lane`'s A fragment of MFMA j: from the full image, or from the
// compact one (the 16 data lanes 20 grp + r, r < 4, read their slot, the
// others the zero slot).
template <int IL>
__device__ __forceinline__ uint4 img_frag(const uint4 (&img)[8][IL], int j, int lane) {
  if (IL == 64) return img[j][lane];
  const int grp = lane >> 4, m = lane & 15;
  return img[j][(m >> 2) == grp ? 4 * grp + (m & 3) : 16];
}

__device__ __forceinline__ uint32_t dword_of(const uint4& v, int j) {
  return j == 0 ? v.x : j == 1 ? v.y : j == 2 ? v.z : v.w;
}

// One super-block column of RB row blocks: the A image, the row blocks' MFMA
// chains interleaved (consecutive MFMAs independent), then the scales.
template <int RB>
__device__ __forceinline__ void mv_column(const MvCol<Q4_K, RB>& c, float4 xv, const MvLane& L,
                                          uint4 (&img)[8][RB == 4 ? 64 : 17], float* xsum, MvHdr<Q4_K>* hdr, int lane,
                                          float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  __builtin_amdgcn_wave_barrier();
  const float invS = build_image<Q4_K>(xv, L, xsum);
  if (RB == 4) hdr->h[lane] = c.h;
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float2 X = *reinterpret_cast<const float2*>(&xsum[2 * g]);
  uint4 H[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) H[rb] = RB == 4 ? hdr->h[16 * rb + n] : c.h;
  __builtin_amdgcn_wave_barrier();
  mf4 D[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 8; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t q = dword_of(j < 4 ? c.a[rb] : c.b[rb], j & 3);
      const uint32_t t = q >> 8;
      D[rb] = mfma_f16(A[j], make_uint4(q & 0x000F000Fu, t & 0x000F000Fu, q & 0x00F000F0u, t & 0x00F000F0u), D[rb]);
    }
  }
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 h = H[rb];
    const float sa = __builtin_fmaf(D[rb][1], 1.f / 2048.f, D[rb][0]);
    const float sb = __builtin_fmaf(D[rb][3], 1.f / 2048.f, D[rb][2]);
    const uint32_t psc = L.upper ? h.w : h.y, pm = L.upper ? h.w : h.z;
    const uint32_t scp = ((psc >> L.b0) & L.m1) | ((h.y >> (L.b0 + 2u)) & L.m2);
    const uint32_t mp = ((pm >> L.mshift) & L.m1) | ((h.z >> (L.b0 + 2u)) & L.m2);
    const float sca = (float)(scp & 0xFFu), scb = (float)((scp >> 8) & 0xFFu);
    const float ma = (float)(mp & 0xFFu), mb = (float)((mp >> 8) & 0xFFu);
    const float T = __builtin_fmaf(scb, sb, sca * sa);
    const float M = __builtin_fmaf(mb, X.y, ma * X.x);
    const float d = f16_ada(h.x & 0xFFFFu) * 16777216.f, dmin = f16_ada(h.x >> 16);
    acc[rb] = __builtin_fmaf(__builtin_fmaf(d, T, -(dmin * M)), invS, acc[rb]);
  }
}

template <int RB>
__device__ __forceinline__ void mv_column(const MvCol<Q6_K, RB>& c, float4 xv, const MvLane& L,
                                          uint4 (&img)[8][RB == 4 ? 64 : 17], float* xsum, MvHdr<Q6_K>* hdr, int lane,
                                          float (&acc)[RB]) {
  const int g = lane >> 4, n = lane & 15;
  __builtin_amdgcn_wave_barrier();
  const float invS = build_image<Q6_K>(xv, L, xsum);
  if (RB == 4) {
    hdr->sc[lane] = c.sc;
    hdr->d[lane] = c.d;
  }
  __builtin_amdgcn_wave_barrier();
  uint4 A[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) A[j] = img_frag(img, j, lane);
  const float4 X = *reinterpret_cast<const float4*>(&xsum[4 * g]);  // sub-blocks k = 0..3 of quarter g
  uint2 SC[RB];
  uint32_t DD[RB];
  const bool half1 = g >= 2;  // the scales of half 1 are dwords 2, 3 of the scale chunk
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const uint4 s4 = RB == 4 ? hdr->sc[16 * rb + n] : c.sc;
    SC[rb] = half1 ? make_uint2(s4.z, s4.w) : make_uint2(s4.x, s4.y);
    DD[rb] = RB == 4 ? hdr->d[16 * rb + n] : c.d;
  }
  __builtin_amdgcn_wave_barrier();
  mf4 D0[RB], D1[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) D0[rb] = D1[rb] = mf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) {
      const uint32_t a = dword_of(c.a[rb], j), b = dword_of(c.b[rb], j), q = dword_of(c.q[rb], j);
      // 6-bit codes of sub-blocks k = 0..3 as bytes (as Block<Q6_K>::dot).
      const uint32_t z0 = (a & 0x0F0F0F0Fu) | ((q << 4) & 0x30303030u);
      const uint32_t z1 = (b & 0x0F0F0F0Fu) | ((q << 2) & 0x30303030u);
      const uint32_t z2 = ((a >> 4) & 0x0F0F0F0Fu) | (q & 0x30303030u);
      const uint32_t z3 = ((b >> 4) & 0x0F0F0F0Fu) | ((q >> 2) & 0x30303030u);
      D0[rb] = mfma_f16(A[j], make_uint4(bytes02(z0), bytes13(z0), bytes02(z1), bytes13(z1)), D0[rb]);
      D1[rb] = mfma_f16(A[4 + j], make_uint4(bytes02(z2), bytes13(z2), bytes02(z3), bytes13(z3)), D1[rb]);
    }
  }
  const int tb = 8 * (g & 1);  // byte t of each scale dword
  constexpr float K32 = 32.f / 16777216.f;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const float s0 = __builtin_fmaf(D0[rb][1], 1.f / 2048.f, D0[rb][0]);
    const float s1 = __builtin_fmaf(D0[rb][3], 1.f / 2048.f, D0[rb][2]);
    const float s2 = __builtin_fmaf(D1[rb][1], 1.f / 2048.f, D1[rb][0]);
    const float s3 = __builtin_fmaf(D1[rb][3], 1.f / 2048.f, D1[rb][2]);
    // int8 scales sc[8h + t + 2k]: dword 2h holds k = 0, 1; dword 2h + 1 holds k = 2, 3.
    const float c0 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].x, tb, 8);
    const float c1 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].x, tb + 16, 8);
    const float c2 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].y, tb, 8);
    const float c3 = (float)(int32_t)__builtin_amdgcn_sbfe(SC[rb].y, tb + 16, 8);
    // The codes are stored offset by 32: sum (q - 32) x = sum q x - 32 sum x.
    float T = c0 * __builtin_fmaf(-K32, X.x, s0);
    T = __builtin_fmaf(c1, __builtin_fmaf(-K32, X.y, s1), T);
    T = __builtin_fmaf(c2, __builtin_fmaf(-K32, X.z, s2), T);
    T = __builtin_fmaf(c3, __builtin_fmaf(-K32, X.w, s3), T);
    const float d = f16_ada(DD[rb]) * 16777216.f;
    acc[rb] = __builtin_fmaf(d * T, invS, acc[rb]);
  }
}

// The LDS one wave uses: its A image, sub-block sums and row headers.
template <int KA, int KB>
struct MvShared {
  uint4 img[8][64];
  float xsum[16];
  union {
    MvHdr<KA> a;
    MvHdr<KB> b;
  } hdr;
};

// The LDS one wave of the 16-row kernels uses: the compact A image and the
// sub-block sums (headers come straight from the lane's own row).
struct MvShared16 {
  uint4 img[8][17];
  float xsum[16];
};

// Row `lane` of tile `tile`'s partial dot over super-block columns sb0 ..
// sb0 + spw - 1 of packed matrix P (nsb columns), computed by this wave.
// How a wave walks its columns: one column; two register sets in turn (the
// next column's loads in flight during this one's work); one register set,
// columns one after another (fewer registers, so more waves per CU).
constexpr int MV_ONE = 0, MV_PF = 1, MV_SEQ = 2;

//
// RB = 4: the wave covers the whole 64-row tile and lane l returns row l.
// RB = 1: it covers 16-row block rb0 of the tile and lane l returns row
// 16 rb0 + l % 16.
template <int KIND, int PIPE, int RB = 4>
__device__ __forceinline__ float mv_mfma_rows(const uint8_t* __restrict__ P, int nsb, int tile, int sb0, int spw,
                                              const float* __restrict__ x, uint4 (&img)[8][RB == 4 ? 64 : 17],
                                              float* xsum, MvHdr<KIND>* hdr, int lane, int rb0 = 0) {
  constexpr int GB = 64 * Block<KIND>::BYTES;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (RB == 4 || lane < 17) img[j][lane] = make_uint4(0u, 0u, 0u, 0u);
  const MvLane L = mv_lane<KIND>(img, lane);

  float acc[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) acc[rb] = 0.f;
  const uint8_t* gp = P + ((size_t)tile * nsb + sb0) * GB;
  const float* xp = x + (size_t)sb0 * 256 + 4 * lane;

  MvCol<KIND, RB> c0;
  float4 x0;
  c0.load(gp, lane, rb0);
  __builtin_memcpy(&x0, __builtin_assume_aligned(xp, 16), 16);
  if (PIPE == MV_ONE) {
    mv_column(c0, x0, L, img, xsum, hdr, lane, acc);
  } else if (PIPE == MV_SEQ) {  // columns one after another: one register set, more waves per CU
    for (int s = 0; s < spw; ++s) {
      if (s > 0) {
        asm volatile("" ::: "memory");  // the next column's loads stay after this column's work
        c0.load(gp + (size_t)s * GB, lane, rb0);
        __builtin_memcpy(&x0, __builtin_assume_aligned(xp + (size_t)s * 256, 16), 16);
      }
      mv_column(c0, x0, L, img, xsum, hdr, lane, acc);
    }
  } else {
    // Two register sets used in turn: the next column's loads are in flight
    // while the current one is multiplied, with no copies between them.
    MvCol<KIND, RB> c1;
    float4 x1;
    for (int s = 0; s < spw; s += 2) {
      const int s1 = s + 1 < spw ? s + 1 : s;
      c1.load(gp + (size_t)s1 * GB, lane, rb0);
      __builtin_memcpy(&x1, __builtin_assume_aligned(xp + (size_t)s1 * 256, 16), 16);
      asm volatile("" ::: "memory");  // keep these loads issued here
      mv_column(c0, x0, L, img, xsum, hdr, lane, acc);
      if (s + 2 < spw) {
        c0.load(gp + (size_t)(s + 2) * GB, lane, rb0);
        __builtin_memcpy(&x0, __builtin_assume_aligned(xp + (size_t)(s + 2) * 256, 16), 16);
        asm volatile("" ::: "memory");
      }
      if (s + 1 < spw) mv_column(c1, x1, L, img, xsum, hdr, lane, acc);
    }
  }

  // Lane (n, g) holds rows 16 rb + n over its quarter: add the four quarters
  // (ascending g).
  float* red = reinterpret_cast<float*>(&img[0][0]);
  __builtin_amdgcn_wave_barrier();
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) red[rb * 64 + lane] = acc[rb];
  __builtin_amdgcn_wave_barrier();
  const float* rr = red + (RB == 4 ? (lane >> 4) * 64 : 0) + (lane & 15);
  return ((rr[0] + rr[16]) + rr[32]) + rr[48];
}

template <int KIND, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                     const float* __restrict__ x, float* __restrict__ y, int spw,
                                                     float* __restrict__ part, unsigned* __restrict__ count) {
  __shared__ MvShared<KIND, KIND> sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int tile = blockIdx.x;
  const float rowsum = mv_mfma_rows<KIND, PIPE>(P, nsb, tile, (blockIdx.y * NW + w) * spw, spw, x, sh[w].img,
                                              sh[w].xsum, &sh[w].hdr.a, lane);
  mv_epilogue<NW>(rowsum, tile, tile, out_rows, y, part, count);
}

// Two matrices that multiply the same x (q|k and v of attention): tiles
// [0, tiles_a) of the grid are matrix A's (kind KA), the rest matrix B's.
template <int KA, int KB, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma2(const uint8_t* __restrict__ Pa, int out_a, float* __restrict__ ya,
                                                      const uint8_t* __restrict__ Pb, int out_b, float* __restrict__ yb,
                                                      int tiles_a, int nsb, const float* __restrict__ x, int spw,
                                                      float* __restrict__ part, unsigned* __restrict__ count) {
  __shared__ MvShared<KA, KB> sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int gtile = blockIdx.x;
  const int sb0 = (blockIdx.y * NW + w) * spw;
  if (gtile < tiles_a) {
    const float r = mv_mfma_rows<KA, PIPE>(Pa, nsb, gtile, sb0, spw, x, sh[w].img, sh[w].xsum, &sh[w].hdr.a, lane);
    mv_epilogue<NW>(r, gtile, gtile, out_a, ya, part, count);
  } else {
    const float r =
        mv_mfma_rows<KB, PIPE>(Pb, nsb, gtile - tiles_a, sb0, spw, x, sh[w].img, sh[w].xsum, &sh[w].hdr.b, lane);
    mv_epilogue<NW>(r, gtile, gtile - tiles_a, out_b, yb, part, count);
  }
}

// 16-row workgroups: workgroup b takes rows 16 b .. 16 b + 15 (block b % 4
// of tile b / 4) over every super-block column, its NW waves splitting the
// columns, and the waves meet in LDS only -- no partial sums through memory,
// whose device-coherent store, counter and reload cost about 1.5 us per
// launch on MI355X.  Each wave builds its own activation image per column, so
// the image is amortised over 16 rows instead of 64: the choice for matrices
// too small to need the 64-row kernels' throughput.
template <int NW>
__device__ __forceinline__ void mv16_epilogue(float r, int blk, int out_rows, float* __restrict__ y) {
  __shared__ float red16[NW][16];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (NW > 1) {
    if (lane < 16) red16[w][lane] = r;
    __syncthreads();
    if (w != 0) return;
    float t = red16[0][lane & 15];
#pragma unroll
    for (int k = 1; k < NW; ++k) t += red16[k][lane & 15];
    r = t;
  }
  const int row = 16 * blk + lane;
  if (lane < 16 && row < out_rows) y[row] = r;
}

template <int KIND, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma16(const uint8_t* __restrict__ P, int nsb, int out_rows,
                                                       const float* __restrict__ x, float* __restrict__ y, int spw) {
  __shared__ MvShared16 sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = blockIdx.x;
  const float r = mv_mfma_rows<KIND, PIPE, 1>(P, nsb, blk >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KIND>*)nullptr, lane, blk & 3);
  mv16_epilogue<NW>(r, blk, out_rows, y);
}

// Two matrices that multiply the same x: blocks [0, blocks_a) are matrix A's.
template <int KA, int KB, int NW, int PIPE>
__global__ __launch_bounds__(64 * NW) void kq_mv_mfma2_16(const uint8_t* __restrict__ Pa, int out_a,
                                                         float* __restrict__ ya, const uint8_t* __restrict__ Pb,
                                                         int out_b, float* __restrict__ yb, int blocks_a, int nsb,
                                                         const float* __restrict__ x, int spw) {
  __shared__ MvShared16 sh[NW];
  const int lane = threadIdx.x & 63;
  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int blk = blockIdx.x;
  if (blk < blocks_a) {
    const float r = mv_mfma_rows<KA, PIPE, 1>(Pa, nsb, blk >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KA>*)nullptr, lane, blk & 3);
    mv16_epilogue<NW>(r, blk, out_a, ya);
  } else {
    const int b = blk - blocks_a;
    const float r = mv_mfma_rows<KB, PIPE, 1>(Pb, nsb, b >> 2, w * spw, spw, x, sh[w].img, sh[w].xsum,
                                              (MvHdr<KB>*)nullptr, lane, b & 3);
    mv16_epilogue<NW>(r, b, out_b, yb);
  }
}

// 0: the MFMA kernel for Q4_K and Q6_K, 1: the VALU kernel (comparison and tuning).
static std::atomic<int> g_engine{0};

void set_matvec_engine(int engine) { g_engine = engine; }

bool matvec_mfma_takes(int kind) { return (kind == Q4_K || kind == Q6_K) && g_engine.load() == 0; }

// The kernel a plan runs: NW waves per workgroup and the column walk.
static int mv_pipe(const PackedPlan& p) { return p.spw == 1 ? MV_ONE : p.seq ? MV_SEQ : MV_PF; }

// Dynamic LDS that leaves room for at most ceil(blocks / CUs) workgroups per
// CU: the dispatcher otherwise stacks several small workgroups on one CU
// while others idle (Q4_K 4096x4096, 256 blocks: 4.7 us stacked, 4.3 us one
// per CU).  The kernels do not use it.  Per kernel, once: its static LDS and
// the dynamic LDS it may take (the device's per-workgroup limit minus the
// static part, opted into; 0 if any query fails, which only turns the
// spreading off).
struct LdsRoom {
  size_t stat = 0, dyn_max = 0;
};

// min_static: the kernel's static LDS as this file lays it out, a floor in
// case the runtime reports less; 1 KB of the limit is left unused.
static LdsRoom lds_room_of(const void* kernel, size_t min_static) {
  LdsRoom r;
  hipFuncAttributes fa;
  int dev = 0, smem = 0;
  if (hipFuncGetAttributes(&fa, kernel) == hipSuccess && hipGetDevice(&dev) == hipSuccess &&
      hipDeviceGetAttribute(&smem, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess) {
    const size_t stat = std::max<size_t>(fa.sharedSizeBytes, min_static);
    if ((size_t)smem > stat + 1024 &&
        hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, smem - (int)stat - 1024) ==
            hipSuccess) {
      r.stat = stat;
      r.dyn_max = (size_t)smem - stat - 1024;
    }
  }
  (void)hipGetLastError();
  return r;
}

// One per kernel (K is the kernel itself, so each instantiation has its own).
template <auto K, int NW>
static LdsRoom lds_room() {
  static const LdsRoom r =
      lds_room_of(reinterpret_cast<const void*>(K), (size_t)NW * (sizeof(MvShared16) + 16 * sizeof(float)));
  return r;
}

static int device_attr(hipDeviceAttribute_t a, int fallback) {
  int dev = 0, v = 0;
  const bool ok = hipGetDevice(&dev) == hipSuccess && hipDeviceGetAttribute(&v, a, dev) == hipSuccess && v > 0;
  (void)hipGetLastError();
  return ok ? v : fallback;
}

// Never more than the kernel's own dynamic allowance (room.dyn_max), so static
// plus dynamic LDS stays within the per-workgroup limit.
static size_t mv16_spread_lds(int blocks, const LdsRoom& room) {
  static const int cus = device_attr(hipDeviceAttributeMultiprocessorCount, 256);
  static const int lds_cu = device_attr(hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, 160 * 1024);
  const size_t per_cu = std::max<size_t>(1, ((size_t)blocks + cus - 1) / cus);
  const size_t share = (size_t)lds_cu / per_cu, need = room.stat + 2048;
  if (share <= need) return 0;
  return std::min(room.dyn_max, (share - need) / 1024 * 1024);
}

template <int KIND>
static hipError_t launch_mfma16_kind(const PackedPlan& p, const uint8_t* w, int in_dim, int out_dim, const float* x,
                                     float* y, hipStream_t s) {
  const dim3 grid((out_dim + 15) / 16);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
#define KQ_GO(N, PIPE)                                                                                     \
  hipLaunchKernelGGL((kq_mv_mfma16<KIND, N, PIPE>), grid, dim3(64 * N),                                    \
                     mv16_spread_lds((int)grid.x, lds_room<kq_mv_mfma16<KIND, N, PIPE>, N>()), s, w, nsb, out_dim, x, \
                     y, p.spw)
#define KQ_NW(N)                                  \
  case N:                                         \
    if (pipe == MV_ONE) {                         \
      KQ_GO(N, MV_ONE);                           \
    } else if (pipe == MV_SEQ) {                  \
      KQ_GO(N, MV_SEQ);                           \
    } else {                                      \
      KQ_GO(N, MV_PF);                            \
    }                                             \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(14) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

template <int KIND>
static hipError_t launch_mfma_kind(const uint8_t* w, int in_dim, int out_dim, const float* x, float* y, float* part,
                                   unsigned* count, hipStream_t s) {
  const PackedPlan p = mfma_plan(KIND, in_dim, out_dim);
  if (p.blk16) return launch_mfma16_kind<KIND>(p, w, in_dim, out_dim, x, y, s);
  const dim3 grid((out_dim + 63) / 64, p.ks);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
#define KQ_GO(N, PIPE) \
  hipLaunchKernelGGL((kq_mv_mfma<KIND, N, PIPE>), grid, dim3(64 * N), 0, s, w, nsb, out_dim, x, y, p.spw, part, count)
#define KQ_NW(N)                                                                                \
  case N:                                                                                       \
    if (pipe == MV_ONE) KQ_GO(N, MV_ONE);                                                       \
    else if constexpr (N == 16) return hipErrorInvalidValue; /* 16 waves: one column only */    \
    else if (pipe == MV_SEQ) KQ_GO(N, MV_SEQ);                                                  \
    else if constexpr (N <= 4 || (N == 8 && KIND != Q6_K)) KQ_GO(N, MV_PF);                     \
    else return hipErrorInvalidValue; /* two register sets: <= 8 waves per group, 4 for Q6_K */ \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

bool matvec2_mfma_takes(int kind_a, int kind_b) { return matvec_mfma_takes(kind_a) && matvec_mfma_takes(kind_b); }

template <int KA, int KB>
static hipError_t launch_mfma_pair(const uint8_t* a, int out_a, float* ya, const uint8_t* b, int out_b, float* yb,
                                   int in_dim, const float* x, float* part, unsigned* count, hipStream_t s) {
  const int tiles_a = (out_a + 63) / 64, tiles_b = (out_b + 63) / 64;
  // The split of the wider kind's registers (Q6_K when either is).
  constexpr int KW = KA == Q6_K || KB == Q6_K ? Q6_K : Q4_K;
  const PackedPlan p = mfma_plan(KW, in_dim, (tiles_a + tiles_b) * 64);
  const int nsb = in_dim / 256, pipe = mv_pipe(p);
  if (p.blk16) {
    const int blocks_a = (out_a + 15) / 16;
    const dim3 grid16(blocks_a + (out_b + 15) / 16);
#define KQ_GO(N, PIPE)                                                                                  \
  hipLaunchKernelGGL((kq_mv_mfma2_16<KA, KB, N, PIPE>), grid16, dim3(64 * N),                            \
                     mv16_spread_lds((int)grid16.x, lds_room<kq_mv_mfma2_16<KA, KB, N, PIPE>, N>()), s, a, out_a, \
                     ya, b, out_b, yb, blocks_a, nsb, x, p.spw)
#define KQ_NW(N)                                  \
  case N:                                         \
    if (pipe == MV_ONE) {                         \
      KQ_GO(N, MV_ONE);                           \
    } else if (pipe == MV_SEQ) {                  \
      KQ_GO(N, MV_SEQ);                           \
    } else {                                      \
      KQ_GO(N, MV_PF);                            \
    }                                             \
    break;
    switch (p.nw) {
      KQ_NW(16) KQ_NW(14) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
      default: return hipErrorInvalidValue;
    }
#undef KQ_NW
#undef KQ_GO
    return hipGetLastError();
  }
  const dim3 grid(tiles_a + tiles_b, p.ks);
#define KQ_GO(N, PIPE)                                                                                            \
  hipLaunchKernelGGL((kq_mv_mfma2<KA, KB, N, PIPE>), grid, dim3(64 * N), 0, s, a, out_a, ya, b, out_b, yb, tiles_a, \
                     nsb, x, p.spw, part, count)
#define KQ_NW(N)                                                          \
  case N:                                                                 \
    if (pipe == MV_ONE) KQ_GO(N, MV_ONE);                                 \
    else if constexpr (N == 16) return hipErrorInvalidValue;              \
    else if (pipe == MV_SEQ) KQ_GO(N, MV_SEQ);                            \
    else if constexpr (N <= 4 || (N == 8 && KW != Q6_K)) KQ_GO(N, MV_PF); \
    else return hipErrorInvalidValue;                                     \
    break;
  switch (p.nw) {
    KQ_NW(16) KQ_NW(8) KQ_NW(4) KQ_NW(2) KQ_NW(1)
    default: return hipErrorInvalidValue;
  }
#undef KQ_NW
#undef KQ_GO
  return hipGetLastError();
}

hipError_t launch_matvec2_mfma(int kind_a, const void* Pa, int out_a, float* ya, int kind_b, const void* Pb, int out_b,
                               float* yb, int in_dim, const float* x, float* part, unsigned* count, hipStream_t s) {
  const uint8_t* a = (const uint8_t*)Pa;
  const uint8_t* b = (const uint8_t*)Pb;
  if (kind_a == Q4_K && kind_b == Q6_K) return launch_mfma_pair<Q4_K, Q6_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q4_K && kind_b == Q4_K) return launch_mfma_pair<Q4_K, Q4_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q6_K && kind_b == Q6_K) return launch_mfma_pair<Q6_K, Q6_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  if (kind_a == Q6_K && kind_b == Q4_K) return launch_mfma_pair<Q6_K, Q4_K>(a, out_a, ya, b, out_b, yb, in_dim, x, part, count, s);
  return hipErrorNotSupported;
}

hipError_t launch_matvec_mfma(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y, float* part,
                              unsigned* count, hipStream_t s) {
  const uint8_t* w = (const uint8_t*)P;
  switch (kind) {
    case Q4_K: return launch_mfma_kind<Q4_K>(w, in_dim, out_dim, x, y, part, count, s);
    case Q6_K: return launch_mfma_kind<Q6_K>(w, in_dim, out_dim, x, y, part, count, s);
    default: return hipErrorNotSupported;
  }
}

}  // namespace kq
