// kq_kernels.h -- host-side launchers of the device kernels (namespace kq).
// All launchers are asynchronous on the given stream and allocate nothing.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>

namespace kq {

struct MvConfig {
  int rows_per_wave = 2;  // rows per lane group per step: 1, 2 or 4
  int waves_per_cu = 16;  // resident waves launched per CU (upper bound)
};

// Launch shape chosen for a batch-1 matvec of this kind and shape.
MvConfig default_mv_config(int kind, int in_dim, int out_dim);

// xq[r][i] = sum of x[r][16i .. 16i+15] for rows r < rows (in_dim % 16 == 0).
hipError_t launch_xsum(const float* x, int in_dim, int rows, float* xq, hipStream_t s);

// y[out] = W[out][in] x[in] for a quantized W (kinds 0..5); xq from launch_xsum.
hipError_t launch_matvec(int kind, const void* W, int in_dim, int out_dim, const float* x, const float* xq,
                         float* y, hipStream_t s, const MvConfig& cfg);

// Y[b][out] = W X[b] for b < batch, on the vector ALUs; XQ from launch_xsum.
hipError_t launch_matmul_valu(int kind, const void* W, int in_dim, int out_dim, int batch, const float* X,
                              const float* XQ, float* Y, hipStream_t s);

// Y[b][out] = W X[b] with MFMA tiles (kinds 0..4); returns hipErrorNotSupported
// for shapes the MFMA kernels do not cover.
hipError_t launch_matmul_mfma(int kind, const void* W, int in_dim, int out_dim, int batch, const float* X,
                              float* Y, hipStream_t s);

// y = W x for a row-major f32 W.
hipError_t launch_dense(const float* W, int in_dim, int out_dim, const float* x, float* y, hipStream_t s);

// dst[out][in] = dequantized W, bit-identical to the CPU decoders.
hipError_t launch_dequant(int kind, const void* W, int in_dim, int out_dim, float* dst, hipStream_t s);

// ---- lane-interleaved ("packed") layout, kq_packed.h ----

// Launch split of a packed matvec: spw super-block columns per wave, nw waves
// per workgroup, ks workgroups per 64-row tile (nw * ks * spw == in_dim / 256).
struct PackedPlan {
  int nw, ks, spw;
  bool seq = false;    // MFMA kernel: columns one after another (one register set) even when spw > 1
  bool blk16 = false;  // MFMA kernel: 16-row workgroups over all columns (nw waves, spw columns each, ks = 1)
};
PackedPlan packed_plan(int in_dim, int out_dim);
// The split of the MFMA matvec (kq_mv_mfma.hip) for a kind.
PackedPlan mfma_plan(int kind, int in_dim, int out_dim);
// Tuning: 0 = the plan's choice, 1 = 64-row workgroups, 2 = 16-row workgroups.
void set_mfma_rows(int mode);
// Tuning: 0 = the plan's choice, 1 = prefetching waves, 2 = sequential columns
// (for splits with more than one column per wave).
void set_mfma_pipeline(int mode);
// Per-thread override of packed_plan for tuning (nw a power of two <= 16,
// nw * ks dividing in_dim / 256; anything else, or 0, restores the choice).
void set_packed_plan_override(int nw, int ks);
// The override's workgroups per tile (0: none); the small-batch MFMA product
// takes it as its column split too.
int packed_plan_override_ks();

// Bytes of the packed image of a [out_dim][in_dim] matrix (rows rounded up to
// a multiple of 64); 0 for an invalid kind or shape.
size_t packed_bytes(int kind, int in_dim, int out_dim);

// Workspace a packed matvec of this shape needs: partial sums (floats) and
// per-tile arrival counters (unsigned, one per 256 bytes; zero before the
// first launch, and every launch leaves them zero again).
size_t packed_workspace_floats(int in_dim, int out_dim);
size_t packed_counters(int out_dim);

// Two packed matrices that multiply the same x, in one launch: y_a = A x,
// y_b = B x (workspace and counters sized for out_a + out_b rows rounded up
// to tiles).  hipErrorNotSupported for kind pairs without a fused kernel.
bool matvec2_supported(int kind_a, int kind_b);
hipError_t launch_matvec2_packed(int kind_a, const void* Pa, int out_a, float* ya, int kind_b, const void* Pb,
                                 int out_b, float* yb, int in_dim, const float* x, float* part, unsigned* count,
                                 hipStream_t s);

// Small-batch products on MFMA over packed W (kq_mmq.hip): kinds with an
// MFMA kernel, workspace bytes for `batch` <= 64 activation rows, and the
// launcher (hipErrorNotSupported for other kinds).  `count` is a per-tile
// arrival-counter array as for launch_matvec_packed (zero before first use,
// left zero).
bool mfma_kind(int kind);
size_t mfma_workspace_bytes(int in_dim, int out_dim, int batch);
hipError_t launch_matmul_mfma_packed(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X,
                                     float* Y, void* work, unsigned* count, hipStream_t s, bool stream_once);

// Up to 16 activation rows per launch on MFMA, dense in rows and vectors
// (kq_mm16.hip): kinds it takes, workspace bytes (activation images and
// partials), and the launcher; `count` as above.
// Up to 4 vectors with the batch-1 matrix-core arithmetic on 16-row
// workgroups, each column's weights read once for all of them
// (kq_mv_mfma.hip); Q4_K and Q6_K (matvec_nv_takes).
bool matvec_nv_takes(int kind, int in_dim, int out_dim);
hipError_t launch_matvec_mfma_nv(int kind, const void* P, int in_dim, int out_dim, int nv, const float* x, float* y,
                                 hipStream_t s);
// Small batches of 2..64 vectors over packed Q4_K / Q6_K on the matrix
// cores with the batch-1 work split (kq_mmv.hip): every weight byte read once,
// no workspace, no pre-pass.  x must be 16-byte aligned.
bool mmv_kind(int kind);
// Vectors per launch for larger batches: 32 for Q6_K on 64-row tiles (whose
// four-group launch would run on 4 waves), else 64.
int mmv_step(int kind, int in_dim, int out_dim);
hipError_t launch_matmul_mmv(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                             hipStream_t s);
// Small batches of up to 64 vectors over packed Q4_K / Q6_K, one wave per
// (64-row tile, super-block column) (kq_mmw.hip): the activation split of
// kq_xsplit, then four columns per workgroup summed in LDS and mmw_ks column
// groups per tile summed through partials.  `work` holds
// mmw_workspace_bytes; `count` one counter per tile, zero before first use
// and left zero.  in_dim must be a multiple of 1024.
bool mmw_takes(int kind, int in_dim);
int mmw_ks(int in_dim, int out_dim);
size_t mmw_workspace_bytes(int in_dim, int out_dim, int batch);
hipError_t launch_matmul_mmw(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                             void* work, unsigned* count, hipStream_t s);
bool mm16_kind(int kind);
size_t mm16_workspace_bytes(int in_dim, int out_dim);
hipError_t launch_matmul_mm16(int kind, const void* P, int in_dim, int out_dim, int batch, const float* X, float* Y,
                              void* work, unsigned* count, hipStream_t s, bool stream_once);

// ggml layout -> packed (unpack = false) or back (unpack = true).
// Y[b][out] = W X[b] for nb <= 8 vectors over packed W on VALU
// (kq_packed_multi.hip); row b is bit-identical to launch_matvec_packed on
// X[b].  part: multi_workspace_floats floats; count as for the matvec.
size_t multi_workspace_floats(int in_dim, int out_dim);
hipError_t launch_matmul_packed_valu(int kind, const void* P, int in_dim, int out_dim, int nb, const float* X, float* Y,
                                     float* part, unsigned* count, hipStream_t s);

hipError_t launch_pack(int kind, const void* src, int in_dim, int out_dim, void* dst, bool unpack, hipStream_t s);

// Batch-1 packed matvec on MFMA (kq_mv_mfma.hip), same arguments, workspace
// and counters as launch_matvec_packed, which routes here for the kinds it
// takes.  set_matvec_engine(1) keeps every kind on the VALU kernel
// (comparison), 0 restores the default.
void set_matvec_engine(int engine);
bool matvec_mfma_takes(int kind);
// The 16-row matrix-core matvec with its x formed in the launch: x =
// RMSNorm(H + r) with weights g (r may be null; H is not written).  Q4_K and
// Q6_K whose batch-1 plan is 16-row workgroups of at least 4 waves, in_dim
// <= 4096 (matvec_norm_takes).
bool matvec_norm_takes(int kind, int in_dim, int out_dim);
hipError_t launch_matvec_norm(int kind, const void* P, int in_dim, int out_dim, const float* H, const float* r,
                              const float* g, float* y, hipStream_t s);
hipError_t launch_matvec_mfma(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y, float* part,
                              unsigned* count, hipStream_t s);
// The fused pair on MFMA when both kinds are MFMA kinds (launch_matvec2_packed
// routes here).
bool matvec2_mfma_takes(int kind_a, int kind_b);
hipError_t launch_matvec2_mfma(int kind_a, const void* Pa, int out_a, float* ya, int kind_b, const void* Pb, int out_b,
                               float* yb, int in_dim, const float* x, float* part, unsigned* count, hipStream_t s);

// y = W x for packed W; x is 16-byte aligned.  Launches that share a
// workspace must be ordered (one stream).
hipError_t launch_matvec_packed(int kind, const void* P, int in_dim, int out_dim, const float* x, float* y,
                                float* part, unsigned* count, hipStream_t s);

}  // namespace kq
