/*
 * aspidagpu.h -- C ABI of libaspidagpu.so, the MI355X (gfx950) implementation
 * of Aspida's quantized-weight GPU path.
 *
 * Weight kinds are LLM_Weight.Kind_Code's (src/llm/llm_weight.adb:277-292):
 *   0 = Q4_K (144 B / 256), 1 = Q6_K (210 B), 2 = Q5_K (176 B),
 *   3 = Q3_K (110 B), 4 = Q2_K (84 B), 5 = Q8_0 (8 x 34 B per 256 elements).
 * A weight is row-major [out_dim][in_dim / 256 super-blocks] (GGUF ne0 =
 * in_dim, ne1 = out_dim); activations are contiguous f32, batched ones
 * [batch][in_dim] / [batch][out_dim].  `long` is 64-bit (LP64), Ada's
 * Interfaces.C.long.
 *
 * Host-pointer entry points (the reference ABI) are synchronous and
 * thread-safe.  Weights are mirrored into HBM on first use, keyed by host
 * pointer; the caller must call aspida_gpu_free_weight(w) before freeing or
 * reusing the host bytes of w, and must not free a weight while another
 * thread's call is using it.  On invalid arguments or a HIP failure the
 * output is filled with quiet NaN, a line is printed to stderr and the
 * calling thread's aspida_gpu_last_error() becomes non-zero.
 */
#ifndef ASPIDAGPU_H
#define ASPIDAGPU_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---- reference ABI (symbols resolved by src/llm/llm_gpu.adb:100-146 and
 *      src/llm/llm_qwen_gpu.adb:257-266, 340) ------------------------------ */

/* y[out_dim] = W x.  Replaces gpu/gpu_matvec.cu:502-530.  in_dim must be a
 * multiple of 256 and wbytes >= out_dim * (in_dim / 256) * block bytes.
 * Kind 4 runs Q2_K and kind 5 Q8_0 (the reference sent every kind >= 4 to
 * its Q2_K kernel). */
void aspida_gpu_matvec(const void *w, long wbytes, int kind, int in_dim, int out_dim,
                       const float *x, float *y);

/* Y[batch][out_dim] = X[batch][in_dim] W^T.  Replaces gpu/gpu_matvec.cu:534-553;
 * any batch >= 1 is served (the reference clamped batch to 32); batch < 1 is a
 * no-op as in the reference. */
void aspida_gpu_matmul(const void *w, long wbytes, int kind, int in_dim, int out_dim, int batch,
                       const float *x, float *y);

/* y = W x for a dense row-major f32 W [out_dim][in_dim] (e.g. the f32 MoE
 * router).  Replaces gpu/gpu_matvec.cu:925-935. */
void aspida_gpu_dense_matvec(const void *w, long wbytes, int in_dim, int out_dim,
                             const float *x, float *y);

/* Drop the HBM mirror of host weight w; idempotent, a no-op for unknown w.
 * Replaces gpu/gpu_matvec.cu:494-500. */
void aspida_gpu_free_weight(const void *w);

/* Routed + shared expert FFN of one MoE layer for one token, routing supplied
 * by the caller: y = sum_k top_w[k] * Down_e(silu(Gate_e x) * Up_e x)
 * (e = top_idx[k], 0-based, ascending k) + g * SharedDown(silu(SharedGate x)
 * * SharedUp x), g = sigmoid(shared_gate_inp . x) when gate_inp_len > 1 and
 * shared_gate_inp is non-null, else 1.  Routed expert tensors are
 * [n_exp][rows][cols] with bytes / n_exp per expert.  Replaces
 * gpu/gpu_matvec.cu:1673-1758; top_k may be up to 32 (the reference silently
 * truncated it to 8); dim and intermed must be multiples of 256.  When gate,
 * up, shared gate and shared up share one kind and down and shared down
 * another, the experts are mirrored in the packed layout and run by the
 * grouped kernels of aspida_moe_experts_packed_dev. */
void aspida_gpu_moe_experts(const float *x, int dim, int top_k, int intermed, int n_exp,
                            const int *top_idx, const float *top_w,
                            const void *gate_w, long gate_bytes, int gate_kind,
                            const void *up_w, long up_bytes, int up_kind,
                            const void *down_w, long down_bytes, int down_kind,
                            const void *shg_w, long shg_bytes, int shg_kind,
                            const void *shu_w, long shu_bytes, int shu_kind,
                            const void *shd_w, long shd_bytes, int shd_kind,
                            const float *shared_gate_inp, int gate_inp_len, float *y);

/* Return and clear the calling thread's last error (0 = none).  Same
 * signature and "return and clear" contract as gpu/gpu_matvec.cu:2348-2352. */
int aspida_gpu_last_error(void);

/* ---- device-pointer entry points (no counterpart in the reference ABI: for
 *      callers whose weights and activations already live in HBM, e.g. a
 *      resident decode chain).  Asynchronous on `stream` (a hipStream_t, NULL =
 *      null stream); return 0 or a negative errno / positive hipError_t. ---- */

/* xq[r][i] = sum of x[r][16 i .. 16 i + 15], r < rows: the per-group
 * activation sums the K-quant kernels take (in_dim % 16 == 0). */
int aspida_kq_xsum_dev(const float *x, int in_dim, int rows, float *xq, void *stream);

/* Device form of aspida_gpu_matvec; xq from aspida_kq_xsum_dev(x). */
int aspida_kq_matvec_dev(int kind, const void *w, int in_dim, int out_dim, const float *x,
                         const float *xq, float *y, void *stream);

/* Lane-interleaved ("packed") layout of the batch-1 decode kernels: tiles of
 * 64 rows, each tile's super-block column stored as 16-byte chunk planes with
 * one chunk per row, so a wave reads 1 KB per load and each lane owns one
 * row.  Same bytes as the ggml layout, regrouped (rows past out_dim in the
 * last tile are zero).  The same math as QMatVec
 * (src/llm/llm_dequant.adb:808-932) and the reference's batch-1 kernels
 * (gpu/gpu_matvec.cu:149-383), over a layout of this library's own.
 * aspida_kq_packed_bytes: size of the packed image (0 for a bad kind/shape).
 * aspida_kq_pack_dev / aspida_kq_unpack_dev: ggml <-> packed, on `stream`. */
long long aspida_kq_packed_bytes(int kind, int in_dim, int out_dim);
int aspida_kq_pack_dev(int kind, const void *w, int in_dim, int out_dim, void *packed, void *stream);
int aspida_kq_unpack_dev(int kind, const void *packed, int in_dim, int out_dim, void *w, void *stream);

/* Launch split aspida_kq_matvec_packed_dev uses for this shape: waves per
 * workgroup (the kernel is kq_mv_packed<kind, waves>), workgroups per 64-row
 * tile and super-block columns per wave (their product is in_dim / 256). */
/* The kernel and split aspida_kq_matvec_packed_dev uses for a kind and shape
 * under the current engine (aspida_kq_set_mv_engine): returns 1 for the
 * matrix-core kernel on 64-row workgroups kq_mv_mfma<kind, waves, walk> (walk
 * 0: one column per wave, 1: prefetching columns), 2 for the same kernel
 * taking its columns one after another (walk 2), 3 and 4 for the same two
 * walks of the 16-row-workgroup kernel kq_mv_mfma16<kind, waves, walk>
 * (groups_per_tile is then 1), 0 for the vector kernel
 * kq_mv_packed<kind, waves, prefetch>, or -EINVAL.  No reference counterpart. */
int aspida_kq_matvec_plan(int kind, int in_dim, int out_dim, int *waves_per_group, int *groups_per_tile,
                          int *columns_per_wave);
int aspida_kq_packed_plan(int in_dim, int out_dim, int *waves_per_group, int *groups_per_tile,
                          int *columns_per_wave);

/* y[out_dim] = W x for packed W: the batch-1 decode path.  Per-group
 * activation sums are formed inside the kernel (no xq).  x must be 16-byte
 * aligned.  The library keeps a small workspace per stream (allocated on the
 * first call for a stream and shape, so warm up before graph capture);
 * calls on one stream are ordered, calls on different streams are
 * independent. */
int aspida_kq_matvec_packed_dev(int kind, const void *packed, int in_dim, int out_dim, const float *x,
                                float *y, void *stream);

/* Allocation-free form of aspida_kq_matvec_packed_dev: same kernels, launch
 * split and results (bit for bit), but the workspace -- per-tile arrival
 * counters and cross-workgroup partial sums -- lives in a fixed device array
 * of this library (6 MiB, one copy per GPU, held until the process ends), so
 * the call never allocates device memory: no hipMalloc, hipFree or allocating
 * library routine.  No counterpart in the reference.  For callers that cannot
 * allocate: code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Limit: out_dim up to 262,144 rows and at most 1,310,720
 * partial sums (tiles x workgroups per tile x 64); larger shapes return
 * -E2BIG and launch nothing.  Every call on one GPU shares the array, so calls
 * that overlap in time on one GPU (different streams or threads) race and
 * give wrong results: order them on one stream.  x must be 16-byte aligned. */
int aspida_kq_matvec_packed_noalloc_dev(int kind, const void *packed, int in_dim, int out_dim, const float *x,
                                        float *y, void *stream);

/* y_a = A x and y_b = B x for two packed matrices that share the input (e.g.
 * the q|k and v projections of a decoder layer), in one launch for the kind
 * pairs (Q4_K, Q6_K), (Q5_K, Q6_K) and equal kinds Q4_K, Q5_K, Q6_K, Q8_0;
 * other pairs run as two launches.  Same results as two calls of
 * aspida_kq_matvec_packed_dev. */
int aspida_kq_matvec2_packed_dev(int kind_a, const void *packed_a, int out_a, float *y_a, int kind_b,
                                 const void *packed_b, int out_b, float *y_b, int in_dim, const float *x,
                                 void *stream);

/* Y[batch][out_dim] = X[batch][in_dim] W^T for packed W: the small-batch
 * path.  Small batches run on a multi-vector VALU kernel, each row
 * bit-identical to aspida_kq_matvec_packed_dev on it: up to 4 rows for Q4_K
 * and Q6_K, whose larger batches run on MFMA (activations split into f16
 * hi + lo, exact integer codes, f32 scales; 64 rows per launch), and 8 rows
 * per launch for the other kinds.
 * x must be 16-byte aligned; workspace as for aspida_kq_matvec_packed_dev.
 * The same math as the reference's batched kernels (gpu/gpu_matvec.cu:234-382)
 * without its batch limit of 32. */
int aspida_kq_matmul_packed_dev(int kind, const void *packed, int in_dim, int out_dim, int batch,
                                const float *x, float *y, void *stream);

/* Device form of aspida_gpu_matmul; xq from aspida_kq_xsum_dev(x, .., batch). */
int aspida_kq_matmul_dev(int kind, const void *w, int in_dim, int out_dim, int batch,
                         const float *x, const float *xq, float *y, void *stream);

/* Small-batch product forced onto the vector-ALU kernels (the reference
 * numerics path the MFMA kernels are checked against). */
int aspida_kq_matmul_valu_dev(int kind, const void *w, int in_dim, int out_dim, int batch,
                              const float *x, const float *xq, float *y, void *stream);

/* dst[out_dim][in_dim] = dequantized W, bit-identical to the CPU decoders
 * Decode_Q*K_Block (src/llm/llm_dequant.adb:122-554) and Dequant_Q8_0
 * (606-630), including their Inf/NaN -> +0.0 reading of f16 scales. */
int aspida_kq_dequant_dev(int kind, const void *w, int in_dim, int out_dim, float *dst, void *stream);

/* Device form of aspida_gpu_dense_matvec. */
int aspida_dense_matvec_dev(const float *w, int in_dim, int out_dim, const float *x, float *y,
                            void *stream);

/* MoE router for T tokens: logits[t][e] = router_w[e][:] . x[t][:] (f32,
 * [n_exp][dim]), stable softmax, greedy top-k (strict >, lowest index wins
 * ties), renormalised weights (src/llm/llm_moe.adb:136-197).  Writes
 * logits[T][n_exp], top_idx[T][top_k] (0-based) and top_w[T][top_k].
 * n_exp <= 1024, top_k <= 32, dim % 4 == 0, router_w and x 16-byte aligned.
 * Uses the stream's workspace like aspida_kq_matvec_packed_dev (allocated on
 * the first call for a stream and T, so warm up before graph capture). */
int aspida_moe_route_dev(const float *router_w, int n_exp, int dim, int T, int top_k, const float *x,
                         float *logits, int *top_idx, float *top_w, void *stream);

/* Floats of `work` aspida_moe_experts_dev needs. */
long aspida_moe_work_floats(int T, int dim, int top_k, int intermed);

/* Device form of aspida_gpu_moe_experts for T tokens: x [T][dim], top_idx /
 * top_w [T][top_k], y [T][dim]; routed expert e of a projection starts at
 * byte e * *_stride of its tensor; shared_gate_inp may be NULL (ungated). */
int aspida_moe_experts_dev(const float *x, int T, int dim, int top_k, int intermed, int n_exp,
                           const int *top_idx, const float *top_w,
                           const void *gate_w, long gate_stride, int gate_kind,
                           const void *up_w, long up_stride, int up_kind,
                           const void *down_w, long down_stride, int down_kind,
                           const void *shg_w, int shg_kind, const void *shu_w, int shu_kind,
                           const void *shd_w, int shd_kind, const float *shared_gate_inp,
                           float *work, float *y, void *stream);

/* Grouped MoE over packed experts.  Same arithmetic contract as
 * aspida_moe_experts_dev (LLM_MoE.Forward steps 4-5,
 * src/llm/llm_moe.adb:249-299; the reference shim's moe_experts,
 * gpu/gpu_matvec.cu:1673-1760), but the expert matrices are in the packed
 * layout (aspida_moe_pack_experts_dev) and each expert's weights are read once
 * per launch however many of the T tokens chose it.  Gate, up, shared gate
 * and shared up are of kind gu_kind, down and shared down of down_kind.
 * dim and intermed multiples of 256, top_k <= 32.  x 16-byte aligned, work
 * 256-byte aligned with aspida_moe_packed_work_bytes bytes.  Deterministic:
 * each y[t] sums its slots in ascending k, shared expert last.  top_idx
 * entries outside [0, n_exp) leave that token's y unwritten. */
long aspida_moe_packed_work_bytes(int T, int dim, int intermed, int top_k);
int aspida_moe_pack_experts_dev(int kind, const void *src, long src_stride, int in_dim, int out_dim, int n,
                                void *dst, void *stream);
int aspida_moe_experts_packed_dev(const float *x, int T, int dim, int top_k, int intermed, int n_exp,
                                  const int *top_idx, const float *top_w, const void *gate_p,
                                  const void *up_p, int gu_kind, const void *down_p, int down_kind,
                                  const void *shg_p, const void *shu_p, const void *shd_p,
                                  const float *shared_gate_inp, void *work, float *y, void *stream);

/* Resident decode chain: an ordered list of packed matvecs (steps) run by ONE
 * persistent launch, with no launch boundary between them -- e.g. every
 * weight matrix of a decoder pass.  A step whose x lies inside an earlier
 * step's y (its producer: the latest earlier step whose y overlaps x; x must
 * lie wholly inside it) waits, per 256-element column, only for the 64-row
 * tiles of the producer that write those elements, while the weight loads
 * of the following columns are already in flight; other steps read x as
 * given.  No step may write memory that an earlier step reads or writes, or
 * its own x.  Same arithmetic per row as aspida_kq_matvec_packed_dev (a
 * different, fixed order of the per-column sums; deterministic).  No
 * counterpart in the reference, whose per-call ABI this path replaces for
 * callers that keep weights and activations in HBM
 * (aspida_gpu_matvec, gpu/gpu_matvec.cu:502-530, called per matrix).
 * aspida_kq_chain_create validates the steps and allocates the chain's
 * flags and partial sums (NULL on error, see aspida_gpu_last_error);
 * aspida_kq_chain_run launches it on `stream` and allocates nothing (runs of
 * one chain must be ordered); aspida_kq_chain_check synchronises and returns
 * 1 if a dependency wait gave up since the last check (outputs of that run
 * unreliable; only when the device could not keep every workgroup
 * resident), else 0; aspida_kq_chain_workgroups: the launch's workgroups. */
typedef struct aspida_kq_step {
  int kind, in_dim, out_dim, reserved;
  const void *packed;   /* aspida_kq_pack_dev layout */
  const float *x;       /* [in_dim], 16-byte aligned */
  float *y;             /* [out_dim] */
} aspida_kq_step;
void *aspida_kq_chain_create(const aspida_kq_step *steps, int nsteps);
int aspida_kq_chain_run(void *chain, void *stream);
int aspida_kq_chain_check(void *chain);
int aspida_kq_chain_workgroups(void *chain);
void aspida_kq_chain_destroy(void *chain);

/* ---- resident model chain (the reference's chain ABI) -----------------------
 * One decode step of a whole MoE model on device-resident weights: the
 * embedding row; per layer nx = RMSNorm(H, attn_norm), H += Mix nx, then
 * nr = RMSNorm(H, post_norm), H += MoE(nr) (LLM_Qwen_Blk.Step,
 * src/llm/llm_qwen_blk.adb:125-170, with LLM_MoE.Forward's router, top-k and
 * experts); then logits = LM RMSNorm(H, final_norm) (src/llm/llm_qwen.adb:
 * 1199-1203).  RMSNorm eps 1e-6.  Weights are given as host pointers and
 * copied into HBM at registration (quantised matrices repacked, a quantised
 * router decoded to f32); the chain owns those copies until
 * aspida_gpu_chain_reset.  The first forward of a lane count runs eagerly;
 * later ones replay a HIP graph captured after it (ASPIDA_NO_GRAPH in the
 * environment, or aspida_kq_chain_set_graphs(0), keeps every forward eager).
 * The reference registers each layer's mixer (attention or delta-net) through
 * aspida_gpu_chain_fattn / aspida_gpu_chain_dnet, which this library does not
 * export: a layer and its mixer -- one matvec -- are registered with
 * aspida_kq_chain_layer instead, so the Ada host's Chain_Available
 * (src/llm/llm_qwen_gpu.adb:554-560) stays false and it keeps its per-layer
 * paths.  Errors: registration failures mark the chain not ready
 * (aspida_gpu_chain_ready() == 0 until a reset); a failed forward fills the
 * logits with NaN; both set aspida_gpu_last_error. */

/* Drop every registered layer and the model.  Replaces gpu/gpu_matvec.cu:2063-2066. */
void aspida_gpu_chain_reset(void);

/* Attach the MoE block to the last registered layer (no-op with no layer).
 * Weight kinds as above (router_k may also be -1: f32 [n_exp][dim]); routed
 * tensors hold n_exp experts of bytes / n_exp each; sgi is the shared-expert
 * gate input when sgi_len > 1 (then sgi_len == dim), else the shared expert is
 * ungated.  n_exp <= 1024, top_k <= 32, intermed % 256 == 0.  Gate, up and
 * the shared gate/up of one kind and both downs of another run on the grouped
 * kernels over packed experts, other mixes on the per-projection kernels.
 * Replaces gpu/gpu_matvec.cu:2143-2199. */
void aspida_gpu_chain_moe(const void *router_w, long router_b, int router_k,
                          const void *gate_w, long gate_b, int gate_k,
                          const void *up_w, long up_b, int up_k,
                          const void *down_w, long down_b, int down_k,
                          const void *shg_w, long shg_b, int shg_k,
                          const void *shu_w, long shu_b, int shu_k,
                          const void *shd_w, long shd_b, int shd_k,
                          const float *sgi, long sgi_b, int sgi_len,
                          int n_exp, int top_k, int intermed);

/* Embedding table (f32 [embed_b / (4 dim)][dim]), final norm (f32 [dim]) and
 * output head ([vocab][dim] of kind lm_k, -1 = f32).  Replaces
 * gpu/gpu_matvec.cu:2201-2211. */
void aspida_gpu_chain_model(const float *embed, long embed_b, const float *fnorm, long fnorm_b,
                            const void *lm, long lm_b, int lm_k, int dim, int vocab);

/* 1 when a model, at least one layer and no failed registration.  Replaces
 * gpu/gpu_matvec.cu:2213. */
int aspida_gpu_chain_ready(void);

/* A generation's start and end: drop the captured graphs.  attn_handles is
 * unused (the matvec mixers keep no per-generation state).  Replace
 * gpu/gpu_matvec.cu:2328-2340. */
void aspida_gpu_chain_begin(const int *attn_handles);
void aspida_gpu_chain_end(void);

/* logits[vocab] of one token whose embedding row is embed_row; pos and
 * attn_handles are unused (see aspida_gpu_chain_begin).  Synchronous.
 * Replaces gpu/gpu_matvec.cu:2356-2400. */
void aspida_gpu_chain_forward(int embed_row, int pos, const int *attn_handles, float *logits);

/* logits[B][vocab] of B lanes (rows[B]) in one step: the matvecs become
 * small-batch products and the MoE blocks run the B tokens together (each
 * expert's weights read once per layer).  1 <= B <= 64 and B * top_k <= 1024;
 * B < 1 is a no-op as in the reference (which clamped B to its lane limit
 * instead of failing).  Replaces gpu/gpu_matvec.cu:2783-2961. */
void aspida_gpu_chain_forward_batch(int B, const int *rows, const int *pos, const int *handles, float *logits);

/* A layer (this library's stand-in for chain_fattn / chain_dnet): attention
 * and post-attention norms (f32 [dim], an_b = pn_b = 4 dim bytes, dim % 256 ==
 * 0) and the mixer, a [dim][dim] matrix of kind mix_k (-1 = f32), or none when
 * mix_w is NULL.  Returns 0 or an error (the chain is then not ready).  No
 * reference counterpart. */
int aspida_kq_chain_layer(const float *attn_norm, long an_b, const float *post_norm, long pn_b,
                          const void *mix_w, long mix_b, int mix_k);

/* The residual stream H[B][dim] after the embedding and the first n_layers
 * layers (0 <= n_layers <= layer count), run eagerly: the chain's state
 * step by step.  Returns 0 or an error.  No reference counterpart. */
int aspida_kq_chain_forward_layers(int B, const int *rows, int n_layers, float *hidden);

/* Graph replay on (1) or off (0) for later forwards; drops captured graphs.
 * aspida_kq_chain_graphs: graphs currently captured.  No reference
 * counterpart. */
int aspida_kq_chain_set_graphs(int on);
int aspida_kq_chain_graphs(void);

/* ---- GGUF tensor layout (host only) ----------------------------------------
 * A reader of GGUF model files for locating and checking real weights: the
 * header, metadata and tensor descriptors with the reference loader's rules
 * (LLM_GGUF.Open_From_Source, src/llm/llm_gguf.adb:317-560; byte sizes per
 * Checked_Byte_Size, 238-258; type codes per To_GGML_Type, 266-291).  A
 * tensor's kind is this library's code (0 Q4_K, 1 Q6_K, 2 Q5_K, 3 Q3_K,
 * 4 Q2_K, 5 Q8_0; LLM_Weight.Kind_Code, src/llm/llm_weight.adb:277-292) or -1;
 * dims[0] is ne0 (in_dim of a weight), dims[1] ne1 (out_dim). */
typedef struct aspida_gguf aspida_gguf;
typedef struct aspida_gguf_tensor_info {
  const char *name;       /* valid until aspida_gguf_close */
  int ggml_type, kind, n_dims;
  long long dims[4];
  long long file_offset;  /* absolute byte offset of the data in the file */
  long long bytes;
} aspida_gguf_tensor_info;
/* NULL on a malformed or unreadable file; aspida_gguf_error() says why. */
aspida_gguf *aspida_gguf_open(const char *path);
const char *aspida_gguf_error(void);
void aspida_gguf_close(aspida_gguf *g);
int aspida_gguf_version(const aspida_gguf *g);
long long aspida_gguf_alignment(const aspida_gguf *g);
long long aspida_gguf_data_start(const aspida_gguf *g);
long long aspida_gguf_tensor_count(const aspida_gguf *g);
long long aspida_gguf_meta_count(const aspida_gguf *g);
/* A metadata value as text (arrays as "[array: N]"), or NULL. */
const char *aspida_gguf_meta(const aspida_gguf *g, const char *key);
/* Index of the tensor named `name`, or -1. */
long long aspida_gguf_find(const aspida_gguf *g, const char *name);
int aspida_gguf_tensor(const aspida_gguf *g, long long i, aspida_gguf_tensor_info *out);
/* Copy tensor i's bytes to dst (cap >= its byte size); returns the byte count
 * or a negative errno. */
long long aspida_gguf_read(const aspida_gguf *g, long long i, void *dst, long long cap);

/* ---- test and tuning hooks (no reference counterpart) ----------------------
 * The aspida_kq_set_* overrides below are per calling thread: each changes
 * the kernel choice of the launches the calling thread makes from then on,
 * and no other thread's.  They exist for tests and tuning runs; production
 * callers leave them at their defaults. */

/* Small-batch workspace check, host only (launches nothing): the bytes of
 * activation split and partial sums the library allocates for a batched
 * product of this kind, shape and batch (*allocated), and the most any single
 * launch of that product uses (*needed).  Returns 0 or -EINVAL. */
int aspida_kq_matmul_workspace(int kind, int in_dim, int out_dim, int batch, long long *allocated,
                               long long *needed);

/* Split override for the packed kernels (aspida_kq_packed_plan): waves per
 * workgroup (a power of two <= 16) and workgroups per tile, applied to every
 * shape whose in_dim / 256 they divide; 0, 0 restores the built-in choice.
 * Per calling thread; for tuning and tests. */
int aspida_kq_set_packed_plan(int waves_per_group, int groups_per_tile);

/* Engine of the batch-1 packed matvec (aspida_kq_matvec_packed_dev and the
 * calls built on it): 0 = matrix cores (MFMA) for Q4_K and Q6_K, the vector
 * kernel for the other kinds (the default); 1 = the vector kernel for every
 * kind.
 * Per calling thread; for comparison and tests.  No reference counterpart.
 * Returns 0, or -EINVAL for another value. */
int aspida_kq_set_mv_engine(int engine);

/* Engine of the packed small-batch product (batch > 1 in
 * aspida_kq_matmul_packed_dev and aspida_gpu_matmul): 0 = the built-in choice
 * (Q4_K and Q6_K: up to 4 vectors on the batch-1 matrix-core kernel where
 * the batch-1 plan is 16-row workgroups, else the one-pass kernel -- Q6_K
 * keeps the batch-1 kernel at 2 vectors -- then the one-pass kernel up to
 * 16 vectors (on matrices of at least 8192 64-row-by-256-column blocks,
 * such as output heads, the 16-vector matrix-core kernel instead, Q6_K from
 * 5 vectors); above 16 the one-pass kernel for Q6_K -- in launches of 32
 * vectors where it takes 64-row tiles; above 32 vectors on at most 1024
 * such blocks the wave-per-column kernel (6) -- and the 64-vector matrix-core
 * kernel for Q4_K; other kinds on the vector kernel); 1 = the vector kernel; 2 = the 64-vector and 3 = the
 * 16-vector matrix-core kernel; 4 = the one-pass matrix-core kernel (up to
 * 64 vectors per weight pass); 5 = the batch-1 matrix-core kernel on up to 4
 * vectors per launch; 6 = the wave-per-column matrix-core kernel (Q4_K and
 * Q6_K with in_dim a multiple of 1024: one wave per 64-row tile and
 * 256-element column, activations split in a pre-pass); for the kinds that
 * have one (others stay on the vector kernel).
 * Per calling thread; for comparison and tests.  No reference counterpart.
 * Returns 0, or -EINVAL for another value. */
int aspida_kq_set_mm_engine(int engine);

/* Workgroup shape of the matrix-core matvec: 0 = the built-in choice (16-row
 * workgroups over all columns for matrices of up to two such blocks per
 * compute unit, 64-row workgroups above), 1 = 64-row, 2 = 16-row workgroups.
 * Per calling thread; for tuning and tests.  No reference counterpart.
 * Returns 0 or -EINVAL. */
int aspida_kq_set_mfma_rows(int mode);

/* Tuning of the matrix-core matvec's splits with several columns per wave:
 * 0 = the built-in choice, 1 = prefetching waves (two register sets),
 * 2 = columns one after another (one register set, more waves per CU).
 * Per calling thread.  No reference counterpart.  Returns 0 or -EINVAL. */
int aspida_kq_set_mfma_pipeline(int mode);

/* Launch-shape override for batch-1 matvecs: rows per lane group per step
 * (1, 2 or 4) and resident waves launched per CU (1..64); rows_per_wave <= 0
 * restores the built-in choice.  Per calling thread; for tuning and tests. */
int aspida_kq_set_mv_config(int rows_per_wave, int waves_per_cu);

#ifdef __cplusplus
}
#endif
#endif
