/*
 * kq_oracle.h -- CPU restatement of Aspida's quantized-weight CPU path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code.  It is used by tests/ (as the parity checker), by
 * __graft_entry__.smoke() (as the checker of one small GPU call) and by
 * bench.py's cpu_baseline leg (the timed CPU path reported beside the GPU).
 *
 * Kind codes follow LLM_Weight.Kind_Code (src/llm/llm_weight.adb:277-292):
 *   0 = Q4_K, 1 = Q6_K, 2 = Q5_K, 3 = Q3_K, 4 = Q2_K, 5 = Q8_0, -1 = dense f32.
 */
#ifndef KQ_ORACLE_H
#define KQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Bytes per 256-element super-block (Q8_0: eight 34-byte blocks). */
int kqo_block_bytes(int kind);

/* IEEE half from two little-endian bytes, with Aspida's Inf/NaN -> +0.0 rule. */
float kqo_f16_to_f32(uint8_t lo, uint8_t hi);

/* Decode one 256-element super-block (or eight Q8_0 blocks) into out[256]. */
int kqo_decode_block(int kind, const uint8_t *blk, float *out);

/* Dequantize out_dim rows of in_dim elements into dst[out_dim * in_dim]. */
int kqo_dequant_rows(int kind, const uint8_t *w, int in_dim, int out_dim, float *dst);

/* Streaming fused matvec y[o] = sum_i W[o, i] * x[i] (LLM_Dequant.QMatVec),
 * rows split across nthreads workers by LLM_Pool.Run's chunking rule
 * (min_grain rows or fewer run serially).  nthreads <= 0 means 1.
 * Returns 0, or a negative code for the guards QMatVec raises on. */
int kqo_qmatvec(int kind, const uint8_t *w, int in_dim, int out_dim,
                const float *x, float *y, int nthreads, int min_grain);

/* Batched form: Y[b][o] for b < batch, each row a kqo_qmatvec. */
int kqo_qmatmul(int kind, const uint8_t *w, int in_dim, int out_dim, int batch,
                const float *x, float *y, int nthreads);

/* Dense f32 row-major matvec, ascending sequential sum per row. */
void kqo_dense_matvec(const float *w, int in_dim, int out_dim, const float *x, float *y);

/* LLM_Pool.Run chunk boundaries: writes up to ncpu (lo, hi) pairs (inclusive)
 * for the range [first, last]; returns the number of chunks. */
int kqo_pool_chunks(int first, int last, int min_grain, int ncpu, int *lo, int *hi);

/* LLM_RMSNorm.Forward: y = (x / sqrt(mean(x^2) + eps)) * w, sum of squares in
 * ascending order. */
void kqo_rmsnorm(const float *x, const float *w, int n, float eps, float *y);

/* Router: softmax over logits, greedy top-k (strict >, lowest index wins ties),
 * renormalised weights.  Writes top_idx (0-based) and top_w. */
void kqo_route(const float *logits, int n_exp, int top_k, int *top_idx, float *top_w);

/* LLM_MoE.Forward for one token.  Expert tensors are [n_exp][rows][cols] in
 * their kinds (dense f32 allowed, kind -1); the router weight is f32
 * [n_exp][dim]; shared_gate_inp may be NULL (ungated shared expert).
 * Also returns the routing it chose (top_idx/top_w, top_k entries). */
int kqo_moe_forward(const float *x, int dim, int intermed, int n_exp, int top_k,
                    const float *router_w,
                    const void *gate_w, int gate_kind, const void *up_w, int up_kind,
                    const void *down_w, int down_kind,
                    const void *shg_w, int shg_kind, const void *shu_w, int shu_kind,
                    const void *shd_w, int shd_kind,
                    const float *shared_gate_inp, int gate_inp_len,
                    float *y, int *top_idx, float *top_w, int nthreads);

/* The expert half of the MoE layer with routing supplied by the caller, i.e.
 * what aspida_gpu_moe_experts computes (gpu_matvec.cu:1673-1758). */
int kqo_moe_experts(const float *x, int dim, int top_k, int intermed, int n_exp,
                    const int *top_idx, const float *top_w,
                    const void *gate_w, int gate_kind, const void *up_w, int up_kind,
                    const void *down_w, int down_kind,
                    const void *shg_w, int shg_kind, const void *shu_w, int shu_kind,
                    const void *shd_w, int shd_kind,
                    const float *shared_gate_inp, int gate_inp_len,
                    float *y, int nthreads);

#ifdef __cplusplus
}
#endif
#endif
