/*
 * kq_oracle.c -- CPU restatement of Aspida's K-quant CPU path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP library and the
 * timed CPU baseline.  The shipped library never links or calls this file.
 *
 * Each function follows the Ada unit it restates, cited file:line into the
 * reference tree (src/llm/...).  Build with -ffp-contract=off: the Ada
 * decoders evaluate "scale * q - min" as a product then a difference, and the
 * fused dot keeps four separate f32 lanes; both are reproduced literally.
 */
#include "kq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

int kqo_block_bytes(int kind)
{
    switch (kind) {
    case 0: return 144;   /* Q4_K */
    case 1: return 210;   /* Q6_K */
    case 2: return 176;   /* Q5_K */
    case 3: return 110;   /* Q3_K */
    case 4: return 84;    /* Q2_K */
    case 5: return 272;   /* Q8_0: 8 x 34 B per 256 elements */
    default: return -1;
    }
}

/* F16_To_F32, src/llm/llm_dequant.adb:33-57.  Exponent 31 (Inf/NaN) maps to
 * +0.0; subnormals and normals are exact. */
float kqo_f16_to_f32(uint8_t lo, uint8_t hi)
{
    const int sign = hi & 0x80;
    const int expo = (hi & 0x7C) >> 2;
    const int mant = ((hi & 3) << 8) + lo;
    float v;
    if (expo == 0) {
        if (mant == 0)
            return sign ? -0.0f : 0.0f;
        v = (float)mant / 1024.0f * ldexpf(1.0f, -14);
    } else if (expo == 31) {
        return 0.0f;
    } else {
        v = (float)(mant + 1024) / 1024.0f * ldexpf(1.0f, expo - 15);
    }
    return sign ? -v : v;
}

static inline float rd_f16(const uint8_t *p) { return kqo_f16_to_f32(p[0], p[1]); }

/* Get_SM / Scale_Min: the j-th 6-bit (scale, min) pair of the 12 packed bytes
 * shared by Q4_K and Q5_K (llm_dequant.adb:369-380, 436-447, 514-525). */
static inline void scale_min_k4(const uint8_t *sc, int j, int *s, int *m)
{
    if (j < 4) {
        *s = sc[j] & 63;
        *m = sc[j + 4] & 63;
    } else {
        *s = (sc[j + 4] & 0x0F) | ((sc[j - 4] >> 6) << 4);
        *m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
}

/* Decode_Q4K_Block, llm_dequant.adb:504-554. */
static void decode_q4k(const uint8_t *b, float *out)
{
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *qs = b + 16;
    for (int g = 0; g < 4; ++g) {
        int s1, m1, s2, m2;
        scale_min_k4(sc, 2 * g, &s1, &m1);
        scale_min_k4(sc, 2 * g + 1, &s2, &m2);
        const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        const float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        const uint8_t *q = qs + 32 * g;
        for (int l = 0; l < 32; ++l)
            out[64 * g + l] = d1 * (float)(q[l] & 0x0F) - mm1;
        for (int l = 0; l < 32; ++l)
            out[64 * g + 32 + l] = d2 * (float)(q[l] >> 4) - mm2;
    }
}

/* Decode_Q5K_Block, llm_dequant.adb:426-498. */
static void decode_q5k(const uint8_t *b, float *out)
{
    const float d = rd_f16(b), dmin = rd_f16(b + 2);
    const uint8_t *sc = b + 4, *qh = b + 16, *qs = b + 48;
    for (int g = 0; g < 4; ++g) {
        int s1, m1, s2, m2;
        scale_min_k4(sc, 2 * g, &s1, &m1);
        scale_min_k4(sc, 2 * g + 1, &s2, &m2);
        const float d1 = d * (float)s1, mm1 = dmin * (float)m1;
        const float d2 = d * (float)s2, mm2 = dmin * (float)m2;
        for (int l = 0; l < 32; ++l) {
            const unsigned q = qs[32 * g + l];
            const unsigned lo = (q & 0x0F) + (((qh[l] >> (2 * g)) & 1u) << 4);
            const unsigned hi = (q >> 4) + (((qh[l] >> (2 * g + 1)) & 1u) << 4);
            out[64 * g + l] = d1 * (float)lo - mm1;
            out[64 * g + 32 + l] = d2 * (float)hi - mm2;
        }
    }
}

/* Decode_Q6K_Block, llm_dequant.adb:122-184. */
static void decode_q6k(const uint8_t *b, float *out)
{
    const uint8_t *ql = b, *qh = b + 128;
    const int8_t *sc = (const int8_t *)(b + 192);
    const float d = rd_f16(b + 208);
    for (int h = 0; h < 2; ++h) {
        const uint8_t *QL = ql + 64 * h, *QH = qh + 32 * h;
        const int8_t *SC = sc + 8 * h;
        float *Y = out + 128 * h;
        for (int ig = 0; ig < 2; ++ig) {
            const float ds1 = d * (float)SC[ig + 0];
            const float ds2 = d * (float)SC[ig + 2];
            const float ds3 = d * (float)SC[ig + 4];
            const float ds4 = d * (float)SC[ig + 6];
            for (int l = 16 * ig; l < 16 * ig + 16; ++l) {
                const unsigned a = QL[l], c = QL[l + 32], hb = QH[l];
                const int q1 = (int)((a & 0x0F) | ((hb & 3u) << 4)) - 32;
                const int q2 = (int)((c & 0x0F) | (((hb >> 2) & 3u) << 4)) - 32;
                const int q3 = (int)((a >> 4) | (((hb >> 4) & 3u) << 4)) - 32;
                const int q4 = (int)((c >> 4) | (((hb >> 6) & 3u) << 4)) - 32;
                Y[l] = ds1 * (float)q1;
                Y[l + 32] = ds2 * (float)q2;
                Y[l + 64] = ds3 * (float)q3;
                Y[l + 96] = ds4 * (float)q4;
            }
        }
    }
}

static inline uint32_t le32(const uint8_t *p)
{
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

/* Element P of a 256-element super-block in the shared Q2_K/Q3_K interleave:
 * 128-half NH, 2-bit field J, 16-group G, lane L (llm_dequant.adb:247-256). */
#define KQ_SPLIT(P, NH, J, G, L)                                   \
    const int NH = (P) / 128, J = ((P) % 128) / 32,                \
              G = ((P) % 32) / 16, L = (P) % 16

/* Decode_Q3K_Block, llm_dequant.adb:207-268. */
static void decode_q3k(const uint8_t *b, float *out)
{
    const uint8_t *hm = b, *qs = b + 32, *scb = b + 96;
    const float d = rd_f16(b + 108);
    const uint32_t km1 = 0x03030303u, km2 = 0x0F0F0F0Fu;
    const uint32_t a0 = le32(scb), a1 = le32(scb + 4), tmp = le32(scb + 8);
    uint32_t s[4];
    s[0] = (a0 & km2) | ((tmp & km1) << 4);
    s[1] = (a1 & km2) | (((tmp >> 2) & km1) << 4);
    s[2] = ((a0 >> 4) & km2) | (((tmp >> 4) & km1) << 4);
    s[3] = ((a1 >> 4) & km2) | (((tmp >> 6) & km1) << 4);
    for (int p = 0; p < 256; ++p) {
        KQ_SPLIT(p, nh, j, g, l);
        const int low2 = (qs[nh * 32 + g * 16 + l] >> (2 * j)) & 3;
        const int hbit = (hm[g * 16 + l] >> (nh * 4 + j)) & 1;
        const int sg = low2 + 4 * hbit - 4;
        const int iss = nh * 8 + j * 2 + g;
        const int scale = (int)((s[iss / 4] >> (8 * (iss % 4))) & 0xFF) - 32;
        out[p] = d * (float)scale * (float)sg;
    }
}

/* Decode_Q2K_Block, llm_dequant.adb:291-322. */
static void decode_q2k(const uint8_t *b, float *out)
{
    const uint8_t *sc = b, *qs = b + 16;
    const float d = rd_f16(b + 80), dmin = rd_f16(b + 82);
    for (int p = 0; p < 256; ++p) {
        KQ_SPLIT(p, nh, j, g, l);
        const int iss = nh * 8 + j * 2 + g;
        const unsigned s = sc[iss];
        const float q2 = (float)((qs[nh * 32 + g * 16 + l] >> (2 * j)) & 3);
        const float dl = d * (float)(s & 0x0F);
        const float ml = dmin * (float)(s >> 4);
        out[p] = dl * q2 - ml;
    }
}

/* Dequant_Q8_0, llm_dequant.adb:606-630 (32-element blocks of f16 d + int8). */
static void decode_q8_0x8(const uint8_t *b, float *out)
{
    for (int k = 0; k < 8; ++k) {
        const uint8_t *blk = b + 34 * k;
        const float d = rd_f16(blk);
        for (int j = 0; j < 32; ++j)
            out[32 * k + j] = d * (float)(int8_t)blk[2 + j];
    }
}

int kqo_decode_block(int kind, const uint8_t *blk, float *out)
{
    switch (kind) {
    case 0: decode_q4k(blk, out); return 0;
    case 1: decode_q6k(blk, out); return 0;
    case 2: decode_q5k(blk, out); return 0;
    case 3: decode_q3k(blk, out); return 0;
    case 4: decode_q2k(blk, out); return 0;
    case 5: decode_q8_0x8(blk, out); return 0;
    default: return -1;
    }
}

int kqo_dequant_rows(int kind, const uint8_t *w, int in_dim, int out_dim, float *dst)
{
    const int bpb = kqo_block_bytes(kind);
    if (bpb < 0 || in_dim % 256 != 0)
        return -1;
    const int nb = in_dim / 256;
    const size_t row_bytes = (size_t)nb * bpb;
    for (int o = 0; o < out_dim; ++o)
        for (int b = 0; b < nb; ++b)
            kqo_decode_block(kind, w + (size_t)o * row_bytes + (size_t)b * bpb,
                             dst + (size_t)o * in_dim + (size_t)b * 256);
    return 0;
}

/* ---- LLM_Pool.Run (src/llm/llm_pool.adb:91-160) ------------------------- */

int kqo_pool_chunks(int first, int last, int min_grain, int ncpu, int *lo, int *hi)
{
    const int count = last - first + 1;
    if (count <= 0)
        return 0;
    const int n_workers = ncpu - 1 > 0 ? ncpu - 1 : 0;
    if (count < min_grain || n_workers == 0) {       /* serial fallback, 103-106 */
        lo[0] = first;
        hi[0] = last;
        return 1;
    }
    const int nn = (n_workers + 1) < count ? (n_workers + 1) : count;
    const int chunk = (count + nn - 1) / nn;
    int n = 0;
    for (int i = 1; i <= nn; ++i) {
        const int l = first + (i - 1) * chunk;
        if (l > last)
            break;
        const int h = first + i * chunk - 1;
        lo[n] = l;
        hi[n] = h < last ? h : last;
        ++n;
    }
    return n;
}

typedef void (*range_fn)(void *ctx, int lo, int hi);
struct range_job { range_fn fn; void *ctx; int lo, hi; };

static void *range_thread(void *p)
{
    struct range_job *j = (struct range_job *)p;
    j->fn(j->ctx, j->lo, j->hi);
    return NULL;
}

/* Run fn over [first, last] in LLM_Pool's chunks; chunk 1 on the caller. */
static void pool_run(range_fn fn, void *ctx, int first, int last, int min_grain, int nthreads)
{
    if (nthreads < 1)
        nthreads = 1;
    int lo[512], hi[512];
    if (nthreads > 512)
        nthreads = 512;
    const int n = kqo_pool_chunks(first, last, min_grain, nthreads, lo, hi);
    if (n <= 1) {
        if (n == 1)
            fn(ctx, lo[0], hi[0]);
        return;
    }
    pthread_t th[512];
    struct range_job jobs[512];
    int started[512];
    for (int i = 1; i < n; ++i) {
        jobs[i].fn = fn; jobs[i].ctx = ctx; jobs[i].lo = lo[i]; jobs[i].hi = hi[i];
        started[i] = pthread_create(&th[i], NULL, range_thread, &jobs[i]) == 0;
        if (!started[i])
            fn(ctx, lo[i], hi[i]);
    }
    fn(ctx, lo[0], hi[0]);
    for (int i = 1; i < n; ++i)
        if (started[i])
            pthread_join(th[i], NULL);
}

/* ---- QMatVec (llm_dequant.adb:808-932) ------------------------------------ */

struct qmv_ctx {
    int kind, in_dim, nb, bpb;
    size_t row_bytes;
    const uint8_t *w;
    const float *x;
    float *y;
};

/* Rows_Op.Execute, llm_dequant.adb:869-925. */
static void qmv_rows(void *p, int lo, int hi)
{
    const struct qmv_ctx *c = (const struct qmv_ctx *)p;
    float bk[256];
    for (int o = lo; o <= hi; ++o) {
        const uint8_t *row = c->w + (size_t)o * c->row_bytes;
        if (c->kind == 5) {
            /* Q8_0 is not fused: Fill one row, then an ascending dot (909-923). */
            float acc = 0.0f;
            for (int b = 0; b < c->nb; ++b) {
                decode_q8_0x8(row + (size_t)b * c->bpb, bk);
                for (int i = 0; i < 256; ++i)
                    acc = acc + bk[i] * c->x[b * 256 + i];
            }
            c->y[o] = acc;
            continue;
        }
        /* Four interleaved accumulator lanes, combined as (A0+A1)+(A2+A3). */
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
        for (int b = 0; b < c->nb; ++b) {
            kqo_decode_block(c->kind, row + (size_t)b * c->bpb, bk);
            const float *xl = c->x + (size_t)b * 256;
            for (int k = 0; k < 64; ++k) {
                a0 = a0 + bk[4 * k + 0] * xl[4 * k + 0];
                a1 = a1 + bk[4 * k + 1] * xl[4 * k + 1];
                a2 = a2 + bk[4 * k + 2] * xl[4 * k + 2];
                a3 = a3 + bk[4 * k + 3] * xl[4 * k + 3];
            }
        }
        c->y[o] = (a0 + a1) + (a2 + a3);
    }
}

int kqo_qmatvec(int kind, const uint8_t *w, int in_dim, int out_dim,
                const float *x, float *y, int nthreads, int min_grain)
{
    const int bpb = kqo_block_bytes(kind);
    if (bpb < 0)
        return -1;
    if (in_dim % 256 != 0)      /* 840-844: K-quant in-dim not a multiple of 256 */
        return -2;
    if (out_dim < 0)
        return -3;
    struct qmv_ctx c;
    c.kind = kind; c.in_dim = in_dim; c.nb = in_dim / 256; c.bpb = bpb;
    c.row_bytes = (size_t)c.nb * bpb; c.w = w; c.x = x; c.y = y;
    pool_run(qmv_rows, &c, 0, out_dim - 1, min_grain, nthreads);
    return 0;
}

int kqo_qmatmul(int kind, const uint8_t *w, int in_dim, int out_dim, int batch,
                const float *x, float *y, int nthreads)
{
    for (int b = 0; b < batch; ++b) {
        const int rc = kqo_qmatvec(kind, w, in_dim, out_dim, x + (size_t)b * in_dim,
                                   y + (size_t)b * out_dim, nthreads, 2048);
        if (rc)
            return rc;
    }
    return 0;
}

/* Dense_MatVec (llm_weight.adb) and QMatVec's generic F32 fallback
 * (llm_dequant.adb:909-923): one accumulator, ascending index. */
void kqo_dense_matvec(const float *w, int in_dim, int out_dim, const float *x, float *y)
{
    for (int o = 0; o < out_dim; ++o) {
        const float *r = w + (size_t)o * in_dim;
        float acc = 0.0f;
        for (int i = 0; i < in_dim; ++i)
            acc = acc + r[i] * x[i];
        y[o] = acc;
    }
}

/* ---- LLM_MoE.Forward (src/llm/llm_moe.adb:111-302) ------------------------ */

/* LLM_RMSNorm.Forward, src/llm/llm_rmsnorm.adb:10-41: Sum_Sq accumulated in
 * ascending order (a product, then the sum), Rms = Sqrt (Sum_Sq / N + Eps),
 * y(I) = (x(I) / Rms) * w(I).  The Ada default Eps is 1.0e-6
 * (llm_rmsnorm.ads:19). */
void kqo_rmsnorm(const float *x, const float *w, int n, float eps, float *y)
{
    float sum_sq = 0.0f;
    for (int i = 0; i < n; ++i)
        sum_sq = sum_sq + x[i] * x[i];
    const float rms = sqrtf(sum_sq / (float)n + eps);
    for (int i = 0; i < n; ++i)
        y[i] = (x[i] / rms) * w[i];
}

static float silu(float v) { return v / (1.0f + expf(-v)); }   /* llm_moe.adb:88 */

/* Steps 2-3 of Forward (llm_moe.adb:153-197), in place on p[n_exp]. */
void kqo_route(const float *logits, int n_exp, int top_k, int *top_idx, float *top_w)
{
    float *r = (float *)malloc(sizeof(float) * (size_t)n_exp);
    char *used = (char *)calloc((size_t)n_exp, 1);
    float max_l = logits[0], sum_e = 0.0f, sum_w = 0.0f;
    for (int e = 1; e < n_exp; ++e)
        if (logits[e] > max_l)
            max_l = logits[e];
    for (int e = 0; e < n_exp; ++e) {
        r[e] = expf(logits[e] - max_l);
        sum_e = sum_e + r[e];
    }
    for (int e = 0; e < n_exp; ++e)
        r[e] = r[e] / sum_e;
    for (int k = 0; k < top_k; ++k) {
        int best_e = -1;
        float best_v = -3.40282347e38f;          /* Float'First */
        for (int e = 0; e < n_exp; ++e)
            if (!used[e] && r[e] > best_v) {
                best_v = r[e];
                best_e = e;
            }
        if (best_e < 0)                           /* all-NaN row: keep index valid */
            best_e = 0;
        top_idx[k] = best_e;
        top_w[k] = best_v;
        used[best_e] = 1;
        sum_w = sum_w + best_v;
    }
    for (int k = 0; k < top_k; ++k)
        top_w[k] = top_w[k] / sum_w;
    free(r);
    free(used);
}

/* One projection of an expert tensor: rows x cols, slice e of n_exp. */
static void proj(const void *w, int kind, int e, int rows, int cols, const float *x,
                 float *y, int nthreads, int min_grain)
{
    if (kind < 0) {
        const float *base = (const float *)w + (size_t)e * rows * cols;
        kqo_dense_matvec(base, cols, rows, x, y);
        return;
    }
    const size_t bpe = (size_t)rows * (cols / 256) * kqo_block_bytes(kind);
    kqo_qmatvec(kind, (const uint8_t *)w + (size_t)e * bpe, cols, rows, x, y,
                nthreads, min_grain);
}

struct experts_ctx {
    const float *x;
    int dim, intermed;
    const int *top_idx;
    const float *top_w;
    const void *gate_w, *up_w, *down_w;
    int gate_kind, up_kind, down_kind;
    float *exp_y;     /* [top_k][dim] */
};

/* Experts_Op.Execute, llm_moe.adb:253-268 (nested matvecs run serially). */
static void experts_rows(void *p, int lo, int hi)
{
    const struct experts_ctx *c = (const struct experts_ctx *)p;
    float *g = (float *)malloc(sizeof(float) * (size_t)c->intermed);
    float *u = (float *)malloc(sizeof(float) * (size_t)c->intermed);
    float *yd = (float *)malloc(sizeof(float) * (size_t)c->dim);
    for (int k = lo; k <= hi; ++k) {
        const int e = c->top_idx[k];
        proj(c->gate_w, c->gate_kind, e, c->intermed, c->dim, c->x, g, 1, 1 << 30);
        proj(c->up_w, c->up_kind, e, c->intermed, c->dim, c->x, u, 1, 1 << 30);
        for (int j = 0; j < c->intermed; ++j)
            g[j] = silu(g[j]) * u[j];
        proj(c->down_w, c->down_kind, e, c->dim, c->intermed, g, yd, 1, 1 << 30);
        for (int i = 0; i < c->dim; ++i)
            c->exp_y[(size_t)k * c->dim + i] = c->top_w[k] * yd[i];
    }
    free(g);
    free(u);
    free(yd);
}

int kqo_moe_experts(const float *x, int dim, int top_k, int intermed, int n_exp,
                    const int *top_idx, const float *top_w,
                    const void *gate_w, int gate_kind, const void *up_w, int up_kind,
                    const void *down_w, int down_kind,
                    const void *shg_w, int shg_kind, const void *shu_w, int shu_kind,
                    const void *shd_w, int shd_kind,
                    const float *shared_gate_inp, int gate_inp_len,
                    float *y, int nthreads)
{
    (void)n_exp;
    if (top_k < 1 || dim < 1 || intermed < 1)
        return -1;
    for (int k = 0; k < top_k; ++k)
        if (top_idx[k] < 0 || top_idx[k] >= n_exp)
            return -2;
    float *exp_y = (float *)malloc(sizeof(float) * (size_t)top_k * dim);
    struct experts_ctx c = { x, dim, intermed, top_idx, top_w, gate_w, up_w, down_w,
                             gate_kind, up_kind, down_kind, exp_y };
    pool_run(experts_rows, &c, 0, top_k - 1, 2, nthreads);      /* Min_Grain => 2 */
    for (int i = 0; i < dim; ++i)
        y[i] = 0.0f;
    for (int k = 0; k < top_k; ++k)                              /* ascending K */
        for (int i = 0; i < dim; ++i)
            y[i] = y[i] + exp_y[(size_t)k * dim + i];
    free(exp_y);

    /* Step 5, shared expert with the optional sigmoid gate (280-299). */
    float *g = (float *)malloc(sizeof(float) * (size_t)intermed);
    float *u = (float *)malloc(sizeof(float) * (size_t)intermed);
    float *ys = (float *)malloc(sizeof(float) * (size_t)dim);
    proj(shg_w, shg_kind, 0, intermed, dim, x, g, nthreads, 2048);
    proj(shu_w, shu_kind, 0, intermed, dim, x, u, nthreads, 2048);
    for (int j = 0; j < intermed; ++j)
        g[j] = silu(g[j]) * u[j];
    proj(shd_w, shd_kind, 0, dim, intermed, g, ys, nthreads, 2048);
    float shared_gate = 1.0f;
    if (gate_inp_len > 1 && shared_gate_inp) {
        float gs = 0.0f;
        for (int d = 0; d < dim; ++d)
            gs = gs + shared_gate_inp[d] * x[d];
        shared_gate = 1.0f / (1.0f + expf(-gs));
    }
    for (int i = 0; i < dim; ++i)
        y[i] = y[i] + shared_gate * ys[i];
    free(g);
    free(u);
    free(ys);
    return 0;
}

int kqo_moe_forward(const float *x, int dim, int intermed, int n_exp, int top_k,
                    const float *router_w,
                    const void *gate_w, int gate_kind, const void *up_w, int up_kind,
                    const void *down_w, int down_kind,
                    const void *shg_w, int shg_kind, const void *shu_w, int shu_kind,
                    const void *shd_w, int shd_kind,
                    const float *shared_gate_inp, int gate_inp_len,
                    float *y, int *top_idx, float *top_w, int nthreads)
{
    if (top_k > n_exp)          /* Create_MoE: Top_K := min(8, N_Experts) */
        top_k = n_exp;
    float *logits = (float *)malloc(sizeof(float) * (size_t)n_exp);
    kqo_dense_matvec(router_w, dim, n_exp, x, logits);         /* step 1 */
    kqo_route(logits, n_exp, top_k, top_idx, top_w);           /* steps 2-3 */
    free(logits);
    return kqo_moe_experts(x, dim, top_k, intermed, n_exp, top_idx, top_w,
                           gate_w, gate_kind, up_w, up_kind, down_w, down_kind,
                           shg_w, shg_kind, shu_w, shu_kind, shd_w, shd_kind,
                           shared_gate_inp, gate_inp_len, y, nthreads);
}
