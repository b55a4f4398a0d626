/*
 * CPU oracle for the ternary BitLinear hot path -- TEST INFRASTRUCTURE ONLY.
 * (see bm_oracle.h for what pins each function)
 *
 * Numerics follow the reference's scalar build exactly: x86-64 SSE float
 * arithmetic, no FMA contraction (the reference compiles kernel.c with
 * -std=gnu11 -O3 and no -mfma, Makefile:4, :92-93), libm expf/logf/sqrtf.
 * Rows are distributed over OpenMP threads; every row's arithmetic is
 * independent of the distribution, as it is under the reference's pool.
 */
#include "bm_oracle.h"

#include <math.h>
#include <stdbool.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ */
/* PRNG (src/utils.c:117-140)                                           */
/* ------------------------------------------------------------------ */
uint64_t orc_rng_next(uint64_t *state)
{
    uint64_t x = *state;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *state = x;
    return x * 0x2545F4914F6CDD1DULL;
}

/* ------------------------------------------------------------------ */
/* Sampler (src/model.c:37-361): temperature, min_p, top_k (bucket      */
/* histogram + min-heap), top_p, CDF draw                               */
/* ------------------------------------------------------------------ */
typedef struct {
    int id;
    float val;
} orc_cand_t;

/* descending by value; equal values compare equal (src/model.c:37-43) */
static int orc_desc(const void *pa, const void *pb)
{
    const float d = ((const orc_cand_t *) pb)->val - ((const orc_cand_t *) pa)->val;
    if (d > 0)
        return 1;
    return d < 0 ? -1 : 0;
}

/* min-heap on val: the node moves below the smaller child, the left one
 * when both are smaller and equal (src/model.c:50-65) */
static void orc_heap_down(orc_cand_t *h, int n, int i)
{
    for (;;) {
        int m = i;
        const int l = 2 * i + 1;
        if (l < n && h[l].val < h[m].val)
            m = l;
        if (l + 1 < n && h[l + 1].val < h[m].val)
            m = l + 1;
        if (m == i)
            return;
        orc_cand_t t = h[i];
        h[i] = h[m];
        h[m] = t;
        i = m;
    }
}

/* keep the k largest of c[0..n) in c[0..k), heap-ordered (src/model.c:238-250) */
static void orc_heap_keep(orc_cand_t *c, int n, int k)
{
    for (int i = k / 2 - 1; i >= 0; i--)
        orc_heap_down(c, k, i);
    for (int i = k; i < n; i++)
        if (c[i].val > c[0].val) {
            c[0] = c[i];
            orc_heap_down(c, k, 0);
        }
}

static float orc_uniform(uint64_t *rng)
{
    return (float) (orc_rng_next(rng) >> 11) * (1.0f / 9007199254740992.0f);
}

/* filter_and_sample with min_p = 0 (src/model.c:67-127) */
static int orc_draw(const orc_cand_t *c, int n, float top_p, int top_k, uint64_t *rng)
{
    if (top_p < 1.0f) {
        double acc = 0.0;
        int i = 0;
        while (i < n) {
            acc += c[i].val;
            i++;
            if (acc >= top_p)
                break;
        }
        n = i;
    }
    if (top_k > 0 && n > top_k)
        n = top_k;
    double total = 0.0;
    for (int i = 0; i < n; i++)
        total += c[i].val;
    const float r = orc_uniform(rng) * (float) total;
    double cdf = 0.0;
    for (int i = 0; i < n; i++) {
        cdf += c[i].val;
        if (r < cdf)
            return c[i].id;
    }
    return c[n - 1].id;
}

static int orc_first_max(const float *v, int n)
{
    int best = 0;
    for (int i = 1; i < n; i++)
        if (v[i] > v[best])
            best = i;
    return best;
}

/* softmax of c[0..n) against `top`: expf(v - top), divided by the double
 * sum taken in array order (src/model.c:253-266, 293-300) */
static void orc_softmax(orc_cand_t *c, int n, float top)
{
    double z = 0.0;
    for (int i = 0; i < n; i++) {
        c[i].val = expf(c[i].val - top);
        z += c[i].val;
    }
    const float inv = 1.0f / (float) z;
    for (int i = 0; i < n; i++)
        c[i].val *= inv;
}

int orc_sample(float *logits, int vocab, float temp, float min_p, float top_p, int top_k,
               uint64_t *rng)
{
    if (temp < 0.05f) {
        int best = 0;
        float top = -1e9f;
        for (int i = 0; i < vocab; i++)
            if (logits[i] > top) {
                top = logits[i];
                best = i;
            }
        return best;
    }
    const float inv_t = 1.0f / temp;
    float top = -1e30f;
    for (int i = 0; i < vocab; i++) {
        logits[i] *= inv_t;
        if (logits[i] > top)
            top = logits[i];
    }
    float floor_v = -1e30f;
    if (min_p >= 1.0f)
        floor_v = top;
    else if (min_p > 0.0f)
        floor_v = top + logf(min_p);

    orc_cand_t *c = malloc((size_t) vocab * sizeof(*c));
    int tok;
    if (top_k > 0 && top_k <= 256) {
        int count[128] = {0};
        const float per_unit = 127.0f / 20.0f;
        for (int i = 0; i < vocab; i++) {
            if (!(logits[i] >= floor_v))
                continue;
            int b = (int) ((top - logits[i]) * per_unit);
            b = b > 127 ? 127 : b;
            b = b < 0 ? 0 : b;
            count[b]++;
        }
        int cut = 127, seen = 0;
        for (int b = 0; b < 128; b++) {
            seen += count[b];
            if (seen >= top_k) {
                cut = b;
                break;
            }
        }
        float lo = top - (float) (cut + 1) / per_unit;
        if (!(lo > floor_v))
            lo = floor_v;
        int n = 0;
        for (int i = 0; i < vocab; i++)
            if (logits[i] >= lo)
                c[n++] = (orc_cand_t) {i, logits[i]};
        if (n == 0) {
            tok = orc_first_max(logits, vocab);
        } else {
            if (n > top_k) {
                orc_heap_keep(c, n, top_k);
                n = top_k;
            }
            float lm = -1e30f;
            for (int i = 0; i < n; i++)
                if (c[i].val > lm)
                    lm = c[i].val;
            orc_softmax(c, n, lm);
            if (top_p < 1.0f)
                qsort(c, n, sizeof(*c), orc_desc);
            tok = orc_draw(c, n, top_p, 0, rng);
        }
    } else {
        int n = 0;
        for (int i = 0; i < vocab; i++)
            if (logits[i] >= floor_v)
                c[n++] = (orc_cand_t) {i, logits[i]};
        if (n == 0) {
            tok = orc_first_max(logits, vocab);
        } else {
            orc_softmax(c, n, top);
            tok = -1;
            if (top_p >= 1.0f && (top_k <= 0 || top_k >= n)) {
                tok = orc_draw(c, n, top_p, top_k, rng);
            } else {
                if (top_p < 1.0f && n > 256) {
                    orc_cand_t part[256];
                    orc_cand_t *tmp = malloc((size_t) n * sizeof(*tmp));
                    memcpy(tmp, c, (size_t) n * sizeof(*tmp));
                    orc_heap_keep(tmp, n, 256);
                    memcpy(part, tmp, sizeof(part));
                    free(tmp);
                    qsort(part, 256, sizeof(part[0]), orc_desc);
                    double acc = 0.0;
                    for (int i = 0; i < 256 && tok < 0; i++) {
                        acc += part[i].val;
                        if (acc >= top_p)
                            tok = orc_draw(part, 256, top_p, top_k, rng);
                    }
                }
                if (tok < 0) {
                    qsort(c, n, sizeof(*c), orc_desc);
                    tok = orc_draw(c, n, top_p, top_k, rng);
                }
            }
        }
    }
    free(c);
    return tok;
}

/* ------------------------------------------------------------------ */
/* a1: ternary decode tables (src/quantization.c:12-53)                 */
/* ------------------------------------------------------------------ */
int orc_decode_weight(int bits)
{
    /* 00 -> -1, 01 -> 0, 10 -> +1, 11 -> +1 (clipped) */
    int v = bits - 1;
    return v > 1 ? 1 : v;
}

static int8_t g_unpack[256][4];
static uint8_t g_pmask[256], g_nmask[256];
static bool g_luts_ready;

static void luts_init(void)
{
    if (g_luts_ready)
        return;
    for (int b = 0; b < 256; b++) {
        uint8_t p = 0, n = 0;
        for (int j = 0; j < 4; j++) {
            int w = orc_decode_weight((b >> (2 * j)) & 3);
            g_unpack[b][j] = (int8_t) w;
            if (w > 0)
                p |= (uint8_t) (1u << j);
            else if (w < 0)
                n |= (uint8_t) (1u << j);
        }
        g_pmask[b] = p;
        g_nmask[b] = n;
    }
    g_luts_ready = true;
}

void orc_luts(int8_t *unpack, uint8_t *pmask, uint8_t *nmask)
{
    luts_init();
    memcpy(unpack, g_unpack, sizeof(g_unpack));
    memcpy(pmask, g_pmask, sizeof(g_pmask));
    memcpy(nmask, g_nmask, sizeof(g_nmask));
}

/* ------------------------------------------------------------------ */
/* a3: RMSNorm with fused max |out| (src/kernel.c:72-129)               */
/* ------------------------------------------------------------------ */
float orc_rms_norm(const float *x, int size, const float *weight, float *out)
{
    /* four interleaved sequential chains, combined ((s0+s1)+s2)+s3, then
     * the tail elements added one by one (src/kernel.c:77-89) */
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int i = 0;
    for (; i + 4 <= size; i += 4)
        for (int j = 0; j < 4; j++) {
            float p = x[i + j] * x[i + j];
            s[j] = s[j] + p;
        }
    float sum_sq = ((s[0] + s[1]) + s[2]) + s[3];
    for (; i < size; i++) {
        float p = x[i] * x[i];
        sum_sq = sum_sq + p;
    }

    float rms = 1.0f / sqrtf(sum_sq / (float) size + 1e-6f); /* :91 */

    /* out = (x * rms) * w, left to right; max |out| is order free */
    float max_abs = 0.0f;
    for (i = 0; i < size; i++) {
        float v = (x[i] * rms) * weight[i];
        out[i] = v;
        float a = fabsf(v);
        if (a > max_abs)
            max_abs = a;
    }
    return max_abs;
}

/* ------------------------------------------------------------------ */
/* a4: int8 quantization, ties away from zero (src/kernel.c:358-386)    */
/* ------------------------------------------------------------------ */
float orc_quantize(const float *x_norm, int n, float max_abs, int8_t *x_quant)
{
    float scale_x = 127.0f / (max_abs + 1e-5f);
    for (int i = 0; i < n; i++) {
        float v = x_norm[i] * scale_x;
        int iv = (int) (v + (v >= 0 ? 0.5f : -0.5f));
        if (iv > 127)
            iv = 127;
        if (iv < -128)
            iv = -128;
        x_quant[i] = (int8_t) iv;
    }
    return scale_x;
}

/* ------------------------------------------------------------------ */
/* a5-a7: T-MAC LUT GEMV with 256-group (1024-column) blocking          */
/* ------------------------------------------------------------------ */
enum { ORC_BLOCK_GROUPS = 256 }; /* TMAC_BLOCK_SIZE, src/kernel.c:12 */

int orc_tmac_slice_count(int cols)
{
    int n_groups = cols / 4;
    return (n_groups + ORC_BLOCK_GROUPS - 1) / ORC_BLOCK_GROUPS;
}

/* lut[mask] = sum of the 4 activations selected by mask
 * (build_tmac_lut, src/kernel.c:136-157) */
static void build_lut16(const int8_t *x, int32_t *lut)
{
    for (int m = 0; m < 16; m++) {
        int32_t s = 0;
        for (int j = 0; j < 4; j++)
            if (m & (1 << j))
                s += x[j];
        lut[m] = s;
    }
}

void orc_tmac_totals(const int8_t *x_quant,
                     const uint8_t *packed,
                     int rows,
                     int cols,
                     int32_t *slice_totals,
                     int32_t *rem_totals)
{
    luts_init();
    int stride = (cols + 3) / 4;
    int n_groups = cols / 4;
    int n_slices = orc_tmac_slice_count(cols);

    int32_t (*luts)[16] = malloc((size_t) (n_groups ? n_groups : 1) *
                                 sizeof(*luts));
    for (int g = 0; g < n_groups; g++)
        build_lut16(x_quant + 4 * g, luts[g]);

#pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const uint8_t *row = packed + (size_t) r * stride;
        for (int s = 0; s < n_slices; s++) {
            int g0 = s * ORC_BLOCK_GROUPS;
            int g1 = g0 + ORC_BLOCK_GROUPS;
            if (g1 > n_groups)
                g1 = n_groups;
            int32_t t = 0;
            for (int g = g0; g < g1; g++)
                t += luts[g][g_pmask[row[g]]] - luts[g][g_nmask[row[g]]];
            slice_totals[(size_t) r * n_slices + s] = t;
        }
        /* remainder columns via UNPACK_LUT (src/kernel.c:430-447) */
        int32_t rt = 0;
        for (int c = 4 * n_groups; c < cols; c++)
            rt += g_unpack[row[n_groups]][c & 3] * x_quant[c];
        rem_totals[r] = rt;
    }
    free(luts);
}

void orc_tmac_rows_f32(const int8_t *x_quant,
                       const uint8_t *packed,
                       int rows,
                       int cols,
                       float inv_scale,
                       float *out)
{
    int n_slices = orc_tmac_slice_count(cols);
    int32_t *st = malloc((size_t) rows * (n_slices ? n_slices : 1) *
                         sizeof(int32_t));
    int32_t *rt = malloc((size_t) rows * sizeof(int32_t));
    orc_tmac_totals(x_quant, packed, rows, cols, st, rt);
    bool has_rem = (cols % 4) != 0;
    for (int r = 0; r < rows; r++) {
        float o = 0.0f; /* out zeroed, then += per block (:407-425) */
        for (int s = 0; s < n_slices; s++) {
            float part = (float) st[(size_t) r * n_slices + s] * inv_scale;
            o = o + part;
        }
        if (has_rem) {
            float part = (float) rt[r] * inv_scale;
            o = o + part;
        }
        out[r] = o;
    }
    free(st);
    free(rt);
}

void orc_bitlinear_forward(const float *x,
                           int n,
                           const uint8_t *packed,
                           int rows,
                           int cols,
                           float w_scale,
                           const float *norm_w,
                           float *out,
                           float *x_norm_buf,
                           int8_t *x_quant_buf)
{
    if (n != cols)
        abort(); /* BITLINEAR_CHECK, src/bitmamba.h:219-231 */
    float max_abs = orc_rms_norm(x, n, norm_w, x_norm_buf);
    float scale_x = orc_quantize(x_norm_buf, n, max_abs, x_quant_buf);
    float inv_scale = 1.0f / (scale_x * w_scale); /* :391 */
    orc_tmac_rows_f32(x_quant_buf, packed, rows, cols, inv_scale, out);
}

void orc_bitlinear_forward_batch(const float *x_batch,
                                 int n_tokens,
                                 int n,
                                 const uint8_t *packed,
                                 int rows,
                                 int cols,
                                 float w_scale,
                                 const float *norm_w,
                                 float *out_batch,
                                 float *x_norm_buf,
                                 int8_t *x_quant_batch,
                                 int quant_stride)
{
    for (int t = 0; t < n_tokens; t++)
        orc_bitlinear_forward(x_batch + (size_t) t * n, n, packed, rows, cols,
                              w_scale, norm_w, out_batch + (size_t) t * rows,
                              x_norm_buf,
                              x_quant_batch + (size_t) t * quant_stride);
}

void orc_ternary_gemm_i32(const int8_t *xq,
                          int M,
                          int ldx,
                          const uint8_t *packed,
                          int N,
                          int K,
                          int32_t *out)
{
    int stride = (K + 3) / 4;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < N; r++) {
        const uint8_t *row = packed + (size_t) r * stride;
        for (int m = 0; m < M; m++) {
            const int8_t *xm = xq + (size_t) m * ldx;
            int32_t t = 0;
            for (int k = 0; k < K; k++)
                t += orc_decode_weight((row[k >> 2] >> (2 * (k & 3))) & 3) *
                     xm[k];
            out[(size_t) m * N + r] = t;
        }
    }
}

/* ------------------------------------------------------------------ */
/* a15: SSM inner step (src/kernel.c:34-70, src/bitmamba.h:234-243)     */
/* ------------------------------------------------------------------ */
static inline float orc_silu(float x)
{
    return x / (1.0f + expf(-x));
}

static inline float orc_softplus(float x)
{
    if (x > 20.0f)
        return x;
    return logf(1.0f + expf(x));
}

void orc_ssm_inner(const float *proj,
                   int d_inner,
                   int n_heads,
                   const float *dt_bias,
                   const float *A_precomp,
                   const float *conv_w_t,
                   const float *conv_b,
                   float *cs0,
                   const float *cs1,
                   const float *cs2,
                   float *ssm_state,
                   const float *D,
                   float *y,
                   int idx_start,
                   int idx_end)
{
    int head_dim = d_inner / n_heads;
    const float *z = proj;
    const float *xin = proj + d_inner;
    const float *B = proj + 2 * d_inner;
    const float *C = B + n_heads;
    const float *dt = C + n_heads;
    const float *w0 = conv_w_t, *w1 = conv_w_t + d_inner;
    const float *w2 = conv_w_t + 2 * d_inner, *w3 = conv_w_t + 3 * d_inner;

    for (int idx = idx_start; idx < idx_end; idx++) {
        int h = idx / head_dim;
        float dt_val = orc_softplus(dt[h] + dt_bias[h]);
        float decay = expf(A_precomp[h] * dt_val);
        float Bdt = B[h] * dt_val;
        float C_val = C[h];

        float xv = xin[idx];
        float conv = conv_b[idx] + cs0[idx] * w0[idx];
        conv = conv + cs1[idx] * w1[idx];
        conv = conv + cs2[idx] * w2[idx];
        conv = conv + xv * w3[idx];
        cs0[idx] = xv; /* cs_write == cs0: the oldest tap is replaced */

        float xa = orc_silu(conv);
        float st = ssm_state[idx] * decay + xa * Bdt;
        ssm_state[idx] = st;
        y[idx] = (st * C_val + xa * D[idx]) * orc_silu(z[idx]);
    }
}

/* ------------------------------------------------------------------ */
/* BIT2 loader (src/model.c:367-932) and scalar model (src/block.c,     */
/* src/model.c:1045-1314)                                               */
/* ------------------------------------------------------------------ */
#define ORC_MAGIC 0x42495432
#define ORC_MAX_DIM (1 << 20)
#define ORC_MAX_VOCAB 256000

typedef struct {
    const float *data;
    const uint8_t *packed;
    int rows, cols;
    size_t n_elements;
    bool is_bitnet;
    float scale;
} orc_tensor_t;

typedef struct {
    orc_tensor_t in_norm, in_proj, conv_w, conv_b, dt_bias, A_log, D, out_norm,
        out_proj;
    float *conv_w_t;   /* [4][d_inner] */
    float *conv_state; /* [3][d_inner] */
    float *ssm_state;  /* [d_inner] */
    float *A_precomp;  /* [n_heads] */
    int conv_pos;
} orc_layer_t;

struct orc_model {
    int vocab, d_model, n_layers, n_heads, d_inner;
    orc_tensor_t embed, norm_f, lm_norm, lm_head;
    orc_layer_t *L;
    float *x, *next_x, *proj, *y, *feat, *logits, *xn;
    int8_t *xq;
};

static int rd_i32(const uint8_t *p)
{
    int v;
    memcpy(&v, p, 4);
    return v;
}

static float rd_f32(const uint8_t *p)
{
    float v;
    memcpy(&v, p, 4);
    return v;
}

/* read_tensor_mmap (src/model.c:367-475); returns bytes consumed or 0 */
static size_t rd_tensor(const uint8_t *p, const uint8_t *end, orc_tensor_t *t)
{
    memset(t, 0, sizeof(*t));
    t->scale = 1.0f;
    const uint8_t *s = p;
    if (end - p < 4)
        return 0;
    int type = rd_i32(p);
    p += 4;
    if (type == 2) {
        if (end - p < 12)
            return 0;
        t->is_bitnet = true;
        t->rows = rd_i32(p);
        t->cols = rd_i32(p + 4);
        t->scale = rd_f32(p + 8);
        p += 12;
        if (!isfinite(t->scale) || t->scale <= 0.0f)
            return 0;
        if (t->rows <= 0 || t->rows > ORC_MAX_DIM || t->cols <= 0 ||
            t->cols > ORC_MAX_DIM)
            return 0;
        size_t bytes = (size_t) t->rows * (size_t) ((t->cols + 3) / 4);
        if (bytes > (size_t) (end - p))
            return 0;
        t->packed = p;
        t->n_elements = (size_t) t->rows * t->cols;
        p += bytes;
    } else {
        if (end - p < 4)
            return 0;
        int ndim = rd_i32(p);
        p += 4;
        if (ndim < 0 || ndim > 4)
            return 0;
        if ((size_t) (end - p) < (size_t) ndim * 4)
            return 0;
        size_t total = 1;
        for (int i = 0; i < ndim; i++) {
            int d = rd_i32(p);
            p += 4;
            if (d <= 0 || d > ORC_MAX_DIM)
                return 0;
            total *= (size_t) d;
            if (i == 0)
                t->rows = d;
            if (i == 1)
                t->cols = d;
        }
        if (total * 4 > (size_t) (end - p))
            return 0;
        t->data = (const float *) p;
        t->n_elements = total;
        p += total * 4;
    }
    return (size_t) (p - s);
}

void orc_model_free(orc_model_t *m)
{
    if (!m)
        return;
    if (m->L) {
        for (int i = 0; i < m->n_layers; i++) {
            free(m->L[i].conv_w_t);
            free(m->L[i].conv_state);
            free(m->L[i].ssm_state);
            free(m->L[i].A_precomp);
        }
        free(m->L);
    }
    free(m->x);
    free(m->next_x);
    free(m->proj);
    free(m->y);
    free(m->feat);
    free(m->logits);
    free(m->xn);
    free(m->xq);
    free(m);
}

orc_model_t *orc_model_load(const void *blob, size_t len)
{
    const uint8_t *p = (const uint8_t *) blob, *end = p + len;
    if (len < 20 || rd_i32(p) != ORC_MAGIC)
        return NULL;
    orc_model_t *m = calloc(1, sizeof(*m));
    m->vocab = rd_i32(p + 4);
    m->d_model = rd_i32(p + 8);
    m->n_layers = rd_i32(p + 12);
    m->n_heads = rd_i32(p + 16);
    p += 20;
    if (m->vocab <= 0 || m->vocab > ORC_MAX_VOCAB || m->d_model <= 0 ||
        m->d_model > ORC_MAX_DIM || m->n_layers <= 0 || m->n_layers > 256 ||
        m->n_heads <= 0 || m->n_heads > ORC_MAX_DIM) {
        free(m);
        return NULL;
    }
    int dm = m->d_model, di = 2 * dm, nh = m->n_heads;
    m->d_inner = di;

    size_t c = rd_tensor(p, end, &m->embed);
    if (!c) {
        free(m);
        return NULL;
    }
    p += c;
    m->L = calloc((size_t) m->n_layers, sizeof(orc_layer_t));
#define RD(t)                          \
    do {                               \
        c = rd_tensor(p, end, (t));    \
        if (!c)                        \
            goto fail;                 \
        p += c;                        \
    } while (0)
    for (int i = 0; i < m->n_layers; i++) {
        orc_layer_t *b = &m->L[i];
        RD(&b->in_norm);
        RD(&b->in_proj);
        RD(&b->conv_w);
        RD(&b->conv_b);
        RD(&b->dt_bias);
        RD(&b->A_log);
        RD(&b->D);
        RD(&b->out_norm);
        RD(&b->out_proj);
    }
    RD(&m->norm_f);
    RD(&m->lm_norm);
    RD(&m->lm_head);
#undef RD

    /* shape/type validation (src/model.c:630-784) */
    if (m->norm_f.n_elements < (size_t) dm ||
        m->lm_norm.n_elements < (size_t) dm)
        goto fail;
    if (m->embed.n_elements < (size_t) m->vocab * dm)
        goto fail;
    if (m->lm_head.rows != m->vocab || m->lm_head.cols != dm)
        goto fail;
    if (di % nh != 0)
        goto fail;
    for (int i = 0; i < m->n_layers; i++) {
        orc_layer_t *b = &m->L[i];
        if (b->in_norm.n_elements < (size_t) dm)
            goto fail;
        if (b->in_proj.cols != dm || b->in_proj.rows != 2 * di + 3 * nh)
            goto fail;
        if (b->out_proj.rows != dm || b->out_proj.cols != di)
            goto fail;
        if (b->conv_w.n_elements < (size_t) di * 4 ||
            b->conv_b.n_elements < (size_t) di ||
            b->dt_bias.n_elements < (size_t) nh ||
            b->A_log.n_elements < (size_t) nh ||
            b->D.n_elements < (size_t) di ||
            b->out_norm.n_elements < (size_t) di)
            goto fail;
        if (!b->in_proj.is_bitnet || !b->out_proj.is_bitnet)
            goto fail;
        if (b->in_norm.is_bitnet || b->out_norm.is_bitnet ||
            b->conv_w.is_bitnet || b->conv_b.is_bitnet ||
            b->dt_bias.is_bitnet || b->A_log.is_bitnet || b->D.is_bitnet)
            goto fail;
    }
    if (m->embed.is_bitnet || m->norm_f.is_bitnet || m->lm_norm.is_bitnet ||
        !m->lm_head.is_bitnet)
        goto fail;

    /* precompute A = -exp(A_log) and the [tap][channel] conv transpose
     * (src/model.c:786-805); zeroed recurrent state (src/block.c:11-26) */
    for (int i = 0; i < m->n_layers; i++) {
        orc_layer_t *b = &m->L[i];
        b->A_precomp = malloc((size_t) nh * sizeof(float));
        for (int h = 0; h < nh; h++)
            b->A_precomp[h] = -expf(b->A_log.data[h]);
        b->conv_w_t = malloc((size_t) 4 * di * sizeof(float));
        for (int tap = 0; tap < 4; tap++)
            for (int ch = 0; ch < di; ch++)
                b->conv_w_t[tap * di + ch] = b->conv_w.data[ch * 4 + tap];
        b->conv_state = calloc((size_t) 3 * di, sizeof(float));
        b->ssm_state = calloc((size_t) di, sizeof(float));
        b->conv_pos = 0;
    }
    int max_proj = 2 * di + 3 * nh;
    m->x = calloc((size_t) dm, sizeof(float));
    m->next_x = calloc((size_t) dm, sizeof(float));
    m->proj = calloc((size_t) max_proj, sizeof(float));
    m->y = calloc((size_t) di, sizeof(float));
    m->feat = calloc((size_t) dm, sizeof(float));
    m->logits = calloc((size_t) m->vocab, sizeof(float));
    m->xn = calloc((size_t) di, sizeof(float));
    m->xq = calloc((size_t) di + 32, 1);
    return m;
fail:
    orc_model_free(m);
    return NULL;
}

/* ssm_scan_token (src/block.c:83-108): ring taps, then advance conv_pos */
static void scan_token(orc_model_t *m, orc_layer_t *b, const float *proj,
                       float *y)
{
    int di = m->d_inner;
    int pos = b->conv_pos;
    int t1 = (pos + 1 < 3) ? pos + 1 : pos + 1 - 3;
    int t2 = (pos + 2 < 3) ? pos + 2 : pos + 2 - 3;
    float *cs0 = b->conv_state + (size_t) pos * di;
    orc_ssm_inner(proj, di, m->n_heads, b->dt_bias.data, b->A_precomp,
                  b->conv_w_t, b->conv_b.data, cs0,
                  b->conv_state + (size_t) t1 * di,
                  b->conv_state + (size_t) t2 * di, b->ssm_state, b->D.data, y,
                  0, di);
    b->conv_pos = (pos + 1 < 3) ? pos + 1 : 0;
}

static void bl(orc_model_t *m, const float *x, int n, const orc_tensor_t *w,
               const orc_tensor_t *norm, float *out)
{
    orc_bitlinear_forward(x, n, w->packed, w->rows, w->cols, w->scale,
                          norm->data, out, m->xn, m->xq);
}

void orc_model_prefill(orc_model_t *m, const int32_t *tokens, int n_tokens)
{
    if (n_tokens <= 0)
        return;
    int dm = m->d_model, di = m->d_inner;
    int proj_dim = 2 * di + 3 * m->n_heads;
    float *xb = malloc((size_t) n_tokens * dm * sizeof(float));
    float *ob = malloc((size_t) n_tokens * dm * sizeof(float));
    float *pb = malloc((size_t) n_tokens * proj_dim * sizeof(float));
    float *yb = malloc((size_t) n_tokens * di * sizeof(float));
    for (int t = 0; t < n_tokens; t++) {
        int tok = tokens[t];
        if (tok < 0 || tok >= m->vocab)
            tok = 0;
        memcpy(xb + (size_t) t * dm, m->embed.data + (size_t) tok * dm,
               (size_t) dm * sizeof(float));
    }
    for (int i = 0; i < m->n_layers; i++) {
        orc_layer_t *b = &m->L[i];
        /* block_step_batch (src/block.c:378-447), scalar branch */
        for (int t = 0; t < n_tokens; t++)
            bl(m, xb + (size_t) t * dm, dm, &b->in_proj, &b->in_norm,
               pb + (size_t) t * proj_dim);
        for (int t = 0; t < n_tokens; t++)
            scan_token(m, b, pb + (size_t) t * proj_dim, yb + (size_t) t * di);
        for (int t = 0; t < n_tokens; t++)
            bl(m, yb + (size_t) t * di, di, &b->out_proj, &b->out_norm,
               ob + (size_t) t * dm);
        for (size_t j = 0; j < (size_t) n_tokens * dm; j++)
            xb[j] = xb[j] + ob[j];
    }
    free(xb);
    free(ob);
    free(pb);
    free(yb);
}

int orc_model_step(orc_model_t *m,
                   int token,
                   const int *history,
                   int history_len,
                   float penalty)
{
    int dm = m->d_model, di = m->d_inner;
    if (token < 0 || token >= m->vocab)
        return 0;
    memcpy(m->x, m->embed.data + (size_t) token * dm,
           (size_t) dm * sizeof(float));
    for (int i = 0; i < m->n_layers; i++) {
        orc_layer_t *b = &m->L[i];
        /* block_step, unfused branch (src/block.c:361-371) */
        bl(m, m->x, dm, &b->in_proj, &b->in_norm, m->proj);
        scan_token(m, b, m->proj, m->y);
        bl(m, m->y, di, &b->out_proj, &b->out_norm, m->next_x);
        for (int j = 0; j < dm; j++)
            m->x[j] = m->x[j] + m->next_x[j];
    }
    orc_rms_norm(m->x, dm, m->norm_f.data, m->feat);
    bl(m, m->feat, dm, &m->lm_head, &m->lm_norm, m->logits);

    /* repetition penalty once per distinct token, protected ids exempt
     * (src/model.c:1272-1305) */
    static const int prot[4] = {50256, 198, 628, 13};
    unsigned char *seen = calloc((size_t) m->vocab, 1);
    for (int i = 0; i < history_len; i++) {
        int past = history[i];
        if (past < 0 || past >= m->vocab || seen[past])
            continue;
        seen[past] = 1;
        bool is_prot = false;
        for (int p = 0; p < 4; p++)
            if (prot[p] == past)
                is_prot = true;
        if (!is_prot && penalty > 0.0f) {
            if (m->logits[past] > 0)
                m->logits[past] = m->logits[past] / penalty;
            else
                m->logits[past] = m->logits[past] * penalty;
        }
    }
    free(seen);

    /* greedy: first maximum wins (src/model.c:143-154) */
    int best = 0;
    float max_l = -1e9f;
    for (int i = 0; i < m->vocab; i++)
        if (m->logits[i] > max_l) {
            max_l = m->logits[i];
            best = i;
        }
    return best;
}

const float *orc_model_logits(const orc_model_t *m)
{
    return m->logits;
}

int orc_model_config(const orc_model_t *m, int which)
{
    switch (which) {
    case 0:
        return m->vocab;
    case 1:
        return m->d_model;
    case 2:
        return m->n_layers;
    case 3:
        return m->n_heads;
    default:
        return m->d_inner;
    }
}

int orc_model_layer_state(const orc_model_t *m,
                          int layer,
                          float *conv_state,
                          float *ssm_state)
{
    const orc_layer_t *b = &m->L[layer];
    memcpy(conv_state, b->conv_state, (size_t) 3 * m->d_inner * sizeof(float));
    memcpy(ssm_state, b->ssm_state, (size_t) m->d_inner * sizeof(float));
    return b->conv_pos;
}

/* glibc expf / logf over an array (the functions scalar_ssm_inner calls) */
void orc_expf_array(const float *in, float *out, size_t n)
{
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++)
        out[i] = expf(in[i]);
}

void orc_logf_array(const float *in, float *out, size_t n)
{
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++)
        out[i] = logf(in[i]);
}
