/*
 * Harness around the reference's own C sources (compiled where they lie by
 * oracle/Makefile into oracle/_ref/libbmref.so).  Test infrastructure only:
 * it is used to pin the oracle restatement and as the timed CPU baseline.
 *
 * It exposes flat entry points (plain pointers and sizes) over the
 * reference's kernel dispatch table and model API:
 *   - dispatch selection: dispatch_init() (src/dispatch.c:15-52), optionally
 *     overwritten with the scalar kernels and a NULL bitlinear_prepare so that
 *     block_step takes its unfused path (src/block.c:280, 361-371);
 *   - bitlinear / rms_norm / ssm_inner through g_kernels
 *     (src/dispatch.h:86-97);
 *   - model_load / model_prefill / model_forward_step / model_free
 *     (src/bitmamba.h:282-294) for end-to-end greedy streams.
 */
#include <stdlib.h>
#include <string.h>

#include "bitmamba.h"
#include "dispatch.h"
#include "threadpool.h"

static int32_t *g_lut_buf;

/* kind: 0 = scalar (the oracle semantics), 1 = whatever dispatch_init picks
 * on this CPU (AVX2+FMA on x86-64). */
const char *bmref_init(int threads, int kind)
{
    /* the wait policy is set before any worker exists: a worker reads it in
     * its idle loop (src/threadpool.c:183-206), and one that has not run yet
     * must not start under a policy other than the one the pool dispatches
     * with */
    bm_set_poll(0);
    bm_set_threads(threads);
    dispatch_init();
    init_lut();
    if (kind == 0) {
        g_kernels.rms_norm = scalar_rms_norm;
        g_kernels.bitlinear_forward = scalar_bitlinear_forward;
        g_kernels.bitlinear_forward_batch = scalar_bitlinear_forward_batch;
        g_kernels.bitlinear_prepare = NULL;
        g_kernels.bitlinear_row_worker = NULL;
        g_kernels.ssm_inner = scalar_ssm_inner;
        g_kernels.name = "scalar";
    }
    if (!g_lut_buf)
        g_lut_buf = xmalloc_aligned(256 * 16 * sizeof(int32_t), 64);
    scalar_set_lut_buf(g_lut_buf);
    return g_kernels.name;
}

/* pool wait policy: 0 = condvar, 100 = pure spin (the reference default).
 * The pool is stopped and started again under the new policy: a worker asleep
 * on its condvar (poll < 100) is never signalled once the policy is 100,
 * since a pure-spin dispatch skips the condvars (src/threadpool.c:195-206,
 * 484-490), so changing the policy under a live pool loses every worker that
 * slept -- including a worker that had not yet run when the pool was made. */
void bmref_set_poll(int intensity)
{
    int n = bm_get_threads();
    bm_thread_pool_free();
    bm_set_poll(intensity);
    if (n > 1)
        bm_set_threads(n);
}

void bmref_shutdown(void)
{
    bm_thread_pool_free();
}

int bmref_threads(void)
{
    return bm_get_threads();
}

static void make_weight(tensor_t *w,
                        const uint8_t *packed,
                        int rows,
                        int cols,
                        float scale)
{
    memset(w, 0, sizeof(*w));
    w->packed_data = packed;
    w->rows = rows;
    w->cols = cols;
    w->n_elements = (size_t) rows * cols;
    w->is_bitnet = true;
    w->scale = scale;
}

static void make_vec(tensor_t *t, const float *data, int n)
{
    memset(t, 0, sizeof(*t));
    t->data = data;
    t->rows = n;
    t->n_elements = (size_t) n;
    t->scale = 1.0f;
}

float bmref_rms_norm(const float *x, int n, const float *w, float *out)
{
    return g_kernels.rms_norm(x, n, w, out);
}

void bmref_bitlinear_forward(const float *x,
                             int n,
                             const uint8_t *packed,
                             int rows,
                             int cols,
                             float scale,
                             const float *norm_w,
                             float *out,
                             float *x_norm_buf,
                             int8_t *x_quant_buf)
{
    tensor_t w, nw;
    make_weight(&w, packed, rows, cols, scale);
    make_vec(&nw, norm_w, n);
    g_kernels.bitlinear_forward(x, n, &w, &nw, out, x_norm_buf, x_quant_buf);
}

void bmref_bitlinear_forward_batch(const float *x,
                                   int n_tokens,
                                   int n,
                                   const uint8_t *packed,
                                   int rows,
                                   int cols,
                                   float scale,
                                   const float *norm_w,
                                   float *out,
                                   float *x_norm_buf,
                                   int8_t *x_quant,
                                   int quant_stride)
{
    tensor_t w, nw;
    make_weight(&w, packed, rows, cols, scale);
    make_vec(&nw, norm_w, n);
    g_kernels.bitlinear_forward_batch(x, n_tokens, n, &w, &nw, out, x_norm_buf,
                                      x_quant, quant_stride);
}

/* Row kernel alone on a given int8 vector (no quantization): the AVX2
 * decomposed worker when available, used for the int8-input stress shape. */
int bmref_row_worker_available(void)
{
    return g_kernels.bitlinear_row_worker != NULL;
}

void bmref_rows_int8(const int8_t *x_quant,
                     const uint8_t *packed,
                     int rows,
                     int cols,
                     float inv_scale,
                     float *out)
{
    bitlinear_row_work_t work = {
        .x_quant = x_quant,
        .packed_data = packed,
        .out = out,
        .inv_scale = inv_scale,
        .rows = rows,
        .cols = cols,
        .packed_stride = (cols + 3) / 4,
        .chunk_ctr = NULL,
        .chunk_size = 0,
    };
    bm_parallel_for(rows, g_kernels.bitlinear_row_worker, &work);
}

void bmref_ssm_inner(const ssm_inner_args_t *a, int idx_start, int idx_end)
{
    g_kernels.ssm_inner(a, idx_start, idx_end);
}

void bmref_rng_seed(uint64_t s)
{
    rng_seed(s);
}

uint64_t bmref_rng_next(void)
{
    return rng_next();
}

void bmref_lut(int8_t *unpack /* [256*4] */,
               uint8_t *pmask /* [256] */,
               uint8_t *nmask /* [256] */)
{
    init_lut();
    memcpy(unpack, UNPACK_LUT, sizeof(UNPACK_LUT));
    memcpy(pmask, TMAC_P_MASK, sizeof(TMAC_P_MASK));
    memcpy(nmask, TMAC_N_MASK, sizeof(TMAC_N_MASK));
}

/* ---- model API ---- */

void *bmref_model_load(const char *path)
{
    bitmamba_model_t *m = calloc(1, sizeof(*m));
    if (!m)
        return NULL;
    m->use_gpu = false;
    if (!model_load(m, path)) {
        free(m);
        return NULL;
    }
    return m;
}

void bmref_model_free(void *h)
{
    if (!h)
        return;
    model_free((bitmamba_model_t *) h);
    free(h);
}

void bmref_model_prefill(void *h, const int32_t *tokens, int n)
{
    model_prefill((bitmamba_model_t *) h, tokens, n);
}

int bmref_model_step(void *h,
                     int token,
                     const int *history,
                     int history_len,
                     float penalty)
{
    return model_forward_step((bitmamba_model_t *) h, token, history,
                              history_len, penalty, 0.0f, 0.0f, 1.0f, 0);
}

/* model_forward_step with the reference's sampler (temp >= 0.05 samples
 * with the global generator seeded by bmref_rng_seed). */
int bmref_model_step_sample(void *h,
                            int token,
                            const int *history,
                            int history_len,
                            float penalty,
                            float temp,
                            float min_p,
                            float top_p,
                            int top_k)
{
    return model_forward_step((bitmamba_model_t *) h, token, history,
                              history_len, penalty, temp, min_p, top_p, top_k);
}

const float *bmref_model_logits(void *h)
{
    return ((bitmamba_model_t *) h)->logits;
}

int bmref_model_vocab(void *h)
{
    return ((bitmamba_model_t *) h)->config.vocab_size;
}

/* Copy of one layer's recurrent state: conv_state [(d_conv-1)*d_inner],
 * ssm_state [d_inner], conv_pos. */
int bmref_model_layer_state(void *h,
                            int layer,
                            float *conv_state,
                            float *ssm_state)
{
    bitmamba_model_t *m = (bitmamba_model_t *) h;
    bitmamba_block_t *b = &m->layers[layer];
    memcpy(conv_state, b->conv_state,
           (size_t) (b->d_conv - 1) * b->d_inner * sizeof(float));
    memcpy(ssm_state, b->ssm_state, (size_t) b->d_inner * sizeof(float));
    return b->conv_pos;
}

/* the inverse of bmref_model_layer_state */
void bmref_model_set_layer_state(void *h,
                                 int layer,
                                 const float *conv_state,
                                 const float *ssm_state,
                                 int conv_pos)
{
    bitmamba_model_t *m = (bitmamba_model_t *) h;
    bitmamba_block_t *b = &m->layers[layer];
    memcpy(b->conv_state, conv_state,
           (size_t) (b->d_conv - 1) * b->d_inner * sizeof(float));
    memcpy(b->ssm_state, ssm_state, (size_t) b->d_inner * sizeof(float));
    b->conv_pos = conv_pos;
}

/* ---------------------------------------------------------------------------
 * The HIP backend wired into this build's own plugin table, as a reference
 * tree built with HAS_HIP would do it (the table's types must agree): the
 * caller passes bm_hip_register from libbitmamba_hip.so, which then owns
 * rms_norm / bitlinear_forward / bitlinear_forward_batch and leaves
 * bitlinear_prepare and bitlinear_row_worker NULL (src/dispatch.c:15-52,
 * src/block.c:361-371, src/model.c:1258-1262).  bmref_init() restores the
 * CPU table.
 * ------------------------------------------------------------------------- */
#define BM_HIP_HAVE_TENSOR_T
#include "bm_hip.h"

_Static_assert(sizeof(kernel_dispatch_t) == sizeof(bm_hip_dispatch_t),
               "kernel_dispatch_t and bm_hip_dispatch_t must have one layout");

int bmref_use_hip(bool (*reg)(bm_hip_dispatch_t *))
{
    return reg((bm_hip_dispatch_t *) &g_kernels) ? 1 : 0;
}

const char *bmref_kernels_name(void)
{
    return g_kernels.name;
}

/* the mmap'd model file of a loaded model (what bm_hip_set_mmap registers
 * at the Metal spot of model_load, src/model.c:840-851) */
int bmref_model_image(void *h, void **addr, size_t *size)
{
    const bitmamba_model_t *m = (const bitmamba_model_t *) h;
    *addr = m->mmap_addr;
    *size = m->mmap_size;
    return m->mmap_addr != NULL;
}

/* ---------------------------------------------------------------------------
 * model_prefill through the HIP backend's batch context, in the order
 * model_prefill_metal drives Metal's (src/model.c:934-1041), as a tree built
 * with HAS_HIP would call it: the embeddings go into the X buffer; the first
 * submit runs layer 0's in_proj; then, per layer, the CPU scans every
 * token's SSM step (block_ssm_scan, src/block.c:486-489) and one submit runs
 * the layer's out_proj, the residual add and the next layer's in_proj.  The
 * library's entry points come in a table, so that this build does not link
 * the library.  0, or -1 when the context could not be made or a step was
 * refused (where the reference would fall back to its CPU prefill).
 * ------------------------------------------------------------------------- */
typedef struct {
    bm_hip_batch_ctx_t *(*begin)(int, int, int, int, int);
    float *(*ptr)(bm_hip_batch_ctx_t *, int);
    bool (*encode_bitlinear)(bm_hip_batch_ctx_t *, int, int, const uint8_t *,
                             int, int, float, const float *, int);
    void (*encode_residual)(bm_hip_batch_ctx_t *, int);
    void (*submit_and_wait)(bm_hip_batch_ctx_t *);
    void (*end)(bm_hip_batch_ctx_t *);
} bmref_batch_api_t;

static bool batch_proj(const bmref_batch_api_t *api,
                       bm_hip_batch_ctx_t *ctx,
                       int src,
                       int dim,
                       const tensor_t *w,
                       const tensor_t *norm,
                       int dst)
{
    return api->encode_bitlinear(ctx, src, dim, w->packed_data, w->rows,
                                 w->cols, w->scale, norm->data, dst);
}

int bmref_model_prefill_batch(void *h,
                              const int32_t *tokens,
                              int n,
                              const bmref_batch_api_t *api)
{
    bitmamba_model_t *m = (bitmamba_model_t *) h;
    const int d_model = m->config.d_model;
    const int d_inner = d_model * BM_EXPAND_FACTOR;
    const int n_layers = m->config.n_layers;
    int max_proj = 0;
    for (int i = 0; i < n_layers; i++)
        if (m->layers[i].in_proj.rows > max_proj)
            max_proj = m->layers[i].in_proj.rows;
    bm_hip_batch_ctx_t *ctx =
        api->begin(n, d_model, max_proj, d_inner, d_inner + 32);
    if (!ctx)
        return -1;
    float *x = api->ptr(ctx, BM_HIP_BUF_X);
    float *proj = api->ptr(ctx, BM_HIP_BUF_PROJ);
    float *y = api->ptr(ctx, BM_HIP_BUF_Y);
    for (int t = 0; t < n; t++) {
        int tok = tokens[t];
        if (tok < 0 || tok >= m->config.vocab_size)
            tok = 0;
        memcpy(x + (size_t) t * d_model, m->embed.data + (size_t) tok * d_model,
               (size_t) d_model * sizeof(float));
    }
    int rc = -1;
    bitmamba_block_t *b0 = &m->layers[0];
    if (!batch_proj(api, ctx, BM_HIP_BUF_X, d_model, &b0->in_proj,
                    &b0->in_proj_norm, BM_HIP_BUF_PROJ))
        goto done;
    api->submit_and_wait(ctx);
    for (int i = 0; i < n_layers; i++) {
        bitmamba_block_t *b = &m->layers[i];
        for (int t = 0; t < n; t++)
            block_ssm_scan(b, proj + (size_t) t * b->in_proj.rows,
                           y + (size_t) t * d_inner);
        if (!batch_proj(api, ctx, BM_HIP_BUF_Y, d_inner, &b->out_proj,
                        &b->out_proj_norm, BM_HIP_BUF_OUT))
            goto done;
        api->encode_residual(ctx, n * d_model);
        if (i + 1 < n_layers) {
            bitmamba_block_t *nb = &m->layers[i + 1];
            if (!batch_proj(api, ctx, BM_HIP_BUF_X, d_model, &nb->in_proj,
                            &nb->in_proj_norm, BM_HIP_BUF_PROJ))
                goto done;
        }
        api->submit_and_wait(ctx);
    }
    rc = 0;
done:
    api->end(ctx);
    return rc;
}
