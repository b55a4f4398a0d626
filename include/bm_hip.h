/*
 * bm_hip.h -- C ABI of the MI355X (gfx950) BitLinear backend.
 *
 * Drop-in for the ternary BitLinear hot path of jserv/bitmamba.c.  The
 * backend takes the slot the Metal backend fills in the reference
 * (src/metal/bm_metal.h:14-99) and registers its kernels in the reference's
 * plugin table kernel_dispatch_t g_kernels (src/dispatch.h:86-100).
 *
 * Every entry point takes plain pointers and sizes.  Functions whose names
 * start with hip_ have exactly the function-pointer types of the dispatch
 * table and take HOST pointers (synchronous, like the CPU kernels they
 * replace).  Functions ending in _dev take DEVICE pointers and a HIP stream
 * (void *, NULL = the library's stream) and are asynchronous.
 *
 * Errors: contract violations (dimension mismatch, non-BitNet weights) exit
 * the process like BITLINEAR_CHECK (src/bitmamba.h:219-231); a HIP runtime
 * failure inside a hip_ kernel entry point also prints and exits -- outputs
 * are never silently zeroed (contrast src/metal/bm_metal.c:549-553).
 * Lifecycle and _dev functions return false / a negative code instead, with
 * the reason in bm_hip_last_error().
 */
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's tensor view (src/bitmamba.h:65-74).  The layout below is
 * the one the reference compiles; define BM_HIP_HAVE_TENSOR_T when the
 * reference's own bitmamba.h is already included. */
#ifndef BM_HIP_HAVE_TENSOR_T
struct tensor {
    const float *data;          /* float32 weights */
    const uint8_t *packed_data; /* packed 2-bit weights, [rows][ceil(cols/4)] */
    int rows;
    int cols;
    size_t n_elements;
    bool is_bitnet;
    float scale;
};
#endif

/* ------------------------------------------------------------------ */
/* Lifecycle -- mirrors src/metal/bm_metal.h:14-24, 44-45               */
/* ------------------------------------------------------------------ */

/* bm_metal_init (src/metal/bm_metal.h:15): selects device 0, creates the
 * library stream.  false if no gfx950 device is usable. */
bool bm_hip_init(void);
/* bm_metal_available (src/metal/bm_metal.h:18) */
bool bm_hip_available(void);
/* bm_metal_set_mmap (src/metal/bm_metal.h:24): registers a model image.
 * When the image parses as BIT2 (src/model.c:477-932 layout) every packed
 * tensor is copied once into its own 256-byte-aligned device buffer with
 * the 2-bit code 11 rewritten to 10 (same value, src/quantization.c:27-31),
 * and every float tensor is copied too; hip_* calls then find them by host
 * pointer.  Tensors outside a registered image are uploaded on every call
 * (their host memory may be reused for other data).  Registered host memory
 * must not change afterwards. */
bool bm_hip_set_mmap(const void *base, size_t size);
/* bm_metal_cleanup (src/metal/bm_metal.h:45) */
void bm_hip_cleanup(void);
/* Reason for the last false / negative return. */
const char *bm_hip_last_error(void);

/* ------------------------------------------------------------------ */
/* Dispatch-table kernels (host pointers, synchronous)                  */
/* ------------------------------------------------------------------ */

/* rms_norm_fn_t (src/dispatch.h:20-23); semantics of scalar_rms_norm
 * (src/kernel.c:72-129), bit-exact. */
float hip_rms_norm(const float *x, int size, const float *weight, float *out);

/* bitlinear_forward_fn_t (src/dispatch.h:25-31); semantics of
 * scalar_bitlinear_forward (src/kernel.c:346-448), bit-exact fp32 output.
 * x_norm_buf[n] and x_quant_buf[n] receive what the scalar kernel leaves
 * there. */
void hip_bitlinear_forward(const float *x,
                           int n,
                           const struct tensor *w,
                           const struct tensor *norm_w,
                           float *out,
                           float *x_norm_buf,
                           int8_t *x_quant_buf);

/* bitlinear_forward_batch_fn_t (src/dispatch.h:33-42); semantics of
 * scalar_bitlinear_forward_batch (src/kernel.c:322-338).  x_norm_buf holds
 * the last token's normalized input afterwards, as in the reference. */
void hip_bitlinear_forward_batch(const float *x_batch,
                                 int n_tokens,
                                 int n,
                                 const struct tensor *w,
                                 const struct tensor *norm_w,
                                 float *out_batch,
                                 float *x_norm_buf,
                                 int8_t *x_quant_batch,
                                 int quant_stride);

/* Layout mirror of kernel_dispatch_t (src/dispatch.h:87-95). */
typedef struct {
    void *rms_norm;
    void *bitlinear_forward;
    void *bitlinear_forward_batch;
    void *bitlinear_prepare;
    void *bitlinear_row_worker;
    void *ssm_inner;
    const char *name;
} bm_hip_dispatch_t;

/* The GPU branch of dispatch_init (src/dispatch.c:15-52): sets rms_norm,
 * bitlinear_forward and bitlinear_forward_batch to the hip_ entries,
 * bitlinear_prepare and bitlinear_row_worker to NULL (so block_step takes
 * its unfused path, src/block.c:280, 361-371, and the LM head calls
 * bitlinear_forward, src/model.c:1258-1262), keeps ssm_inner, and sets
 * name = "hip".  Returns false (table untouched) if the backend is not
 * available. */
bool bm_hip_register(bm_hip_dispatch_t *table);

/* bm_metal_bitlinear_forward_batch (src/metal/bm_metal.h:31-42): the same
 * computation as hip_bitlinear_forward_batch from raw tensor fields. */
void bm_hip_bitlinear_forward_batch(const float *x_batch,
                                    int n_tokens,
                                    int n,
                                    const uint8_t *packed_data,
                                    int rows,
                                    int cols,
                                    float w_scale,
                                    const float *norm_weight,
                                    float *out_batch,
                                    float *x_norm_buf,
                                    int8_t *x_quant_batch,
                                    int quant_stride);

/* ------------------------------------------------------------------ */
/* Batch context: the Metal backend's prefill batching                  */
/* (src/metal/bm_metal.h:57-99), driven as model_prefill_metal drives   */
/* it (src/model.c:934-1041).                                           */
/* ------------------------------------------------------------------ */

/* Buffer ids (BM_BUF_X .. BM_BUF_OUT, src/metal/bm_metal.h:58-63) */
enum {
    BM_HIP_BUF_X = 0,    /* n_tokens * d_model floats */
    BM_HIP_BUF_PROJ = 1, /* n_tokens * max_proj floats */
    BM_HIP_BUF_Y = 2,    /* n_tokens * d_inner floats */
    BM_HIP_BUF_OUT = 3,  /* n_tokens * d_model floats */
};
typedef struct bm_hip_batch_ctx bm_hip_batch_ctx_t;

/* bm_metal_batch_begin: the four buffers, zeroed.  NULL before bm_hip_init
 * or on a failed allocation (the caller falls back to the CPU). */
bm_hip_batch_ctx_t *bm_hip_batch_begin(int n_tokens,
                                       int d_model,
                                       int max_proj,
                                       int d_inner,
                                       int quant_stride);
/* bm_metal_batch_ptr: host pointer to a buffer (NULL for another id).  The
 * buffers live on the device with a pinned host copy: what the caller
 * writes there before bm_hip_submit_and_wait reaches the steps of that
 * submit, and what the steps write is there when it returns. */
float *bm_hip_batch_ptr(bm_hip_batch_ctx_t *ctx, int buf_id);
/* bm_metal_encode_bitlinear: queue RMSNorm + int8 + the blocked product of
 * the n_tokens rows of src (X or Y, row stride input_dim) into dst (PROJ or
 * OUT, row stride rows), bit-exact with scalar_bitlinear_forward_batch
 * (src/kernel.c:322-338).  Runs nothing.  False, as in Metal, for a bad id,
 * cols % 16 != 0, no image registered by bm_hip_set_mmap, packed_data or
 * norm_weight outside it; also when input_dim != cols or the rows do not
 * fit the buffers. */
bool bm_hip_encode_bitlinear(bm_hip_batch_ctx_t *ctx,
                             int src_id,
                             int input_dim,
                             const uint8_t *packed_data,
                             int rows,
                             int cols,
                             float w_scale,
                             const float *norm_weight,
                             int dst_id);
/* bm_metal_encode_residual: queue X[i] += OUT[i] for i < count. */
void bm_hip_encode_residual(bm_hip_batch_ctx_t *ctx, int count);
/* bm_metal_submit_and_wait: run the queued steps in order and wait; a
 * failure is reported on stderr ("[HIP] Batch submit error") and in
 * bm_hip_last_error(). */
void bm_hip_submit_and_wait(bm_hip_batch_ctx_t *ctx);
/* bm_metal_batch_end */
void bm_hip_batch_end(bm_hip_batch_ctx_t *ctx);

/* ------------------------------------------------------------------ */
/* Device memory helpers (for callers without a HIP runtime of their    */
/* own; no counterpart in the reference)                                */
/* ------------------------------------------------------------------ */
void *bm_hip_malloc(size_t bytes);
void bm_hip_free(void *dev);
int bm_hip_memcpy_h2d(void *dev, const void *host, size_t bytes);
int bm_hip_memcpy_d2h(void *host, const void *dev, size_t bytes);
int bm_hip_memset(void *dev, int value, size_t bytes);
int bm_hip_synchronize(void);
/* Rewrites 2-bit code 11 to 10 in place (device buffer of `bytes`). */
int bm_hip_canonicalize_dev(uint8_t *packed, size_t bytes, void *stream);

/* Timing and calibration (no reference counterpart; the reference times
 * with CLOCK_MONOTONIC, src/utils.c:90-95): HIP events on a stream (NULL =
 * the library's stream), and a plain 16-byte copy kernel whose HBM counters
 * calibrate traffic measurements. */
void *bm_hip_stream(void);
void *bm_hip_event_create(void);
void bm_hip_event_destroy(void *ev);
int bm_hip_event_record(void *ev, void *stream);
float bm_hip_event_elapsed_ms(void *start, void *stop);
int bm_hip_copy_dev(void *dst, const void *src, size_t bytes, void *stream);
/* int8 MFMA ceiling: `blocks` blocks of 256 threads, each wave `iters` x 16
 * v_mfma_i32_32x32x32_i8 (65536 ops each); ternary != 0 uses hashed int8
 * activations against codes 0..2 like the prefill GEMM.  `sink` (one int,
 * device) is written only on an impossible value. */
int bm_hip_mfma_peak_dev(int blocks, int iters, int ternary, int *sink, void *stream);

/* ------------------------------------------------------------------ */
/* Device-pointer kernels (asynchronous on `stream`)                    */
/* ------------------------------------------------------------------ */

/* Per-token RMSNorm + absmax int8 quantization, bit-exact with
 * src/kernel.c:72-129 + 356-386, for M tokens of n values (row stride
 * x_stride floats).  Writes x_quant[m*quant_stride + i] and scale_x[m];
 * x_norm (nullable) gets [m*n + i].  Also fills the activation workspace
 * `act` (bm_hip_act_bytes(M, n) bytes) used by the _dev products below. */
size_t bm_hip_act_bytes(int M, int n);
int bm_hip_quantize_dev(const float *x,
                        int M,
                        int n,
                        int x_stride,
                        const float *norm_w,
                        float *x_norm,
                        int8_t *x_quant,
                        int quant_stride,
                        float *scale_x,
                        void *act,
                        void *stream);

/* Fast mode of the same (opt-in; not the reference's bits): the sum of
 * squares as one pairwise tree over the n values -- the reduction class of
 * the Metal backend's rms_norm_quantize (src/metal/bm_shaders.metal:40-60)
 * -- instead of the scalar kernel's four sequential chains
 * (src/kernel.c:77-89).  For n = 1024, 2048, 4096; other n give the
 * sequential sum. */
int bm_hip_quantize_fast_dev(const float *x,
                             int M,
                             int n,
                             int x_stride,
                             const float *norm_w,
                             float *x_norm,
                             int8_t *x_quant,
                             int quant_stride,
                             float *scale_x,
                             void *act,
                             void *stream);

/* Ternary BitLinear product on quantized activations (the act workspace
 * from bm_hip_quantize_dev): out[m*N + r] (fp32) with the scalar kernel's
 * 1024-column block epilogue (src/kernel.c:255-256, 407-447), bit-exact.
 * `canonical` != 0 promises the packed bytes hold no code 11. */
int bm_hip_bitlinear_act_dev(const void *act,
                             const float *scale_x,
                             int M,
                             const uint8_t *packed,
                             int N,
                             int K,
                             float w_scale,
                             int canonical,
                             float *out,
                             void *stream);

/* Quantize + product in one call (device pointers): scalar_bitlinear_
 * forward_batch semantics for M tokens. `act` as above.  One token on
 * canonical weights (K % 64 == 0, K <= 8192) runs as a single launch that
 * leaves `act` untouched. */
int bm_hip_bitlinear_dev(const float *x,
                         int M,
                         int K,
                         const float *norm_w,
                         const uint8_t *packed,
                         int N,
                         float w_scale,
                         int canonical,
                         float *out,
                         int8_t *x_quant,
                         int quant_stride,
                         float *scale_x,
                         void *act,
                         void *stream);

/* No counterpart in the reference: bm_hip_bitlinear_dev without any
 * allocation, for callers that cannot allocate (code under HIP stream
 * capture, tight serving loops).  The per-token scale and the activation
 * workspace (or int8 copy) live in a device array of the library's own,
 * bm_hip_noalloc_scratch_bytes() = 8 MiB per GPU, held until the process
 * ends; a call needing more (M * (K-row workspace) beyond it) returns -2.
 * Needs bm_hip_init() first (-1 otherwise).  Calls that overlap on one GPU
 * share the array and race.  Same semantics and output as
 * bm_hip_bitlinear_dev (out[m*N + r], bit-exact). */
int bm_hip_bitlinear_noalloc_dev(const float *x,
                                 int M,
                                 int K,
                                 const float *norm_w,
                                 const uint8_t *packed,
                                 int N,
                                 float w_scale,
                                 int canonical,
                                 float *out,
                                 void *stream);
size_t bm_hip_noalloc_scratch_bytes(void);

/* Exact int32 product of int8 activations and ternary weights:
 * out[m*N + r] = sum_k xq[m*ldx + k] * decode(W[r][k]) (stress shape;
 * activations need no quantization).  M = 1 (K % 64 == 0, K <= 8192) runs
 * as one GEMV launch that reads xq itself and leaves `act` untouched; few
 * tokens (K % 128 == 0, rows of xq on 16 bytes) one int8 MFMA launch that
 * also reads xq itself; other shapes prepare `act` first and run the int8
 * MFMA GEMM.  Needs bm_hip_i8_act_bytes(M, K) bytes of `act`. */
size_t bm_hip_i8_act_bytes(int M, int K);
int bm_hip_ternary_gemm_i32_dev(const int8_t *xq,
                                int M,
                                int ldx,
                                const uint8_t *packed,
                                int N,
                                int K,
                                int canonical,
                                int32_t *out,
                                void *act,
                                void *stream);

/* ------------------------------------------------------------------ */
/* Device-resident model: the reference's model API (src/bitmamba.h:    */
/* 282-294, src/model.c:477-1314) with weights, activations and the    */
/* recurrent state in HBM.  Greedy or sampled next tokens              */
/* (src/model.c:132-361) with the repetition penalty.                  */
/* ------------------------------------------------------------------ */
typedef struct bm_hip_model bm_hip_model_t;

/* model_load (src/model.c:477-932) from a BIT2 image in memory: same
 * validation; weights copied to one device arena (packed tensors with code
 * 11 rewritten to 10), A = -expf(A_log) and the conv transpose computed at
 * load.  NULL on failure (reason in bm_hip_last_error()). */
bm_hip_model_t *bm_hip_model_load(const void *image, size_t size);
/* model_free (src/model.c:1316-1372) */
void bm_hip_model_free(bm_hip_model_t *m);
/* 0 vocab, 1 d_model, 2 n_layers, 3 n_heads, 4 d_inner */
int bm_hip_model_config(const bm_hip_model_t *m, int which);
/* zero recurrent state and ring position (block_init_cache,
 * src/block.c:11-26) */
int bm_hip_model_reset(bm_hip_model_t *m);
/* model_prefill (src/model.c:1045-1153): n tokens through every layer,
 * batched BitLinear + token-serial SSM; no LM head.  0 or -1. */
int bm_hip_model_prefill(bm_hip_model_t *m, const int32_t *tokens, int n);
/* model_forward_step (src/model.c:1175-1314) with the sampler set by
 * bm_hip_model_set_sampler: returns the next token; history[history_len]
 * as the reference's caller keeps it (the last 256 tokens are used). */
int bm_hip_model_step(bm_hip_model_t *m,
                      int token,
                      const int *history,
                      int history_len,
                      float penalty);
/* Fast mode (on != 0; off by default): every later prefill, step,
 * generate and decode sums the squares of each RMSNorm of d_model 1024,
 * 2048 or 4096 (and d_inner of the same) as a pairwise tree, as
 * bm_hip_quantize_fast_dev does, instead of the reference's sequential
 * chains.  Results then differ from the reference in the last bits of
 * 1/rms and occasionally by one int8 step.  0. */
int bm_hip_model_set_fast(bm_hip_model_t *m, int on);
/* Measurement (no counterpart in the reference; for benchmarks and
 * profiles): one kernel of the decode step, launched reps times back to
 * back on the model's stream after two untimed launches, timed with events
 * on that stream.  which: 0 = in_proj + SSM step of `layer`, 1 = out_proj
 * (+ residual) of `layer`, 2 = the LM head (greedy candidates); layer -1
 * takes the layers in turn (0, 1, .., n_layers - 1, 0, ..), so that each
 * launch reads weights that the previous launches did not.  Writes the
 * average microseconds per launch to *avg_us.  The recurrent state and the
 * activations change: reset the model (or load a saved state) afterwards.
 * 0, or -1 (bm_hip_last_error) for bad arguments or widths that take the
 * generic kernels. */
int bm_hip_model_time_kernel(bm_hip_model_t *m, int which, int layer, int reps, float *avg_us);
/* Sampling parameters of every later step, generate and decode: the
 * temp, min_p, top_p, top_k arguments of model_forward_step
 * (src/model.c:1175-1183), sampled on the device by sample_advanced
 * (src/model.c:132-361).  temp < 0.05 is greedy (the default). */
int bm_hip_model_set_sampler(bm_hip_model_t *m,
                             float temp,
                             float min_p,
                             float top_p,
                             int top_k);
/* sample_advanced (src/model.c:132-361) on its own: one token from
 * logits[vocab] (device memory, 16-byte aligned; scaled in place by 1/temp
 * as the reference leaves them), advancing the XorShift64* state *rng
 * (device memory, src/utils.c:117-140); temp < 0.05 is the greedy branch.
 * workspace: bm_hip_sample_workspace_bytes(vocab) bytes of device memory
 * (the reference's probs buffer, twice).  The token goes to token_out[0]
 * (device memory); enqueued on `stream`, no synchronization.  0, or -1 for
 * vocab outside 1..256000, misaligned logits or a null pointer. */
size_t bm_hip_sample_workspace_bytes(int vocab);
int bm_hip_sample_advanced(float *logits,
                           int vocab,
                           float temp,
                           float min_p,
                           float top_p,
                           int top_k,
                           uint64_t *rng,
                           void *workspace,
                           int32_t *token_out,
                           void *stream);
/* rng_seed (src/utils.c:121-124) for the model's device generator; the
 * model starts with the reference's default state. */
int bm_hip_model_seed(bm_hip_model_t *m, uint64_t seed);
/* Recurrent state as a BMST image (state_save / state_load,
 * src/chat.c:1160-1271): u32 magic 0x424D5354, n_layers, d_inner, d_conv,
 * then per layer conv_state[(d_conv-1)*d_inner], ssm_state[d_inner] (fp32)
 * and conv_pos (int).  File I/O stays with the caller.  save returns the
 * bytes written (bm_hip_model_state_bytes) or -1; load returns 0, or -1
 * leaving the state untouched on a bad magic or dimensions and reset to
 * zero on a truncated image or a bad ring position, as the reference does.
 * Layers at different ring positions are rejected (the device model keeps
 * one position; the reference's layers always share it). */
size_t bm_hip_model_state_bytes(const bm_hip_model_t *m);
int bm_hip_model_state_save(const bm_hip_model_t *m, void *out, size_t len);
int bm_hip_model_state_load(bm_hip_model_t *m, const void *in, size_t len);
/* copies the logits of the last step (after the penalty; divided by the
 * temperature when the step sampled, like the reference's) */
int bm_hip_model_logits(const bm_hip_model_t *m, float *out);
/* copies one layer's conv_state [3][d_inner] and ssm_state [d_inner];
 * returns the ring position */
int bm_hip_model_layer_state(const bm_hip_model_t *m,
                             int layer,
                             float *conv_state,
                             float *ssm_state);
/* The inverse: one layer's conv ring [3][d_inner], ssm state [d_inner] and
 * ring position (the block cache fields of src/bitmamba.h:84-87) into the
 * device model.  The device keeps one ring position for all layers, as the
 * reference's layers advance together.  With bm_hip_model_layer_state this
 * is the prefill hook for model_prefill (the Metal spot, src/model.c:
 * 1050-1055): push the blocks' state, bm_hip_model_prefill, pull it back.
 * 0, or -1 with bm_hip_last_error(). */
int bm_hip_model_set_layer_state(bm_hip_model_t *m,
                                 int layer,
                                 const float *conv_state,
                                 const float *ssm_state,
                                 int conv_pos);
/* The decode loop of src/main.c:443-500 on the device: prefill
 * prompt[0..n-2], history = prompt, then n_steps steps (greedy or sampled,
 * bm_hip_model_set_sampler) from
 * prompt[n-1], each step one replay of a captured hipGraph with no host
 * synchronization.  Writes the tokens; *decode_ms = device time of the
 * steps (prefill excluded, as the reference's tok/s).  Returns the number of
 * tokens (cut after the first 50256 or 0 when stop_on_eos), -1 on error.
 * With stop_on_eos the step that picks the end token is the last that
 * changes anything, as in the reference's loop (src/main.c:473-500): the
 * recurrent state, ring position, history, logits and sampler state stay
 * where that step left them although the device replays the step graph
 * n_steps times (a done word in the control block turns the later steps'
 * stores off).  This holds for d_model and d_inner multiples of 64 up to
 * 8192 (the fused step kernels); other widths run all n_steps and only the
 * returned list is cut.  bm_hip_model_decode and bm_hip_model_step then
 * continue from the end token. */
int bm_hip_model_generate(bm_hip_model_t *m,
                          const int32_t *prompt,
                          int n_prompt,
                          int n_steps,
                          float penalty,
                          int stop_on_eos,
                          int32_t *out_tokens,
                          double *decode_ms);
/* n_steps more steps from the current device state (also after a
 * generate that stopped at an end token); tokens readable with
 * bm_hip_model_tokens. */
int bm_hip_model_decode(bm_hip_model_t *m,
                        int n_steps,
                        float penalty,
                        double *decode_ms);
int bm_hip_model_tokens(const bm_hip_model_t *m, int32_t *out, int n);

/* Diagnostic (no reference counterpart): evaluates the device scalar
 * functions of the SSM step on n device floats, for checks against the host:
 * fn 0 = expf, 1 = logf (restatements of glibc's), 2 = fp32 division of each
 * even/odd input pair in both orders (out[i] = in[i] / in[i ^ 1]; a last
 * unpaired input is divided by itself), 3 = silu, x / (1 + expf(-x)),
 * 4 = sqrt.  Returns -1 for any other fn. */
int bm_hip_libm_eval_dev(int fn,
                         const float *in,
                         float *out,
                         size_t n,
                         void *stream);

/* ------------------------------------------------------------------ */
/* Synthetic BIT2 images (counterpart: the writer scripts/export-bin.py  */
/* :99-199; no libm, bit-reproducible on any host)                      */
/* ------------------------------------------------------------------ */
enum {
    BM_SYNTH_UNIFORM = 0,   /* p(-1)=p(0)=p(+1)=1/3 */
    BM_SYNTH_P0_40 = 1,     /* p(0)=0.4, p(+-1)=0.3 */
    BM_SYNTH_P0_60 = 2,     /* p(0)=0.6, p(+-1)=0.2 */
    BM_SYNTH_RAW_BYTES = 3, /* all four 2-bit codes, 11 included */
};

typedef struct {
    int vocab;
    int d_model;
    int n_layers;
    int n_heads;
    int in_proj_rows; /* 0: 2*d_inner + 3*n_heads (src/model.c:683-701) */
    int ternary_dist; /* BM_SYNTH_* */
    float fp_sigma;   /* std of every float tensor */
    float ternary_scale;
    uint64_t seed;
} bm_synth_config_t;

size_t bm_bit2_synth_size(const bm_synth_config_t *c);
int bm_bit2_synth_write(const bm_synth_config_t *c, void *dst, size_t len);
void bm_synth_ternary(uint64_t seed,
                      int tensor,
                      int rows,
                      int cols,
                      int dist,
                      uint8_t *packed);
void bm_synth_normal(uint64_t seed,
                     int tensor,
                     size_t n,
                     float sigma,
                     float *out);
void bm_synth_int8(uint64_t seed, int tensor, size_t n, int8_t *out);
void bm_synth_prompt(uint64_t seed, int vocab, int n, int32_t *tokens);

#ifdef __cplusplus
}
#endif
