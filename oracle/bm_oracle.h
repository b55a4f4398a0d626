/*
 * CPU oracle for the ternary BitLinear hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference's scalar path (jserv/bitmamba.c,
 * src/kernel.c, src/quantization.c, src/block.c, src/model.c).  Only the
 * tests, __graft_entry__.smoke() and the cpu_baseline leg of bench.py load
 * it, and only to check results or time the CPU; the product library never
 * links it.
 *
 * Pinning (each function is checked by something other than itself):
 *   orc_luts / orc_decode_weight   exhaustive 256-byte KAT vs the compiled
 *                                  reference (oracle/_ref) and the closed
 *                                  form min(code-1, 1)
 *   orc_rms_norm                   bit-exact vs _ref on seeded vectors,
 *                                  golden fixtures; invariants (scale
 *                                  invariance of the int8 output, max maps
 *                                  to +-127)
 *   orc_bitlinear_forward[_batch]  bit-exact vs _ref (scalar) + fixtures;
 *                                  int32 slice totals vs numpy brute force
 *   orc_ternary_gemm_i32           numpy brute force (closed form)
 *   orc_ssm_inner                  bit-exact vs _ref scalar_ssm_inner
 *   orc_model_*                    bit-exact logits + identical greedy
 *                                  streams vs _ref model_load/prefill/
 *                                  forward_step on synthetic BIT2 files
 *   orc_sample                     identical draws vs _ref model_forward_step
 *                                  sampling the same logits from the same
 *                                  generator state, on every path (top-k
 *                                  heap, top-p partial and full sort,
 *                                  min_p, greedy); closed forms: min_p = 1
 *                                  keeps only the max, top_k = 1 is greedy
 * No function is left unpinned.
 */
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* XorShift64* (src/utils.c:117-140), with the state passed explicitly. */
uint64_t orc_rng_next(uint64_t *state);
/* sample_advanced (src/model.c:132-361) with filter_and_sample: returns the
 * drawn token; logits are scaled by 1/temp in place like the reference's */
int orc_sample(float *logits, int vocab, float temp, float min_p, float top_p, int top_k,
               uint64_t *rng);

/* 2-bit code -> {-1, 0, +1, +1} (src/quantization.c:27-31). */
int orc_decode_weight(int bits);
/* UNPACK_LUT[256][4], TMAC_P_MASK[256], TMAC_N_MASK[256]
 * (src/quantization.c:33-53). */
void orc_luts(int8_t *unpack, uint8_t *pmask, uint8_t *nmask);

/* scalar_rms_norm (src/kernel.c:72-129): returns max |out|. */
float orc_rms_norm(const float *x, int size, const float *weight, float *out);

/* Quantize step of scalar_bitlinear_forward (src/kernel.c:358-386).
 * Returns scale_x. */
float orc_quantize(const float *x_norm, int n, float max_abs, int8_t *x_quant);

/* Integer part of the T-MAC GEMV (src/kernel.c:131-316, 388-447) on an
 * already-quantized vector: per-row totals of each 1024-column block
 * (slice_totals[r * n_slices + s], n_slices = ceil((cols/4)/256)) and the
 * remainder-column total (rem_totals[r], zero when cols % 4 == 0). */
int orc_tmac_slice_count(int cols);
void orc_tmac_totals(const int8_t *x_quant,
                     const uint8_t *packed,
                     int rows,
                     int cols,
                     int32_t *slice_totals,
                     int32_t *rem_totals);

/* scalar_bitlinear_forward (src/kernel.c:346-448). */
void orc_bitlinear_forward(const float *x,
                           int n,
                           const uint8_t *packed,
                           int rows,
                           int cols,
                           float w_scale,
                           const float *norm_w,
                           float *out,
                           float *x_norm_buf,
                           int8_t *x_quant_buf);

/* scalar_bitlinear_forward_batch (src/kernel.c:322-338). */
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
                                 int quant_stride);

/* Epilogue of the int8-input path: out = sum_s fl(total_s * inv_scale)
 * in block order, then the remainder (src/kernel.c:255-256, 407-447). */
void orc_tmac_rows_f32(const int8_t *x_quant,
                       const uint8_t *packed,
                       int rows,
                       int cols,
                       float inv_scale,
                       float *out);

/* Plain int32 ternary product out[m][r] = sum_k xq[m][k]*decode(W[r][k]). */
void orc_ternary_gemm_i32(const int8_t *xq,
                          int M,
                          int ldx,
                          const uint8_t *packed,
                          int N,
                          int K,
                          int32_t *out);

/* scalar_ssm_inner (src/kernel.c:34-70) over [idx_start, idx_end).
 * proj: [z(d_inner) | x(d_inner) | B(h) | C(h) | dt(h)] (src/block.c:54-58);
 * conv_w_t: [4][d_inner]; cs0/cs1/cs2 oldest..newest taps; cs_write = cs0. */
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
                   int idx_end);

/* ---- model (BIT2 loader + scalar prefill / greedy step) ---- */
typedef struct orc_model orc_model_t;

/* Parses a BIT2 image held in memory (the caller keeps it alive) with the
 * validation of src/model.c:367-932.  Returns NULL on a malformed image. */
orc_model_t *orc_model_load(const void *blob, size_t len);
void orc_model_free(orc_model_t *m);
/* model_prefill, scalar branch (src/model.c:1045-1153). */
void orc_model_prefill(orc_model_t *m, const int32_t *tokens, int n_tokens);
/* model_forward_step with temp < 0.05 (greedy, src/model.c:1175-1314). */
int orc_model_step(orc_model_t *m,
                   int token,
                   const int *history,
                   int history_len,
                   float penalty);
const float *orc_model_logits(const orc_model_t *m);
int orc_model_config(const orc_model_t *m, int which);
/* copies one layer's conv_state/ssm_state; returns conv_pos */
int orc_model_layer_state(const orc_model_t *m,
                          int layer,
                          float *conv_state,
                          float *ssm_state);

/* libm expf / logf applied elementwise (the values the SSM step sees) */
void orc_expf_array(const float *in, float *out, size_t n);
void orc_logf_array(const float *in, float *out, size_t n);

#ifdef __cplusplus
}
#endif
