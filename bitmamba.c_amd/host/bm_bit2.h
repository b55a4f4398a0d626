/*
 * BIT2 model image parsing for the device arena (internal header).
 * Layout and validation follow src/model.c:367-784 (reader) and
 * scripts/export-bin.py:110-199 (writer).
 */
#pragma once

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct {
    const float *data;     /* float tensor payload (may be unaligned) */
    const uint8_t *packed; /* ternary payload, [rows][ceil(cols/4)] */
    int rows, cols;
    size_t n_elements;
    bool is_bitnet;
    float scale;
} bm_bit2_tensor_t;

/* Tensor order of the image: embed, then per layer the nine BM_L_* entries,
 * then norm_f, lm_head.norm, lm_head. */
enum {
    BM_L_IN_NORM = 0,
    BM_L_IN_PROJ,
    BM_L_CONV_W,
    BM_L_CONV_B,
    BM_L_DT_BIAS,
    BM_L_A_LOG,
    BM_L_D,
    BM_L_OUT_NORM,
    BM_L_OUT_PROJ,
    BM_L_COUNT
};

typedef struct {
    int vocab, d_model, n_layers, n_heads;
    int n_tensors;
    bm_bit2_tensor_t *tensors; /* 1 + 9*n_layers + 3 entries */
} bm_bit2_view_t;

static inline const bm_bit2_tensor_t *bm_bit2_layer(const bm_bit2_view_t *v,
                                                    int layer,
                                                    int which)
{
    return &v->tensors[1 + BM_L_COUNT * layer + which];
}

/* 0 on success; -1 malformed structure; -2 shapes/types rejected by the
 * reference loader's validation. */
int bm_bit2_parse(const void *base, size_t size, bm_bit2_view_t *out);
void bm_bit2_view_free(bm_bit2_view_t *v);

#ifdef __cplusplus
}
#endif
