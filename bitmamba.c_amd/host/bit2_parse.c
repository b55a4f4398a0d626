/*
 * BIT2 image parser: the structure of read_tensor_mmap and the checks of
 * model_load (src/model.c:367-475, 630-784), over an image in memory.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "bm_bit2.h"

enum { MAGIC = 0x42495432, MAX_DIM = 1 << 20, MAX_VOCAB = 256000 };

static int get_i32(const uint8_t *p)
{
    int v;
    memcpy(&v, p, 4);
    return v;
}

static size_t parse_tensor(const uint8_t *p,
                           const uint8_t *end,
                           bm_bit2_tensor_t *t)
{
    const uint8_t *s = p;
    memset(t, 0, sizeof(*t));
    t->scale = 1.0f;
    if (end - p < 4)
        return 0;
    int type = get_i32(p);
    p += 4;
    if (type == 2) {
        if (end - p < 12)
            return 0;
        t->is_bitnet = true;
        t->rows = get_i32(p);
        t->cols = get_i32(p + 4);
        memcpy(&t->scale, p + 8, 4);
        p += 12;
        if (!isfinite(t->scale) || t->scale <= 0.0f)
            return 0;
        if (t->rows <= 0 || t->rows > MAX_DIM || t->cols <= 0 ||
            t->cols > MAX_DIM)
            return 0;
        size_t bytes = (size_t) t->rows * (size_t) ((t->cols + 3) / 4);
        if (bytes > (size_t) (end - p))
            return 0;
        t->packed = p;
        t->n_elements = (size_t) t->rows * (size_t) t->cols;
        p += bytes;
    } else {
        if (end - p < 4)
            return 0;
        int ndim = get_i32(p);
        p += 4;
        if (ndim < 0 || ndim > 4 || (size_t) (end - p) < (size_t) ndim * 4)
            return 0;
        size_t total = 1;
        for (int i = 0; i < ndim; i++) {
            int d = get_i32(p);
            p += 4;
            if (d <= 0 || d > MAX_DIM)
                return 0;
            total *= (size_t) d;
            if (i == 0)
                t->rows = d;
            if (i == 1)
                t->cols = d;
        }
        if (total > (size_t) (end - p) / 4)
            return 0;
        t->data = (const float *) p;
        t->n_elements = total;
        p += total * 4;
    }
    return (size_t) (p - s);
}

void bm_bit2_view_free(bm_bit2_view_t *v)
{
    if (!v)
        return;
    free(v->tensors);
    v->tensors = NULL;
    v->n_tensors = 0;
}

int bm_bit2_parse(const void *base, size_t size, bm_bit2_view_t *v)
{
    memset(v, 0, sizeof(*v));
    const uint8_t *p = (const uint8_t *) base, *end = p + size;
    if (!base || size < 20 || get_i32(p) != MAGIC)
        return -1;
    v->vocab = get_i32(p + 4);
    v->d_model = get_i32(p + 8);
    v->n_layers = get_i32(p + 12);
    v->n_heads = get_i32(p + 16);
    p += 20;
    if (v->vocab <= 0 || v->vocab > MAX_VOCAB || v->d_model <= 0 ||
        v->d_model > MAX_DIM || v->n_layers <= 0 || v->n_layers > 256 ||
        v->n_heads <= 0 || v->n_heads > MAX_DIM)
        return -1;
    v->n_tensors = 1 + BM_L_COUNT * v->n_layers + 3;
    v->tensors = calloc((size_t) v->n_tensors, sizeof(bm_bit2_tensor_t));
    if (!v->tensors)
        return -1;
    for (int i = 0; i < v->n_tensors; i++) {
        size_t c = parse_tensor(p, end, &v->tensors[i]);
        if (!c) {
            bm_bit2_view_free(v);
            return -1;
        }
        p += c;
    }

    int dm = v->d_model, di = 2 * dm, nh = v->n_heads;
    const bm_bit2_tensor_t *embed = &v->tensors[0];
    const bm_bit2_tensor_t *fin = &v->tensors[1 + BM_L_COUNT * v->n_layers];
    if (fin[0].n_elements < (size_t) dm || fin[1].n_elements < (size_t) dm)
        goto bad;
    if (embed->n_elements < (size_t) v->vocab * dm)
        goto bad;
    if (fin[2].rows != v->vocab || fin[2].cols != dm)
        goto bad;
    if (di % nh != 0)
        goto bad;
    for (int l = 0; l < v->n_layers; l++) {
        const bm_bit2_tensor_t *t = bm_bit2_layer(v, l, 0);
        if (t[BM_L_IN_NORM].n_elements < (size_t) dm)
            goto bad;
        if (t[BM_L_IN_PROJ].cols != dm ||
            t[BM_L_IN_PROJ].rows != 2 * di + 3 * nh)
            goto bad;
        if (t[BM_L_OUT_PROJ].rows != dm || t[BM_L_OUT_PROJ].cols != di)
            goto bad;
        if (t[BM_L_CONV_W].n_elements < (size_t) di * 4 ||
            t[BM_L_CONV_B].n_elements < (size_t) di ||
            t[BM_L_DT_BIAS].n_elements < (size_t) nh ||
            t[BM_L_A_LOG].n_elements < (size_t) nh ||
            t[BM_L_D].n_elements < (size_t) di ||
            t[BM_L_OUT_NORM].n_elements < (size_t) di)
            goto bad;
        if (!t[BM_L_IN_PROJ].is_bitnet || !t[BM_L_OUT_PROJ].is_bitnet)
            goto bad;
        for (int k = 0; k < BM_L_COUNT; k++)
            if (k != BM_L_IN_PROJ && k != BM_L_OUT_PROJ && t[k].is_bitnet)
                goto bad;
    }
    if (embed->is_bitnet || fin[0].is_bitnet || fin[1].is_bitnet ||
        !fin[2].is_bitnet)
        goto bad;
    return 0;
bad:
    bm_bit2_view_free(v);
    return -2;
}
