/*
 * Deterministic synthetic BIT2 model images.
 *
 * Writes the on-disk layout that scripts/export-bin.py:110-199 produces and
 * src/model.c:477-932 loads:
 *   header  int32 magic 0x42495432, vocab, d_model, n_layers, n_heads
 *   tensors embed; per layer in_proj.norm, in_proj, conv1d.weight,
 *           conv1d.bias, dt_bias, A_log, D, out_proj.norm, out_proj;
 *           norm_f, lm_head.norm, lm_head
 *   float   int32 type 0, int32 ndim, int32 dims[ndim], float32 data
 *   ternary int32 type 2, int32 rows, int32 cols, float32 scale,
 *           uint8 packed[rows][ceil(cols/4)], column c in bits 2*(c%4) of
 *           byte c/4, code = w + 1 (export-bin.py:99-107)
 *
 * Values are bit-reproducible on any host: no libm, integer PRNG only.
 *   - every (tensor, row) draws from its own XorShift64* stream
 *     (src/utils.c:117-140) seeded by splitmix64 of (seed, tensor, row), so
 *     rows can be generated in parallel without changing a single bit;
 *     float tensors use 1024-element rows;
 *   - normals: Irwin-Hall, z = (sum of 12 draws of 24 bits - 6*2^24) / 2^24,
 *     value = (float)((double)z * sigma);
 *   - ternary: {-1,0,+1} with the distribution selected by `dist`.
 */
#include <stdint.h>
#include <string.h>

#include "bm_hip.h"

static uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ULL;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ULL;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBULL;
    return x ^ (x >> 31);
}

static uint64_t xs_next(uint64_t *s)
{
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1DULL;
}

static uint64_t stream_seed(uint64_t seed, int tensor, int64_t row)
{
    uint64_t s = splitmix64(seed ^ splitmix64(((uint64_t) (uint32_t) tensor
                                               << 40) ^
                                              (uint64_t) row));
    return s ? s : 0x853c49e6748fea9bULL;
}

static float normal_draw(uint64_t *s, double sigma)
{
    int64_t acc = 0;
    for (int k = 0; k < 12; k++)
        acc += (int64_t) (xs_next(s) >> 40);
    acc -= 6LL << 24;
    return (float) ((double) acc * (sigma / 16777216.0));
}

/* code = w + 1: 0 -> -1, 1 -> 0, 2 -> +1 */
static int ternary_code(uint64_t *s, int dist)
{
    uint64_t r = xs_next(s);
    switch (dist) {
    case BM_SYNTH_P0_40: { /* p(0)=0.4, p(+-1)=0.3 */
        int v = (int) (r % 10);
        return v < 3 ? 0 : (v < 7 ? 1 : 2);
    }
    case BM_SYNTH_P0_60: { /* p(0)=0.6, p(+-1)=0.2 */
        int v = (int) (r % 5);
        return v == 0 ? 0 : (v < 4 ? 1 : 2);
    }
    case BM_SYNTH_RAW_BYTES: /* every 2-bit code, 11 included */
        return (int) (r & 3);
    default: /* uniform thirds */
        return (int) (r % 3);
    }
}

void bm_synth_ternary(uint64_t seed,
                      int tensor,
                      int rows,
                      int cols,
                      int dist,
                      uint8_t *packed)
{
    int stride = (cols + 3) / 4;
#pragma omp parallel for schedule(dynamic, 64)
    for (int r = 0; r < rows; r++) {
        uint64_t s = stream_seed(seed, tensor, r);
        uint8_t *row = packed + (size_t) r * stride;
        memset(row, 0, (size_t) stride);
        for (int c = 0; c < cols; c++)
            row[c >> 2] |= (uint8_t) (ternary_code(&s, dist) << (2 * (c & 3)));
    }
}

void bm_synth_normal(uint64_t seed,
                     int tensor,
                     size_t n,
                     float sigma,
                     float *out)
{
    int64_t n_rows = (int64_t) ((n + 1023) / 1024);
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < n_rows; r++) {
        uint64_t s = stream_seed(seed, tensor, r);
        size_t e = (size_t) r * 1024 + 1024;
        if (e > n)
            e = n;
        for (size_t i = (size_t) r * 1024; i < e; i++)
            out[i] = normal_draw(&s, sigma);
    }
}

void bm_synth_int8(uint64_t seed, int tensor, size_t n, int8_t *out)
{
    int64_t n_rows = (int64_t) ((n + 1023) / 1024);
#pragma omp parallel for schedule(dynamic, 16)
    for (int64_t r = 0; r < n_rows; r++) {
        uint64_t s = stream_seed(seed, tensor, r);
        size_t e = (size_t) r * 1024 + 1024;
        if (e > n)
            e = n;
        for (size_t i = (size_t) r * 1024; i < e; i++)
            out[i] = (int8_t) ((int) (xs_next(&s) % 255) - 127);
    }
}

/* ---- BIT2 image ---- */

static int in_proj_rows(const bm_synth_config_t *c)
{
    if (c->in_proj_rows > 0)
        return c->in_proj_rows;
    return 2 * (2 * c->d_model) + 3 * c->n_heads;
}

static size_t float_rec(int ndim, size_t n)
{
    return 8 + 4 * (size_t) ndim + 4 * n;
}

static size_t tern_rec(int rows, int cols)
{
    return 16 + (size_t) rows * (size_t) ((cols + 3) / 4);
}

size_t bm_bit2_synth_size(const bm_synth_config_t *c)
{
    if (!c || c->vocab <= 0 || c->d_model <= 0 || c->n_layers <= 0 ||
        c->n_heads <= 0)
        return 0;
    size_t dm = (size_t) c->d_model, di = 2 * dm, nh = (size_t) c->n_heads;
    size_t sz = 20 + float_rec(2, (size_t) c->vocab * dm);
    size_t layer = float_rec(1, dm) + tern_rec(in_proj_rows(c), c->d_model) +
                   float_rec(2, di * 4) + float_rec(1, di) +
                   float_rec(1, nh) * 2 + float_rec(1, di) +
                   float_rec(1, di) + tern_rec(c->d_model, (int) di);
    sz += layer * (size_t) c->n_layers;
    sz += float_rec(1, dm) * 2 + tern_rec(c->vocab, c->d_model);
    return sz;
}

typedef struct {
    uint8_t *p;
    int tensor;
} wr_t;

static void put_i32(wr_t *w, int v)
{
    memcpy(w->p, &v, 4);
    w->p += 4;
}

static void put_f32(wr_t *w, float v)
{
    memcpy(w->p, &v, 4);
    w->p += 4;
}

/* data is generated straight into the (possibly unaligned) image */
static void put_float_tensor(wr_t *w,
                             const bm_synth_config_t *c,
                             int ndim,
                             int d0,
                             int d1)
{
    size_t n = (size_t) d0 * (size_t) (ndim == 2 ? d1 : 1);
    put_i32(w, 0);
    put_i32(w, ndim);
    put_i32(w, d0);
    if (ndim == 2)
        put_i32(w, d1);
    if (((uintptr_t) w->p & 3) == 0) {
        bm_synth_normal(c->seed, w->tensor, n, c->fp_sigma, (float *) w->p);
    } else {
        /* generate in chunks of 1024-element rows to keep the streams */
        float buf[1024];
        for (size_t r = 0; r * 1024 < n; r++) {
            size_t m = n - r * 1024 < 1024 ? n - r * 1024 : 1024;
            uint64_t s = stream_seed(c->seed, w->tensor, (int64_t) r);
            for (size_t i = 0; i < m; i++)
                buf[i] = normal_draw(&s, c->fp_sigma);
            memcpy(w->p + r * 4096, buf, m * 4);
        }
    }
    w->p += 4 * n;
    w->tensor++;
}

static void put_ternary_tensor(wr_t *w,
                               const bm_synth_config_t *c,
                               int rows,
                               int cols)
{
    put_i32(w, 2);
    put_i32(w, rows);
    put_i32(w, cols);
    put_f32(w, c->ternary_scale);
    bm_synth_ternary(c->seed, w->tensor, rows, cols, c->ternary_dist, w->p);
    w->p += (size_t) rows * (size_t) ((cols + 3) / 4);
    w->tensor++;
}

int bm_bit2_synth_write(const bm_synth_config_t *c, void *dst, size_t len)
{
    size_t need = bm_bit2_synth_size(c);
    if (!need || !dst || len < need)
        return -1;
    int dm = c->d_model, di = 2 * dm, nh = c->n_heads;
    wr_t w = {(uint8_t *) dst, 0};
    put_i32(&w, 0x42495432);
    put_i32(&w, c->vocab);
    put_i32(&w, dm);
    put_i32(&w, c->n_layers);
    put_i32(&w, nh);
    put_float_tensor(&w, c, 2, c->vocab, dm); /* embed */
    for (int l = 0; l < c->n_layers; l++) {
        put_float_tensor(&w, c, 1, dm, 0);           /* in_proj.norm */
        put_ternary_tensor(&w, c, in_proj_rows(c), dm); /* in_proj */
        put_float_tensor(&w, c, 2, di, 4);           /* conv1d.weight */
        put_float_tensor(&w, c, 1, di, 0);           /* conv1d.bias */
        put_float_tensor(&w, c, 1, nh, 0);           /* dt_bias */
        put_float_tensor(&w, c, 1, nh, 0);           /* A_log */
        put_float_tensor(&w, c, 1, di, 0);           /* D */
        put_float_tensor(&w, c, 1, di, 0);           /* out_proj.norm */
        put_ternary_tensor(&w, c, dm, di);           /* out_proj */
    }
    put_float_tensor(&w, c, 1, dm, 0);          /* norm_f */
    put_float_tensor(&w, c, 1, dm, 0);          /* lm_head.norm */
    put_ternary_tensor(&w, c, c->vocab, dm);    /* lm_head */
    return (size_t) (w.p - (uint8_t *) dst) == need ? 0 : -1;
}

void bm_synth_prompt(uint64_t seed, int vocab, int n, int32_t *tokens)
{
    uint64_t s = stream_seed(seed, 0x7fffff, 0);
    for (int i = 0; i < n; i++)
        tokens[i] = (int32_t) (xs_next(&s) % (uint64_t) vocab);
}
