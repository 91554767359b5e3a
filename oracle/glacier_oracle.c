/*
 * glacier_oracle.c — CPU restatement of the reference's text-token-loop
 * numerics. TEST INFRASTRUCTURE ONLY: see glacier_oracle.h.
 *
 * Built with -O2 -ffp-contract=off and without fast-math so every f32
 * operation rounds where the reference's Zig code rounds. Zig @Vector
 * accumulators are restated as explicit per-lane arrays, and @reduce(.Add)
 * as a sequential lane-0-first sum.
 */
#define _GNU_SOURCE
#include "glacier_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* threads: row split (int4_matmul.zig:3046-3160 is bit-identical to serial) */
/* ------------------------------------------------------------------------ */
static int g_threads = 1;
void go_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }
int go_get_threads(void) { return g_threads; }

typedef void (*go_range_fn)(void *ctx, size_t begin, size_t end);
typedef struct { go_range_fn fn; void *ctx; size_t begin, end; } go_task;
static void *go_task_run(void *p) {
    go_task *t = (go_task *)p;
    if (t->begin < t->end) t->fn(t->ctx, t->begin, t->end);
    return NULL;
}
static void go_parallel_rows(go_range_fn fn, void *ctx, size_t rows) {
    int nt = g_threads;
    if (nt <= 1 || rows < 256) { fn(ctx, 0, rows); return; }
    if ((size_t)nt > rows) nt = (int)rows;
    pthread_t th[256];
    go_task tasks[256];
    size_t chunk = (rows + nt - 1) / nt;
    for (int i = 0; i < nt; i++) {
        tasks[i].fn = fn; tasks[i].ctx = ctx;
        tasks[i].begin = (size_t)i * chunk;
        tasks[i].end = tasks[i].begin + chunk > rows ? rows : tasks[i].begin + chunk;
        if (tasks[i].begin > rows) tasks[i].begin = rows;
    }
    for (int i = 1; i < nt; i++) pthread_create(&th[i], NULL, go_task_run, &tasks[i]);
    go_task_run(&tasks[0]);
    for (int i = 1; i < nt; i++) pthread_join(th[i], NULL);
}

static size_t ceil_div(size_t a, size_t b) { return a / b + (a % b != 0); }

/* ------------------------------------------------------------------------ */
/* a1: INT4 code                                                            */
/* ------------------------------------------------------------------------ */
/* int4_matmul.zig:22-25 NIBBLE_TO_OFFSET: nibble u -> f32(u - 7). */
static const float NIBBLE_TO_OFFSET[16] = {-7, -6, -5, -4, -3, -2, -1, 0,
                                           1,  2,  3,  4,  5,  6,  7, 8};

/* quant.zig:164-191: two codes per byte, low nibble holds the even index. */
uint8_t go_read_nibble(const uint8_t *buf, size_t idx) {
    uint8_t b = buf[idx / 2];
    return (idx % 2 == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F);
}
void go_write_nibble(uint8_t *buf, size_t idx, uint8_t val) {
    size_t bi = idx / 2;
    if (idx % 2 == 0) buf[bi] = (uint8_t)((buf[bi] & 0xF0) | (val & 0x0F));
    else buf[bi] = (uint8_t)((buf[bi] & 0x0F) | ((val & 0x0F) << 4));
}

/* Zig @round: round half away from zero. */
static float zig_round(float v) { return roundf(v); }

/* quant.zig:36-111 (INT4 branch). qzero = 7, qmin = -7, qmax = 8 when
 * group_size >= 16 else 7. Scale = max(-min/7, max/qmax). */
int go_int4_quantize(const float *src, size_t n, uint32_t group_size,
                     uint8_t *packed, float *scales) {
    if (n == 0) return GO_OK;
    if (group_size == 0) return GO_BAD_GROUP_SIZE;
    const int32_t qzero = 7, qmin = -7;
    const int32_t qmax = group_size >= 16 ? qzero + 1 : qzero;
    memset(packed, 0, ceil_div(n * 4, 8));
    size_t elem = 0, gi = 0;
    while (elem < n) {
        size_t end = elem + ((n - elem) < group_size ? (n - elem) : group_size);
        float mn = 0, mx = 0;
        for (size_t i = elem; i < end; i++) {
            float fv = src[i];
            /* Zig @min/@max on f32 */
            mn = fv < mn ? fv : mn;
            mx = fv > mx ? fv : mx;
        }
        float neg = -mn / (float)(-qmin);
        float pos = mx / (float)qmax;
        float scale = neg > pos ? neg : pos;
        scales[gi] = scale;
        float inv = scale == 0 ? 0.0f : 1.0f / scale;
        for (size_t i = elem; i < end; i++) {
            int32_t q = (int32_t)zig_round(src[i] * inv);
            if (q < qmin) q = qmin;
            if (q > qmax) q = qmax;
            go_write_nibble(packed, i, (uint8_t)(q + qzero));
        }
        elem = end;
        gi++;
    }
    return GO_OK;
}

/* quant.zig:114-162 (INT4 branch): v = f32(u - 7) * scale. */
int go_int4_dequantize(const uint8_t *packed, size_t packed_len,
                       const float *scales, size_t scale_len,
                       uint32_t group_size, size_t n, float *out) {
    if (n == 0) return GO_OK;
    if (group_size == 0) return GO_BAD_GROUP_SIZE;
    if (scale_len < ceil_div(n, group_size)) return GO_TRUNCATED;
    if (packed_len < ceil_div(n * 4, 8)) return GO_TRUNCATED;
    for (size_t i = 0; i < n; i++) {
        int32_t q = (int32_t)go_read_nibble(packed, i) - 7;
        out[i] = (float)q * scales[i / group_size];
    }
    return GO_OK;
}

float go_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1F, man = h & 0x3FF, bits;
    if (exp == 0) {
        if (man == 0) bits = sign;
        else { /* subnormal: value = man * 2^-24, exact in f32 */
            float f = (float)man * 5.9604644775390625e-8f;
            memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (exp == 31) bits = sign | 0x7F800000u | (man << 13);
    else bits = sign | ((exp + 112) << 23) | (man << 13);
    float f; memcpy(&f, &bits, 4); return f;
}

uint16_t go_f32_to_f16(float f) {
    uint32_t x; memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000;
    uint32_t ax = x & 0x7FFFFFFF;
    if (ax > 0x7F800000) return (uint16_t)(sign | 0x7E00);            /* NaN */
    if (ax >= 0x477FF000) return (uint16_t)(sign | 0x7C00);           /* overflow -> inf */
    if (ax < 0x38800000) {                                            /* subnormal / zero */
        if (ax < 0x33000000) return (uint16_t)sign;                   /* < 2^-25 rounds to 0 */
        uint32_t e = ax >> 23, m = (ax & 0x7FFFFF) | 0x800000;
        uint32_t shift = 126 - e;                                     /* 14 + (112 - e) + 0 */
        uint32_t r = m >> shift, rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (r & 1))) r++;
        return (uint16_t)(sign | r);
    }
    uint32_t r = ((ax >> 13) - (112u << 10));
    uint32_t rem = ax & 0x1FFF;
    if (rem > 0x1000 || (rem == 0x1000 && (r & 1))) r++;
    return (uint16_t)(sign | r);
}

/* ------------------------------------------------------------------------ */
/* a2: linearInt4OnTheFly (int4_matmul.zig:215-311)                          */
/* ------------------------------------------------------------------------ */
typedef struct {
    const float *x; const uint8_t *packed; const float *scales; const float *bias;
    float *out; size_t out_f, in_f, group_size, row_idx;
} lin_ctx;

static float reduce8(const float v[8]) {
    float r = v[0];
    for (int j = 1; j < 8; j++) r += v[j];
    return r;
}

static float dequant_element(const uint8_t *packed, const float *scales,
                             size_t idx, size_t group_size) {
    return NIBBLE_TO_OFFSET[go_read_nibble(packed, idx)] * scales[idx / group_size];
}

static void lin_f32_rows(void *p, size_t o0, size_t o1) {
    lin_ctx *c = (lin_ctx *)p;
    const float *x_row = c->x + c->row_idx * c->in_f;
    const size_t in_f = c->in_f, gs = c->group_size;
    for (size_t o = o0; o < o1; o++) {
        float acc = c->bias ? c->bias[o] : 0.0f;
        const size_t w_row_start = o * in_f;
        if (gs % 8 == 0 && w_row_start % gs == 0 && in_f % gs == 0) {
            /* Vec8 accumulator, (w * x) * scale per lane (int4_matmul.zig:277-287) */
            float vacc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
            size_t elem = 0, gidx = w_row_start / gs;
            while (elem < in_f) {
                const size_t gend = elem + gs;
                const float s = c->scales[gidx];
                for (; elem < gend; elem += 8) {
                    const uint8_t *b = c->packed + (w_row_start + elem) / 2;
                    for (int j = 0; j < 8; j++) {
                        uint8_t nib = (j & 1) ? (b[j / 2] >> 4) & 0xF : b[j / 2] & 0xF;
                        float w = NIBBLE_TO_OFFSET[nib];
                        float t = w * x_row[elem + j];
                        t = t * s;
                        vacc[j] += t;
                    }
                }
                gidx++;
            }
            acc += reduce8(vacc);
        } else {
            /* generic path (int4_matmul.zig:289-306) */
            size_t elem = 0;
            while (elem + 8 <= in_f) {
                size_t gidx = w_row_start + elem;
                size_t gi0 = gidx / gs, gi1 = (gidx + 7) / gs;
                if (gidx % 2 != 0 || gi0 != gi1) {
                    acc += x_row[elem] * dequant_element(c->packed, c->scales, gidx, gs);
                    elem += 1;
                    continue;
                }
                float v[8];
                for (int j = 0; j < 8; j++)
                    v[j] = NIBBLE_TO_OFFSET[go_read_nibble(c->packed, gidx + j)] * x_row[elem + j];
                acc += reduce8(v) * c->scales[gi0];
                elem += 8;
            }
            for (; elem < in_f; elem++)
                acc += x_row[elem] * dequant_element(c->packed, c->scales, w_row_start + elem, gs);
        }
        c->out[c->row_idx * c->out_f + o] = acc;
    }
}

int go_linear_int4_f32(const float *x, size_t batch, const uint8_t *packed,
                       const float *scales, const float *bias, float *out,
                       size_t out_f, size_t in_f, size_t group_size) {
    if (group_size == 0) return GO_SHAPE_MISMATCH;
    lin_ctx c = {x, packed, scales, bias, out, out_f, in_f, group_size, 0};
    for (size_t i = 0; i < batch; i++) {
        c.row_idx = i;
        go_parallel_rows(lin_f32_rows, &c, out_f);
    }
    return GO_OK;
}

/* ------------------------------------------------------------------------ */
/* a3: Q8 activations (int4_matmul.zig:335-420)                             */
/* ------------------------------------------------------------------------ */
/* Per activation group: scale = max|x| / 127; q = clamp(@round(x * (1/scale)),
 * -127, 127); an all-zero group stores scale 0 and q = 0 (:380-398). */
int go_q8_quantize(const float *x, size_t in_f, size_t ag, int8_t *q, float *scales) {
    if (ag == 0) return GO_SHAPE_MISMATCH;
    size_t groups = ceil_div(in_f, ag);
    for (size_t g = 0; g < groups; g++) {
        size_t start = g * ag, end = start + ag < in_f ? start + ag : in_f;
        float max_abs = 0;
        for (size_t i = start; i < end; i++) {
            float a = fabsf(x[i]);
            max_abs = a > max_abs ? a : max_abs;
        }
        float scale = max_abs / 127.0f;
        scales[g] = scale;
        if (scale == 0) {
            memset(q + start, 0, end - start);
        } else {
            float inv = 1.0f / scale;
            for (size_t i = start; i < end; i++) {
                int32_t qi = (int32_t)zig_round(x[i] * inv);
                if (qi < -127) qi = -127;
                if (qi > 127) qi = 127;
                q[i] = (int8_t)qi;
            }
        }
    }
    return GO_OK;
}

typedef struct {
    const int8_t *q; const float *as; const uint8_t *packed; const float *ws;
    const float *bias; float *out; size_t out_f, in_f, gs, ag;
} q8_ctx;

static void lin_q8_rows(void *p, size_t r0, size_t r1) {
    q8_ctx *c = (q8_ctx *)p;
    const size_t groups = ceil_div(c->in_f, c->gs);
    for (size_t row = r0; row < r1; row++) {
        float acc = c->bias ? c->bias[row] : 0.0f;
        const size_t row_start = row * c->in_f;
        for (size_t og = 0; og < groups; og++) {
            size_t start = og * c->gs;
            size_t end = start + c->gs < c->in_f ? start + c->gs : c->in_f;
            int32_t dot = 0;
            for (size_t col = start; col < end; col++) {
                size_t idx = row_start + col;
                uint8_t pb = c->packed[idx / 2];
                int32_t nib = (idx & 1) == 0 ? (pb & 0x0f) : (pb >> 4);
                dot += (nib - 7) * (int32_t)c->q[col];
            }
            /* (f32(dot) * w_scale) * a_scale, then acc += (:413) */
            float t = (float)dot * c->ws[(row_start + start) / c->gs];
            t = t * c->as[start / c->ag];
            acc += t;
        }
        c->out[row] = acc;
    }
}

int go_linear_int4_q8(const float *x, size_t batch, const uint8_t *packed,
                      const float *scales, const float *bias, float *out,
                      size_t out_f, size_t in_f, size_t group_size) {
    if (group_size == 0 || in_f % group_size != 0) return GO_SHAPE_MISMATCH;
    const size_t ag = group_size == 8 ? 32 : group_size;
    const size_t agroups = ceil_div(in_f, ag);
    if (in_f > 16384 || agroups > 2048)
        return go_linear_int4_f32(x, batch, packed, scales, bias, out, out_f, in_f, group_size);
    int8_t *q = (int8_t *)malloc(in_f);
    float *as = (float *)malloc(agroups * sizeof(float));
    if (!q || !as) { free(q); free(as); return GO_NO_MEMORY; }
    for (size_t i = 0; i < batch; i++) {
        go_q8_quantize(x + i * in_f, in_f, ag, q, as);
        q8_ctx c = {q, as, packed, scales, bias, out + i * out_f, out_f, in_f, group_size, ag};
        go_parallel_rows(lin_q8_rows, &c, out_f);
    }
    free(q);
    free(as);
    return GO_OK;
}

int go_linear_int4_weight_q8(const float *x, size_t batch, const uint8_t *packed,
                             const float *scales, const float *bias, float *out,
                             size_t out_f, size_t in_f, size_t group_size) {
    /* int4_matmul.zig:461-463: the vocabulary head (out_f > 65536) on a
     * row-major matrix takes linearInt4Weight (f32 activations). */
    if (out_f > 65536)
        return go_linear_int4_f32(x, batch, packed, scales, bias, out, out_f, in_f, group_size);
    return go_linear_int4_q8(x, batch, packed, scales, bias, out, out_f, in_f, group_size);
}

/* ------------------------------------------------------------------------ */
/* a5: rmsNormF32 (kernels.zig:141-220)                                      */
/* ------------------------------------------------------------------------ */
int go_rmsnorm(const float *x, size_t batch, size_t dim, const float *w,
               float eps, float *out) {
    for (size_t i = 0; i < batch; i++) {
        const float *row = x + i * dim;
        float sv[16] = {0};
        size_t k = 0, vec_end = dim - (dim % 16);
        for (; k < vec_end; k += 16)
            for (int j = 0; j < 16; j++) sv[j] += row[k + j] * row[k + j];
        float sum_sq = sv[0];
        for (int j = 1; j < 16; j++) sum_sq += sv[j];
        for (; k < dim; k++) sum_sq += row[k] * row[k];
        float rms = sqrtf(sum_sq / (float)dim + eps);
        float inv = 1.0f / rms;
        for (k = 0; k < dim; k++) {
            float t = row[k] * inv;
            out[i * dim + k] = t * w[k];
        }
    }
    return GO_OK;
}

/* a8: siluMulF32 (kernels.zig:465-520): g * (1 / (1 + exp(-g))) * u. */
void go_silu_mul(const float *g, const float *u, float *out, size_t n) {
    for (size_t k = 0; k < n; k++) {
        float sig = 1.0f / (1.0f + expf(-g[k]));
        float t = g[k] * sig;
        out[k] = t * u[k];
    }
}

/* ------------------------------------------------------------------------ */
/* a6: RoPE (generate.zig:784-832; forward.zig:353-377)                      */
/* ------------------------------------------------------------------------ */
void go_rope_table(size_t positions, size_t head_dim, float theta,
                   float *cos_t, float *sin_t) {
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < positions; pos++)
        for (size_t pair = 0; pair < half; pair++) {
            float exponent = (float)(2 * pair) / (float)head_dim;
            float freq = 1.0f / powf(theta, exponent);
            float angle = (float)pos * freq;
            cos_t[pos * half + pair] = cosf(angle);
            sin_t[pos * half + pair] = sinf(angle);
        }
}

void go_rope_apply(const float *cos_t, const float *sin_t, size_t half,
                   float *row, size_t pos, size_t num_heads, size_t head_dim) {
    if (head_dim / 2 != half) return;
    size_t f = pos * half;
    for (size_t h = 0; h < num_heads; h++) {
        size_t off = h * head_dim;
        for (size_t pair = 0; pair < half; pair++) {
            size_t i0 = off + pair, i1 = off + pair + half;
            float x0 = row[i0], x1 = row[i1];
            float c = cos_t[f + pair], s = sin_t[f + pair];
            float a = x0 * c, b = x1 * s, d = x0 * s, e = x1 * c;
            row[i0] = a - b;
            row[i1] = d + e;
        }
    }
}

void go_rope_apply_direct(float *row, size_t pos, size_t num_heads,
                          size_t head_dim, float theta) {
    size_t half = head_dim / 2;
    for (size_t h = 0; h < num_heads; h++) {
        size_t off = h * head_dim;
        for (size_t kp = 0; kp < half; kp++) {
            float freq = 1.0f / powf(theta, (float)(2 * kp) / (float)head_dim);
            float angle = (float)pos * freq;
            float c = cosf(angle), s = sinf(angle);
            size_t i0 = off + kp, i1 = off + kp + half;
            float x0 = row[i0], x1 = row[i1];
            float a = x0 * c, b = x1 * s, d = x0 * s, e = x1 * c;
            row[i0] = a - b;
            row[i1] = d + e;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* a7: attention (forward.zig:478-533; paged_attention.zig:108-210)          */
/* ------------------------------------------------------------------------ */
typedef struct {
    const void *base;      /* contiguous f32 [kv_seq, kv_dim] or page pool */
    int paged, fp16;
    const int32_t *page_table;
    size_t layer, num_layers, kv_dim;
    int value;             /* 0 = K, 1 = V */
} kv_view;

/* Element pointer math for one K or V row (paged_kv_cache.zig:1421-1444). */
static void kv_row(const kv_view *v, size_t pos, size_t off, size_t n, float *dst) {
    if (!v->paged) {
        const float *src = (const float *)v->base + pos * v->kv_dim + off;
        memcpy(dst, src, n * sizeof(float));
        return;
    }
    size_t page = (size_t)v->page_table[pos / 16], row = pos % 16;
    size_t elem = (((page * v->num_layers + v->layer) * 2 + (size_t)v->value) * 16 + row) * v->kv_dim + off;
    if (v->fp16) {
        const uint16_t *src = (const uint16_t *)v->base + elem;
        for (size_t i = 0; i < n; i++) dst[i] = go_f16_to_f32(src[i]);
    } else {
        memcpy(dst, (const float *)v->base + elem, n * sizeof(float));
    }
}

static int attention_core(const float *q, size_t q_seq, const kv_view *kv,
                          const kv_view *vv, size_t kv_seq, float *out,
                          size_t num_heads, size_t num_kv_heads, size_t head_dim) {
    size_t eff_kv = num_kv_heads == 0 ? num_heads : num_kv_heads;
    if (num_heads == 0 || head_dim == 0 || eff_kv > num_heads || num_heads % eff_kv)
        return GO_SHAPE_MISMATCH;
    if (q_seq == 0 || q_seq > kv_seq) return GO_SHAPE_MISMATCH;
    const size_t q_dim = num_heads * head_dim;
    const size_t group = num_heads / eff_kv;
    const size_t query_start = kv_seq - q_seq;
    const float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = (float *)malloc(kv_seq * sizeof(float));
    float *krow = (float *)malloc(head_dim * sizeof(float));
    if (!scores || !krow) { free(scores); free(krow); return GO_NO_MEMORY; }
    for (size_t h = 0; h < num_heads; h++) {
        const size_t q_head_off = h * head_dim;
        const size_t kv_head_off = (h / group) * head_dim;
        for (size_t i = 0; i < q_seq; i++) {
            const float *qh = q + i * q_dim + q_head_off;
            size_t upto = query_start + i;
            if (upto > kv_seq - 1) upto = kv_seq - 1;
            float max_score = -INFINITY;
            for (size_t j = 0; j <= upto; j++) {
                kv_row(kv, j, kv_head_off, head_dim, krow);
                float dv[8] = {0, 0, 0, 0, 0, 0, 0, 0};
                size_t d = 0, vec_end = head_dim - (head_dim % 8);
                for (; d < vec_end; d += 8)
                    for (int t = 0; t < 8; t++) dv[t] += qh[d + t] * krow[d + t];
                float dot = reduce8(dv);
                for (; d < head_dim; d++) dot += qh[d] * krow[d];
                scores[j] = dot * scale;
                if (scores[j] > max_score) max_score = scores[j];
            }
            float sum_exp = 0;
            for (size_t j = 0; j <= upto; j++) {
                scores[j] = expf(scores[j] - max_score);
                sum_exp += scores[j];
            }
            const float inv = 1.0f / sum_exp;
            float *oh = out + i * q_dim + q_head_off;
            for (size_t d = 0; d < head_dim; d++) oh[d] = 0;
            for (size_t j = 0; j <= upto; j++) {
                const float wgt = scores[j] * inv;
                kv_row(vv, j, kv_head_off, head_dim, krow);
                for (size_t d = 0; d < head_dim; d++) oh[d] += wgt * krow[d];
            }
        }
    }
    free(scores);
    free(krow);
    return GO_OK;
}

int go_attention(const float *q, size_t q_seq, const float *k, const float *v,
                 size_t kv_seq, float *out, size_t num_heads,
                 size_t num_kv_heads, size_t head_dim) {
    size_t eff_kv = num_kv_heads == 0 ? num_heads : num_kv_heads;
    kv_view kk = {k, 0, 0, NULL, 0, 1, eff_kv * head_dim, 0};
    kv_view vv = {v, 0, 0, NULL, 0, 1, eff_kv * head_dim, 1};
    return attention_core(q, q_seq, &kk, &vv, kv_seq, out, num_heads, num_kv_heads, head_dim);
}

int go_attention_paged(const float *q, size_t q_seq, const void *pool, int kv_fp16,
                       const int32_t *page_table, size_t kv_seq, size_t layer,
                       size_t num_layers, float *out, size_t num_heads,
                       size_t num_kv_heads, size_t head_dim) {
    size_t eff_kv = num_kv_heads == 0 ? num_heads : num_kv_heads;
    if (layer >= num_layers) return GO_SHAPE_MISMATCH;
    kv_view kk = {pool, 1, kv_fp16, page_table, layer, num_layers, eff_kv * head_dim, 0};
    kv_view vv = kk;
    vv.value = 1;
    return attention_core(q, q_seq, &kk, &vv, kv_seq, out, num_heads, num_kv_heads, head_dim);
}

/* ------------------------------------------------------------------------ */
/* a12/a13: argmax                                                          */
/* ------------------------------------------------------------------------ */
/* sampling.zig:194-206: first strict maximum; a NaN at index 0 sticks. */
size_t go_argmax(const float *v, size_t n) {
    size_t bi = 0;
    float bv = v[0];
    for (size_t i = 1; i < n; i++)
        if (v[i] > bv) { bv = v[i]; bi = i; }
    return bi;
}

/* sampling.zig:55-105 */
int go_argmax_eligible(const float *logits, size_t n, const uint64_t *words,
                       size_t word_count, size_t *index_out, size_t *rows_out) {
    size_t wc = n / 64 + (n % 64 != 0);
    if (wc == 0 || word_count != wc) return GO_INVALID_MASK;
    if (n % 64 != 0) {
        uint64_t valid_tail = (((uint64_t)1) << (n % 64)) - 1;
        if (words[wc - 1] & ~valid_tail) return GO_INVALID_MASK;
    }
    size_t rows = 0;
    for (size_t w = 0; w < wc; w++) rows += (size_t)__builtin_popcountll(words[w]);
    if (rows == 0 || rows > n) return GO_INVALID_MASK;
    size_t best_i = 0;
    float best_v = 0;
    int have = 0;
    for (size_t w = 0; w < wc; w++) {
        uint64_t rem = words[w];
        while (rem) {
            size_t bit = (size_t)__builtin_ctzll(rem);
            size_t ti = w * 64 + bit;
            float val = logits[ti];
            if (isnan(val)) return GO_ELIGIBLE_NAN;
            if (!have || val > best_v) { best_i = ti; best_v = val; have = 1; }
            rem &= rem - 1;
        }
    }
    *index_out = best_i;
    *rows_out = rows;
    return GO_OK;
}

/* ------------------------------------------------------------------------ */
/* a9-a11: one layer and the greedy token loop                               */
/* ------------------------------------------------------------------------ */
static int project(const go_model *m, const float *x, go_int4_weight w, const float *bias,
                   float *out, size_t out_f, size_t in_f, size_t gs) {
    /* generate.zig:3550-3596 linearInt4Decode with no pool: the .q8 activation
     * (the default, generate.zig:925; prepared_text_session.zig:81-105
     * num_threads = 1) -> linearInt4WeightQ8 with its x86 dispatch; .f32 ->
     * linearInt4Weight (int4_matmul.zig:2957-2981) -> linearInt4OnTheFly */
    if (m->int4_activation_f32)
        return go_linear_int4_f32(x, 1, w.packed, w.scales, bias, out, out_f, in_f, gs);
    return go_linear_int4_weight_q8(x, 1, w.packed, w.scales, bias, out, out_f, in_f, gs);
}

int go_forward_layer(const go_model *m, size_t li, const float *x_row,
                     float *k_cache, float *v_cache, size_t pos,
                     const float *rope_cos, const float *rope_sin, float *out_row) {
    const go_layer *L = &m->layers[li];
    const size_t dim = m->dim, hidden = m->hidden_dim, hd = m->head_dim;
    const size_t kv_dim = (size_t)m->num_kv_heads * hd, gs = m->group_size;
    float *buf = (float *)malloc(sizeof(float) * (dim * 6 + kv_dim * 2 + hidden * 3));
    if (!buf) return GO_NO_MEMORY;
    float *h_norm = buf, *q = h_norm + dim, *attn = q + dim, *proj = attn + dim;
    float *h = proj + dim, *mlp_norm = h + dim, *k = mlp_norm + dim, *v = k + kv_dim;
    float *gate = v + kv_dim, *up = gate + hidden, *act = up + hidden;
    int rc;
    /* generate.zig:1561 */
    go_rmsnorm(x_row, 1, dim, L->input_norm, m->rms_eps, h_norm);
    /* Q, K, V projections (:1668-1700) */
    if ((rc = project(m, h_norm, L->wq, L->bq, q, dim, dim, gs))) goto done;
    if ((rc = project(m, h_norm, L->wk, L->bk, k, kv_dim, dim, gs))) goto done;
    if ((rc = project(m, h_norm, L->wv, L->bv, v, kv_dim, dim, gs))) goto done;
    /* RoPE on k, append row, RoPE on q (:1712-1735) */
    go_rope_apply(rope_cos, rope_sin, hd / 2, k, pos, m->num_kv_heads, hd);
    if (m->kv_fp16)
        for (size_t i = 0; i < kv_dim; i++) {
            k[i] = go_f16_to_f32(go_f32_to_f16(k[i]));
            v[i] = go_f16_to_f32(go_f32_to_f16(v[i]));
        }
    memcpy(k_cache + pos * kv_dim, k, kv_dim * sizeof(float));
    memcpy(v_cache + pos * kv_dim, v, kv_dim * sizeof(float));
    go_rope_apply(rope_cos, rope_sin, hd / 2, q, pos, m->num_heads, hd);
    /* serial attention over filled + 1 rows (:1757) */
    if ((rc = go_attention(q, 1, k_cache, v_cache, pos + 1, attn, m->num_heads,
                           m->num_kv_heads, hd))) goto done;
    /* O projection, residual, post-attention norm (:1763-1768) */
    if ((rc = project(m, attn, L->wo, NULL, proj, dim, dim, gs))) goto done;
    for (size_t i = 0; i < dim; i++) h[i] = x_row[i] + proj[i];
    go_rmsnorm(h, 1, dim, L->post_attn_norm, m->rms_eps, mlp_norm);
    /* gate, up, SiLU * up, down, residual (:1844-1965, x86 branch) */
    if ((rc = project(m, mlp_norm, L->w_gate, NULL, gate, hidden, dim, gs))) goto done;
    if ((rc = project(m, mlp_norm, L->w_up, NULL, up, hidden, dim, gs))) goto done;
    go_silu_mul(gate, up, act, hidden);
    if ((rc = project(m, act, L->w_down, NULL, proj, dim, hidden, gs))) goto done;
    for (size_t i = 0; i < dim; i++) out_row[i] = h[i] + proj[i];
done:
    free(buf);
    return rc;
}

static void hash_u64(go_sha256_ctx *c, uint64_t v) {
    uint8_t b[8];
    for (int i = 0; i < 8; i++) b[i] = (uint8_t)(v >> (8 * i));
    go_sha256_update(c, b, 8);
}
static void hash_u32(go_sha256_ctx *c, uint32_t v) {
    uint8_t b[4];
    for (int i = 0; i < 4; i++) b[i] = (uint8_t)(v >> (8 * i));
    go_sha256_update(c, b, 4);
}

static int generate_impl(const go_model *m, const uint32_t *prompt, size_t prompt_len,
                         size_t max_new, const uint32_t *forced, uint32_t *tokens_out,
                         const int32_t *logits_steps, size_t n_logits_steps, float *logits_out,
                         uint8_t *kv_sha256_out, uint8_t *output_sha256_out) {
    if (prompt_len == 0 || max_new == 0) return GO_SHAPE_MISMATCH;
    const size_t dim = m->dim, L = m->num_layers, hd = m->head_dim;
    const size_t kv_dim = (size_t)m->num_kv_heads * hd, V = m->vocab_size;
    const size_t max_seq = prompt_len + max_new - 1;
    for (size_t i = 0; i < prompt_len; i++)
        if (prompt[i] >= V) return GO_SHAPE_MISMATCH;
    float *kc = (float *)calloc(L * max_seq * kv_dim, sizeof(float));
    float *vc = (float *)calloc(L * max_seq * kv_dim, sizeof(float));
    float *rc_t = (float *)malloc(max_seq * (hd / 2) * sizeof(float));
    float *rs_t = (float *)malloc(max_seq * (hd / 2) * sizeof(float));
    float *x = (float *)malloc(dim * sizeof(float)), *nx = (float *)malloc(dim * sizeof(float));
    float *fh = (float *)malloc(dim * sizeof(float));
    float *logits = (float *)malloc(V * sizeof(float));
    int rc = GO_OK;
    if (!kc || !vc || !rc_t || !rs_t || !x || !nx || !fh || !logits) { rc = GO_NO_MEMORY; goto out; }
    go_rope_table(max_seq, hd, m->rope_theta, rc_t, rs_t);
    size_t pos = 0;
    uint32_t next = 0;
    for (size_t step = 0; step < max_new; step++) {
        /* prefill: tokens of the prompt one at a time (generate.zig:5080-5118);
         * decode: the previously generated token (:5366-5450). */
        size_t n_in = step == 0 ? prompt_len : 1;
        for (size_t t = 0; t < n_in; t++) {
            uint32_t tok = step == 0 ? prompt[t] : next;
            memcpy(x, m->token_embedding + (size_t)tok * dim, dim * sizeof(float));
            for (size_t l = 0; l < L; l++) {
                rc = go_forward_layer(m, l, x, kc + l * max_seq * kv_dim,
                                      vc + l * max_seq * kv_dim, pos, rc_t, rs_t, nx);
                if (rc) goto out;
                memcpy(x, nx, dim * sizeof(float));
            }
            pos++;
        }
        go_rmsnorm(x, 1, dim, m->final_norm, m->rms_eps, fh);
        rc = project(m, fh, m->lm_head, NULL, logits, V, dim, m->group_size);
        if (rc) goto out;
        for (size_t i = 0; i < n_logits_steps; i++)
            if (logits_steps[i] == (int32_t)step)
                memcpy(logits_out + i * V, logits, V * sizeof(float));
        next = (uint32_t)go_argmax(logits, V);
        tokens_out[step] = next;
        if (forced && step + 1 < max_new) next = forced[step];
    }
    if (kv_sha256_out) go_logical_kv_sha256(kc, vc, L, max_seq, kv_dim, pos, kv_sha256_out);
    if (output_sha256_out) go_token_sequence_sha256(tokens_out, max_new, output_sha256_out);
out:
    free(kc); free(vc); free(rc_t); free(rs_t); free(x); free(nx); free(fh); free(logits);
    return rc;
}

int go_generate(const go_model *m, const uint32_t *prompt, size_t prompt_len,
                size_t max_new, uint32_t *tokens_out, const int32_t *logits_steps,
                size_t n_logits_steps, float *logits_out, uint8_t *kv_sha256_out,
                uint8_t *output_sha256_out) {
    return generate_impl(m, prompt, prompt_len, max_new, NULL, tokens_out, logits_steps,
                         n_logits_steps, logits_out, kv_sha256_out, output_sha256_out);
}

int go_generate_forced(const go_model *m, const uint32_t *prompt, size_t prompt_len,
                       size_t max_new, const uint32_t *forced, uint32_t *tokens_out,
                       const int32_t *logits_steps, size_t n_logits_steps, float *logits_out) {
    if (!forced) return GO_SHAPE_MISMATCH;
    for (size_t i = 0; i + 1 < max_new; i++)
        if (forced[i] >= m->vocab_size) return GO_SHAPE_MISMATCH;
    return generate_impl(m, prompt, prompt_len, max_new, forced, tokens_out, logits_steps,
                         n_logits_steps, logits_out, NULL, NULL);
}

/* ------------------------------------------------------------------------ */
/* SHA-256 (FIPS 180-4)                                                      */
/* ------------------------------------------------------------------------ */
static const uint32_t K256[64] = {
    0x428a2f98, 0x71374491, 0xb5c0fbcf, 0xe9b5dba5, 0x3956c25b, 0x59f111f1, 0x923f82a4, 0xab1c5ed5,
    0xd807aa98, 0x12835b01, 0x243185be, 0x550c7dc3, 0x72be5d74, 0x80deb1fe, 0x9bdc06a7, 0xc19bf174,
    0xe49b69c1, 0xefbe4786, 0x0fc19dc6, 0x240ca1cc, 0x2de92c6f, 0x4a7484aa, 0x5cb0a9dc, 0x76f988da,
    0x983e5152, 0xa831c66d, 0xb00327c8, 0xbf597fc7, 0xc6e00bf3, 0xd5a79147, 0x06ca6351, 0x14292967,
    0x27b70a85, 0x2e1b2138, 0x4d2c6dfc, 0x53380d13, 0x650a7354, 0x766a0abb, 0x81c2c92e, 0x92722c85,
    0xa2bfe8a1, 0xa81a664b, 0xc24b8b70, 0xc76c51a3, 0xd192e819, 0xd6990624, 0xf40e3585, 0x106aa070,
    0x19a4c116, 0x1e376c08, 0x2748774c, 0x34b0bcb5, 0x391c0cb3, 0x4ed8aa4a, 0x5b9cca4f, 0x682e6ff3,
    0x748f82ee, 0x78a5636f, 0x84c87814, 0x8cc70208, 0x90befffa, 0xa4506ceb, 0xbef9a3f7, 0xc67178f2};

#define ROR(x, n) (((x) >> (n)) | ((x) << (32 - (n))))
static void sha_block(uint32_t h[8], const uint8_t *p) {
    uint32_t w[64];
    for (int i = 0; i < 16; i++)
        w[i] = ((uint32_t)p[4 * i] << 24) | ((uint32_t)p[4 * i + 1] << 16) |
               ((uint32_t)p[4 * i + 2] << 8) | p[4 * i + 3];
    for (int i = 16; i < 64; i++) {
        uint32_t s0 = ROR(w[i - 15], 7) ^ ROR(w[i - 15], 18) ^ (w[i - 15] >> 3);
        uint32_t s1 = ROR(w[i - 2], 17) ^ ROR(w[i - 2], 19) ^ (w[i - 2] >> 10);
        w[i] = w[i - 16] + s0 + w[i - 7] + s1;
    }
    uint32_t a = h[0], b = h[1], c = h[2], d = h[3], e = h[4], f = h[5], g = h[6], hh = h[7];
    for (int i = 0; i < 64; i++) {
        uint32_t S1 = ROR(e, 6) ^ ROR(e, 11) ^ ROR(e, 25);
        uint32_t ch = (e & f) ^ (~e & g);
        uint32_t t1 = hh + S1 + ch + K256[i] + w[i];
        uint32_t S0 = ROR(a, 2) ^ ROR(a, 13) ^ ROR(a, 22);
        uint32_t mj = (a & b) ^ (a & c) ^ (b & c);
        uint32_t t2 = S0 + mj;
        hh = g; g = f; f = e; e = d + t1; d = c; c = b; b = a; a = t1 + t2;
    }
    h[0] += a; h[1] += b; h[2] += c; h[3] += d; h[4] += e; h[5] += f; h[6] += g; h[7] += hh;
}
void go_sha256_init(go_sha256_ctx *c) {
    static const uint32_t iv[8] = {0x6a09e667, 0xbb67ae85, 0x3c6ef372, 0xa54ff53a,
                                   0x510e527f, 0x9b05688c, 0x1f83d9ab, 0x5be0cd19};
    memcpy(c->h, iv, sizeof iv);
    c->len = 0;
    c->fill = 0;
}
void go_sha256_update(go_sha256_ctx *c, const void *data, size_t len) {
    const uint8_t *p = (const uint8_t *)data;
    c->len += len;
    while (len) {
        size_t take = 64 - c->fill < len ? 64 - c->fill : len;
        memcpy(c->buf + c->fill, p, take);
        c->fill += take; p += take; len -= take;
        if (c->fill == 64) { sha_block(c->h, c->buf); c->fill = 0; }
    }
}
void go_sha256_final(go_sha256_ctx *c, uint8_t out[32]) {
    uint64_t bits = c->len * 8;
    uint8_t pad = 0x80, z = 0;
    go_sha256_update(c, &pad, 1);
    while (c->fill != 56) go_sha256_update(c, &z, 1);
    uint8_t lb[8];
    for (int i = 0; i < 8; i++) lb[i] = (uint8_t)(bits >> (56 - 8 * i));
    go_sha256_update(c, lb, 8);
    for (int i = 0; i < 8; i++) {
        out[4 * i] = (uint8_t)(c->h[i] >> 24); out[4 * i + 1] = (uint8_t)(c->h[i] >> 16);
        out[4 * i + 2] = (uint8_t)(c->h[i] >> 8); out[4 * i + 3] = (uint8_t)c->h[i];
    }
}
void go_sha256(const uint8_t *data, size_t len, uint8_t out[32]) {
    go_sha256_ctx c;
    go_sha256_init(&c);
    go_sha256_update(&c, data, len);
    go_sha256_final(&c, out);
}

/* ------------------------------------------------------------------------ */
/* paged KV geometry and ownership digests                                   */
/* ------------------------------------------------------------------------ */
int go_paged_capacity_ledger(uint64_t L, uint64_t dim, uint64_t max_seq, go_capacity_ledger *o) {
    if (L == 0 || dim == 0 || max_seq == 0) return GO_SHAPE_MISMATCH;
    __uint128_t pc = max_seq / 16 + (max_seq % 16 != 0);
    __uint128_t rounded = pc * 16;
    __uint128_t page_elements = (__uint128_t)L * 2 * 16 * dim;
    __uint128_t payload = page_elements * 4;
    __uint128_t tensor = pc * payload;
    __uint128_t map = pc * 16;               /* sizeof(PageEntry) == 16 */
    __uint128_t alloc = tensor + map;
    __uint128_t contig = (__uint128_t)L * 2 * max_seq * dim * 4 + (__uint128_t)L * 2 * 16;
    if (alloc >> 64 || contig >> 64 || payload >> 64) return GO_SHAPE_MISMATCH;
    o->page_count_capacity = (uint64_t)pc;
    o->page_elements = (uint64_t)page_elements;
    o->page_payload_bytes = (uint64_t)payload;
    o->tensor_capacity_bytes = (uint64_t)tensor;
    o->page_map_bytes = (uint64_t)map;
    o->allocation_capacity_bytes = (uint64_t)alloc;
    o->contiguous_counterfactual_bytes = (uint64_t)contig;
    o->capacity_reclaimed_bytes = contig > alloc ? (uint64_t)(contig - alloc) : 0;
    o->capacity_overhead_bytes = alloc > contig ? (uint64_t)(alloc - contig) : 0;
    o->padded_positions = (uint64_t)(rounded - max_seq);
    return GO_OK;
}

void go_paged_empty_ownership_digest(uint64_t inst, uint64_t L, uint64_t dim,
                                     uint64_t max_seq, uint8_t out[32]) {
    go_sha256_ctx c;
    go_sha256_init(&c);
    go_sha256_update(&c, "glacier-paged-kv-ownership-v1\0", 30);
    hash_u64(&c, inst);
    hash_u64(&c, L);
    hash_u64(&c, dim);
    hash_u64(&c, max_seq);
    hash_u64(&c, 16);
    go_sha256_final(&c, out);
}

void go_paged_append_ownership_digest(const uint8_t before[32], uint64_t inst,
                                      uint64_t logical_page, uint64_t gen, uint8_t out[32]) {
    go_sha256_ctx c;
    go_sha256_init(&c);
    go_sha256_update(&c, "glacier-paged-kv-root-append-v1\0", 32);
    go_sha256_update(&c, before, 32);
    hash_u64(&c, 0x4750524600000001ull); /* page_ref_abi */
    hash_u64(&c, inst);
    hash_u64(&c, logical_page);
    hash_u64(&c, gen);
    go_sha256_final(&c, out);
}

/* logicalKvPrefixSha256 (generate.zig:3150-3172) over the committed prefix:
 * domain, layer count, kv_dim and positions (u64 LE), then per layer the K
 * rows and then the V rows of positions [0, pos) as f32 bit patterns. */
void go_logical_kv_sha256(const float *k, const float *v, size_t L, size_t max_seq, size_t kv_dim,
                          size_t pos, uint8_t out[32]) {
    go_sha256_ctx c;
    go_sha256_init(&c);
    go_sha256_update(&c, "glacier-logical-kv-state-v1\0", 28);
    hash_u64(&c, L);
    hash_u64(&c, kv_dim);
    hash_u64(&c, pos);
    for (size_t l = 0; l < L; l++) {
        const float *kl = k + l * max_seq * kv_dim, *vl = v + l * max_seq * kv_dim;
        for (size_t i = 0; i < pos * kv_dim; i++) { uint32_t b; memcpy(&b, &kl[i], 4); hash_u32(&c, b); }
        for (size_t i = 0; i < pos * kv_dim; i++) { uint32_t b; memcpy(&b, &vl[i], 4); hash_u32(&c, b); }
    }
    go_sha256_final(&c, out);
}

void go_token_sequence_sha256(const uint32_t *tokens, size_t n, uint8_t out[32]) {
    go_sha256_ctx c;
    go_sha256_init(&c);
    go_sha256_update(&c, "glacier-output-token-state-v1\0", 30);
    hash_u64(&c, n);
    for (size_t i = 0; i < n; i++) hash_u32(&c, tokens[i]);
    go_sha256_final(&c, out);
}

/* SplitMix64 (Steele, Lea, Flood 2014) feeding Xoshiro256 (Blackman, Vigna). */
void go_xoshiro256_init(uint64_t seed, uint64_t s[4]) {
    uint64_t st = seed;
    for (int i = 0; i < 4; i++) {
        st += 0x9e3779b97f4a7c15ull;
        uint64_t z = st;
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        s[i] = z ^ (z >> 31);
    }
}
