/*
 * fw_cpu — CPU restatement of forword.c's forward.  TEST INFRASTRUCTURE:
 * only the tests, the smoke check and the benchmark's CPU-baseline leg use it.
 *
 * Build with contraction off (-ffp-contract=off): every a*b+c below that is not
 * an explicit fmaf() must round twice, as in the reference's ISO-C build.
 * Each function cites the reference code whose operation order it follows.
 */
#define _POSIX_C_SOURCE 200809L
#include "fw_cpu.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

/* ── scalar helpers ──────────────────────────────────────────────────────── */

/* half_to_float (quant_matvec.c:22-50): exact, subnormals normalised by shifting. */
float fwc_half_to_float(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 31u, mant = h & 1023u, bits;
    if (ex == 0) {
        if (mant == 0) bits = sign;
        else {
            int e = -14;
            while (!(mant & 1024u)) { mant <<= 1; --e; }
            bits = sign | ((uint32_t)(e + 127) << 23) | ((mant & 1023u) << 13);
        }
    } else if (ex == 31) bits = sign | 0x7f800000u | (mant << 13);
    else bits = sign | ((ex + 112u) << 23) | (mant << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

void fwc_half_to_float_n(const uint16_t *h, float *out, size_t n)
{
    for (size_t i = 0; i < n; i++) out[i] = fwc_half_to_float(h[i]);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/*
 * simd_dot_f32, AVX2+FMA branch (simd.h:27-67) plus the scalar tail
 * (simd.h:151-153): two 8-lane FMA accumulators over 16-wide steps, merged,
 * one more 8-lane FMA step per remaining 8, then the horizontal tree
 * (lo128+hi128, movehl, shuffle) and `0.0f + tree`.
 */
float fwc_dot_f32(const float *a, const float *b, size_t n)
{
    size_t i = 0;
    float sum = 0.0f, acc0[8] = { 0 }, acc1[8] = { 0 };
    for (; i + 16 <= n; i += 16) {
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
        for (int l = 0; l < 8; l++) acc1[l] = fmaf(a[i + 8 + l], b[i + 8 + l], acc1[l]);
    }
    for (int l = 0; l < 8; l++) acc0[l] = acc0[l] + acc1[l];
    for (; i + 8 <= n; i += 8)
        for (int l = 0; l < 8; l++) acc0[l] = fmaf(a[i + l], b[i + l], acc0[l]);
    float s0 = acc0[0] + acc0[4], s1 = acc0[1] + acc0[5], s2 = acc0[2] + acc0[6], s3 = acc0[3] + acc0[7];
    float r = (s0 + s2) + (s1 + s3);
    sum += r;
    for (; i < n; i++) sum += a[i] * b[i];
    return sum;
}

/* dot_q8_0_block, AVX2+FMA branch (quant_matvec.c:65-114). */
static float dot_q8_0(const uint8_t *p, const float *x)
{
    float d = fwc_half_to_float(rd16(p));
    const int8_t *qs = (const int8_t *)(p + 2);
    float prod[32], s[8];
    for (int j = 0; j < 32; j++) prod[j] = fmaf((float)qs[j], x[j], 0.0f);
    for (int l = 0; l < 8; l++) s[l] = (prod[l] + prod[8 + l]) + (prod[16 + l] + prod[24 + l]);
    float t0 = s[0] + s[4], t1 = s[1] + s[5], t2 = s[2] + s[6], t3 = s[3] + s[7];
    return d * ((t0 + t2) + (t1 + t3));
}

/* Q5_0 block decode (decode_small_block, quant_matvec.c:197-213; linear.c:40-56). */
static void decode_q5_0(const uint8_t *p, float *w)
{
    float d = fwc_half_to_float(rd16(p));
    const uint8_t *qh = p + 2, *qs = p + 6;
    for (int j = 0; j < 16; j++) {
        int h0 = (qh[j / 8] >> (j % 8)) & 1;
        int h1 = (qh[(j + 16) / 8] >> ((j + 16) % 8)) & 1;
        int q0 = (qs[j] & 15) | (h0 << 4), q1 = (qs[j] >> 4) | (h1 << 4);
        w[j] = d * (float)(q0 - 16);
        w[j + 16] = d * (float)(q1 - 16);
    }
}

/*
 * Q4_0 block decode.  Not in the reference (quant_matvec.c:52-62 has no case);
 * written from the GGUF block definition in the shape of the reference's other
 * 32-value decoder: w_j = d*(float)(q_j-8), q_j = qs[j]&15, q_{j+16} = qs[j]>>4.
 */
static void decode_q4_0(const uint8_t *p, float *w)
{
    float d = fwc_half_to_float(rd16(p));
    const uint8_t *qs = p + 2;
    for (int j = 0; j < 16; j++) {
        w[j] = d * (float)((qs[j] & 15) - 8);
        w[j + 16] = d * (float)((qs[j] >> 4) - 8);
    }
}

/* q8_0_decode inner loop (quant.c:254-259). */
static void decode_q8_0(const uint8_t *p, float *w)
{
    float d = fwc_half_to_float(rd16(p));
    const int8_t *qs = (const int8_t *)(p + 2);
    for (int j = 0; j < 32; j++) w[j] = d * (float)qs[j];
}

/* get_scale_min_k4 (quant.c:66-85): 6-bit scale and min of group j. */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn)
{
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

/* q4_k_decode, one super-block (quant.c:87-131): y = (d*sc)*q - dmin*m, each
 * product rounded, then the difference. */
static void decode_q4_k(const uint8_t *p, float *y)
{
    const float d = fwc_half_to_float(rd16(p)), dmin = fwc_half_to_float(rd16(p + 2));
    const uint8_t *scales = p + 4, *qs = p + 16;
    for (int g = 0; g < 8; g++) {
        uint8_t sc, mn;
        scale_min_k4(g, scales, &sc, &mn);
        const float ds = d * sc, dm = dmin * mn;
        const uint8_t *q = qs + (g / 2) * 32;
        for (int i = 0; i < 32; i++) {
            const uint8_t v = (g & 1) ? (uint8_t)(q[i] >> 4) : (uint8_t)(q[i] & 15);
            y[g * 32 + i] = ds * v - dm;
        }
    }
}

/* q6_k_decode, one super-block (quant.c:133-188): y = (d*sc)*(q-32). */
static void decode_q6_k(const uint8_t *p, float *y)
{
    const uint8_t *ql = p, *qh = p + 128;
    const int8_t *sc = (const int8_t *)(p + 192);
    const float d = fwc_half_to_float(rd16(p + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t *a = ql + h * 64, *hb = qh + h * 32;
        const int8_t *s = sc + h * 8;
        float *o = y + h * 128;
        for (int l = 0; l < 32; l++) {
            const int q1 = (a[l] & 15) | ((hb[l] & 3) << 4);
            const int q2 = (a[l + 32] & 15) | (((hb[l] >> 2) & 3) << 4);
            const int q3 = (a[l] >> 4) | (((hb[l] >> 4) & 3) << 4);
            const int q4 = (a[l + 32] >> 4) | (((hb[l] >> 6) & 3) << 4);
            o[l] = d * s[l / 16] * (q1 - 32);
            o[l + 32] = d * s[l / 16 + 2] * (q2 - 32);
            o[l + 64] = d * s[l / 16 + 4] * (q3 - 32);
            o[l + 96] = d * s[l / 16 + 6] * (q4 - 32);
        }
    }
}

static size_t block_bytes(uint32_t t)
{
    switch (t) {
    case FORWORD_GGML_Q4_0: return 18;
    case FORWORD_GGML_Q5_0: return 22;
    case FORWORD_GGML_Q8_0: return 34;
    case FORWORD_GGML_Q4_K: return 144;
    case FORWORD_GGML_Q6_K: return 210;
    default: return 0;
    }
}

static size_t block_values(uint32_t t)
{
    return t == FORWORD_GGML_Q4_K || t == FORWORD_GGML_Q6_K ? 256 : 32;
}

static void decode_block(const uint8_t *p, uint32_t type, float *w)
{
    if (type == FORWORD_GGML_Q8_0) decode_q8_0(p, w);
    else if (type == FORWORD_GGML_Q5_0) decode_q5_0(p, w);
    else if (type == FORWORD_GGML_Q4_K) decode_q4_k(p, w);
    else if (type == FORWORD_GGML_Q6_K) decode_q6_k(p, w);
    else decode_q4_0(p, w);
}

int fwc_dequant(const void *blocks, size_t bytes, uint32_t type, float *out, size_t count)
{
    const size_t bb = block_bytes(type), bv = block_values(type);
    if (!blocks || !out || !bb || !bytes || bytes % bb || count % bv || bytes / bb != count / bv)
        return -1;
    const uint8_t *p = (const uint8_t *)blocks;
    for (size_t b = 0; b < bytes / bb; b++, p += bb) decode_block(p, type, out + bv * b);
    return 0;
}

/* dot_quant_block (quant_matvec.c:231-261), with Q4_0 taking the Q5_0 route:
 * decode, then simd_dot_f32 over the block's 32 or 256 values. */
static float dot_block(const uint8_t *p, uint32_t type, const float *x)
{
    float w[256];
    if (type == FORWORD_GGML_Q8_0) return dot_q8_0(p, x);
    decode_block(p, type, w);
    return fwc_dot_f32(w, x, block_values(type));
}

/* ── row-parallel driver ─────────────────────────────────────────────────── */

static int g_threads = 1;
void fwc_set_threads(int n) { g_threads = n < 1 ? 1 : (n > 256 ? 256 : n); }

typedef struct {
    void (*fn)(void *ctx, size_t r0, size_t r1);
    void *ctx;
    size_t r0, r1;
} span_t;

static void *span_run(void *a)
{
    span_t *s = (span_t *)a;
    s->fn(s->ctx, s->r0, s->r1);
    return NULL;
}

/* fn over rows [0, n) split into contiguous spans; each row's arithmetic is
 * independent of the split, so results are identical for any thread count. */
static void par_rows_min(void (*fn)(void *, size_t, size_t), void *ctx, size_t n, size_t min_rows)
{
    int nt = g_threads;
    if (nt > 1 && n >= min_rows) {
        if ((size_t)nt > n) nt = (int)n;
        span_t sp[256];
        pthread_t tid[256];
        int ok[256];
        for (int i = 0; i < nt; i++) {
            sp[i].fn = fn; sp[i].ctx = ctx;
            sp[i].r0 = n * (size_t)i / (size_t)nt;
            sp[i].r1 = n * (size_t)(i + 1) / (size_t)nt;
            ok[i] = i > 0 && pthread_create(&tid[i], NULL, span_run, &sp[i]) == 0;
        }
        span_run(&sp[0]);
        for (int i = 1; i < nt; i++) {
            if (ok[i]) pthread_join(tid[i], NULL);
            else span_run(&sp[i]);
        }
        return;
    }
    fn(ctx, 0, n);
}

static void par_rows(void (*fn)(void *, size_t, size_t), void *ctx, size_t n)
{
    par_rows_min(fn, ctx, n, 64);
}

typedef struct {
    const uint8_t *w;
    uint32_t type;
    const float *x;
    float *y;
    size_t in, bpr, bb, bv;
} qmv_t;

/* quant_matvec row loop (quant_matvec.c:293-309): sequential float sum over blocks. */
static void qmv_rows(void *c, size_t r0, size_t r1)
{
    qmv_t *m = (qmv_t *)c;
    for (size_t r = r0; r < r1; r++) {
        const uint8_t *row = m->w + r * m->bpr * m->bb;
        float sum = 0.0f;
        for (size_t b = 0; b < m->bpr; b++) sum += dot_block(row + b * m->bb, m->type, m->x + m->bv * b);
        m->y[r] = sum;
    }
}

static void f32mv_rows(void *c, size_t r0, size_t r1)
{
    qmv_t *m = (qmv_t *)c;
    const float *w = (const float *)m->w;
    for (size_t r = r0; r < r1; r++) m->y[r] = fwc_dot_f32(w + r * m->in, m->x, m->in);
}

/* quant_matvec (quant_matvec.c:263-312) incl. its argument checks (:274-289);
 * type F32 takes linear_forward's F32 branch (linear.c:173-179). */
int fwc_quant_matvec(const void *w, size_t w_size, uint32_t type, const float *x, float *y,
                     size_t in, size_t out)
{
    if (!w || !x || !y || !in || !out) return -1;
    qmv_t m = { (const uint8_t *)w, type, x, y, in, 0, 0, 0 };
    if (type == FORWORD_GGML_F32) {
        if (out > SIZE_MAX / in / 4 || w_size < out * in * 4) return -1;
        par_rows(f32mv_rows, &m, out);
        return 0;
    }
    m.bb = block_bytes(type);
    m.bv = block_values(type);
    if (!m.bb || in % m.bv) return -1;
    m.bpr = in / m.bv;
    size_t rb = m.bpr * m.bb;
    if (out > SIZE_MAX / rb || w_size < out * rb) return -1;
    par_rows(qmv_rows, &m, out);
    return 0;
}

int fwc_tensor_matvec_f32(const float *w, const float *x, float *y, size_t rows, size_t cols)
{
    if (!w || !x || !y || !rows || !cols) return -1;          /* tensor_ops.c:8-23 */
    for (size_t r = 0; r < rows; r++) y[r] = fwc_dot_f32(w + r * cols, x, cols);
    return 0;
}

/* rms_norm (norm.c:7-16): simd_sum_squares, then simd_mul and simd_scale. */
void fwc_rms_norm(const float *x, const float *w, float *out, size_t n, float eps)
{
    float ss = fwc_dot_f32(x, x, n);
    float scale = 1.0f / sqrtf((ss / (float)n) + eps);
    if (w) {
        for (size_t i = 0; i < n; i++) out[i] = x[i] * w[i];
        for (size_t i = 0; i < n; i++) out[i] = out[i] * scale;
    } else {
        for (size_t i = 0; i < n; i++) out[i] = x[i] * scale;
    }
}

/* rope_apply (rope.c:28-53). */
void fwc_rope_apply(float *qk, size_t pos, size_t n_heads, size_t hd, const float *cos_tab,
                    const float *sin_tab, int neox)
{
    size_t half = hd / 2;
    const float *c = cos_tab + pos * half, *s = sin_tab + pos * half;
    for (size_t h = 0; h < n_heads; h++) {
        float *v = qk + h * hd;
        for (size_t i = 0; i < half; i++) {
            size_t i0 = neox ? i : 2 * i, i1 = neox ? half + i : 2 * i + 1;
            float v0 = v[i0], v1 = v[i1];
            v[i0] = v0 * c[i] - v1 * s[i];
            v[i1] = v0 * s[i] + v1 * c[i];
        }
    }
}

/* softmax (attention.c:18-33): left unnormalised when the sum is <= 0 or not finite. */
void fwc_softmax(float *x, size_t n)
{
    if (!n) return;
    float mx = x[0];
    for (size_t i = 1; i < n; i++) if (x[i] > mx) mx = x[i];
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) { x[i] = expf(x[i] - mx); sum += x[i]; }
    if (sum <= 0.0f || !isfinite(sum)) return;
    float inv = 1.0f / sum;
    for (size_t i = 0; i < n; i++) x[i] *= inv;
}

/* apply_silu (ffn.c:17-25) = tensor_silu (tensor_ops.c:63-81). */
void fwc_silu(float *x, size_t n)
{
    for (size_t i = 0; i < n; i++) {
        float v = x[i];
        float sig = v >= 0.0f ? 1.0f / (1.0f + expf(-v)) : expf(v) / (1.0f + expf(v));
        x[i] = v * sig;
    }
}

/* layer_norm (norm.c:18-40): mean and variance summed in double in index
 * order, then ((x - mean) * scale) * w + b per element, w and b optional. */
void fwc_layer_norm(const float *x, const float *w, const float *b, float *out, size_t n, float eps)
{
    double sum = 0.0;
    for (size_t i = 0; i < n; i++) sum += x[i];
    const float mean = (float)(sum / (double)n);
    double var = 0.0;
    for (size_t i = 0; i < n; i++) {
        const float d = x[i] - mean;
        var += (double)d * d;
    }
    const float scale = 1.0f / sqrtf((float)(var / (double)n) + eps);
    for (size_t i = 0; i < n; i++) {
        float v = (x[i] - mean) * scale;
        if (w) v *= w[i];
        if (b) v += b[i];
        out[i] = v;
    }
}

/* apply_gelu (ffn.c:27-31): 0.5 v (1 + erf(v / sqrt 2)), libm erff. */
void fwc_gelu(float *x, size_t n)
{
    const float inv_sqrt2 = 0.7071067811865476f;
    for (size_t i = 0; i < n; i++) x[i] = 0.5f * x[i] * (1.0f + erff(x[i] * inv_sqrt2));
}

/* apply_gelu_fast (ffn.c:33-42): the tanh form, sqrt(2/pi) (v + 0.044715 v^3). */
void fwc_gelu_fast(float *x, size_t n)
{
    const float c1 = 0.7978845608028654f, c2 = 0.044715f;
    for (size_t i = 0; i < n; i++) {
        const float v = x[i], inner = c1 * (v + c2 * v * v * v);
        x[i] = 0.5f * v * (1.0f + tanhf(inner));
    }
}

/* sampler_argmax (sampler.c:28-32). */
uint32_t fwc_argmax(const float *x, size_t n)
{
    size_t best = 0;
    for (size_t i = 1; i < n; i++) if (x[i] > x[best]) best = i;
    return (uint32_t)best;
}

typedef struct {
    const float *q, *kc, *vc;
    float *out, *scores;        /* scores: [n_head][pos+1] scratch */
    size_t n_head, n_kv, hd, pos;
} attn_t;

/* per-head body of attention_forward (attention.c:142-164), incl. simd_axpy_f32
 * (simd.h:262-275: 8-wide FMA part, then a rounded multiply-add tail). */
static void attn_heads(void *c, size_t h0, size_t h1)
{
    attn_t *a = (attn_t *)c;
    const size_t group = a->n_head / a->n_kv, stride = a->n_kv * a->hd;
    const float scale = 1.0f / sqrtf((float)a->hd);
    for (size_t h = h0; h < h1; h++) {
        size_t kvh = h / group;
        const float *qh = a->q + h * a->hd;
        float *oh = a->out + h * a->hd, *sc = a->scores + h * (a->pos + 1);
        for (size_t t = 0; t <= a->pos; t++) {
            float dot = fwc_dot_f32(qh, a->kc + t * stride + kvh * a->hd, a->hd);
            sc[t] = dot * scale;
        }
        fwc_softmax(sc, a->pos + 1);
        memset(oh, 0, a->hd * sizeof(float));
        for (size_t t = 0; t <= a->pos; t++) {
            const float *vt = a->vc + t * stride + kvh * a->hd;
            float w = sc[t];
            size_t i = 0;
            for (; i + 8 <= a->hd; i += 8)
                for (int l = 0; l < 8; l++) oh[i + l] = fmaf(vt[i + l], w, oh[i + l]);
            for (; i < a->hd; i++) oh[i] += vt[i] * w;
        }
    }
}

void fwc_attention_core(const float *q, const float *kc, const float *vc, float *out, size_t n_head,
                        size_t n_kv, size_t hd, size_t pos, float *scores)
{
    attn_t a = { q, kc, vc, out, scores, n_head, n_kv, hd, pos };
    /* split heads across threads only when the work is large */
    par_rows_min(attn_heads, &a, n_head, pos >= 1024 ? 2 : SIZE_MAX);
}

/* ── model ───────────────────────────────────────────────────────────────── */

typedef struct {
    const uint8_t *p;
    uint32_t type;
    size_t in, out, bytes;
} lin_t;

struct fwc_model {
    forword_gpu_config_t c;
    size_t n_ctx;
    const uint8_t *data;
    size_t data_size;
    lin_t embd, out_w;
    const float *out_norm, *out_norm_b;
    lin_t pos_embd;                        /* GPT-2 learned positions */
    float *qkv_buf;
    struct layer {
        const float *attn_norm, *ffn_norm, *attn_norm_b, *ffn_norm_b;
        const float *bq, *bk, *bv, *bo;    /* F32 biases, null when absent */
        const float *bqkv, *bu, *bd;       /* GPT-2: attn_qkv.bias, ffn_up.bias, ffn_down.bias */
        lin_t q, k, v, o, gate, up, down, qkv;
    } *L;
    const float *cos_tab, *sin_tab;
    float *kv_k, *kv_v;
    float *x, *xn, *attn_out, *ffn_out, *q, *k, *v, *att, *gate, *upb, *scores, *logits, *trace;
    int traced;
};

static const forword_gpu_tensor_t *find(const forword_gpu_tensor_t *t, size_t n, const char *name)
{
    for (size_t i = 0; i < n; i++) if (t[i].name && !strcmp(t[i].name, name)) return &t[i];
    return NULL;
}

static int bind_lin(lin_t *l, const fwc_model_t *m, const forword_gpu_tensor_t *t)
{
    if (!t || t->n_dims < 2 || t->offset > m->data_size || t->byte_size > m->data_size - t->offset) return -1;
    l->p = m->data + t->offset;
    l->type = t->ggml_type;
    l->in = (size_t)t->dims[0];
    l->out = (size_t)t->dims[1];
    l->bytes = (size_t)t->byte_size;
    return 0;
}

static const float *bind_vec(const fwc_model_t *m, const forword_gpu_tensor_t *t, size_t n)
{
    if (!t || t->ggml_type != FORWORD_GGML_F32 || t->byte_size < n * 4 || t->offset > m->data_size ||
        t->byte_size > m->data_size - t->offset) return NULL;
    return (const float *)(m->data + t->offset);
}

void fwc_model_free(fwc_model_t *m)
{
    if (!m) return;
    free(m->L); free(m->kv_k); free(m->kv_v); free(m->x); free(m->xn); free(m->attn_out);
    free(m->ffn_out); free(m->q); free(m->k); free(m->v); free(m->att); free(m->gate); free(m->upb);
    free(m->scores); free(m->logits); free(m->trace); free(m->qkv_buf);
    free(m);
}

fwc_model_t *fwc_model_init(const void *data, size_t data_size, const forword_gpu_tensor_t *t,
                            size_t nt, const forword_gpu_config_t *cfg, size_t max_ctx,
                            const float *cos_tab, const float *sin_tab)
{
    if (!data || !t || !cfg || !max_ctx || !cos_tab || !sin_tab) return NULL;
    const forword_gpu_config_t *c = cfg;
    if ((c->norm_type != FORWORD_NORM_RMS && c->norm_type != FORWORD_NORM_LAYER) ||
        (c->rope_type == FORWORD_ROPE_NONE) != (c->arch == FORWORD_ARCH_GPT2) || !c->n_head_kv ||
        c->n_head % c->n_head_kv || c->head_dim % 2 || c->n_embd != c->n_head * c->head_dim) {
        fprintf(stderr, "fwc_model_init: unsupported model variant\n");
        return NULL;
    }
    fwc_model_t *m = (fwc_model_t *)calloc(1, sizeof(*m));
    if (!m) return NULL;
    m->c = *c;
    m->n_ctx = max_ctx;
    m->data = (const uint8_t *)data;
    m->data_size = data_size;
    m->cos_tab = cos_tab;
    m->sin_tab = sin_tab;
    const forword_gpu_tensor_t *e = find(t, nt, "token_embd.weight");
    const forword_gpu_tensor_t *o = find(t, nt, "output.weight");
    if (!o) o = find(t, nt, "lm_head.weight");
    if (!o) o = e;
    if (bind_lin(&m->embd, m, e) || bind_lin(&m->out_w, m, o)) goto fail;
    m->out_norm = bind_vec(m, find(t, nt, "output_norm.weight"), c->n_embd);
    m->out_norm_b = bind_vec(m, find(t, nt, "output_norm.bias"), c->n_embd);
    const int gpt2 = c->arch == FORWORD_ARCH_GPT2;
    if (gpt2 && bind_lin(&m->pos_embd, m, find(t, nt, "position_embd.weight"))) goto fail;   /* transformer.c:188-205 */
    m->L = calloc(c->n_layer, sizeof(*m->L));
    if (!m->L) goto fail;
    for (uint32_t l = 0; l < c->n_layer; l++) {
        char nm[96];
        struct layer *L = &m->L[l];
#define LIN(field, suffix) snprintf(nm, sizeof nm, "blk.%u." suffix, l); \
        if (bind_lin(&L->field, m, find(t, nt, nm))) goto fail;
        if (gpt2) {                                  /* attention.c:68-96 */
            LIN(qkv, "attn_qkv.weight");
            snprintf(nm, sizeof nm, "blk.%u.attn_qkv.bias", l);
            L->bqkv = bind_vec(m, find(t, nt, nm), 3 * (size_t)c->n_embd);
        } else {
            LIN(q, "attn_q.weight"); LIN(k, "attn_k.weight"); LIN(v, "attn_v.weight");
        }
        LIN(o, "attn_output.weight");
        if (c->use_ffn_gate) {
            LIN(gate, "ffn_gate.weight"); LIN(up, "ffn_up.weight"); LIN(down, "ffn_down.weight");
        } else {                                     /* ffn.c:110-168: fc1 / fc2 names too */
            snprintf(nm, sizeof nm, "blk.%u.ffn_up.weight", l);
            const forword_gpu_tensor_t *tu = find(t, nt, nm);
            snprintf(nm, sizeof nm, "blk.%u.fc1.weight", l);
            if (!tu) tu = find(t, nt, nm);
            snprintf(nm, sizeof nm, "blk.%u.fc2.weight", l);
            const forword_gpu_tensor_t *td = find(t, nt, nm);
            const int fc2 = td != NULL;
            snprintf(nm, sizeof nm, "blk.%u.ffn_down.weight", l);
            if (!td) td = find(t, nt, nm);
            if (bind_lin(&L->up, m, tu) || bind_lin(&L->down, m, td)) goto fail;
            if (gpt2) {                              /* ffn.c:127-140: required for GPT-2 */
                snprintf(nm, sizeof nm, "blk.%u.ffn_up.bias", l); L->bu = bind_vec(m, find(t, nt, nm), c->n_ff);
                snprintf(nm, sizeof nm, "blk.%u.ffn_down.bias", l); L->bd = bind_vec(m, find(t, nt, nm), c->n_embd);
                if (!L->bu || !L->bd) goto fail;
                if (fc2) L->bd = NULL;                                   /* ffn.c:162-166 */
            }
        }
#undef LIN
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.bias", l);       /* transformer.c:212-230 */
        L->attn_norm_b = bind_vec(m, find(t, nt, nm), c->n_embd);
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.bias", l);
        L->ffn_norm_b = bind_vec(m, find(t, nt, nm), c->n_embd);
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.weight", l);
        L->attn_norm = bind_vec(m, find(t, nt, nm), c->n_embd);
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.weight", l);
        L->ffn_norm = bind_vec(m, find(t, nt, nm), c->n_embd);
        /* attention.c:106-122: attn_output.bias whenever present, q/k/v biases
         * when the architecture has them; linear.c:214-221 adds F32 biases only. */
        const size_t kvd = (size_t)c->n_head_kv * c->head_dim;
        snprintf(nm, sizeof nm, "blk.%u.attn_output.bias", l);
        L->bo = bind_vec(m, find(t, nt, nm), c->n_embd);
        if (c->use_qkv_bias) {
            snprintf(nm, sizeof nm, "blk.%u.attn_q.bias", l); L->bq = bind_vec(m, find(t, nt, nm), c->n_embd);
            snprintf(nm, sizeof nm, "blk.%u.attn_k.bias", l); L->bk = bind_vec(m, find(t, nt, nm), kvd);
            snprintf(nm, sizeof nm, "blk.%u.attn_v.bias", l); L->bv = bind_vec(m, find(t, nt, nm), kvd);
        }
    }
    size_t kvd = (size_t)c->n_head_kv * c->head_dim, kvn = (size_t)c->n_layer * max_ctx * kvd;
    m->kv_k = calloc(kvn, 4); m->kv_v = calloc(kvn, 4);
    m->x = calloc(c->n_embd, 4); m->xn = calloc(c->n_embd, 4); m->attn_out = calloc(c->n_embd, 4);
    m->ffn_out = calloc(c->n_embd, 4); m->q = calloc(c->n_embd, 4); m->k = calloc(kvd, 4);
    m->v = calloc(kvd, 4); m->att = calloc(c->n_embd, 4); m->gate = calloc(c->n_ff, 4);
    m->upb = calloc(c->n_ff, 4); m->scores = calloc((size_t)c->n_head * max_ctx, 4);
    m->logits = calloc(c->n_vocab, 4); m->trace = calloc((size_t)2 * c->n_layer * c->n_embd, 4);
    m->qkv_buf = calloc(3 * (size_t)c->n_embd, 4);
    if (!m->qkv_buf) goto fail;
    if (!m->kv_k || !m->kv_v || !m->x || !m->xn || !m->attn_out || !m->ffn_out || !m->q || !m->k ||
        !m->v || !m->att || !m->gate || !m->upb || !m->scores || !m->logits || !m->trace) goto fail;
    return m;
fail:
    fprintf(stderr, "fwc_model_init: missing tensor or out of memory\n");
    fwc_model_free(m);
    return NULL;
}

static int lin(const lin_t *l, const float *x, float *y)
{
    return fwc_quant_matvec(l->p, l->bytes, l->type, x, y, l->in, l->out);
}

/* linear_get_row (linear.c:60-151) for F32/Q8_0/Q5_0, Q4_K/Q6_K (linear.c:137-142); Q4_0 by its definition. */
static int get_row(const lin_t *l, size_t row, float *out)
{
    if (row >= l->out) return -1;
    if (l->type == FORWORD_GGML_F32) { memcpy(out, l->p + row * l->in * 4, l->in * 4); return 0; }
    const size_t bb = block_bytes(l->type), bv = block_values(l->type);
    if (!bb || l->in % bv) return -1;
    const size_t rb = l->in / bv * bb;
    return fwc_dequant(l->p + row * rb, rb, l->type, out, l->in);
}

static void add_bias(float *y, const float *b, size_t n)
{
    if (b) for (size_t i = 0; i < n; i++) y[i] += b[i];
}

/* The block's pre-norm (transformer.c:234-239, 256-261, 275-280). */
static void block_norm(const fwc_model_t *m, const float *w, const float *b)
{
    const forword_gpu_config_t *c = &m->c;
    if (c->norm_type == FORWORD_NORM_LAYER) fwc_layer_norm(m->x, w, b, m->xn, c->n_embd, c->norm_eps);
    else fwc_rms_norm(m->x, w, m->xn, c->n_embd, c->norm_eps);
}

/* ffn_forward (ffn.c:44-177) of m->xn into m->ffn_out: the gated branch
 * (:68-107, silu by default) or the plain one (:108-171, gelu by default, relu). */
static int ffn(fwc_model_t *m, const struct layer *L)
{
    const forword_gpu_config_t *c = &m->c;
    const size_t nf = c->n_ff;
    if (c->use_ffn_gate) {
        if (lin(&L->gate, m->xn, m->gate) || lin(&L->up, m->xn, m->upb)) return -1;
        if (c->act_type == FORWORD_ACT_GELU) fwc_gelu(m->gate, nf);
        else if (c->act_type == FORWORD_ACT_GELU_FAST) fwc_gelu_fast(m->gate, nf);
        else fwc_silu(m->gate, nf);
        for (size_t i = 0; i < nf; i++) m->gate[i] *= m->upb[i];
        return lin(&L->down, m->gate, m->ffn_out);
    }
    if (lin(&L->up, m->xn, m->upb)) return -1;
    add_bias(m->upb, L->bu, nf);
    if (c->act_type == FORWORD_ACT_GELU_FAST) fwc_gelu_fast(m->upb, nf);
    else if (c->act_type == FORWORD_ACT_SILU) fwc_silu(m->upb, nf);
    else if (c->act_type == FORWORD_ACT_RELU) { for (size_t i = 0; i < nf; i++) if (m->upb[i] < 0.0f) m->upb[i] = 0.0f; }
    else fwc_gelu(m->upb, nf);
    if (lin(&L->down, m->upb, m->ffn_out)) return -1;
    add_bias(m->ffn_out, L->bd, c->n_embd);
    return 0;
}

float *fwc_forward(fwc_model_t *m, uint32_t token, size_t pos)
{
    const forword_gpu_config_t *c = &m->c;
    const size_t n = c->n_embd, hd = c->head_dim, kvd = (size_t)c->n_head_kv * hd;
    if (pos >= m->n_ctx || token >= c->n_vocab) return NULL;     /* transformer.c:156-164 */
    if (get_row(&m->embd, token, m->x)) return NULL;             /* transformer.c:167-177 */
    if (c->embd_scale != 1.0f) for (size_t i = 0; i < n; i++) m->x[i] *= c->embd_scale;
    if (c->arch == FORWORD_ARCH_GPT2) {                          /* transformer.c:188-205 */
        if (get_row(&m->pos_embd, pos, m->xn)) return NULL;
        for (size_t i = 0; i < n; i++) m->x[i] += m->xn[i];
    }
    int neox = c->rope_type == FORWORD_ROPE_NEOX;
    for (uint32_t l = 0; l < c->n_layer; l++) {                  /* transformer.c:208-290 */
        struct layer *L = &m->L[l];
        block_norm(m, L->attn_norm, L->attn_norm_b);
        /* attention_forward (attention.c:97-166) */
        if (c->arch == FORWORD_ARCH_GPT2) {                      /* attention.c:68-96: q | k | v */
            if (lin(&L->qkv, m->xn, m->qkv_buf)) return NULL;
            add_bias(m->qkv_buf, L->bqkv, 3 * n);
            memcpy(m->q, m->qkv_buf, n * 4);
            memcpy(m->k, m->qkv_buf + n, n * 4);
            memcpy(m->v, m->qkv_buf + 2 * n, n * 4);
        } else {
            if (lin(&L->q, m->xn, m->q) || lin(&L->k, m->xn, m->k) || lin(&L->v, m->xn, m->v)) return NULL;
            add_bias(m->q, L->bq, n);                            /* linear.c:214-221 */
            add_bias(m->k, L->bk, kvd);
            add_bias(m->v, L->bv, kvd);
        }
        if (c->rope_type != FORWORD_ROPE_NONE) {                 /* attention.c:129-133 */
            fwc_rope_apply(m->q, pos, c->n_head, hd, m->cos_tab, m->sin_tab, neox);
            fwc_rope_apply(m->k, pos, c->n_head_kv, hd, m->cos_tab, m->sin_tab, neox);
        }
        memcpy(fwc_kv_k(m, l, pos), m->k, kvd * 4);
        memcpy(fwc_kv_v(m, l, pos), m->v, kvd * 4);
        fwc_attention_core(m->q, fwc_kv_k(m, l, 0), fwc_kv_v(m, l, 0), m->att, c->n_head,
                           c->n_head_kv, hd, pos, m->scores);
        if (lin(&L->o, m->att, m->attn_out)) return NULL;
        add_bias(m->attn_out, L->bo, n);
        if (c->parallel_res) {                                   /* transformer.c:232-252 */
            if (ffn(m, L)) return NULL;
            for (size_t i = 0; i < n; i++) m->x[i] += m->attn_out[i] + m->ffn_out[i];
            memcpy(m->trace + (2 * (size_t)l) * n, m->x, n * 4);   /* one residual add: both rows */
            memcpy(m->trace + (2 * (size_t)l + 1) * n, m->x, n * 4);
            continue;
        }
        for (size_t i = 0; i < n; i++) m->x[i] += m->attn_out[i];
        memcpy(m->trace + (2 * (size_t)l) * n, m->x, n * 4);
        block_norm(m, L->ffn_norm, L->ffn_norm_b);
        if (ffn(m, L)) return NULL;
        for (size_t i = 0; i < n; i++) m->x[i] += m->ffn_out[i];
        memcpy(m->trace + (2 * (size_t)l + 1) * n, m->x, n * 4);
    }
    if (m->out_norm) {                                           /* transformer.c:293-307 */
        if (c->norm_type == FORWORD_NORM_LAYER) fwc_layer_norm(m->x, m->out_norm, m->out_norm_b, m->xn, n, c->norm_eps);
        else fwc_rms_norm(m->x, m->out_norm, m->xn, n, c->norm_eps);
    } else {
        memcpy(m->xn, m->x, n * 4);
    }
    if (lin(&m->out_w, m->xn, m->logits)) return NULL;          /* transformer.c:310-323 */
    m->traced = 1;
    return m->logits;
}

const float *fwc_trace(const fwc_model_t *m) { return m && m->traced ? m->trace : NULL; }

float *fwc_kv_k(fwc_model_t *m, size_t layer, size_t pos)
{
    size_t kvd = (size_t)m->c.n_head_kv * m->c.head_dim;
    return m->kv_k + (layer * m->n_ctx + pos) * kvd;              /* kv_cache.h:45-47 */
}

float *fwc_kv_v(fwc_model_t *m, size_t layer, size_t pos)
{
    size_t kvd = (size_t)m->c.n_head_kv * m->c.head_dim;
    return m->kv_v + (layer * m->n_ctx + pos) * kvd;
}

int fwc_generate_greedy(fwc_model_t *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                        uint32_t *out_ids)
{
    if (!m || !prompt || !n_prompt || !out_ids) return -1;
    float *lg = NULL;
    for (size_t i = 0; i < n_prompt; i++)                        /* main.c:145-151 */
        if (!(lg = fwc_forward(m, prompt[i], i))) return -1;
    for (size_t g = 0; g < n_gen; g++) {                          /* main.c:173-217 */
        out_ids[g] = fwc_argmax(lg, m->c.n_vocab);
        if (g + 1 < n_gen && !(lg = fwc_forward(m, out_ids[g], n_prompt + g))) return -1;
    }
    return 0;
}

/* ── sampling (sampler.c:12-101) and the sampled generation loop (main.c:173-217) ── */

static uint64_t xorshift64(uint64_t *s)                       /* sampler.c:8-10 */
{
    *s ^= *s << 13;
    *s ^= *s >> 7;
    *s ^= *s << 17;
    return *s;
}

static const float *g_sort_p;
/* cmp_prob_desc (sampler.c:40-45) with ties in index order: glibc's qsort is a
 * stable merge sort for arrays this size, so equal probabilities keep their
 * index order. */
static int cmp_desc_stable(const void *a, const void *b)
{
    const uint32_t ia = *(const uint32_t *)a, ib = *(const uint32_t *)b;
    if (g_sort_p[ib] > g_sort_p[ia]) return 1;
    if (g_sort_p[ib] < g_sort_p[ia]) return -1;
    return ia < ib ? -1 : ia > ib;
}

uint32_t fwc_sample(const float *logits, size_t n, const uint32_t *hist, size_t n_hist, float temperature,
                    float top_p, float penalty, uint64_t *rng)
{
    float *p = (float *)malloc(n * sizeof(float));
    uint32_t *idx = (uint32_t *)malloc(n * sizeof(uint32_t));
    if (!p || !idx) { free(p); free(idx); return 0; }
    memcpy(p, logits, n * sizeof(float));
    if (penalty != 1.0f)                                          /* sampler_rep_penalty, :89-101 */
        for (size_t i = 0; i < n_hist; i++) {
            const uint32_t id = hist[i];
            if (id < n) p[id] = p[id] > 0.0f ? p[id] / penalty : p[id] * penalty;
        }
    uint32_t out;
    if (temperature <= 0.0f) {                                    /* main.c:184-185 */
        out = fwc_argmax(p, n);
    } else {                                                      /* sampler_top_p, :47-87 */
        if (temperature != 1.0f) {
            const float inv = 1.0f / temperature;
            for (size_t i = 0; i < n; i++) p[i] *= inv;
        }
        float mx = p[0];                                          /* sampler_softmax, :18-26 */
        for (size_t i = 1; i < n; i++) if (p[i] > mx) mx = p[i];
        float sum = 0.0f;
        for (size_t i = 0; i < n; i++) { p[i] = expf(p[i] - mx); sum += p[i]; }
        const float inv = 1.0f / sum;
        for (size_t i = 0; i < n; i++) p[i] *= inv;
        for (size_t i = 0; i < n; i++) idx[i] = (uint32_t)i;
        g_sort_p = p;
        qsort(idx, n, sizeof(uint32_t), cmp_desc_stable);
        float cum = 0.0f;
        size_t nucleus = 0;
        for (size_t i = 0; i < n; i++) {
            cum += p[idx[i]];
            nucleus = i + 1;
            if (cum >= top_p) break;
        }
        float norm = 0.0f;
        for (size_t i = 0; i < nucleus; i++) norm += p[idx[i]];
        const float r = (float)(xorshift64(rng) >> 11) / (float)(UINT64_MAX >> 11) * norm;
        out = idx[nucleus - 1];
        cum = 0.0f;
        for (size_t i = 0; i < nucleus; i++) {
            cum += p[idx[i]];
            if (r <= cum) { out = idx[i]; break; }
        }
    }
    free(p);
    free(idx);
    return out;
}

int fwc_generate_sampled(fwc_model_t *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen, float temperature,
                         float top_p, float penalty, uint64_t seed, uint32_t *out_ids)
{
    if (!m || !prompt || !n_prompt || !out_ids) return -1;
    uint64_t rng = seed ? seed : 12345;                           /* main.c:98-99 */
    uint32_t *hist = (uint32_t *)malloc((n_prompt + n_gen) * sizeof(uint32_t));
    if (!hist) return -1;
    memcpy(hist, prompt, n_prompt * sizeof(uint32_t));
    size_t n_hist = n_prompt;
    float *lg = NULL;
    for (size_t i = 0; i < n_prompt; i++)
        if (!(lg = fwc_forward(m, prompt[i], i))) { free(hist); return -1; }
    for (size_t g = 0; g < n_gen; g++) {
        const uint32_t t = fwc_sample(lg, m->c.n_vocab, hist, n_hist, temperature, top_p, penalty, &rng);
        out_ids[g] = t;
        hist[n_hist++] = t;
        if (g + 1 < n_gen && !(lg = fwc_forward(m, t, n_prompt + g))) { free(hist); return -1; }
    }
    free(hist);
    return 0;
}
