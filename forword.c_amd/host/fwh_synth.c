/*
 * Seeded random-init model writer: PRNG, fp16 conversion, GGUF block
 * quantisers and a GGUF v3 image writer.
 *
 * PRNG: splitmix64 (Steele, Lea, Flood 2014) drives every draw.  Normals use
 * the Box-Muller transform in double precision on 24-bit uniforms in (0,1].
 * Every tensor row has its own stream, seeded from (model seed, tensor name,
 * row), so generation is parallel over rows and the bytes do not depend on the
 * thread count.
 *
 * Block layouts (GGUF/ggml definitions; sizes as in gguf.c:211-215):
 *   Q4_0 (18 B): fp16 d, qs[16]; w_j = d*((qs[j]&15)-8), w_{j+16} = d*((qs[j]>>4)-8)
 *   Q5_0 (22 B): fp16 d, qh u32 (LE), qs[16]; 5th bit of code j is bit j of qh
 *   Q8_0 (34 B): fp16 d, int8 qs[32]; w_j = d*qs[j]
 *   Q4_K (144 B per 256): fp16 d, dmin, 12 B of 6-bit group scales/mins, qs[128]
 *   Q6_K (210 B per 256): ql[128], qh[64], int8 scales[16], fp16 d
 * Quantisers follow ggml's reference rounding: Q8_0 d = amax/127 with
 * round-to-nearest codes; Q4_0/Q5_0 take the signed value of largest magnitude
 * m and use d = m/-8 (resp. m/-16), codes min(15, (int8)(x/d + 8.5)) (resp.
 * min(31, (int8)(x/d + 16.5))).
 *
 * Image layout written by fwh_synth_write (satisfies the reference loader,
 * gguf.c:256-353, model_config.c:61-220, tokenizer.c:191-195):
 *   header | metadata (llama.* keys as UINT32/FLOAT32, tokenizer tokens) |
 *   tensor infos | pad to 32 | tensors, each 32-byte aligned, in the order
 *   token_embd, blk.N.{attn_norm, attn_q, attn_k, attn_v, attn_output,
 *   ffn_norm, ffn_gate, ffn_up, ffn_down}, output_norm, output.
 */
#define _GNU_SOURCE
#include "fw_host.h"

#include <math.h>
#include <pthread.h>
#include <stdatomic.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <unistd.h>

/* ── threads ─────────────────────────────────────────────────────────────── */

uint32_t fwh_default_threads(void)
{
    const char *e = getenv("FW_THREADS");
    if (e && atoi(e) > 0) return (uint32_t)atoi(e);
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    if (n < 1) n = 1;
    if (n > 16) n = 16;
    return (uint32_t)n;
}

typedef struct {
    void (*fn)(void *ctx, size_t job);
    void *ctx;
    size_t n_jobs;
    atomic_size_t next;
} pool_t;

static void *pool_worker(void *arg)
{
    pool_t *p = (pool_t *)arg;
    for (;;) {
        size_t j = atomic_fetch_add(&p->next, 1);
        if (j >= p->n_jobs) break;
        p->fn(p->ctx, j);
    }
    return NULL;
}

static void run_parallel(void (*fn)(void *, size_t), void *ctx, size_t n_jobs, uint32_t threads)
{
    pool_t p = { fn, ctx, n_jobs, 0 };
    if (!threads) threads = fwh_default_threads();
    if (threads > n_jobs) threads = (uint32_t)(n_jobs ? n_jobs : 1);
    if (threads <= 1) { pool_worker(&p); return; }
    pthread_t *tid = (pthread_t *)malloc(sizeof(pthread_t) * threads);
    uint32_t started = 0;
    for (uint32_t i = 0; i < threads; i++)
        if (pthread_create(&tid[i], NULL, pool_worker, &p) == 0) started++;
        else break;
    if (!started) pool_worker(&p);
    for (uint32_t i = 0; i < started; i++) pthread_join(tid[i], NULL);
    free(tid);
}

/* ── PRNG ────────────────────────────────────────────────────────────────── */

uint64_t fwh_splitmix64(uint64_t *s)
{
    uint64_t z = (*s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

/* uniform in (0, 1], 24 bits */
static double unif(uint64_t *s) { return (double)((fwh_splitmix64(s) >> 40) + 1) * (1.0 / 16777216.0); }

void fwh_randn(uint64_t seed, float std, float *out, size_t n)
{
    uint64_t s = seed;
    for (size_t i = 0; i < n; i += 2) {
        double u1 = unif(&s), u2 = unif(&s);
        double r = sqrt(-2.0 * log(u1));
        double a = 6.283185307179586 * u2;
        out[i] = (float)(r * cos(a)) * std;
        if (i + 1 < n) out[i + 1] = (float)(r * sin(a)) * std;
    }
}

static uint64_t name_seed(uint64_t seed, const char *name)
{
    uint64_t h = 0xcbf29ce484222325ull;                    /* FNV-1a 64 */
    for (const unsigned char *p = (const unsigned char *)name; *p; p++) { h ^= *p; h *= 0x100000001b3ull; }
    uint64_t s = seed ^ h;
    return fwh_splitmix64(&s);
}

static uint64_t row_seed(uint64_t tseed, uint64_t row)
{
    uint64_t s = tseed + (row + 1) * 0xD1B54A32D192ED03ull;
    return fwh_splitmix64(&s);
}

/* ── fp16 ────────────────────────────────────────────────────────────────── */

uint16_t fwh_f32_to_f16(float f)
{
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t a = x & 0x7fffffffu;
    if (a >= 0x7f800000u) return (uint16_t)(sign | (a > 0x7f800000u ? 0x7e00u : 0x7c00u));
    if (a >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);        /* rounds to +-inf */
    if (a >= 0x38800000u) {                                          /* normal binary16 */
        uint32_t h = (a - (112u << 23)) >> 13;
        uint32_t rem = a & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    uint32_t e = a >> 23;                                            /* subnormal or zero */
    if (e < 102) return (uint16_t)sign;                              /* < 2^-25: rounds to 0 */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t s = 126u - e;                                           /* 14..24 */
    uint32_t q = m >> s;
    uint32_t rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

float fwh_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu, bits;
    if (e == 0x1fu) bits = sign | 0x7f800000u | (m << 13);
    else if (e) bits = sign | ((e + 112u) << 23) | (m << 13);
    else if (!m) bits = sign;
    else {                                  /* subnormal: m * 2^-24, normalise */
        int sh = 0;
        while (!(m & 0x400u)) { m <<= 1; sh++; }
        bits = sign | ((uint32_t)(113 - sh) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* ── quantisers ──────────────────────────────────────────────────────────── */

size_t fwh_block_bytes(uint32_t t)
{
    switch (t) {
    case FORWORD_GGML_Q4_0: return 18;
    case FORWORD_GGML_Q5_0: return 22;
    case FORWORD_GGML_Q8_0: return 34;
    case FORWORD_GGML_Q4_K: return 144;
    case FORWORD_GGML_Q6_K: return 210;
    case FORWORD_GGML_F32: return 4;
    default: return 0;
    }
}

size_t fwh_block_values(uint32_t t)
{
    switch (t) {
    case FORWORD_GGML_Q4_0: case FORWORD_GGML_Q5_0: case FORWORD_GGML_Q8_0: return 32;
    case FORWORD_GGML_Q4_K: case FORWORD_GGML_Q6_K: return 256;
    case FORWORD_GGML_F32: return 1;
    default: return 0;
    }
}

static void put_f16(uint8_t *p, float v)
{
    uint16_t h = fwh_f32_to_f16(v);
    p[0] = (uint8_t)(h & 0xff);
    p[1] = (uint8_t)(h >> 8);
}

static void quant_q8_0(const float *x, uint8_t *b)
{
    float amax = 0.0f;
    for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) amax = a; }
    float d = amax / 127.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(b, d);
    for (int j = 0; j < 32; j++) b[2 + j] = (uint8_t)(int8_t)roundf(x[j] * id);
}

static float signed_absmax(const float *x)
{
    float amax = 0.0f, m = 0.0f;
    for (int j = 0; j < 32; j++) { float a = fabsf(x[j]); if (a > amax) { amax = a; m = x[j]; } }
    return m;
}

static void quant_q4_0(const float *x, uint8_t *b)
{
    float d = signed_absmax(x) / -8.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    put_f16(b, d);
    for (int j = 0; j < 16; j++) {
        int q0 = (int8_t)(x[j] * id + 8.5f), q1 = (int8_t)(x[16 + j] * id + 8.5f);
        if (q0 > 15) q0 = 15;
        if (q1 > 15) q1 = 15;
        b[2 + j] = (uint8_t)(q0 | (q1 << 4));
    }
}

static void quant_q5_0(const float *x, uint8_t *b)
{
    float d = signed_absmax(x) / -16.0f;
    float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint32_t qh = 0;
    put_f16(b, d);
    for (int j = 0; j < 16; j++) {
        int q0 = (int8_t)(x[j] * id + 16.5f), q1 = (int8_t)(x[16 + j] * id + 16.5f);
        if (q0 > 31) q0 = 31;
        if (q1 > 31) q1 = 31;
        b[6 + j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
        qh |= (uint32_t)((q0 >> 4) & 1) << j;
        qh |= (uint32_t)((q1 >> 4) & 1) << (j + 16);
    }
    b[2] = (uint8_t)qh; b[3] = (uint8_t)(qh >> 8); b[4] = (uint8_t)(qh >> 16); b[5] = (uint8_t)(qh >> 24);
}

/* Q4_K super-block (the layout q4_k_decode reads, quant.c:63-131): fp16 d and
 * dmin, 12 bytes of 6-bit scale/min pairs per 32-value group, 128 code bytes
 * (group 2k in the low nibbles of bytes 32k.., group 2k+1 in the high ones).
 * Value = d*sc*q - dmin*m.  A simple encoder: per group the range above its
 * minimum, both quantised against the super-block maxima. */
static void quant_q4_k(const float *x, uint8_t *b)
{
    float scale[8], minv[8], smax = 0.0f, mmax = 0.0f;
    for (int g = 0; g < 8; g++) {
        float lo = x[32 * g], hi = x[32 * g];
        for (int i = 1; i < 32; i++) { lo = fminf(lo, x[32 * g + i]); hi = fmaxf(hi, x[32 * g + i]); }
        minv[g] = lo < 0.0f ? -lo : 0.0f;
        scale[g] = (hi + minv[g]) / 15.0f;
        smax = fmaxf(smax, scale[g]);
        mmax = fmaxf(mmax, minv[g]);
    }
    const float d = smax / 63.0f, dmin = mmax / 63.0f;
    put_f16(b, d);
    put_f16(b + 2, dmin);
    const float dq = fwh_f16_to_f32(fwh_f32_to_f16(d)), mq = fwh_f16_to_f32(fwh_f32_to_f16(dmin));
    uint8_t sc[8], mn[8];
    for (int g = 0; g < 8; g++) {
        int s6 = dq > 0.0f ? (int)lroundf(scale[g] / dq) : 0, m6 = mq > 0.0f ? (int)lroundf(minv[g] / mq) : 0;
        sc[g] = (uint8_t)(s6 < 0 ? 0 : s6 > 63 ? 63 : s6);
        mn[g] = (uint8_t)(m6 < 0 ? 0 : m6 > 63 ? 63 : m6);
    }
    uint8_t *scales = b + 4;
    for (int j = 0; j < 4; j++) {
        scales[j] = (uint8_t)(sc[j] | ((sc[j + 4] >> 4) << 6));
        scales[j + 4] = (uint8_t)(mn[j] | ((mn[j + 4] >> 4) << 6));
        scales[j + 8] = (uint8_t)((sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4));
    }
    uint8_t *qs = b + 16;
    memset(qs, 0, 128);
    for (int g = 0; g < 8; g++) {
        const float ds = dq * sc[g], dm = mq * mn[g];
        for (int i = 0; i < 32; i++) {
            int q = ds > 0.0f ? (int)lroundf((x[32 * g + i] + dm) / ds) : 0;
            q = q < 0 ? 0 : q > 15 ? 15 : q;
            qs[(g / 2) * 32 + i] |= (uint8_t)(g & 1 ? q << 4 : q);
        }
    }
}

/* Q6_K super-block (q6_k_decode, quant.c:133-188): ql[128] low nibbles, qh[64]
 * high bit pairs, int8 scales[16] (one per 16 values), fp16 d.  Value =
 * d*sc*(q - 32); within a half of 128 values, value l+32k (l < 32) has its low
 * nibble in ql[l + 32(k&1)] (high nibble for k >= 2), its high bits in qh[l]
 * bits 2k..2k+1, its scale in scales[l/16 + 2k]. */
static void quant_q6_k(const float *x, uint8_t *b)
{
    float sub[16], smax = 0.0f;
    for (int s = 0; s < 16; s++) {
        float a = 0.0f;
        for (int i = 0; i < 16; i++) a = fmaxf(a, fabsf(x[16 * s + i]));
        sub[s] = a / 31.0f;
        smax = fmaxf(smax, sub[s]);
    }
    const float d = smax / 127.0f;
    put_f16(b + 208, d);
    const float dq = fwh_f16_to_f32(fwh_f32_to_f16(d));
    int8_t *sc = (int8_t *)(b + 192);
    for (int s = 0; s < 16; s++) {
        int v = dq > 0.0f ? (int)lroundf(sub[s] / dq) : 0;
        sc[s] = (int8_t)(v > 127 ? 127 : v);
    }
    memset(b, 0, 192);
    for (int h = 0; h < 2; h++)
        for (int k = 0; k < 4; k++)
            for (int l = 0; l < 32; l++) {
                const int pos = h * 128 + 32 * k + l, s = h * 8 + l / 16 + 2 * k;
                const float st = dq * sc[s];
                int q = st > 0.0f ? (int)lroundf(x[pos] / st) + 32 : 32;
                q = q < 0 ? 0 : q > 63 ? 63 : q;
                uint8_t *ql = b + h * 64 + l + 32 * (k & 1), *qh = b + 128 + h * 32 + l;
                *ql |= (uint8_t)(k >= 2 ? (q & 15) << 4 : (q & 15));
                *qh |= (uint8_t)(((q >> 4) & 3) << (2 * k));
            }
}

size_t fwh_quantize(uint32_t t, const float *src, size_t n, void *dst)
{
    uint8_t *o = (uint8_t *)dst;
    if (t == FORWORD_GGML_F32) { memcpy(dst, src, n * 4); return n * 4; }
    const size_t bb = fwh_block_bytes(t), bv = fwh_block_values(t);
    if (!bb || n % bv) return 0;
    for (size_t i = 0; i < n; i += bv, o += bb) {
        if (t == FORWORD_GGML_Q8_0) quant_q8_0(src + i, o);
        else if (t == FORWORD_GGML_Q4_0) quant_q4_0(src + i, o);
        else if (t == FORWORD_GGML_Q5_0) quant_q5_0(src + i, o);
        else if (t == FORWORD_GGML_Q4_K) quant_q4_k(src + i, o);
        else quant_q6_k(src + i, o);
    }
    return (n / bv) * bb;
}

/* ── GGUF image writer ───────────────────────────────────────────────────── */

enum { T_EMBD = 0, T_ATTN_NORM, T_Q, T_K, T_V, T_O, T_FFN_NORM, T_GATE, T_UP, T_DOWN,
       T_OUT_NORM, T_OUT, T_BIAS };

typedef struct {
    char     name[64];
    int      kind;
    uint32_t type;
    uint64_t cols, rows;    /* dims[0], dims[1] (rows = 1 for 1-D) */
    int      n_dims;
    uint64_t offset, bytes;
} tdesc_t;

typedef struct {
    fwh_synth_spec_t s;
    tdesc_t *t;
    size_t n_t;
    size_t meta_bytes, info_bytes, data_offset, total;
} layout_t;

static uint64_t tbytes(uint32_t type, uint64_t cols, uint64_t rows)
{
    if (type == FORWORD_GGML_F32) return cols * rows * 4;
    return cols / fwh_block_values(type) * fwh_block_bytes(type) * rows;
}

static void add_t(layout_t *L, const char *name, int kind, uint32_t type, uint64_t cols, uint64_t rows,
                  int n_dims)
{
    tdesc_t *d = &L->t[L->n_t++];
    snprintf(d->name, sizeof d->name, "%s", name);
    d->kind = kind; d->type = type; d->cols = cols; d->rows = rows; d->n_dims = n_dims;
    d->bytes = tbytes(type, cols, rows);
}

static size_t str_bytes(size_t len) { return 8 + len; }

static int token_text(uint32_t i, char *buf) { return sprintf(buf, "<t%u>", i); }

/* Architectures the writer emits (model_config.c:10-22 names). */
static const char *synth_arch_name(uint32_t arch)
{
    return arch == FORWORD_ARCH_QWEN2 ? "qwen2" : arch == FORWORD_ARCH_GEMMA ? "gemma"
         : arch == FORWORD_ARCH_PHI2 ? "phi2" : arch == FORWORD_ARCH_GPT2 ? "gpt2" : "llama";
}

static int build_layout(const fwh_synth_spec_t *s, layout_t *L)
{
    memset(L, 0, sizeof *L);
    L->s = *s;
    if (!s->n_embd || !s->n_layer || !s->n_head || !s->n_head_kv || !s->n_ff || !s->n_vocab ||
        s->n_embd % s->n_head || s->n_embd % 32 || s->n_ff % 32 || s->n_head % s->n_head_kv ||
        !fwh_block_bytes(s->linear_type) || !fwh_block_bytes(s->embd_type) ||
        !fwh_block_bytes(s->output_type) || s->n_embd % fwh_block_values(s->linear_type) ||
        s->n_ff % fwh_block_values(s->linear_type) || s->n_embd % fwh_block_values(s->embd_type) ||
        s->n_embd % fwh_block_values(s->output_type) ||
        (s->mix_type && (!fwh_block_bytes(s->mix_type) || s->n_embd % fwh_block_values(s->mix_type) ||
                         s->n_ff % fwh_block_values(s->mix_type))))
        return -1;
    uint64_t hd = s->n_embd / s->n_head, kvd = hd * s->n_head_kv;
    const int phi2 = s->arch == FORWORD_ARCH_PHI2;
    const int gpt2 = s->arch == FORWORD_ARCH_GPT2, ln = phi2 || gpt2;   /* LayerNorm blocks: norm biases */
    if (gpt2 && s->n_head_kv != s->n_head) return -1;                   /* model_config.c:204 */
    L->t = (tdesc_t *)calloc(14 * (size_t)s->n_layer + 8, sizeof(tdesc_t));
    if (!L->t) return -1;
    char nm[64];
#define BIAS(fmt, n) do { snprintf(nm, sizeof nm, fmt, l); add_t(L, nm, T_BIAS, FORWORD_GGML_F32, n, 1, 1); } while (0)
    add_t(L, "token_embd.weight", T_EMBD, s->embd_type, s->n_embd, s->n_vocab, 2);
    if (gpt2) add_t(L, "position_embd.weight", T_EMBD, s->embd_type, s->n_embd, s->n_ctx, 2);
    for (uint32_t l = 0; l < s->n_layer; l++) {
        const uint32_t mixed = s->mix_type && l % 2 == 0 ? s->mix_type : s->linear_type;
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.weight", l); add_t(L, nm, T_ATTN_NORM, FORWORD_GGML_F32, s->n_embd, 1, 1);
        if (ln) BIAS("blk.%u.attn_norm.bias", s->n_embd);
        if (gpt2) {                                   /* one [q | k | v] projection (attention.c:68-96) */
            snprintf(nm, sizeof nm, "blk.%u.attn_qkv.weight", l); add_t(L, nm, T_Q, s->linear_type, s->n_embd, 3 * (uint64_t)s->n_embd, 2);
            BIAS("blk.%u.attn_qkv.bias", 3 * (uint64_t)s->n_embd);
        } else {
            snprintf(nm, sizeof nm, "blk.%u.attn_q.weight", l); add_t(L, nm, T_Q, s->linear_type, s->n_embd, s->n_embd, 2);
            snprintf(nm, sizeof nm, "blk.%u.attn_k.weight", l); add_t(L, nm, T_K, s->linear_type, s->n_embd, kvd, 2);
            snprintf(nm, sizeof nm, "blk.%u.attn_v.weight", l); add_t(L, nm, T_V, mixed, s->n_embd, kvd, 2);
        }
        if (s->arch == FORWORD_ARCH_QWEN2) {
            BIAS("blk.%u.attn_q.bias", s->n_embd); BIAS("blk.%u.attn_k.bias", kvd); BIAS("blk.%u.attn_v.bias", kvd);
        }
        snprintf(nm, sizeof nm, "blk.%u.attn_output.weight", l); add_t(L, nm, T_O, s->linear_type, s->n_embd, s->n_embd, 2);
        if (ln) BIAS("blk.%u.attn_output.bias", s->n_embd);
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.weight", l); add_t(L, nm, T_FFN_NORM, FORWORD_GGML_F32, s->n_embd, 1, 1);
        if (ln) BIAS("blk.%u.ffn_norm.bias", s->n_embd);
        if (!ln) { snprintf(nm, sizeof nm, "blk.%u.ffn_gate.weight", l); add_t(L, nm, T_GATE, s->linear_type, s->n_embd, s->n_ff, 2); }
        snprintf(nm, sizeof nm, "blk.%u.ffn_up.weight", l); add_t(L, nm, T_UP, s->linear_type, s->n_embd, s->n_ff, 2);
        if (gpt2) BIAS("blk.%u.ffn_up.bias", s->n_ff);
        snprintf(nm, sizeof nm, "blk.%u.ffn_down.weight", l); add_t(L, nm, T_DOWN, mixed, s->n_ff, s->n_embd, 2);
        if (gpt2) BIAS("blk.%u.ffn_down.bias", s->n_embd);
    }
#undef BIAS
    add_t(L, "output_norm.weight", T_OUT_NORM, FORWORD_GGML_F32, s->n_embd, 1, 1);
    if (ln) add_t(L, "output_norm.bias", T_BIAS, FORWORD_GGML_F32, s->n_embd, 1, 1);
    if (s->arch != FORWORD_ARCH_GEMMA && !gpt2)
        add_t(L, "output.weight", T_OUT, s->output_type, s->n_embd, s->n_vocab, 2);

    /* metadata: 8 <arch> keys + architecture + name + tokenizer model + tokens */
    const char *arch = synth_arch_name(s->arch);
    const size_t arch_len = strlen(arch), pre = arch_len + 1;            /* "<arch>." prefix */
    size_t m = 0;
    m += str_bytes(strlen("general.architecture")) + 4 + str_bytes(arch_len);
    m += str_bytes(strlen("general.name")) + 4 + str_bytes(strlen("forword-synth"));
    static const char *u32keys[] = { "embedding_length", "block_count", "attention.head_count",
        "attention.head_count_kv", "feed_forward_length", "context_length" };
    for (int i = 0; i < 6; i++) m += str_bytes(pre + strlen(u32keys[i])) + 4 + 4;
    m += str_bytes(pre + strlen("rope.freq_base")) + 4 + 4;
    m += str_bytes(pre + strlen("attention.layer_norm_rms_epsilon")) + 4 + 4;
    m += str_bytes(strlen("tokenizer.ggml.model")) + 4 + str_bytes(5);
    m += str_bytes(strlen("tokenizer.ggml.tokens")) + 4 + 4 + 8;
    char tb[32];
    for (uint32_t i = 0; i < s->n_vocab; i++) m += str_bytes((size_t)token_text(i, tb));
    L->meta_bytes = m;

    size_t info = 0;
    for (size_t i = 0; i < L->n_t; i++) info += str_bytes(strlen(L->t[i].name)) + 4 + 8 * (size_t)L->t[i].n_dims + 4 + 8;
    L->info_bytes = info;
    size_t hdr = 4 + 4 + 8 + 8;
    L->data_offset = (hdr + m + info + 31) & ~(size_t)31;
    uint64_t off = 0;
    for (size_t i = 0; i < L->n_t; i++) {
        L->t[i].offset = off;
        off = (off + L->t[i].bytes + 31) & ~(uint64_t)31;
    }
    L->total = L->data_offset + off;
    return 0;
}

typedef struct { uint8_t *p; } wr_t;
static void w_bytes(wr_t *w, const void *src, size_t n) { memcpy(w->p, src, n); w->p += n; }
static void w_u32(wr_t *w, uint32_t v) { w_bytes(w, &v, 4); }
static void w_u64(wr_t *w, uint64_t v) { w_bytes(w, &v, 8); }
static void w_f32(wr_t *w, float v) { w_bytes(w, &v, 4); }
static void w_str(wr_t *w, const char *s, size_t n) { w_u64(w, n); w_bytes(w, s, n); }
static void w_cstr(wr_t *w, const char *s) { w_str(w, s, strlen(s)); }

/* "<arch>.<suffix>" metadata key (model_config.c:53-57 builds the same names). */
static const char *arch_key(char *buf, size_t n, const char *arch, const char *suffix)
{
    snprintf(buf, n, "%s.%s", arch, suffix);
    return buf;
}

typedef struct {
    const layout_t *L;
    uint8_t *data;          /* start of data section */
    size_t rows_per_job;
    size_t *job_first;      /* first global job index per tensor (n_t + 1 entries) */
    size_t n_jobs;
    int progress;           /* env FW_SYNTH_PROGRESS: a line on stderr per tenth done */
    atomic_size_t done;
} gen_ctx_t;

static void gen_job(void *vctx, size_t job)
{
    gen_ctx_t *c = (gen_ctx_t *)vctx;
    const layout_t *L = c->L;
    size_t ti = 0;
    while (c->job_first[ti + 1] <= job) ti++;
    const tdesc_t *t = &L->t[ti];
    size_t r0 = (job - c->job_first[ti]) * c->rows_per_job;
    size_t r1 = r0 + c->rows_per_job;
    if (r1 > t->rows) r1 = t->rows;
    uint64_t tseed = name_seed(L->s.seed, t->name);
    float *buf = (float *)malloc(sizeof(float) * (t->cols + 1));
    uint64_t row_bytes = t->bytes / t->rows;
    for (size_t r = r0; r < r1; r++) {
        int is_norm = t->kind == T_ATTN_NORM || t->kind == T_FFN_NORM || t->kind == T_OUT_NORM;
        fwh_randn(row_seed(tseed, r), is_norm ? L->s.norm_std : t->kind == T_BIAS ? 4.0f * L->s.w_std : L->s.w_std,
                  buf, t->cols);
        if (is_norm) for (size_t j = 0; j < t->cols; j++) buf[j] += 1.0f;
        fwh_quantize(t->type, buf, t->cols, c->data + t->offset + r * row_bytes);
    }
    free(buf);
    if (c->progress) {
        const size_t d = atomic_fetch_add(&c->done, 1) + 1;
        if (d * 10 / c->n_jobs != (d - 1) * 10 / c->n_jobs)
            fprintf(stderr, "fwh_synth: %zu%% of %zu row blocks written\n", d * 100 / c->n_jobs, c->n_jobs);
    }
}

size_t fwh_synth_size(const fwh_synth_spec_t *spec)
{
    layout_t L;
    if (build_layout(spec, &L)) return 0;
    free(L.t);
    return L.total;
}

size_t fwh_synth_write(const fwh_synth_spec_t *spec, void *out, size_t cap)
{
    layout_t L;
    if (build_layout(spec, &L)) return 0;
    if (cap < L.total) { free(L.t); return 0; }
    const fwh_synth_spec_t *s = &L.s;
    wr_t w = { (uint8_t *)out };
    w_u32(&w, 0x46554747u);
    w_u32(&w, 3);
    w_u64(&w, L.n_t);
    w_u64(&w, 12);
    const char *arch = synth_arch_name(s->arch);
    char key[96];
#define ARCH_KEY(k) arch_key(key, sizeof key, arch, k)
    w_cstr(&w, "general.architecture"); w_u32(&w, 8); w_cstr(&w, arch);
    w_cstr(&w, "general.name"); w_u32(&w, 8); w_cstr(&w, "forword-synth");
    w_cstr(&w, ARCH_KEY("embedding_length")); w_u32(&w, 4); w_u32(&w, s->n_embd);
    w_cstr(&w, ARCH_KEY("block_count")); w_u32(&w, 4); w_u32(&w, s->n_layer);
    w_cstr(&w, ARCH_KEY("attention.head_count")); w_u32(&w, 4); w_u32(&w, s->n_head);
    w_cstr(&w, ARCH_KEY("attention.head_count_kv")); w_u32(&w, 4); w_u32(&w, s->n_head_kv);
    w_cstr(&w, ARCH_KEY("feed_forward_length")); w_u32(&w, 4); w_u32(&w, s->n_ff);
    w_cstr(&w, ARCH_KEY("context_length")); w_u32(&w, 4); w_u32(&w, s->n_ctx);
    w_cstr(&w, ARCH_KEY("rope.freq_base")); w_u32(&w, 6); w_f32(&w, s->rope_freq_base);
    w_cstr(&w, ARCH_KEY("attention.layer_norm_rms_epsilon")); w_u32(&w, 6); w_f32(&w, s->norm_eps);
#undef ARCH_KEY
    w_cstr(&w, "tokenizer.ggml.model"); w_u32(&w, 8); w_cstr(&w, "llama");
    w_cstr(&w, "tokenizer.ggml.tokens"); w_u32(&w, 9); w_u32(&w, 8); w_u64(&w, s->n_vocab);
    char tb[32];
    for (uint32_t i = 0; i < s->n_vocab; i++) { int n = token_text(i, tb); w_str(&w, tb, (size_t)n); }
    for (size_t i = 0; i < L.n_t; i++) {
        const tdesc_t *t = &L.t[i];
        w_cstr(&w, t->name);
        w_u32(&w, (uint32_t)t->n_dims);
        w_u64(&w, t->cols);
        if (t->n_dims == 2) w_u64(&w, t->rows);
        w_u32(&w, t->type);
        w_u64(&w, t->offset);
    }
    uint8_t *base = (uint8_t *)out;
    memset(w.p, 0, (size_t)(base + L.data_offset - w.p));
    uint8_t *data = base + L.data_offset;
    /* zero the inter-tensor padding, then fill tensors in parallel */
    for (size_t i = 0; i < L.n_t; i++) {
        uint64_t end = L.t[i].offset + L.t[i].bytes;
        uint64_t next = i + 1 < L.n_t ? L.t[i + 1].offset : (L.total - L.data_offset);
        if (next > end) memset(data + end, 0, (size_t)(next - end));
    }
    gen_ctx_t c = { &L, data, 64, NULL, 0, 0, 0 };
    c.job_first = (size_t *)calloc(L.n_t + 1, sizeof(size_t));
    for (size_t i = 0; i < L.n_t; i++)
        c.job_first[i + 1] = c.job_first[i] + (L.t[i].rows + c.rows_per_job - 1) / c.rows_per_job;
    c.n_jobs = c.job_first[L.n_t];
    c.progress = getenv("FW_SYNTH_PROGRESS") != NULL;
    run_parallel(gen_job, &c, c.n_jobs, s->threads);
    free(c.job_first);
    size_t total = L.total;
    free(L.t);
    return total;
}

int fwh_synth_write_file(const fwh_synth_spec_t *spec, const char *path)
{
    size_t n = 0;
    void *img = fwh_synth_alloc(spec, &n);
    if (!img) return -1;
    FILE *f = fopen(path, "wb");
    int rc = -1;
    if (f) {
        rc = fwrite(img, 1, n, f) == n ? 0 : -1;
        if (fclose(f)) rc = -1;
    }
    fwh_synth_release(img, n);
    return rc;
}

void *fwh_synth_alloc(const fwh_synth_spec_t *spec, size_t *size_out)
{
    size_t n = fwh_synth_size(spec);
    if (!n) return NULL;
    void *p = mmap(NULL, n, PROT_READ | PROT_WRITE, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (p == MAP_FAILED) return NULL;
    if (fwh_synth_write(spec, p, n) != n) { munmap(p, n); return NULL; }
    if (size_out) *size_out = n;
    return p;
}

void fwh_synth_release(void *image, size_t size)
{
    if (image) munmap(image, size);
}

/* ── microbenchmark matrices ─────────────────────────────────────────────── */

typedef struct {
    uint32_t type;
    size_t rows, cols, bb, blocks_per_row;
    uint64_t seed;
    float scale_std;
    uint32_t subnormal_every;
    uint8_t *dst;
} mat_ctx_t;

static void mat_job(void *vctx, size_t r)
{
    mat_ctx_t *c = (mat_ctx_t *)vctx;
    uint64_t s = row_seed(c->seed, r);
    uint8_t *o = c->dst + r * c->blocks_per_row * c->bb;
    for (size_t b = 0; b < c->blocks_per_row; b++, o += c->bb) {
        double u1 = unif(&s), u2 = unif(&s);
        float z = (float)(sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
        uint16_t h = fwh_f32_to_f16(fabsf(z) * c->scale_std);
        size_t gb = r * c->blocks_per_row + b;
        if (c->subnormal_every && gb % c->subnormal_every == 0)
            h = (uint16_t)(1u + (fwh_splitmix64(&s) & 0x3feu));      /* subnormal, non-zero */
        const int kq = c->type == FORWORD_GGML_Q4_K || c->type == FORWORD_GGML_Q6_K;
        for (size_t k = kq ? 0 : 2; k < c->bb; k += 8) {      /* 32-value blocks: codes after d */
            uint64_t v = fwh_splitmix64(&s);
            size_t n = c->bb - k < 8 ? c->bb - k : 8;
            memcpy(o + k, &v, n);
        }
        /* the fp16 scale fields: d at 0 (Q6_K: at 208), Q4_K's dmin at 2 */
        const size_t d_at = c->type == FORWORD_GGML_Q6_K ? 208 : 0;
        o[d_at] = (uint8_t)h;
        o[d_at + 1] = (uint8_t)(h >> 8);
        if (c->type == FORWORD_GGML_Q4_K) {
            uint16_t hm = fwh_f32_to_f16(fabsf(z) * c->scale_std * 0.5f);
            o[2] = (uint8_t)hm;
            o[3] = (uint8_t)(hm >> 8);
        }
    }
}

size_t fwh_synth_matrix(uint32_t type, size_t rows, size_t cols, uint64_t seed, float scale_std,
                        uint32_t subnormal_every, void *dst, uint32_t threads)
{
    const size_t bb = fwh_block_bytes(type), bv = fwh_block_values(type);
    if (!dst || !bb || type == FORWORD_GGML_F32 || !rows || !cols || cols % bv) return 0;
    mat_ctx_t c = { type, rows, cols, bb, cols / bv, seed, scale_std, subnormal_every, (uint8_t *)dst };
    run_parallel(mat_job, &c, rows, threads);
    return rows * (cols / bv) * bb;
}
