/*
 * ref_driver — drives forword.c's own compiled code (oracle/_ref/libforword_ref.so,
 * built from the reference sources by ref.mk) to write golden vectors.  Used
 * only in the build container by tests/golden/make_golden.py; the outputs are
 * committed as fixtures, this program and the reference build are not.
 *
 * Modes (all binary files are raw little-endian arrays):
 *   gen MODEL MAX_CTX PROMPT.u32 N_GEN OUTDIR LOGIT_STEPS TRACE_STEPS
 *       prefill + greedy as main.c:145-217 with temperature 0, repetition
 *       penalty 1.0 (sampler.c:92) and no EOS stop; per forward f writes a
 *       stats row, logits at the listed forwards, and the residual stream
 *       after every residual add at the listed forwards.  Traced forwards run
 *       the transformer.c:149-326 llama branch through the exported layer
 *       functions and are cross-checked bit-for-bit against transformer_forward.
 *   qmv TYPE IN OUT W X Y           quant_matvec (quant_matvec.c:263-312)
 *   getrow TYPE NCOLS NROWS W OUT   linear_get_row over every row (linear.c:60-151)
 *   rmsnorm N EPS X W OUT           rms_norm (norm.c:7-16)
 *   ropetab NCTX HD BASE OUT        rope_precompute (rope.c:6-17): cos then sin
 *   rope POS NH HD NCTX BASE NEOX QK OUT   rope_apply (rope.c:28-53)
 *   silu N X OUT                    tensor_silu (tensor_ops.c:63-81)
 *   dot N A B OUT                   simd_dot_f32 (simd.h:27-155)
 *   argmax N X OUT                  sampler_argmax (sampler.c:28-32)
 *   q8dec NBYTES IN OUT             q8_0_decode (quant.c:232-263)
 *   sample N TEMP TOPP PEN SEED NHIST LOGITS HIST OUT
 *                                   one decision as main.c:176-188: sampler_rep_penalty
 *                                   over HIST, then sampler_argmax (TEMP <= 0) or
 *                                   sampler_top_p (sampler.c:47-101); OUT = token (u32)
 *                                   and the xorshift64 state after it (u64)
 */
#define _POSIX_C_SOURCE 200809L
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "transformer.h"
#include "attention.h"
#include "ffn.h"
#include "norm.h"
#include "rope.h"
#include "linear.h"
#include "tensor_data.h"
#include "sampler.h"
#include "quant.h"
#include "quant_matvec.h"
#include "tensor_ops.h"
#include "simd.h"

static void *slurp(const char *path, size_t *n)
{
    FILE *f = fopen(path, "rb");
    if (!f) { perror(path); exit(2); }
    fseek(f, 0, SEEK_END);
    long sz = ftell(f);
    fseek(f, 0, SEEK_SET);
    void *p = malloc(sz > 0 ? (size_t)sz : 1);
    if (fread(p, 1, (size_t)sz, f) != (size_t)sz) { perror(path); exit(2); }
    fclose(f);
    if (n) *n = (size_t)sz;
    return p;
}

static void spit(const char *path, const void *p, size_t n)
{
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, 1, n, f) != n) { perror(path); exit(2); }
    fclose(f);
}

static int in_list(const char *list, size_t v)
{
    char buf[1024];
    snprintf(buf, sizeof buf, "%s", list);
    for (char *tok = strtok(buf, ","); tok; tok = strtok(NULL, ","))
        if ((size_t)strtoul(tok, NULL, 10) == v) return 1;
    return 0;
}

/* The block's pre-norm with the reference's own kernels (transformer.c:234-239). */
static void pre_norm(const model_config_t *c, const float *x, const float *w, const float *b, float *out)
{
    if (c->norm_type == NORM_LAYER) layer_norm(x, w, b, out, c->n_embd, c->norm_eps);
    else rms_norm(x, w, out, c->n_embd, c->norm_eps);
}

static const float *vec(const gguf_file_t *g, const char *fmt, size_t l)
{
    char nm[128];
    snprintf(nm, sizeof nm, fmt, l);
    const gguf_tensor_t *t = tensor_find(g, nm);
    return t ? (const float *)tensor_data(g, t, NULL) : NULL;
}

/* transformer.c:149-326 (sequential and parallel residual, RMSNorm and
 * LayerNorm), with the residual stream copied out after each residual add;
 * a parallel-residual layer has one add, recorded in both of its rows. */
static float *traced_forward(transformer_t *t, uint32_t tok, size_t pos, float *trace)
{
    const model_config_t *c = &t->cfg;
    const gguf_file_t *g = &t->g;
    const size_t n = c->n_embd;
    if (linear_get_row(g, tensor_find(g, "token_embd.weight"), tok, t->x)) return NULL;
    if (c->embd_scale != 1.0f)                                      /* transformer.c:179-182 */
        for (size_t i = 0; i < n; i++) t->x[i] *= c->embd_scale;
    if (c->arch == ARCH_GPT2) {                                     /* transformer.c:188-205 */
        if (linear_get_row(g, tensor_find(g, "position_embd.weight"), pos, t->xn)) return NULL;
        for (size_t i = 0; i < n; i++) t->x[i] += t->xn[i];
    }
    for (size_t l = 0; l < c->n_layer; l++) {
        const float *an = vec(g, "blk.%zu.attn_norm.weight", l), *anb = vec(g, "blk.%zu.attn_norm.bias", l);
        const float *fn = vec(g, "blk.%zu.ffn_norm.weight", l), *fnb = vec(g, "blk.%zu.ffn_norm.bias", l);
        pre_norm(c, t->x, an, anb, t->xn);
        if (attention_forward(c, g, &t->kv, t->cos_tab, t->sin_tab, t->xn, t->attn_out, t->scratch, l, pos))
            return NULL;
        if (c->parallel_res) {
            if (ffn_forward(c, g, t->xn, t->ffn_out, t->scratch, l)) return NULL;
            for (size_t i = 0; i < n; i++) t->x[i] += t->attn_out[i] + t->ffn_out[i];
            memcpy(trace + 2 * l * n, t->x, n * 4);
            memcpy(trace + (2 * l + 1) * n, t->x, n * 4);
            continue;
        }
        for (size_t i = 0; i < n; i++) t->x[i] += t->attn_out[i];
        memcpy(trace + 2 * l * n, t->x, n * 4);
        pre_norm(c, t->x, fn, fnb, t->xn);
        if (ffn_forward(c, g, t->xn, t->ffn_out, t->scratch, l)) return NULL;
        for (size_t i = 0; i < n; i++) t->x[i] += t->ffn_out[i];
        memcpy(trace + (2 * l + 1) * n, t->x, n * 4);
    }
    const float *w = vec(g, "output_norm.weight", 0), *b = vec(g, "output_norm.bias", 0);
    if (w) pre_norm(c, t->x, w, b, t->xn);                          /* transformer.c:293-307 */
    else memcpy(t->xn, t->x, n * 4);
    const gguf_tensor_t *ow = tensor_find(g, "output.weight");     /* transformer.c:309-316 */
    if (!ow) ow = tensor_find(g, "lm_head.weight");
    if (!ow) ow = tensor_find(g, "token_embd.weight");
    if (linear_forward(g, ow, NULL, t->xn, t->logits, NULL)) return NULL;
    return t->logits;
}

static int mode_gen(int argc, char **argv)
{
    if (argc < 9) return 2;
    const char *model = argv[2], *outdir = argv[6], *lsteps = argv[7], *tsteps = argv[8];
    size_t max_ctx = strtoul(argv[3], NULL, 10), n_prompt = 0, n_gen = strtoul(argv[5], NULL, 10);
    uint32_t *prompt = (uint32_t *)slurp(argv[4], &n_prompt);
    n_prompt /= 4;
    transformer_t t;
    if (transformer_init(&t, model, max_ctx)) return 3;
    const size_t nv = t.cfg.n_vocab, n = t.cfg.n_embd, L = t.cfg.n_layer;
    size_t n_fwd = n_prompt + n_gen - 1;
    uint32_t *tokens = (uint32_t *)calloc(n_prompt + n_gen, 4);
    double *stats = (double *)calloc(n_fwd * 5, sizeof(double));
    float *trace = (float *)calloc(2 * L * n, 4), *copy = (float *)calloc(nv, 4);
    memcpy(tokens, prompt, n_prompt * 4);
    int mismatch = 0;
    char path[1024];
    for (size_t f = 0; f < n_fwd; f++) {
        uint32_t tok = tokens[f];
        float *lg;
        if (in_list(tsteps, f)) {
            lg = traced_forward(&t, tok, f, trace);
            if (!lg) return 4;
            memcpy(copy, lg, nv * 4);
            lg = transformer_forward(&t, tok, f);
            if (!lg) return 4;
            if (memcmp(copy, lg, nv * 4)) mismatch++;
            snprintf(path, sizeof path, "%s/trace_%zu.f32", outdir, f);
            spit(path, trace, 2 * L * n * 4);
        } else {
            lg = transformer_forward(&t, tok, f);
            if (!lg) return 4;
        }
        if (in_list(lsteps, f)) {
            snprintf(path, sizeof path, "%s/logits_%zu.f32", outdir, f);
            spit(path, lg, nv * 4);
        }
        uint32_t best = sampler_argmax(lg, nv);      /* rep-pen 1.0 is a no-op, sampler.c:92 */
        float second = -INFINITY;
        double sum = 0.0;
        for (size_t i = 0; i < nv; i++) {
            sum += lg[i];
            if (i != best && lg[i] > second) second = lg[i];
        }
        stats[f * 5 + 0] = best;
        stats[f * 5 + 1] = lg[best];
        stats[f * 5 + 2] = second;
        stats[f * 5 + 3] = (double)lg[best] - (double)second;
        stats[f * 5 + 4] = sum;
        if (f + 1 >= n_prompt) tokens[f + 1] = best;
    }
    snprintf(path, sizeof path, "%s/tokens.u32", outdir);
    spit(path, tokens, (n_prompt + n_gen) * 4);
    snprintf(path, sizeof path, "%s/stats.f64", outdir);
    spit(path, stats, n_fwd * 5 * sizeof(double));
    printf("forwards=%zu traced_vs_transformer_forward_mismatch=%d\n", n_fwd, mismatch);
    transformer_free(&t);
    return mismatch ? 5 : 0;
}

int main(int argc, char **argv)
{
    if (argc < 2) return 2;
    const char *m = argv[1];
    size_t sz;
    if (!strcmp(m, "gen")) return mode_gen(argc, argv);
    if (!strcmp(m, "qmv") && argc == 8) {
        uint32_t type = (uint32_t)atoi(argv[2]);
        size_t in = strtoul(argv[3], NULL, 10), out = strtoul(argv[4], NULL, 10);
        void *w = slurp(argv[5], &sz);
        float *x = (float *)slurp(argv[6], NULL), *y = (float *)calloc(out, 4);
        int rc = quant_matvec(w, sz, type, x, y, in, out);
        spit(argv[7], y, out * 4);
        return rc ? 6 : 0;
    }
    if (!strcmp(m, "getrow") && argc == 7) {
        uint32_t type = (uint32_t)atoi(argv[2]);
        size_t cols = strtoul(argv[3], NULL, 10), rows = strtoul(argv[4], NULL, 10);
        void *w = slurp(argv[5], &sz);
        gguf_file_t g;
        memset(&g, 0, sizeof g);
        g.mapping = w; g.file_size = sz; g.data_offset = 0;
        gguf_tensor_t tt;
        memset(&tt, 0, sizeof tt);
        tt.name = (char *)"w"; tt.n_dims = 2; tt.dims[0] = cols; tt.dims[1] = rows;
        tt.ggml_type = type; tt.offset = 0; tt.byte_size = sz;
        float *out = (float *)calloc(rows * cols, 4);
        for (size_t r = 0; r < rows; r++)
            if (linear_get_row(&g, &tt, r, out + r * cols)) return 6;
        spit(argv[6], out, rows * cols * 4);
        return 0;
    }
    if (!strcmp(m, "rmsnorm") && argc == 7) {
        size_t n = strtoul(argv[2], NULL, 10);
        float eps = strtof(argv[3], NULL);
        float *x = (float *)slurp(argv[4], NULL), *w = (float *)slurp(argv[5], NULL);
        float *o = (float *)calloc(n, 4);
        rms_norm(x, w, o, n, eps);
        spit(argv[6], o, n * 4);
        return 0;
    }
    if (!strcmp(m, "ropetab") && argc == 6) {
        size_t nctx = strtoul(argv[2], NULL, 10), hd = strtoul(argv[3], NULL, 10);
        float base = strtof(argv[4], NULL);
        float *t = (float *)calloc(2 * nctx * (hd / 2), 4);
        rope_precompute(t, t + nctx * (hd / 2), nctx, hd, base);
        spit(argv[5], t, 2 * nctx * (hd / 2) * 4);
        return 0;
    }
    if (!strcmp(m, "rope") && argc == 10) {
        size_t pos = strtoul(argv[2], NULL, 10), nh = strtoul(argv[3], NULL, 10);
        size_t hd = strtoul(argv[4], NULL, 10), nctx = strtoul(argv[5], NULL, 10);
        float base = strtof(argv[6], NULL);
        int neox = atoi(argv[7]);
        float *qk = (float *)slurp(argv[8], NULL);
        float *t = (float *)calloc(2 * nctx * (hd / 2), 4);
        rope_precompute(t, t + nctx * (hd / 2), nctx, hd, base);
        rope_apply(qk, pos, nh, hd, t, t + nctx * (hd / 2), neox);
        spit(argv[9], qk, nh * hd * 4);
        return 0;
    }
    if (!strcmp(m, "silu") && argc == 5) {
        size_t n = strtoul(argv[2], NULL, 10);
        float *x = (float *)slurp(argv[3], NULL), *o = (float *)calloc(n, 4);
        tensor_silu(x, o, n);
        spit(argv[4], o, n * 4);
        return 0;
    }
    if (!strcmp(m, "dot") && argc == 6) {
        size_t n = strtoul(argv[2], NULL, 10);
        float *a = (float *)slurp(argv[3], NULL), *b = (float *)slurp(argv[4], NULL);
        float r = simd_dot_f32(a, b, n);
        spit(argv[5], &r, 4);
        return 0;
    }
    if (!strcmp(m, "argmax") && argc == 5) {
        size_t n = strtoul(argv[2], NULL, 10);
        float *x = (float *)slurp(argv[3], NULL);
        uint32_t r = sampler_argmax(x, n);
        spit(argv[4], &r, 4);
        return 0;
    }
    if (!strcmp(m, "q8dec") && argc == 5) {
        size_t n = strtoul(argv[2], NULL, 10);
        void *in = slurp(argv[3], NULL);
        float *o = (float *)calloc(n / 34 * 32, 4);
        if (q8_0_decode(in, n, o, n / 34 * 32)) return 6;
        spit(argv[4], o, n / 34 * 32 * 4);
        return 0;
    }
    if (!strcmp(m, "sample") && argc == 11) {
        size_t n = strtoul(argv[2], NULL, 10), nh = strtoul(argv[7], NULL, 10);
        float temp = strtof(argv[3], NULL), top_p = strtof(argv[4], NULL), pen = strtof(argv[5], NULL);
        uint64_t rng = strtoull(argv[6], NULL, 10);
        float *lg = (float *)slurp(argv[8], NULL);
        uint32_t *hist = nh ? (uint32_t *)slurp(argv[9], NULL) : NULL;
        sampler_rep_penalty(lg, n, hist, nh, pen);
        uint32_t tok = temp <= 0.0f ? sampler_argmax(lg, n) : sampler_top_p(lg, n, temp, top_p, &rng);
        unsigned char out[12];
        memcpy(out, &tok, 4);
        memcpy(out + 4, &rng, 8);
        spit(argv[10], out, 12);
        return 0;
    }
    fprintf(stderr, "ref_driver: bad mode/arguments\n");
    return 2;
}
