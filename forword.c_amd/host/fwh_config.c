/*
 * Model config from GGUF metadata with model_config_load's rules
 * (model_config.c:61-220):
 *   - `general.architecture` picks the key prefix and the arch id (:11-23,65-72);
 *   - dimension keys are read only when UINT32/INT32, float keys only when
 *     FLOAT32; any other type silently falls back to the default (:34-51);
 *   - head_dim = n_embd / n_head (:100); n_rot defaults to head_dim (:103-104);
 *   - eps: `attention.layer_norm_rms_epsilon`, and if that yields exactly the
 *     1e-5 default, `attention.layer_norm_epsilon` (:107-113);
 *   - n_vocab from `tokenizer.ggml.token_type_count`, else dims[1] of
 *     output.weight / lm_head.weight, else dims[0] of a 1-D one (:133-146);
 *   - per-architecture defaults (:148-217).
 * RoPE tables follow rope_precompute (rope.c:6-17): theta = pos / base^(2i/hd)
 * in float with libm powf/cosf/sinf, so a host built against the same libm
 * produces the reference's tables bit for bit.
 */
#define _POSIX_C_SOURCE 200809L
#include "fw_host.h"

#include <math.h>
#include <stdio.h>
#include <string.h>

static const struct { const char *name; uint32_t id; } k_arch[] = {
    { "llama", FORWORD_ARCH_LLAMA }, { "qwen2", FORWORD_ARCH_QWEN2 },
    { "mistral", FORWORD_ARCH_MISTRAL }, { "gemma", FORWORD_ARCH_GEMMA },
    { "gemma2", FORWORD_ARCH_GEMMA }, { "phi2", FORWORD_ARCH_PHI2 },
    { "phi3", FORWORD_ARCH_PHI3 }, { "starcoder", FORWORD_ARCH_STARCODER },
    { "falcon", FORWORD_ARCH_FALCON }, { "gpt2", FORWORD_ARCH_GPT2 },
};

static uint32_t meta_u32(const fwh_gguf_t *g, const char *arch, const char *suffix, uint32_t def)
{
    char key[160];
    uint32_t v;
    if (arch) snprintf(key, sizeof key, "%s.%s", arch, suffix);
    else snprintf(key, sizeof key, "%s", suffix);
    return fwh_gguf_get_u32(g, key, &v) == 0 ? v : def;
}

static float meta_f32(const fwh_gguf_t *g, const char *arch, const char *suffix, float def)
{
    char key[160];
    float v;
    snprintf(key, sizeof key, "%s.%s", arch, suffix);
    return fwh_gguf_get_f32(g, key, &v) == 0 ? v : def;
}

int fwh_config(const fwh_gguf_t *g, forword_gpu_config_t *c)
{
    char arch[64];
    memset(c, 0, sizeof(*c));
    if (fwh_gguf_get_str(g, "general.architecture", arch, sizeof arch) != 0) {
        fprintf(stderr, "fwh_config: missing general.architecture\n");
        return -1;
    }
    c->arch = FORWORD_ARCH_UNKNOWN;
    for (size_t i = 0; i < sizeof k_arch / sizeof k_arch[0]; i++)
        if (!strcmp(k_arch[i].name, arch)) { c->arch = k_arch[i].id; break; }

    c->n_embd = meta_u32(g, arch, "embedding_length", 0);
    if (!c->n_embd) { fprintf(stderr, "fwh_config: missing n_embd\n"); return -1; }
    c->n_layer = meta_u32(g, arch, "block_count", 0);
    if (!c->n_layer) { fprintf(stderr, "fwh_config: missing n_layer\n"); return -1; }
    c->n_head = meta_u32(g, arch, "attention.head_count", 0);
    if (!c->n_head) { fprintf(stderr, "fwh_config: missing n_head\n"); return -1; }
    c->n_head_kv = meta_u32(g, arch, "attention.head_count_kv", c->n_head);
    c->n_ff = meta_u32(g, arch, "feed_forward_length", 0);
    c->n_ctx = meta_u32(g, arch, "context_length", 2048);
    c->head_dim = c->n_embd / c->n_head;
    c->n_rot = meta_u32(g, arch, "rope.dimension_count", c->head_dim);

    c->norm_eps = meta_f32(g, arch, "attention.layer_norm_rms_epsilon", 1e-5f);
    if (c->norm_eps == 1e-5f)
        c->norm_eps = meta_f32(g, arch, "attention.layer_norm_epsilon", 1e-5f);
    c->rope_freq_base = meta_f32(g, arch, "rope.freq_base", 10000.0f);
    c->rope_freq_scale = meta_f32(g, arch, "rope.scale_linear", 1.0f);

    c->n_vocab = meta_u32(g, NULL, "tokenizer.ggml.token_type_count", 0);
    if (!c->n_vocab) {
        const forword_gpu_tensor_t *t = fwh_gguf_tensors(g);
        size_t n = fwh_gguf_n_tensors(g);
        for (size_t i = 0; i < n; i++) {
            if (!strcmp(t[i].name, "output.weight") || !strcmp(t[i].name, "lm_head.weight")) {
                if (t[i].n_dims >= 2) c->n_vocab = (uint32_t)t[i].dims[1];
                else c->n_vocab = (uint32_t)t[i].dims[0];
                break;
            }
        }
    }
    if (!c->n_vocab) {
        /* transformer_init falls back to the tokenizer's vocabulary size
         * (transformer.c:59-60), i.e. the length of tokenizer.ggml.tokens. */
        int64_t nt = fwh_gguf_array_len(g, "tokenizer.ggml.tokens");
        if (nt > 0) c->n_vocab = (uint32_t)nt;
    }

    switch (c->arch) {
    case FORWORD_ARCH_LLAMA: case FORWORD_ARCH_MISTRAL: case FORWORD_ARCH_PHI3:
    case FORWORD_ARCH_STARCODER:
        c->norm_type = FORWORD_NORM_RMS; c->act_type = FORWORD_ACT_SILU; c->use_ffn_gate = 1;
        c->rope_type = FORWORD_ROPE_NORMAL; c->embd_scale = 1.0f;
        break;
    case FORWORD_ARCH_QWEN2:
        c->norm_type = FORWORD_NORM_RMS; c->act_type = FORWORD_ACT_SILU; c->use_ffn_gate = 1;
        c->rope_type = FORWORD_ROPE_NORMAL; c->use_qkv_bias = 1; c->embd_scale = 1.0f;
        if (c->rope_freq_base < 10001.0f) c->rope_freq_base = 1000000.0f;
        break;
    case FORWORD_ARCH_GEMMA:
        c->norm_type = FORWORD_NORM_RMS; c->act_type = FORWORD_ACT_GELU_FAST; c->use_ffn_gate = 1;
        c->rope_type = FORWORD_ROPE_NORMAL; c->embd_scale = sqrtf((float)c->n_embd);
        break;
    case FORWORD_ARCH_PHI2:
        c->norm_type = FORWORD_NORM_LAYER; c->act_type = FORWORD_ACT_GELU_FAST; c->use_ffn_gate = 0;
        c->rope_type = FORWORD_ROPE_NEOX; c->parallel_res = 1; c->embd_scale = 1.0f;
        break;
    case FORWORD_ARCH_FALCON:
        c->norm_type = FORWORD_NORM_LAYER; c->act_type = FORWORD_ACT_GELU; c->use_ffn_gate = 0;
        c->rope_type = FORWORD_ROPE_NORMAL; c->embd_scale = 1.0f;
        break;
    case FORWORD_ARCH_GPT2:
        c->norm_type = FORWORD_NORM_LAYER; c->act_type = FORWORD_ACT_GELU; c->use_ffn_gate = 0;
        c->rope_type = FORWORD_ROPE_NONE; c->use_qkv_bias = 1; c->embd_scale = 1.0f;
        c->n_head_kv = c->n_head; c->n_rot = 0;
        break;
    default:
        c->norm_type = FORWORD_NORM_RMS; c->act_type = FORWORD_ACT_SILU; c->use_ffn_gate = 1;
        c->rope_type = FORWORD_ROPE_NORMAL; c->embd_scale = 1.0f;
        break;
    }
    return 0;
}

size_t fwh_resolve_ctx(const forword_gpu_config_t *c, size_t max_ctx)
{
    if (!max_ctx) max_ctx = c->n_ctx < 4096 ? c->n_ctx : 4096;
    if (max_ctx > c->n_ctx) max_ctx = c->n_ctx;
    return max_ctx;
}

void fwh_rope_tables(float *cos_tab, float *sin_tab, size_t n_ctx, size_t head_dim, float freq_base)
{
    size_t half = head_dim / 2;
    for (size_t pos = 0; pos < n_ctx; pos++) {
        for (size_t i = 0; i < half; i++) {
            float theta = (float)pos / powf(freq_base, (float)(2 * i) / (float)head_dim);
            cos_tab[pos * half + i] = cosf(theta);
            sin_tab[pos * half + i] = sinf(theta);
        }
    }
}
