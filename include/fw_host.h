/*
 * fw_host.h — host side of the forword MI355X decode path (plain C, no GPU).
 *
 * In a forword.c build the host is the reference's own code: gguf.c opens and
 * mmaps the file, model_config.c reads the config, transformer.c:73-89 builds
 * the RoPE tables, and transformer.c hands all of it to forword_gpu_init (see
 * the integration notes).  This library is the same host role for this
 * repository's tests, benchmark and CLI, written from the GGUF format and the
 * reference's documented behaviour:
 *   - fwh_gguf_*   : GGUF v2/v3 reader over a file mmap or a memory image
 *                    (behaviour of gguf_open, gguf.c:256-353, and tensor_data,
 *                    tensor_data.c:25-62);
 *   - fwh_config   : model_config_load's keys, defaults and type rules
 *                    (model_config.c:61-220);
 *   - fwh_rope_tables : rope_precompute (rope.c:6-17);
 *   - fwh_synth_*  : seeded random-init GGUF writer with its own PRNG and
 *                    Q4_0/Q5_0/Q8_0 quantisers (test and benchmark inputs; the
 *                    reference has no writer).
 */
#ifndef FW_HOST_H
#define FW_HOST_H

#include <stddef.h>
#include <stdint.h>
#include "forword_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ── GGUF reader ─────────────────────────────────────────────────────────── */

typedef struct fwh_gguf fwh_gguf_t;

/* Open and parse a GGUF file (mmap, read-only).  NULL on error; errbuf gets a message. */
fwh_gguf_t *fwh_gguf_open(const char *path, char *errbuf, size_t errcap);
/* Parse a GGUF image already in memory (borrowed: must outlive the handle). */
fwh_gguf_t *fwh_gguf_open_memory(const void *image, size_t size, char *errbuf, size_t errcap);
void fwh_gguf_close(fwh_gguf_t *g);

uint32_t fwh_gguf_version(const fwh_gguf_t *g);
uint32_t fwh_gguf_alignment(const fwh_gguf_t *g);
uint64_t fwh_gguf_data_offset(const fwh_gguf_t *g);
/* Pointer to the data section (mapping + data_offset) and its size. */
const void *fwh_gguf_data(const fwh_gguf_t *g, size_t *size_out);
size_t fwh_gguf_n_tensors(const fwh_gguf_t *g);
/* Descriptor table (n_tensors entries), offsets relative to the data section. */
const forword_gpu_tensor_t *fwh_gguf_tensors(const fwh_gguf_t *g);
/* Index of a tensor by exact name, -1 if absent (tensor_find, tensor_data.c:8-23). */
long fwh_gguf_find_tensor(const fwh_gguf_t *g, const char *name);

/* Metadata lookup: value type (GGUF value type id) or -1 if the key is absent. */
int fwh_gguf_kv_type(const fwh_gguf_t *g, const char *key);
int fwh_gguf_get_u32(const fwh_gguf_t *g, const char *key, uint32_t *out);   /* UINT32/INT32 only */
int fwh_gguf_get_f32(const fwh_gguf_t *g, const char *key, float *out);      /* FLOAT32 only */
/* String value copied into buf (NUL-terminated). */
int fwh_gguf_get_str(const fwh_gguf_t *g, const char *key, char *buf, size_t cap);
/* Element count of an array value, -1 if absent or not an array. */
int64_t fwh_gguf_array_len(const fwh_gguf_t *g, const char *key);

/* ── Model config (model_config_load semantics) ─────────────────────────── */
int fwh_config(const fwh_gguf_t *g, forword_gpu_config_t *cfg);
/* KV length as transformer_init resolves it (transformer.c:43-52): 0 -> min(n_ctx,4096),
 * clamped to n_ctx.  Returns 0 when invalid. */
size_t fwh_resolve_ctx(const forword_gpu_config_t *cfg, size_t max_ctx);

/* ── RoPE tables (rope_precompute, rope.c:6-17) ─────────────────────────── */
void fwh_rope_tables(float *cos_tab, float *sin_tab, size_t n_ctx, size_t head_dim,
                     float freq_base);

/* ── fp16 helpers ────────────────────────────────────────────────────────── */
uint16_t fwh_f32_to_f16(float f);  /* round to nearest even, IEEE binary16 */
float    fwh_f16_to_f32(uint16_t h);

/* ── Deterministic PRNG (splitmix64) and normals (Box-Muller) ───────────── */
uint64_t fwh_splitmix64(uint64_t *state);
/* n normals N(0, std) into out, stream fully determined by seed. */
void fwh_randn(uint64_t seed, float std, float *out, size_t n);

/* ── Quantisers (GGUF/ggml block formats) ───────────────────────────────── */
size_t fwh_block_bytes(uint32_t ggml_type);    /* 18/22/34 for Q4_0/Q5_0/Q8_0, 144/210 for Q4_K/Q6_K,
                                                  4 for F32, 0 unknown */
size_t fwh_block_values(uint32_t ggml_type);   /* values per block: 32, 256 for Q4_K/Q6_K, 1 for F32 */
/* Quantise n (multiple of 32) floats into dst; returns bytes written, 0 on error. */
size_t fwh_quantize(uint32_t ggml_type, const float *src, size_t n, void *dst);

/* ── Synthetic model writer ─────────────────────────────────────────────── */
typedef struct {
    uint32_t n_embd, n_ff, n_layer, n_head, n_head_kv, n_vocab, n_ctx;
    float    rope_freq_base;      /* written as llama.rope.freq_base */
    float    norm_eps;            /* written as llama.attention.layer_norm_rms_epsilon */
    uint32_t linear_type;         /* attn_{q,k,v,output}, ffn_{gate,up,down} */
    uint32_t embd_type;           /* token_embd.weight */
    uint32_t output_type;         /* output.weight */
    uint64_t seed;
    float    w_std;               /* linear/embedding weights N(0, w_std) before quantisation */
    float    norm_std;            /* norm weights 1 + N(0, norm_std), F32 */
    uint32_t threads;             /* 0 = default */
    uint32_t arch;                /* FORWORD_ARCH_*: 0 or LLAMA = llama; QWEN2 adds F32
                                     blk.N.attn_{q,k,v}.bias ~ N(0, 4*w_std); GEMMA writes
                                     no output.weight (the head reuses token_embd); PHI2
                                     writes no ffn_gate and adds F32 biases to the norms
                                     (attn, ffn, output) and to attn_output; GPT2 as phi2
                                     plus position_embd, one attn_qkv (+bias), ffn_up/down
                                     biases and no output.weight (n_head_kv must equal n_head) */
    uint32_t mix_type;            /* 0 = every linear is linear_type; else attn_v and ffn_down of
                                     the even layers are this type (the per-tensor mix of
                                     llama.cpp's *_M files, e.g. Q6_K among Q4_K) */
} fwh_synth_spec_t;

/* Exact byte size of the GGUF image fwh_synth_write would produce. */
size_t fwh_synth_size(const fwh_synth_spec_t *spec);
/* Write the GGUF image into buf (cap >= fwh_synth_size). Returns bytes or 0. */
size_t fwh_synth_write(const fwh_synth_spec_t *spec, void *buf, size_t cap);
/* Write the GGUF image to a file. Returns 0 / -1. */
int fwh_synth_write_file(const fwh_synth_spec_t *spec, const char *path);
/* Anonymous-mmap'd image (for multi-GB models); release with fwh_synth_release. */
void *fwh_synth_alloc(const fwh_synth_spec_t *spec, size_t *size_out);
void  fwh_synth_release(void *image, size_t size);

/*
 * Microbenchmark matrix: rows x cols of `ggml_type` blocks with codes uniform
 * over the format's range (Q4_0 0..15, Q5_0 0..31, Q8_0 -128..127) and fp16
 * scales |N(0,1)|*scale_std.  `subnormal_every` > 0 forces every k-th block
 * scale to a subnormal fp16.  Returns bytes written (rows*cols/32*bb) or 0.
 */
size_t fwh_synth_matrix(uint32_t ggml_type, size_t rows, size_t cols, uint64_t seed,
                        float scale_std, uint32_t subnormal_every, void *dst, uint32_t threads);

/* Threads used by the parallel helpers when 0 is passed (env FW_THREADS, else min(16, cores)). */
uint32_t fwh_default_threads(void);

#ifdef __cplusplus
}
#endif
#endif /* FW_HOST_H */
