/*
 * forword_gpu.h — C ABI of the MI355X (gfx950) decode path for forword.c.
 *
 * The reference runs one token through the model with
 *     float *transformer_forward(transformer_t *t, uint32_t token_id, size_t pos);
 * (transformer.h:48, transformer.c:149-326).  This library is the drop-in
 * replacement for that call and for the kernels below it (quant_matvec.c,
 * attention.c + kv_cache.h, rope.c, norm.c, ffn.c, tensor_ops.c).  The host
 * side (gguf.c loader, model_config.c, tokenizer.c, sampler.c, main.c) stays
 * unchanged and hands this library plain descriptors of what it already owns:
 * the mmap'd GGUF data section, the tensor table and the model config.
 *
 * Conventions (same as the reference, transformer.c:157-176, linear.c:210):
 *   - int-returning calls give 0 on success and -1 on error;
 *   - pointer-returning calls give NULL on error;
 *   - on error a message is printed to stderr and kept for
 *     forword_gpu_last_error(); nothing aborts and no exception crosses the ABI.
 * Threading: one handle = one HIP stream = one calling thread; a handle is not
 * reentrant (the reference is single-threaded too).
 */
#ifndef FORWORD_GPU_H
#define FORWORD_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml block/scalar type ids used on the path (gguf.c:155-174). */
enum {
    FORWORD_GGML_F32  = 0,
    FORWORD_GGML_Q4_0 = 2,
    FORWORD_GGML_Q5_0 = 6,
    FORWORD_GGML_Q8_0 = 8,
    FORWORD_GGML_Q4_K = 12,   /* 256-value super-blocks (quant.c:63-189) */
    FORWORD_GGML_Q6_K = 14
};

/* Architecture / variant enums, same numeric values as model_config.h:12-38. */
enum { FORWORD_ARCH_UNKNOWN = 0, FORWORD_ARCH_GPT2, FORWORD_ARCH_LLAMA, FORWORD_ARCH_QWEN2,
       FORWORD_ARCH_MISTRAL, FORWORD_ARCH_GEMMA, FORWORD_ARCH_PHI2, FORWORD_ARCH_PHI3,
       FORWORD_ARCH_STARCODER, FORWORD_ARCH_FALCON };
enum { FORWORD_NORM_RMS = 0, FORWORD_NORM_LAYER };
enum { FORWORD_ACT_SILU = 0, FORWORD_ACT_GELU, FORWORD_ACT_GELU_FAST, FORWORD_ACT_RELU };
enum { FORWORD_ROPE_NORMAL = 0, FORWORD_ROPE_NEOX, FORWORD_ROPE_NONE };

/*
 * One tensor descriptor: the fields of gguf_tensor_t (gguf.h:16-24) that the
 * forward reads.  `offset` is relative to the GGUF data section, exactly as in
 * the reference (gguf.c:308, tensor_data.c:45).
 */
typedef struct {
    const char *name;
    uint32_t    n_dims;
    uint64_t    dims[4];      /* dims[0] = columns (in), dims[1] = rows (out), linear.c:169-170 */
    uint32_t    ggml_type;
    uint64_t    offset;
    uint64_t    byte_size;
} forword_gpu_tensor_t;

/* The fields of model_config_t (model_config.h:47-89) that the forward reads. */
typedef struct {
    uint32_t arch;            /* FORWORD_ARCH_*                                  */
    uint32_t n_vocab, n_ctx, n_embd, n_layer, n_head, n_head_kv, n_ff, head_dim, n_rot;
    uint32_t norm_type;       /* FORWORD_NORM_*                                  */
    uint32_t act_type;        /* FORWORD_ACT_*                                   */
    uint32_t rope_type;       /* FORWORD_ROPE_*                                  */
    int32_t  use_ffn_gate, use_qkv_bias, use_alibi, parallel_res;
    float    norm_eps, rope_freq_base, rope_freq_scale, embd_scale;
} forword_gpu_config_t;

typedef struct forword_gpu forword_gpu_t;

/* ── Model-level entry points ────────────────────────────────────────────── */

/*
 * Create a handle: upload the GGUF data section (`data`, `data_size` bytes,
 * i.e. mapping + data_offset, gguf.c:339-342) as one device buffer with the
 * tensor offsets preserved, resolve every tensor the forward needs once
 * (tensor_find/tensor_data, tensor_data.c:8-62), allocate the fp32 KV cache in
 * the reference layout [layer][pos][kv_head][head_dim] zero-filled
 * (kv_cache.h:25-37), and upload the host RoPE tables cos_tab/sin_tab of
 * max_ctx*(head_dim/2) floats (rope.c:6-17, transformer.c:73-89).
 * `max_ctx` is the already-resolved KV length (transformer.c:43-52).
 * Replaces the device-side half of transformer_init (transformer.c:14-128).
 * Every block `model_config.c:148-217` describes runs: RMSNorm or LayerNorm
 * (with biases), sequential or parallel residual, gated or plain FFN with
 * silu / gelu / gelu-tanh / relu (GPT-2's with biases), pairwise, NEOX or no
 * RoPE, q/k/v (separate or GPT-2's fused attn_qkv) and output-projection
 * biases, GPT-2's learned position rows, an embedding scale, a head tied to
 * token_embd.  Unknown norm or RoPE codes return -1.
 * head_dim 32/48/64/80/96/128/256 with any GQA group; n_embd and n_ff
 * multiples of the weight block (32 or 256 values).
 */
int forword_gpu_init(forword_gpu_t **out,
                     const void *data, size_t data_size,
                     const forword_gpu_tensor_t *tensors, size_t n_tensors,
                     const forword_gpu_config_t *cfg, size_t max_ctx,
                     const float *cos_tab, const float *sin_tab);

/* Release the handle (transformer_free, transformer.c:130-147). NULL is a no-op. */
void forword_gpu_free(forword_gpu_t *h);

/*
 * One token at position `pos` -> logits[n_vocab] in host memory owned by the
 * handle, valid until the next call (transformer_forward, transformer.c:149-326;
 * ownership transformer.h:45-47).  NULL if pos >= max_ctx or token >= n_vocab
 * (transformer.c:156-164) or on a HIP error.
 */
float *forword_gpu_forward(forword_gpu_t *h, uint32_t token_id, size_t pos);

/*
 * Same step, but only the greedy choice comes back: *next = lowest index of the
 * maximum logit (sampler_argmax, sampler.c:28-32; main.c:184-185 with
 * temperature <= 0 and repetition penalty 1.0, sampler.c:92).
 */
int forword_gpu_forward_argmax(forword_gpu_t *h, uint32_t token_id, size_t pos,
                               uint32_t *next);

/*
 * The CLI's prefill + greedy loop (main.c:145-151, 173-217) run device-resident:
 * prompt[0..n_prompt) at positions 0..n_prompt-1, then n_gen greedy tokens.
 * Costs n_prompt + n_gen - 1 forwards (the last sampled token is not forwarded,
 * main.c:214).  Repetition penalty 1.0 and no EOS stop: out_ids[0..n_gen) are
 * the n_gen argmax tokens.  Requires n_prompt >= 1 and n_prompt+n_gen-1 <= max_ctx.
 */
int forword_gpu_generate_greedy(forword_gpu_t *h, const uint32_t *prompt, size_t n_prompt,
                                size_t n_gen, uint32_t *out_ids);

/*
 * The CLI's generation loop with its sampler, device-resident (main.c:145-217
 * with sampler.c:12-101): prompt[0..n_prompt) token by token, then n_gen
 * tokens, each drawn from the current logits after the repetition penalty over
 * the prompt and the tokens drawn so far (sampler_rep_penalty, once per
 * occurrence), greedily when temperature <= 0 (sampler_argmax) or by top-p with
 * the xorshift64 stream seeded by `seed` (0 -> 12345 as main.c:98-99).  No EOS or
 * stop-string check (main.c:190-208 is the caller's): out_ids[0..n_gen) are the
 * drawn tokens.  Draws equal the reference's except where the random number
 * falls within float rounding of a cumulative-probability boundary (the softmax
 * normaliser is a parallel sum).  Any nucleus size, up to the whole vocabulary
 * (large ones are sorted in a device buffer of the next power of two >= n_vocab
 * keys).  Costs n_prompt + n_gen - 1 forwards.
 */
int forword_gpu_generate(forword_gpu_t *h, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                         float temperature, float top_p, float repetition_penalty, uint64_t seed,
                         uint32_t *out_ids);

/*
 * Continue the greedy loop of the last forword_gpu_generate_greedy for n_steps
 * more forwards, each fed the previous argmax (main.c:173-217, decode part).
 * With out_ids != NULL the n_steps new tokens are copied out and the call
 * waits; with out_ids == NULL the steps are only queued on the handle's stream
 * (for timing with stream events) and the call returns at once.
 */
int forword_gpu_decode(forword_gpu_t *h, size_t n_steps, uint32_t *out_ids);

/*
 * Start a greedy loop at an arbitrary position: forward `token` at `pos` and
 * continue for n_steps forwards in all, each fed the previous argmax
 * (main.c:173-217 entered after a prefill done by other means, e.g.
 * forword_gpu_kv_write of rows [0, pos)).  Composition of transformer_forward
 * and sampler_argmax with no single counterpart in forword.c.  out_ids as in
 * forword_gpu_decode; forword_gpu_decode may continue the loop afterwards.
 */
int forword_gpu_decode_from(forword_gpu_t *h, uint32_t token, size_t pos, size_t n_steps, uint32_t *out_ids);

/*
 * Batched prompt forward: tokens[0..n_tokens) at positions pos0..pos0+n_tokens-1
 * in one pass per layer (every weight matrix read once per 512 tokens, the
 * linears as matrix-core GEMMs), writing their KV rows; returns the logits of
 * the last token, owned by the handle as for forword_gpu_forward.  Replaces the
 * token-by-token prefill loop main.c:145-151 (n_tokens transformer_forward
 * calls, transformer.c:149-326) and is equal to it within the floating-point
 * tolerance (the linears sum in another order).  NULL on invalid arguments
 * (positions past max_ctx, token >= n_vocab) or a HIP error.  A greedy loop
 * continues with forword_gpu_decode_from(h, argmax, pos0 + n_tokens, ...).
 */
float *forword_gpu_prefill(forword_gpu_t *h, const uint32_t *tokens, size_t n_tokens, size_t pos0);

/* Same pass, only the greedy choice of the last token's logits comes back. */
int forword_gpu_prefill_argmax(forword_gpu_t *h, const uint32_t *tokens, size_t n_tokens, size_t pos0,
                               uint32_t *next);

/*
 * Write / read rows of the device KV cache for one layer: positions
 * [pos0, pos0+n_pos), each row n_head_kv*head_dim floats, K post-RoPE
 * (kv_k/kv_v, kv_cache.h:45-51; the append in attention.c:135-140).
 * Either of k / v may be NULL to leave that half untouched.
 */
int forword_gpu_kv_write(forword_gpu_t *h, size_t layer, size_t pos0, size_t n_pos,
                         const float *k, const float *v);
int forword_gpu_kv_read(forword_gpu_t *h, size_t layer, size_t pos0, size_t n_pos,
                        float *k, float *v);

/*
 * Residual stream of the most recent forward: out[2*n_layer][n_embd], row 2l is
 * x after layer l's attention residual (transformer.c:271-272), row 2l+1 after
 * its FFN residual (transformer.c:287-288).  Returns -1 before the first forward.
 */
int forword_gpu_layer_trace(forword_gpu_t *h, float *out);

/* The KV length the handle was created with (kv.n_ctx, kv_cache.h:18). */
size_t forword_gpu_n_ctx(const forword_gpu_t *h);

/* The hipStream_t (as void*) all of the handle's work is queued on. */
void *forword_gpu_stream(const forword_gpu_t *h);

/*
 * Which implementation runs the token step (no counterpart in forword.c, whose
 * step is one C function): 1 = one persistent cooperative kernel per up to 64
 * steps (models whose layer linears share one Q4_0/Q5_0/Q8_0/Q4_K type, or
 * Q4_K with some attn_v/ffn_down in Q6_K; a Q4_0/Q5_0/Q8_0/Q4_K/Q6_K lm-head;
 * n_embd and n_ff multiples of 64, of 256 with K types, head_dim 32/64/128,
 * any GQA group);
 * 0 = one kernel per phase replayed from a hipGraph.  Setting the environment
 * variable FORWORD_GPU_MEGAKERNEL=0 before forword_gpu_init selects 0.
 */
int forword_gpu_step_impl(const forword_gpu_t *h);

/*
 * Wait for the work queued on the handle's stream and report whether it ran
 * to the end: -1 when a persistent step launch gave up at a bounded wait (its
 * results, and those of the launches queued after it, are invalid; the error
 * state is reset so the handle can be used again), 0 otherwise.  The decode
 * calls that only queue work (out_ids == NULL) leave this check to the caller.
 * No counterpart in forword.c, whose step cannot fail this way.
 */
int forword_gpu_status(forword_gpu_t *h);

/*
 * Profiling aid of the persistent step kernel (no counterpart in forword.c):
 * with FORWORD_GPU_PHASE_TIMES=1 set before forword_gpu_init, the kernel
 * stamps the wall clock after every phase.  Writes the mean duration in
 * microseconds of each phase over the steps of the last launch into us[0..n)
 * in step order (per layer: QKV, attention, WO, FFN, down; then the lm-head),
 * each measured barrier to barrier, and returns the number written (-1 when
 * nothing was stamped).
 */
int forword_gpu_phase_times(forword_gpu_t *h, double *us, size_t n);

/* Message of the last failed call on this thread ("" if none). */
const char *forword_gpu_last_error(void);

/* ── Operator-level entry points (device pointers, explicit stream) ─────────
 * `stream` is a hipStream_t passed as void* (NULL = the null stream).  Each
 * call validates sizes exactly like its CPU counterpart and returns -1 on the
 * same conditions. */

/* y[out] = W[out][in] . x[in] for block-quantised W (quant_matvec,
 * quant_matvec.c:263-312, argument list quant_matvec.h:7-15).
 * Types: Q4_0, Q5_0, Q8_0, and F32. */
int forword_gpu_quant_matvec(const void *weights, size_t weights_size, uint32_t ggml_type,
                             const float *input, float *output,
                             size_t input_size, size_t output_size, void *stream);

/* Bit-exact block dequantisation: q8_0_decode (quant.c:232-263), the Q5_0
 * decoder (quant_matvec.c:192-229, linear.c:40-56) and Q4_0 from the GGUF
 * format definition.  output_count = 32 * blocks. */
int forword_gpu_dequant(const void *blocks, size_t blocks_size, uint32_t ggml_type,
                        float *output, size_t output_count, void *stream);

/* One dequantised row of a [rows][n_cols] matrix (linear_get_row, linear.c:60-151). */
int forword_gpu_get_row(const void *weights, size_t weights_size, uint32_t ggml_type,
                        size_t n_cols, size_t row, float *output, void *stream);

/* out = (x*w) * 1/sqrt(mean(x^2)+eps) (rms_norm, norm.c:7-16).  w may be NULL. */
int forword_gpu_rms_norm(const float *x, const float *weight, float *out, size_t n,
                         float eps, void *stream);

/* In-place RoPE of n_heads heads at position pos from the cos/sin tables
 * (rope_apply, rope.c:28-53).  neox_style != 0 pairs (i, half+i). */
int forword_gpu_rope_apply(float *qk, size_t pos, size_t n_heads, size_t head_dim,
                           const float *cos_tab, const float *sin_tab, int neox_style,
                           void *stream);

/*
 * Decode attention core for one layer at position pos (attention.c:142-164):
 * q[n_head][head_dim] against the cache rows 0..pos of k_cache/v_cache (one
 * layer's slice, [n_ctx][n_head_kv][head_dim]); out[n_head][head_dim].
 * GQA maps query head h to kv head h / (n_head/n_head_kv) (attention.c:142,147).
 */
int forword_gpu_attention(const float *q, const float *k_cache, const float *v_cache,
                          float *out, size_t n_head, size_t n_head_kv, size_t head_dim,
                          size_t n_ctx, size_t pos, void *stream);

/*
 * forword_gpu_attention without allocating: no counterpart in the reference.
 * For callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, validation and results as forword_gpu_attention; the split
 * partials (n_head x splits x (head_dim + 2) floats, splits as that call
 * chooses them) live in a fixed 8 MiB device array per GPU, and a call whose
 * partials exceed it returns -1.  The array is shared by every call on that
 * GPU: calls that overlap on one GPU race.
 */
int forword_gpu_attention_noalloc(const float *q, const float *k_cache, const float *v_cache,
                                  float *out, size_t n_head, size_t n_head_kv, size_t head_dim,
                                  size_t n_ctx, size_t pos, void *stream);

/* out = silu(gate) * up, n elements (ffn.c:88-91,103-104 with apply_silu ffn.c:17-25). */
int forword_gpu_silu_mul(const float *gate, const float *up, float *out, size_t n, void *stream);

/* h[n_ff] = silu(W_gate . x) * (W_up . x), the gated FFN up to the down
 * projection (ffn.c:82-104) as one fused GEMV; both weights of one ggml type,
 * [n_ff][n_in] each. */
int forword_gpu_ffn_swiglu(const void *w_gate, const void *w_up, size_t weights_size, uint32_t ggml_type,
                           const float *x, float *h, size_t n_in, size_t n_ff, void *stream);

/* tensor_ops.c counterparts (tensor_ops.h:6-33). */
int forword_gpu_tensor_matvec_f32(const float *weights, const float *x, float *y,
                                  size_t rows, size_t cols, void *stream);
int forword_gpu_tensor_add(const float *a, const float *b, float *out, size_t n, void *stream);
int forword_gpu_tensor_rms_norm(const float *x, const float *weight, float *out, size_t n,
                                float epsilon, void *stream);
int forword_gpu_tensor_silu(const float *x, float *out, size_t n, void *stream);

/* *out_index = lowest index of the maximum of logits[0..n) (sampler_argmax,
 * sampler.c:28-32: strict '>' scan from index 0, so a NaN never wins and a NaN
 * at index 0 makes the answer 0).  out_index is a device pointer. */
int forword_gpu_argmax(const float *logits, size_t n, uint32_t *out_index, void *stream);

/* ── Device memory plumbing (no counterpart in the reference: the CPU code
 * works on host memory).  Used by callers of the operator-level entry points. */
void *forword_gpu_dev_alloc(size_t bytes);
int   forword_gpu_dev_free(void *ptr);
int   forword_gpu_memcpy_h2d(void *dst, const void *src, size_t bytes);
int   forword_gpu_memcpy_d2h(void *dst, const void *src, size_t bytes);
int   forword_gpu_memset(void *dst, int value, size_t bytes);
int   forword_gpu_synchronize(void *stream);

#ifdef __cplusplus
}
#endif
#endif /* FORWORD_GPU_H */
