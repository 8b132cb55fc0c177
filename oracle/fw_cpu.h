/*
 * fw_cpu — CPU restatement of forword.c's per-token forward.  TEST
 * INFRASTRUCTURE ONLY: the oracle the HIP path is checked against and the
 * CPU baseline of the benchmark.  Nothing in the product calls it.
 *
 * Every function reproduces the reference's fp32 operation order on its
 * AVX2+FMA build (`-O2 -std=c11 -march=native`, which turns floating-point
 * contraction off, so FMAs exist only where the reference calls an FMA
 * intrinsic).  The citation on each function is the code it restates.
 *
 * Pinning (what checks each function independently of this restatement):
 *   fwc_half_to_float   all 65536 inputs vs numpy float16->float32
 *   fwc_dot_f32         test_runner.c:207-223 (lengths 1..67), float64 bound
 *   fwc_dequant Q8_0    test_runner.c:110-126 KAT, reference q8_0_decode over all codes
 *   fwc_dequant Q5_0    reference Q5_0 decoder over all codes and bit positions
 *   fwc_dequant Q4_0    parity unpinned by the reference (no Q4_0 decoder exists,
 *                       quant_matvec.c:52-62); pinned by the GGUF format closed form
 *                       d*(q-8) over all 16 codes, linearity and one-hot columns
 *   fwc_quant_matvec    test_runner.c:161-178 KAT (=64), reference quant_matvec
 *                       bit-exact on Q8_0/Q5_0; Q4_0 as above
 *   fwc_rms_norm        test_runner.c:30-41 invariant, reference rms_norm bit-exact
 *   fwc_rope_apply      test_runner.c:60-90 (pos 0 identity), reference bit-exact
 *   fwc_softmax/attention/ffn/forward  reference transformer_forward bit-exact
 *                       (golden fixtures of the llama, qwen2, gemma, phi2 and
 *                       gpt2 blocks), per-layer residual stream; the gpt2
 *                       fixture pins learned positions, the fused attn_qkv and
 *                       the FFN biases
 *   fwc_layer_norm      the phi2 fixture (bit-exact through the whole forward)
 *   fwc_gelu_fast       the gemma and phi2 fixtures; float64 closed form
 *   fwc_gelu            float64 closed form only (no fixture selects it)
 *   fwc_argmax          test_runner.c:93-96, tie and NaN rules
 */
#ifndef FW_CPU_H
#define FW_CPU_H

#include <stddef.h>
#include <stdint.h>
#include "../include/forword_gpu.h"

#ifdef __cplusplus
extern "C" {
#endif

float    fwc_half_to_float(uint16_t h);
void     fwc_half_to_float_n(const uint16_t *h, float *out, size_t n);
float    fwc_dot_f32(const float *a, const float *b, size_t n);
int      fwc_dequant(const void *blocks, size_t bytes, uint32_t type, float *out, size_t count);
int      fwc_quant_matvec(const void *w, size_t w_size, uint32_t type, const float *x, float *y,
                          size_t in, size_t out);
void     fwc_rms_norm(const float *x, const float *w, float *out, size_t n, float eps);
void     fwc_rope_apply(float *qk, size_t pos, size_t n_heads, size_t hd, const float *cos_tab,
                        const float *sin_tab, int neox);
void     fwc_softmax(float *x, size_t n);
void     fwc_silu(float *x, size_t n);
void     fwc_gelu(float *x, size_t n);
void     fwc_gelu_fast(float *x, size_t n);
void     fwc_layer_norm(const float *x, const float *w, const float *b, float *out, size_t n, float eps);
uint32_t fwc_argmax(const float *x, size_t n);
/* attention core (attention.c:142-164) over one layer's KV slice */
void     fwc_attention_core(const float *q, const float *kc, const float *vc, float *out,
                            size_t n_head, size_t n_kv, size_t hd, size_t pos, float *scores);
/* tensor_ops.c restatements */
int      fwc_tensor_matvec_f32(const float *w, const float *x, float *y, size_t rows, size_t cols);

/* Row-parallel worker count for matvecs (results are identical for any count). */
void     fwc_set_threads(int n);

typedef struct fwc_model fwc_model_t;
fwc_model_t *fwc_model_init(const void *data, size_t data_size, const forword_gpu_tensor_t *tensors,
                            size_t n_tensors, const forword_gpu_config_t *cfg, size_t max_ctx,
                            const float *cos_tab, const float *sin_tab);
void     fwc_model_free(fwc_model_t *m);
/* transformer_forward: logits owned by the model, NULL on error. */
float   *fwc_forward(fwc_model_t *m, uint32_t token, size_t pos);
/* residual stream after each residual add of the last forward: [2*n_layer][n_embd] */
const float *fwc_trace(const fwc_model_t *m);
float   *fwc_kv_k(fwc_model_t *m, size_t layer, size_t pos);   /* row [n_kv*hd] */
float   *fwc_kv_v(fwc_model_t *m, size_t layer, size_t pos);
/* prefill + greedy (rep-pen 1.0, no EOS): out_ids[n_gen] */
int      fwc_generate_greedy(fwc_model_t *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                             uint32_t *out_ids);
/* one sampling decision (sampler.c:12-101, main.c:176-188): repetition penalty over
 * hist, then argmax (temperature <= 0) or top-p with the xorshift64 state *rng */
uint32_t fwc_sample(const float *logits, size_t n, const uint32_t *hist, size_t n_hist, float temperature,
                    float top_p, float penalty, uint64_t *rng);
/* prefill + sampled generation (main.c:145-217 without EOS/stop strings), seed 0 -> 12345 */
int      fwc_generate_sampled(fwc_model_t *m, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                              float temperature, float top_p, float penalty, uint64_t seed, uint32_t *out_ids);

#ifdef __cplusplus
}
#endif
#endif
