// Host-side launch interface of the gfx950 kernels (internal to libforword_gpu.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fw {

// ggml type ids on the path (gguf.c:155-174)
enum : uint32_t { kF32 = 0, kQ4_0 = 2, kQ5_0 = 6, kQ8_0 = 8, kQ4_K = 12, kQ6_K = 14 };
// Q6_K rows re-laid out for the persistent step kernel (no ggml counterpart):
// each 64-value quarter of a super-block as one 56-byte, 4-byte-aligned record,
// 224 bytes per super-block (see repack_q6k).
constexpr uint32_t kQ6_KR = 0x10e;

// Device-resident step state read by every kernel of a token step, so one
// captured graph serves every position.
struct StepState {
    uint32_t token;      // token fed at this step
    uint32_t pos;        // its position
    uint32_t n_prompt;   // greedy loop: prompt length
    uint32_t next;       // argmax of this step's logits
    uint32_t greedy;     // 1 inside generate_greedy: advance token/pos on device
    uint32_t pad[3];
};

enum Epi : int { EPI_STORE = 0, EPI_QKV = 1, EPI_RESID = 2, EPI_SWIGLU = 3 };

// Activation codes of the gated FFN (ffn.c:88-101): silu (also the default for
// any other code), gelu with erf (ffn.c:27-31), gelu with tanh (ffn.c:33-42).
enum FfnAct : uint32_t { ACT_SILU = 0, ACT_GELU = 1, ACT_GELU_TANH = 2, ACT_RELU = 3 };

// One GEMV launch over up to three weight matrices that share the input x and
// the column count (fused QKV; gate+up).  Rows of matrix s are rows[s].
struct QmvArgs {
    const uint8_t *w[3];
    uint32_t rows[3];
    uint32_t n_seg;
    uint32_t role_base;        // QKV: role of matrix 0 (0 = Q, 1 = K, 2 = V) when launched apart
    uint32_t n_cols;
    uint64_t row_bytes;
    uint32_t n_groups;
    uint32_t group_base[4];
    const float *x;
    float *out[3];             // STORE: per-matrix outputs; QKV: by role q, K cache, V cache (layer slices)
                               // RESID: residual stream x (updated in place); SWIGLU: h
    float *trace;              // RESID: copy of the updated residual (may be null)
    const float *cos_tab, *sin_tab;
    const float *bias[3];      // QKV: F32 bias by role (attn_{q,k,v}.bias) added before RoPE;
                               // STORE: by segment; RESID: bias[0] added to the product; or null
    const float *addend;       // RESID: x += addend + product (parallel residual), or null
    float *trace2;             // RESID: second copy of the updated residual (may be null)
    const StepState *state;
    uint32_t head_dim;
    uint32_t kv_dim;           // n_head_kv * head_dim (K/V cache row length)
    // Input RMSNorm folded into the load of x (norm.c:7-16): x_j -> (x_j*norm_w[j])*scale,
    // scale read from *norm_scale.  Off when norm_w is null.
    const float *norm_w;
    const float *norm_scale;
    // RESID only: publish 1/sqrt(mean(x_new^2)+eps) of the updated residual for the
    // next RMSNorm (off when scale_out is null): per-block partials in pss[], the
    // last block to take a ticket sums them in block order.
    float *pss;
    uint32_t *ticket;
    float *scale_out;
    float norm_eps;
    uint32_t act;              // SWIGLU: FfnAct of the gate (silu / gelu / gelu-tanh)
    uint32_t store_act;        // STORE: 0, or 1 + FfnAct applied after the bias (plain FFN up, ffn.c:143-160)
};

// Rows computed by one wave of the GEMV kernels.
constexpr int kRowsPerWave = 4;

hipError_t launch_qmv(uint32_t type, int epi, QmvArgs a, hipStream_t s);
// Fill group bookkeeping of QmvArgs for the given epilogue.
void qmv_plan(QmvArgs &a, int epi);
// Whether matrices of this type/column count/base alignment use the
// paired-block (dword-aligned) path.
bool qmv_pair_ok(uint32_t type, uint32_t n_cols, const void *base);

hipError_t launch_rmsnorm(const float *x, const float *w, float *out, uint32_t n, float eps,
                          hipStream_t s);
// RMSNorm of `rows` consecutive rows of n floats (one workgroup each).
hipError_t launch_rmsnorm_rows(const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps,
                               hipStream_t s);
hipError_t launch_embed(const uint8_t *w, uint32_t type, uint32_t n_cols, uint32_t n_rows,
                        const StepState *st, const uint32_t *token_override, float embd_scale, float *x,
                        float *scale_out, float norm_eps, hipStream_t s);
hipError_t launch_get_row(const uint8_t *w, uint32_t type, uint32_t n_cols, uint32_t row, float *out,
                          hipStream_t s);
hipError_t launch_dequant(const uint8_t *blocks, uint32_t type, uint64_t n_blocks, float *out,
                          hipStream_t s);

// Split-K decode attention: partials [n_head][n_splits][head_dim + 2], then combine.
uint32_t attn_splits(uint32_t max_ctx, uint32_t n_kv);
// Attention kernels: head_dim 32/48/64/80/96/128/256, any GQA group (walked in
// sub-groups of attn_sub_group query heads per workgroup).
bool attn_supported(uint32_t head_dim, uint32_t group);
uint32_t attn_epl(uint32_t head_dim);
uint32_t attn_sub_group(uint32_t head_dim, uint32_t group);
hipError_t launch_attention(const float *q, const float *kc, const float *vc, float *part, float *out,
                            uint32_t n_head, uint32_t n_kv, uint32_t head_dim, uint32_t n_splits,
                            const StepState *st, uint32_t pos_host, hipStream_t s);

// y = W x for Q4_0 / Q5_0 / Q8_0 rows of whole block pairs (fw_gemv.hip);
// hipErrorNotSupported for other types, shapes or alignments (the caller then
// uses the general kernel).
hipError_t launch_gemv(uint32_t type, const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                       uint32_t n_cols, hipStream_t s);
hipError_t launch_set_state(StepState *st, const StepState &v, hipStream_t s);
hipError_t launch_argmax(const float *x, uint32_t n, float *pv, uint32_t *pi, uint32_t *counter,
                         uint32_t *out, StepState *st, const uint32_t *prompt, uint32_t *ids,
                         uint32_t n_blocks, hipStream_t s);
uint32_t argmax_blocks(uint32_t n);

hipError_t launch_rope(float *qk, uint32_t pos, uint32_t n_heads, uint32_t head_dim, const float *cos_tab,
                       const float *sin_tab, int neox, hipStream_t s);
hipError_t launch_silu_mul(const float *g, const float *u, float *out, uint64_t n, hipStream_t s);
// out = act(x + bias[i % period]) in place or not, FfnAct code (ffn.c:143-160, plain FFN;
// the bias is GPT-2's ffn_up.bias, may be null).
hipError_t launch_act(const float *x, float *out, uint64_t n, uint32_t act, hipStream_t s,
                      const float *bias = nullptr, uint32_t period = 1);
// x[r] += position-embedding row (st ? st->pos : p0) + r, r < rows (transformer.c:188-205).
hipError_t launch_pos_add(const uint8_t *w, uint32_t type, uint64_t row_bytes, uint32_t n, const StepState *st,
                          uint32_t p0, uint32_t rows, float *x, hipStream_t s);
// layer_norm (norm.c:18-40) of `rows` consecutive rows of n floats; w and b may be null.
hipError_t launch_layernorm(const float *x, const float *w, const float *b, float *out, uint32_t n, float eps,
                            hipStream_t s, uint32_t rows = 1);
// x += (a + bias[i % n]) + b2 over count floats (bias, b2 may be null).
hipError_t launch_resid_add(float *x, const float *a, const float *bias, const float *b2, uint64_t count, uint32_t n,
                            hipStream_t s);
// NEOX RoPE (rope.c:44-51) at the step's position: q heads in place and the K
// cache row at pos of this layer.
hipError_t launch_rope_neox_step(float *q, float *kc_layer, uint32_t n_head, uint32_t n_kv, uint32_t hd,
                                 const float *cos_tab, const float *sin_tab, const StepState *st, hipStream_t s);
// out = act(g) * u with an FfnAct code (ffn.c:88-104).
hipError_t launch_act_mul(const float *g, const float *u, float *out, uint64_t n, uint32_t act, hipStream_t s);
hipError_t launch_silu(const float *x, float *out, uint64_t n, hipStream_t s);
hipError_t launch_add(const float *a, const float *b, float *out, uint64_t n, hipStream_t s);

// Device-resident sampling (fw_sample.hip): the xorshift64 state of the
// generation loop and an error flag (a top-p decision without any candidate).
struct SampleState {
    uint64_t rng;
    uint32_t err;
    uint32_t pad;
};
// Blocks of the sampler's element-wise kernels (part needs 512 floats).
uint32_t samp_blocks(uint32_t n);
// One decision on logits[n]: repetition penalty by history counts, greedy
// (temperature <= 0) or top-p; the token goes to ids[g], st->token and counts.
// buf: n floats; part: 512 floats; bcnt/bsum: 1024 zeroed buckets (cleared again);
// gkeys: the next power of two >= n 64-bit keys (candidates beyond the cap that
// the LDS sort holds are sorted there).
hipError_t launch_sample(const float *logits, uint32_t n, const uint32_t *counts, float temperature, float top_p,
                         float penalty, float *buf, float *part, uint32_t *bcnt, unsigned long long *bsum,
                         uint64_t *gkeys, uint32_t cap, SampleState *ss, StepState *st, uint32_t *ids, uint32_t g,
                         uint32_t *counts_rw, hipStream_t s);

// Batched prompt forward (fw_prefill.hip).
// Up to three weight matrices of one type and column count computed as one
// output of end[n_seg-1] rows: matrix i gives rows end[i-1] .. end[i]-1.
struct GemmW {
    const uint8_t *w[3];
    uint64_t rb[3];
    uint32_t end[3];
    uint32_t n_seg;
};
hipError_t launch_gemm_qs(uint32_t type, const float *x, uint32_t ldx, const GemmW &g, float *y, uint32_t ldy,
                          uint32_t n_tok, uint32_t n_in, bool accumulate, hipStream_t s);
// Y[t][r] (+)= Σ_k X[t][k]·W[r][k] for t < n_tok, r < n_out: X fp32 rows ldx
// apart, W Q4_0/Q5_0/Q8_0 rows of n_in columns, Y rows ldy apart.
hipError_t launch_gemm_q(uint32_t type, const float *x, uint32_t ldx, const uint8_t *w, uint64_t row_bytes, float *y,
                         uint32_t ldy, uint32_t n_tok, uint32_t n_out, uint32_t n_in, bool accumulate,
                         hipStream_t s);
// X[t] = embedding row tokens[t] (times embd_scale when it is not 1).
hipError_t launch_embed_rows(const uint8_t *w, uint32_t type, uint32_t n_cols, const uint32_t *tokens,
                             uint32_t n_tok, float embd_scale, float *x, hipStream_t s);
// Rows [q | k | v] ld floats apart at positions pos0..: RoPE on q in place, K
// (rotated) and V appended to the layer's cache rows.
hipError_t launch_rope_append(float *qkv, const float *bias, int neox, uint32_t ld, uint32_t n_tok, uint32_t n_head,
                              uint32_t n_kv, uint32_t hd,
                              uint32_t pos0, const float *cos_tab, const float *sin_tab, float *kc_layer,
                              float *vc_layer, hipStream_t s);
// Causal attention of the n_tok rows' queries over cache rows 0..pos0+t.
hipError_t launch_attn_prefill(const float *qkv, uint32_t ld, uint32_t n_tok, const float *kc_layer,
                               const float *vc_layer, float *out, uint32_t n_head, uint32_t n_kv, uint32_t hd,
                               uint32_t pos0, hipStream_t s);
} // namespace fw
