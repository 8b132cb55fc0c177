// forword_gpu_* C ABI: the per-token forward of forword.c on one MI355X.
//
// transformer_forward (transformer.c:149-326) becomes one token step queued on
// the handle's stream: embedding row -> per layer [RMSNorm, fused QKV GEMV +
// RoPE + KV append, split-K attention, Wo GEMV + residual, RMSNorm, fused
// gate/up GEMV + SiLU*up, down GEMV + residual] -> RMSNorm -> lm-head GEMV ->
// argmax.  The step reads token and position from a small device-resident
// StepState, so the greedy loop (main.c:145-217) runs on the device: the
// argmax feeds the next token without a host round trip.
//
// Two implementations of the step: for models whose layer linears share one
// Q4_0/Q5_0/Q8_0/Q4_K type (Q4_K with some Q6_K attn_v/ffn_down included), a
// persistent cooperative kernel runs whole steps (up to 64 per launch) with
// grid barriers between phases (fw_step.hip); otherwise
// (or with FORWORD_GPU_MEGAKERNEL=0) one kernel per phase, captured once as a
// hipGraph and replayed per position.
#include "fw_kernels.h"
#include "fw_step.h"
#include "forword_gpu.h"

#include <hip/hip_runtime.h>
#include <algorithm>
#include <math.h>
#include <mutex>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <vector>

using namespace fw;

static thread_local char g_err[512] = "";

static void set_err(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
    fprintf(stderr, "forword_gpu: %s\n", g_err);
}

#define HIPCHK(call, what)                                                               \
    do {                                                                                 \
        hipError_t e_ = (call);                                                          \
        if (e_ != hipSuccess) {                                                          \
            set_err("%s: %s", what, hipGetErrorString(e_));                              \
            return -1;                                                                   \
        }                                                                                \
    } while (0)

extern "C" const char *forword_gpu_last_error(void) { return g_err; }

namespace {

struct Lin {
    const uint8_t *w = nullptr;
    uint32_t type = 0, in = 0, out = 0;
    uint64_t row_bytes = 0;
};

struct Layer {
    const float *attn_norm = nullptr, *ffn_norm = nullptr;
    const float *attn_norm_b = nullptr, *ffn_norm_b = nullptr;   // LayerNorm biases, or null
    const float *bo = nullptr;     // attn_output.bias, or null
    const float *bu = nullptr, *bd = nullptr;   // GPT-2 ffn_up.bias / ffn_down.bias, or null
    const float *bqkv = nullptr;   // attn_q|k|v.bias concatenated [n_embd + 2 kv_dim] (qwen2), or null
    Lin q, k, v, o, gate, up, down;
};

uint64_t type_row_bytes(uint32_t type, uint64_t cols)
{
    switch (type) {
    case kF32: return cols * 4;
    case kQ4_0: return cols / 32 * 18;
    case kQ5_0: return cols / 32 * 22;
    case kQ8_0: return cols / 32 * 34;
    case kQ4_K: return cols / 256 * 144;
    case kQ6_K: return cols / 256 * 210;
    default: return 0;
    }
}

// The gated FFN's activation (ffn.c:88-101): GELU and GELU-tanh by their codes,
// silu for silu and for every other code (the switch's default).
static uint32_t ffn_act_code(const forword_gpu_config_t &c)
{
    return c.act_type == FORWORD_ACT_GELU        ? fw::ACT_GELU
         : c.act_type == FORWORD_ACT_GELU_FAST ? fw::ACT_GELU_TANH
                                               : fw::ACT_SILU;
}

// The plain FFN's activation (ffn.c:143-160): GELU-tanh, silu, relu by their
// codes, GELU (erf) for GELU and every other code.
static uint32_t plain_act_code(const forword_gpu_config_t &c)
{
    return c.act_type == FORWORD_ACT_GELU_FAST ? fw::ACT_GELU_TANH
         : c.act_type == FORWORD_ACT_SILU      ? fw::ACT_SILU
         : c.act_type == FORWORD_ACT_RELU      ? fw::ACT_RELU
                                               : fw::ACT_GELU;
}

// Values per block of a block type (gguf.c:211-223); 1 for F32, 0 unknown.
uint32_t type_block_values(uint32_t type)
{
    switch (type) {
    case kF32: return 1;
    case kQ4_0: case kQ5_0: case kQ8_0: return 32;
    case kQ4_K: case kQ6_K: return 256;
    default: return 0;
    }
}

} // namespace

struct forword_gpu {
    forword_gpu_config_t cfg{};
    size_t n_ctx = 0;
    hipStream_t stream = nullptr;
    uint8_t *d_data = nullptr;
    size_t data_size = 0;
    Lin embd, out;
    const float *out_norm = nullptr;
    std::vector<Layer> L;
    float *d_k = nullptr, *d_v = nullptr, *d_cos = nullptr, *d_sin = nullptr;
    float *d_x = nullptr, *d_xn = nullptr, *d_q = nullptr, *d_att = nullptr, *d_h = nullptr;
    float *d_logits = nullptr, *d_part = nullptr, *d_trace = nullptr, *d_pv = nullptr;
    uint32_t *d_pi = nullptr, *d_counter = nullptr, *d_argmax = nullptr, *d_prompt = nullptr, *d_ids = nullptr;
    float *d_pss = nullptr, *d_scale = nullptr;      // RMSNorm scale published by the residual kernels
    float *d_bias = nullptr;                         // per-layer q|k|v biases (qwen2)
    const float *out_norm_b = nullptr;               // output_norm.bias (LayerNorm), or null
    Lin pos_embd;                                    // GPT-2 learned positions (w null otherwise)
    // Blocks other than the RMSNorm / gated-FFN / sequential / pairwise-RoPE one
    // (LayerNorm, parallel residual, plain FFN, NEOX RoPE, output-projection
    // bias) run the explicit per-phase step (enqueue_step_generic).
    bool generic = false;
    float *d_ao = nullptr;                           // attention output kept for the parallel residual
    uint32_t *d_ticket = nullptr;
    StepState *d_state = nullptr, *h_state = nullptr;   // h_state: the host's mirror, set on the device by kernel
    StepState host_state{};                             // argument (launch_set_state), never copied by DMA
    float *h_logits = nullptr;
    uint32_t *h_u32 = nullptr;
    uint32_t n_splits = 1, am_blocks = 1;
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    bool traced = false;
    // persistent step kernel
    bool mk = false;
    uint32_t mk_wg = 0, mk_tl = 0, mk_th = 0, mk_tm = 0, mk_epoch = 0;
    size_t mk_lds = 0, mk_tq_bytes = 0, mk_tkv_bytes = 0, mk_tpart_bytes = 0;
    MkArgs mka{};
    uint32_t *d_bar = nullptr, *d_mk_err = nullptr, *d_mk_tickets = nullptr, *d_ami = nullptr;
    float *d_amv = nullptr;
    uint64_t *d_tx = nullptr, *d_tatt = nullptr;   // tagged activations of the persistent kernel
    uint64_t *d_tq = nullptr, *d_tkv = nullptr, *d_tpart = nullptr;   // and of its attention
    float *d_hf = nullptr;                          // its FFN activations
    uint32_t *d_hflag = nullptr;                    // and their per-workgroup flags
    MkLayer *d_layers = nullptr;
    uint64_t *d_prof = nullptr;          // phase stamps of the last launch (FORWORD_GPU_PHASE_TIMES=1)
    uint32_t prof_steps = 0;
    // Failure injection for tests (FORWORD_GPU_ABORT_LAUNCH=k, read at init):
    // persistent launch k (1-based) starts with the error word set, so every
    // bounded wait in it takes its exit and forword_gpu_status reports it.
    uint32_t mk_abort_at = 0, mk_launches = 0;
    // sampled generation (allocated on first use): probabilities, reductions, buckets,
    // history counts, PRNG state, sampled ids
    float *d_sbuf = nullptr, *d_spart = nullptr;
    unsigned long long *d_bsum = nullptr;           // bucket weights, 2^-40 units
    uint64_t *d_gkeys = nullptr;                     // top-p candidates beyond the LDS sort
    uint32_t *d_bcnt = nullptr, *d_counts = nullptr, *d_sids = nullptr;
    SampleState *d_ss = nullptr;
    // batched prefill: activations of up to kPrefillChunk tokens (allocated on first use)
    float *d_pf = nullptr;
    uint32_t *d_pf_tok = nullptr;
    std::vector<void *> allocs;
};

static int dalloc(forword_gpu_t *h, void **p, size_t bytes, const char *what)
{
    hipError_t e = hipMalloc(p, bytes ? bytes : 4);
    if (e != hipSuccess) {
        set_err("hipMalloc(%zu) for %s: %s", bytes, what, hipGetErrorString(e));
        return -1;
    }
    h->allocs.push_back(*p);
    return 0;
}

static const forword_gpu_tensor_t *find_t(const forword_gpu_tensor_t *t, size_t n, const char *name)
{
    for (size_t i = 0; i < n; i++)
        if (t[i].name && !strcmp(t[i].name, name)) return &t[i];
    return nullptr;
}

// Bind a linear weight with its expected [in, out] shape (linear.c:169-170).
static int bind_lin(forword_gpu_t *h, Lin &l, const forword_gpu_tensor_t *t, const char *name, uint64_t in,
                    uint64_t out)
{
    if (!t) { set_err("missing tensor %s", name); return -1; }
    if (!type_block_values(t->ggml_type)) {
        set_err("tensor %s: unsupported ggml type %u", name, t->ggml_type);
        return -1;
    }
    if (t->n_dims < 2 || t->dims[0] != in || t->dims[1] != out) {
        set_err("tensor %s: shape [%llu, %llu], expected [%llu, %llu]", name, (unsigned long long)t->dims[0],
                (unsigned long long)(t->n_dims > 1 ? t->dims[1] : 1), (unsigned long long)in,
                (unsigned long long)out);
        return -1;
    }
    if (in % type_block_values(t->ggml_type)) {
        set_err("tensor %s: columns not a multiple of the %u-value block", name, type_block_values(t->ggml_type));
        return -1;
    }
    uint64_t rb = type_row_bytes(t->ggml_type, in);
    if (in >= (1u << 31) || out >= (1u << 31) || t->offset > h->data_size ||
        rb * out > h->data_size - t->offset) {
        set_err("tensor %s: data outside the data section", name);
        return -1;
    }
    l.w = h->d_data + t->offset;
    l.type = t->ggml_type;
    l.in = (uint32_t)in;
    l.out = (uint32_t)out;
    l.row_bytes = rb;
    return 0;
}

static int bind_vec(forword_gpu_t *h, const float **p, const forword_gpu_tensor_t *t, const char *name, uint64_t n,
                    bool required)
{
    if (!t) {
        if (required) { set_err("missing tensor %s", name); return -1; }
        *p = nullptr;
        return 0;
    }
    if (t->ggml_type != kF32 || t->offset > h->data_size || n * 4 > h->data_size - t->offset ||
        (t->offset & 3)) {
        set_err("tensor %s: expected %llu F32 values inside the data section", name, (unsigned long long)n);
        return -1;
    }
    *p = reinterpret_cast<const float *>(h->d_data + t->offset);
    return 0;
}

// ── one token step ───────────────────────────────────────────────────────────

// The block's pre-norm written out (transformer.c:234-239, 256-261, 275-280).
static hipError_t launch_block_norm(const forword_gpu_t *h, const float *x, const float *w, const float *b, float *out,
                                    hipStream_t s, uint32_t rows = 1)
{
    const forword_gpu_config_t &c = h->cfg;
    if (c.norm_type == FORWORD_NORM_LAYER) return launch_layernorm(x, w, b, out, c.n_embd, c.norm_eps, s, rows);
    return launch_rmsnorm_rows(x, w, out, c.n_embd, rows, c.norm_eps, s);
}

// One token step of any supported block (transformer.c:149-326): LayerNorm or
// RMSNorm written out to xn, sequential or parallel residual, gated or plain
// FFN, pairwise or NEOX RoPE, biases of q/k/v and of the output projection.
static hipError_t enqueue_step_generic(forword_gpu_t *h)
{
    const forword_gpu_config_t &c = h->cfg;
    const uint32_t n = c.n_embd, hd = c.head_dim, kvd = c.n_head_kv * hd;
    const bool neox = c.rope_type == FORWORD_ROPE_NEOX, par = c.parallel_res != 0;
    hipStream_t s = h->stream;
    hipError_t e;
#define TRY(x) do { e = (x); if (e != hipSuccess) return e; } while (0)
    TRY(launch_embed(h->embd.w, h->embd.type, n, h->embd.out, h->d_state, nullptr, c.embd_scale, h->d_x,
                     h->d_scale, c.norm_eps, s));                                       // transformer.c:167-182
    if (h->pos_embd.w)                                                                  // transformer.c:188-205
        TRY(launch_pos_add(h->pos_embd.w, h->pos_embd.type, h->pos_embd.row_bytes, n, h->d_state, 0, 1, h->d_x, s));
    const bool rope = c.rope_type != FORWORD_ROPE_NONE;
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const Layer &Ly = h->L[l];
        float *kc = h->d_k + (size_t)l * h->n_ctx * kvd, *vc = h->d_v + (size_t)l * h->n_ctx * kvd;
        TRY(launch_block_norm(h, h->d_x, Ly.attn_norm, Ly.attn_norm_b, h->d_xn, s));
        const Lin *qkv[3] = { &Ly.q, &Ly.k, &Ly.v };                                   // attention.c:97-140
        const bool fused = Ly.q.type == Ly.k.type && Ly.k.type == Ly.v.type;
        for (uint32_t s0 = 0; s0 < 3; s0 += fused ? 3 : 1) {
            QmvArgs a{};
            a.n_seg = fused ? 3 : 1;
            for (uint32_t i = 0; i < a.n_seg; i++) { a.w[i] = qkv[s0 + i]->w; a.rows[i] = qkv[s0 + i]->out; }
            a.role_base = s0;
            a.n_cols = n;
            a.row_bytes = qkv[s0]->row_bytes;
            a.x = h->d_xn;
            a.out[0] = h->d_q; a.out[1] = kc; a.out[2] = vc;
            if (rope && !neox) { a.cos_tab = h->d_cos; a.sin_tab = h->d_sin; }
            if (Ly.bqkv) { a.bias[0] = Ly.bqkv; a.bias[1] = Ly.bqkv + n; a.bias[2] = Ly.bqkv + n + kvd; }
            a.state = h->d_state;
            a.head_dim = hd;
            a.kv_dim = kvd;
            qmv_plan(a, EPI_QKV);
            TRY(launch_qmv(qkv[s0]->type, EPI_QKV, a, s));
        }
        if (rope && neox) TRY(launch_rope_neox_step(h->d_q, kc, c.n_head, c.n_head_kv, hd, h->d_cos, h->d_sin, h->d_state, s));
        TRY(launch_attention(h->d_q, kc, vc, h->d_part, h->d_att, c.n_head, c.n_head_kv, hd, h->n_splits,
                             h->d_state, 0, s));                                        // attention.c:142-164
        {
            QmvArgs a{};                                                                // attention.c:166
            a.n_seg = 1; a.w[0] = Ly.o.w; a.rows[0] = Ly.o.out; a.n_cols = Ly.o.in; a.row_bytes = Ly.o.row_bytes;
            a.x = h->d_att; a.bias[0] = Ly.bo;
            if (par) {                                                                  // kept for the parallel add
                a.out[0] = h->d_ao;
                qmv_plan(a, EPI_STORE);
                TRY(launch_qmv(Ly.o.type, EPI_STORE, a, s));
            } else {                                                                    // transformer.c:271-272
                a.out[0] = h->d_x; a.trace = h->d_trace + (size_t)(2 * l) * n;
                qmv_plan(a, EPI_RESID);
                TRY(launch_qmv(Ly.o.type, EPI_RESID, a, s));
                TRY(launch_block_norm(h, h->d_x, Ly.ffn_norm, Ly.ffn_norm_b, h->d_xn, s));   // transformer.c:275-280
            }
        }
        if (c.use_ffn_gate) {                                                           // ffn.c:68-104
            QmvArgs a{};
            a.n_seg = 2; a.w[0] = Ly.gate.w; a.w[1] = Ly.up.w; a.rows[0] = a.rows[1] = c.n_ff;
            a.n_cols = n; a.row_bytes = Ly.gate.row_bytes; a.x = h->d_xn; a.out[0] = h->d_h;
            a.act = ffn_act_code(c);
            qmv_plan(a, EPI_SWIGLU);
            TRY(launch_qmv(Ly.gate.type, EPI_SWIGLU, a, s));
        } else {                                                                        // ffn.c:108-160
            QmvArgs a{};
            a.n_seg = 1; a.w[0] = Ly.up.w; a.rows[0] = c.n_ff; a.n_cols = n; a.row_bytes = Ly.up.row_bytes;
            a.x = h->d_xn; a.out[0] = h->d_h; a.bias[0] = Ly.bu;
            a.store_act = 1 + plain_act_code(c);                                       // act(W x + b) in the epilogue
            qmv_plan(a, EPI_STORE);
            TRY(launch_qmv(Ly.up.type, EPI_STORE, a, s));
        }
        {
            QmvArgs a{};                                                                // ffn.c:106/168, transformer.c:250/287
            a.n_seg = 1; a.w[0] = Ly.down.w; a.rows[0] = n; a.n_cols = c.n_ff; a.row_bytes = Ly.down.row_bytes;
            a.x = h->d_h; a.out[0] = h->d_x; a.trace = h->d_trace + (size_t)(2 * l + 1) * n;
            a.bias[0] = Ly.bd;
            if (par) { a.addend = h->d_ao; a.trace2 = h->d_trace + (size_t)(2 * l) * n; }
            qmv_plan(a, EPI_RESID);
            TRY(launch_qmv(Ly.down.type, EPI_RESID, a, s));
        }
    }
    const float *xh = h->d_x;                                                          // transformer.c:293-307
    if (h->out_norm) {
        TRY(launch_block_norm(h, h->d_x, h->out_norm, h->out_norm_b, h->d_xn, s));
        xh = h->d_xn;
    }
    {
        QmvArgs a{};                                                                    // transformer.c:309-323
        a.n_seg = 1; a.w[0] = h->out.w; a.rows[0] = h->out.out; a.n_cols = n; a.row_bytes = h->out.row_bytes;
        a.x = xh; a.out[0] = h->d_logits; a.state = h->d_state;
        qmv_plan(a, EPI_STORE);
        TRY(launch_qmv(h->out.type, EPI_STORE, a, s));
    }
    TRY(launch_argmax(h->d_logits, c.n_vocab, h->d_pv, h->d_pi, h->d_counter, h->d_argmax, h->d_state, h->d_prompt,
                      h->d_ids, h->am_blocks, s));
#undef TRY
    return hipSuccess;
}

static hipError_t enqueue_step(forword_gpu_t *h)
{
    if (h->generic) return enqueue_step_generic(h);
    const forword_gpu_config_t &c = h->cfg;
    const uint32_t n = c.n_embd, hd = c.head_dim, kvd = c.n_head_kv * hd;
    hipStream_t s = h->stream;
    hipError_t e;
#define TRY(x) do { e = (x); if (e != hipSuccess) return e; } while (0)
    // Every RMSNorm (transformer.c:261,279,293-304) is folded into the GEMV that
    // consumes it: the kernel writing x (embedding, Wo and down residuals)
    // publishes the scale, the next GEMV applies (x*w)*scale as it loads x.
    TRY(launch_embed(h->embd.w, h->embd.type, n, h->embd.out, h->d_state, nullptr, c.embd_scale, h->d_x,
                     h->d_scale, c.norm_eps, s));
    for (uint32_t l = 0; l < c.n_layer; l++) {
        const Layer &Ly = h->L[l];
        float *kc = h->d_k + (size_t)l * h->n_ctx * kvd, *vc = h->d_v + (size_t)l * h->n_ctx * kvd;
        // attention_forward (attention.c:124-140): Q/K/V, RoPE, KV append at pos
        const Lin *qkv[3] = { &Ly.q, &Ly.k, &Ly.v };
        const bool fused = Ly.q.type == Ly.k.type && Ly.k.type == Ly.v.type;
        for (uint32_t s0 = 0; s0 < 3; s0 += fused ? 3 : 1) {
            QmvArgs a{};
            a.n_seg = fused ? 3 : 1;
            for (uint32_t i = 0; i < a.n_seg; i++) { a.w[i] = qkv[s0 + i]->w; a.rows[i] = qkv[s0 + i]->out; }
            a.role_base = s0;
            a.n_cols = n;
            a.row_bytes = qkv[s0]->row_bytes;
            a.x = h->d_x;
            a.norm_w = Ly.attn_norm; a.norm_scale = h->d_scale;
            a.out[0] = h->d_q; a.out[1] = kc; a.out[2] = vc;
            a.cos_tab = h->d_cos; a.sin_tab = h->d_sin;
            if (Ly.bqkv) { a.bias[0] = Ly.bqkv; a.bias[1] = Ly.bqkv + n; a.bias[2] = Ly.bqkv + n + kvd; }
            a.state = h->d_state;
            a.head_dim = hd;
            a.kv_dim = kvd;
            qmv_plan(a, EPI_QKV);
            TRY(launch_qmv(qkv[s0]->type, EPI_QKV, a, s));
        }
        TRY(launch_attention(h->d_q, kc, vc, h->d_part, h->d_att, c.n_head, c.n_head_kv, hd, h->n_splits,
                             h->d_state, 0, s));                                        // attention.c:142-164
        {
            QmvArgs a{};                                                                // attention.c:166 + transformer.c:271
            a.n_seg = 1; a.w[0] = Ly.o.w; a.rows[0] = Ly.o.out; a.n_cols = Ly.o.in; a.row_bytes = Ly.o.row_bytes;
            a.x = h->d_att; a.out[0] = h->d_x; a.trace = h->d_trace + (size_t)(2 * l) * n;
            a.pss = h->d_pss; a.ticket = h->d_ticket; a.scale_out = h->d_scale; a.norm_eps = c.norm_eps;
            qmv_plan(a, EPI_RESID);
            TRY(launch_qmv(Ly.o.type, EPI_RESID, a, s));
        }
        {
            QmvArgs a{};                                                                // ffn.c:82-104
            a.n_seg = 2; a.w[0] = Ly.gate.w; a.w[1] = Ly.up.w; a.rows[0] = a.rows[1] = c.n_ff;
            a.n_cols = n; a.row_bytes = Ly.gate.row_bytes; a.x = h->d_x; a.out[0] = h->d_h;
            a.norm_w = Ly.ffn_norm; a.norm_scale = h->d_scale;
            a.act = ffn_act_code(c);
            qmv_plan(a, EPI_SWIGLU);
            TRY(launch_qmv(Ly.gate.type, EPI_SWIGLU, a, s));
        }
        {
            QmvArgs a{};                                                                // ffn.c:106 + transformer.c:287
            a.n_seg = 1; a.w[0] = Ly.down.w; a.rows[0] = n; a.n_cols = c.n_ff; a.row_bytes = Ly.down.row_bytes;
            a.x = h->d_h; a.out[0] = h->d_x; a.trace = h->d_trace + (size_t)(2 * l + 1) * n;
            a.pss = h->d_pss; a.ticket = h->d_ticket; a.scale_out = h->d_scale; a.norm_eps = c.norm_eps;
            qmv_plan(a, EPI_RESID);
            TRY(launch_qmv(Ly.down.type, EPI_RESID, a, s));
        }
    }
    {
        QmvArgs a{};                                                                    // transformer.c:293-323
        a.n_seg = 1; a.w[0] = h->out.w; a.rows[0] = h->out.out; a.n_cols = n; a.row_bytes = h->out.row_bytes;
        a.x = h->d_x; a.out[0] = h->d_logits; a.state = h->d_state;
        a.norm_w = h->out_norm; a.norm_scale = h->d_scale;       // no output_norm: logits of x itself
        qmv_plan(a, EPI_STORE);
        TRY(launch_qmv(h->out.type, EPI_STORE, a, s));
    }
    TRY(launch_argmax(h->d_logits, c.n_vocab, h->d_pv, h->d_pi, h->d_counter, h->d_argmax, h->d_state, h->d_prompt,
                      h->d_ids, h->am_blocks, s));
#undef TRY
    return hipSuccess;
}

static constexpr uint32_t kMkStepsPerLaunch = 64;

// Queue n token steps.
static int run_steps(forword_gpu_t *h, size_t n)
{
    if (h->mk) {
        while (n) {
            const uint32_t k = n > kMkStepsPerLaunch ? kMkStepsPerLaunch : (uint32_t)n;
            MkArgs a = h->mka;
            a.epoch0 = h->mk_epoch;
            a.n_steps = k;
            if (h->mk_abort_at && ++h->mk_launches == h->mk_abort_at)
                HIPCHK(hipMemsetD32Async(h->d_mk_err, 1, 1, h->stream), "persistent step launch");
            HIPCHK(mk_launch(a, h->mk_tl, h->mk_th, h->mk_tm, h->mk_wg, h->mk_lds, h->stream), "persistent step launch");
            h->prof_steps = k;
            h->mk_epoch += k * mk_barriers_per_step(h->cfg.n_layer);
            n -= k;
        }
        return 0;
    }
    for (size_t i = 0; i < n; i++) {
        if (h->exec) HIPCHK(hipGraphLaunch(h->exec, h->stream), "hipGraphLaunch");
        else HIPCHK(enqueue_step(h), "token step launch");
    }
    return 0;
}

// After the stream has drained: did a persistent launch give up at a barrier?
// Then its results are invalid; reset the barrier state for the next launch.
static int mk_check(forword_gpu_t *h)
{
    if (!h->mk) return 0;
    uint32_t err = 0;
    HIPCHK(hipMemcpy(&err, h->d_mk_err, 4, hipMemcpyDeviceToHost), "persistent step status");
    if (!err) return 0;
    // the epoch restarts at 0, so every flag and tagged word goes back to 0 too
    (void)hipMemset(h->d_bar, 0, (size_t)h->mk_wg * 128);
    (void)hipMemset(h->d_mk_tickets, 0, 64 * 4);
    (void)hipMemset(h->d_mk_err, 0, 4);
    (void)hipMemset(h->d_tx, 0, (size_t)h->cfg.n_embd * 8);
    (void)hipMemset(h->d_tatt, 0, (size_t)h->cfg.n_embd * 8);
    (void)hipMemset(h->d_hflag, 0, (size_t)h->mk_wg * 128);
    (void)hipMemset(h->d_tq, 0, h->mk_tq_bytes);
    (void)hipMemset(h->d_tkv, 0, h->mk_tkv_bytes);
    (void)hipMemset(h->d_tpart, 0, h->mk_tpart_bytes);
    (void)hipDeviceSynchronize();
    h->mk_epoch = 0;
    set_err("persistent step kernel: a grid barrier timed out; results of the last call are invalid");
    return -1;
}

// Set up the persistent step kernel when the model and the device allow it
// (else the per-phase kernels run).
static int setup_mk(forword_gpu_t *h)
{
    const char *env = getenv("FORWORD_GPU_MEGAKERNEL");
    if ((env && !strcmp(env, "0")) || h->generic) return 0;
    const forword_gpu_config_t &c = h->cfg;
    const uint32_t n = c.n_embd, hd = c.head_dim, L = c.n_layer;
    // one linear type; attn_v / ffn_down may be Q6_K in some layers (the Q4_K_M
    // layout), run from re-laid-out copies as the kernel's second layer type
    const uint32_t tl = h->L[0].q.type;
    uint32_t tm = 0;
    for (const Layer &Ly : h->L) {
        for (const Lin *l : { &Ly.q, &Ly.k, &Ly.o, &Ly.gate, &Ly.up })
            if (l->type != tl) return 0;
        for (const Lin *l : { &Ly.v, &Ly.down }) {
            if (l->type == tl) continue;
            if (l->type != kQ6_K) return 0;
            tm = kQ6_KR;
        }
    }
    // attention units: a KV head's query heads in power-of-two sub-groups (any group)
    const uint32_t group = c.n_head / c.n_head_kv;
    uint32_t gs = 8;
    while (group % gs) gs >>= 1;
    const uint32_t units = c.n_head_kv * (group / gs);
    // a Q6_K lm-head runs from a re-laid-out copy (whole super-blocks per row required)
    const bool head_q6k = h->out.type == kQ6_K;
    const uint32_t th = head_q6k ? kQ6_KR : h->out.type;
    if (!mk_supported(n, c.n_ff, hd, group, tl, th, h->embd.type, tm) || units > 64) return 0;
    int dev = 0, cus = 0;                    // one workgroup per CU; each barrier flag is polled by one thread
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1 ||
        cus > (int)kMkPollers) {
        (void)hipGetLastError();
        return 0;
    }

    MkArgs &a = h->mka;
    a.n_layer = L;
    // row strides of the linear type (layer 0's ffn_down may be of the second type)
    a.rb_embd = type_row_bytes(tl, n);
    a.rb_ff = type_row_bytes(tl, c.n_ff);
    a.head_w = h->out.w; a.head_rb = h->out.row_bytes; a.out_norm = h->out_norm;
    a.qa_lin = mk_q_align(tl); a.qa_head = mk_q_align(th);
    a.rb_mix_embd = (uint64_t)(n / 256) * 224; a.rb_mix_ff = (uint64_t)(c.n_ff / 256) * 224;
    a.embd = h->embd.w; a.embd_type = h->embd.type; a.embd_row_bytes = h->embd.row_bytes; a.embd_scale = c.embd_scale;
    a.n_embd = n; a.n_ff = c.n_ff; a.n_head = c.n_head; a.n_kv = c.n_head_kv; a.head_dim = hd;
    a.n_vocab = c.n_vocab; a.n_ctx = (uint32_t)h->n_ctx; a.eps = c.norm_eps;
    a.kc = h->d_k; a.vc = h->d_v; a.cos_tab = h->d_cos; a.sin_tab = h->d_sin;
    a.bqkv = h->d_bias;
    a.act = ffn_act_code(c);
    a.logits = h->d_logits; a.trace = h->d_trace;
    a.state = h->d_state; a.prompt = h->d_prompt; a.ids = h->d_ids; a.argmax_out = h->d_argmax;
    // (attention unit, split) items: about one per workgroup, >= 8 positions per split
    a.attn_gs = gs;
    a.attn_units = units;
    uint32_t ns = (uint32_t)cus / units;
    const uint32_t by_ctx = (uint32_t)((h->n_ctx + 7) / 8);
    if (ns > by_ctx) ns = by_ctx;
    if (ns > 256) ns = 256;
    if (ns < 1) ns = 1;
    a.n_splits = ns;
    // Below position 4096 half-size sub-groups: twice the units with half the
    // heads each, so an item's scores and softmax take half as long; each K/V
    // row is then read by two units, which costs more than it saves from a few
    // thousand positions on (8B shape: +2 % at position 2K, -5 % at 8K, -17 %
    // at 32K with half-size sub-groups throughout).
    a.attn_gs_short = gs > 1 ? gs / 2 : 1;
    a.attn_units_short = c.n_head_kv * (group / a.attn_gs_short);
    uint32_t ns_short = (uint32_t)cus / a.attn_units_short;
    if (ns_short > by_ctx) ns_short = by_ctx;
    if (ns_short < 1) ns_short = 1;
    a.n_splits_short = ns_short < ns ? ns_short : ns;
    a.attn_long_pos = 4096;
    const size_t lds = mk_lds_bytes(a, (uint32_t)cus, tl, th, tm);
    const int wg = lds ? mk_max_workgroups(tl, th, tm, lds) : 0;
    if (wg != cus) {
        fprintf(stderr, "forword_gpu: persistent step kernel cannot launch (LDS %zu B); using per-phase kernels\n", lds);
        return 0;
    }

    std::vector<MkLayer> layers(L);
    for (uint32_t l = 0; l < L; l++) {
        const Layer &Ly = h->L[l];
        layers[l] = MkLayer{ Ly.q.w, Ly.k.w, Ly.v.w, Ly.o.w, Ly.gate.w, Ly.up.w, Ly.down.w, Ly.attn_norm, Ly.ffn_norm,
                             0u, 0u };
        // the second-type tensors of this layer, re-laid out
        for (int which = 0; which < 2 && tm; which++) {
            const Lin &li = which ? Ly.down : Ly.v;
            if (li.type == tl) continue;
            const uint32_t n_sb = li.in / 256;
            uint8_t *rp = nullptr;
            if (dalloc(h, (void **)&rp, (size_t)li.out * n_sb * 224, "Q6_K layer records")) return -1;
            if (launch_repack_q6k(li.w, li.row_bytes, li.out, n_sb, rp, h->stream) != hipSuccess) {
                set_err("persistent step kernel: Q6_K repack launch failed");
                return -1;
            }
            (which ? layers[l].wd : layers[l].wv) = rp;
            layers[l].mix |= which ? MK_MIX_DOWN : MK_MIX_V;
        }
    }
    h->mk_tq_bytes = (size_t)c.n_head * hd * 8;
    h->mk_tkv_bytes = (size_t)2 * c.n_head_kv * hd * 8;
    h->mk_tpart_bytes = (size_t)c.n_head * ns * (hd + 2) * 8;
    if (dalloc(h, (void **)&h->d_layers, layers.size() * sizeof(MkLayer), "layer table") ||
        dalloc(h, (void **)&h->d_bar, (size_t)wg * 128, "barrier flags") ||
        dalloc(h, (void **)&h->d_mk_tickets, 64 * 4, "tickets") || dalloc(h, (void **)&h->d_mk_err, 4, "barrier status") ||
        dalloc(h, (void **)&h->d_amv, (size_t)wg * 4, "argmax") || dalloc(h, (void **)&h->d_ami, (size_t)wg * 4, "argmax") ||
        dalloc(h, (void **)&h->d_tpart, h->mk_tpart_bytes, "tagged attention partials") ||
        dalloc(h, (void **)&h->d_tq, h->mk_tq_bytes, "tagged q") || dalloc(h, (void **)&h->d_tkv, h->mk_tkv_bytes, "tagged K/V row") ||
        dalloc(h, (void **)&h->d_tx, (size_t)n * 8, "tagged x") ||
        dalloc(h, (void **)&h->d_tatt, (size_t)n * 8, "tagged attention output") ||
        dalloc(h, (void **)&h->d_hf, (size_t)c.n_ff * 4 * kMkStepsPerLaunch * L, "ffn activations") ||
        dalloc(h, (void **)&h->d_hflag, (size_t)wg * 128, "ffn activation flags"))
        return -1;
    if (head_q6k) {
        const uint32_t n_sb = n / 256;
        uint8_t *rp = nullptr;
        if (dalloc(h, (void **)&rp, (size_t)c.n_vocab * n_sb * 224, "lm-head Q6_K records")) return -1;
        if (launch_repack_q6k(h->out.w, h->out.row_bytes, c.n_vocab, n_sb, rp, h->stream) != hipSuccess) {
            set_err("persistent step kernel: lm-head repack launch failed");
            return -1;
        }
        a.head_w = rp;
        a.head_rb = (uint64_t)n_sb * 224;
    }
    a.tx = h->d_tx; a.tatt = h->d_tatt; a.hf = h->d_hf; a.hflag = h->d_hflag;
    a.tq = h->d_tq; a.tkv = h->d_tkv; a.tpart = h->d_tpart;
    if (hipMemcpy(h->d_layers, layers.data(), layers.size() * sizeof(MkLayer), hipMemcpyHostToDevice) != hipSuccess ||
        hipMemset(h->d_bar, 0, (size_t)wg * 128) != hipSuccess || hipMemset(h->d_mk_tickets, 0, 64 * 4) != hipSuccess ||
        hipMemset(h->d_mk_err, 0, 4) != hipSuccess || hipMemset(h->d_tx, 0, (size_t)n * 8) != hipSuccess ||
        hipMemset(h->d_tatt, 0, (size_t)n * 8) != hipSuccess || hipMemset(h->d_hflag, 0, (size_t)wg * 128) != hipSuccess ||
        hipMemset(h->d_tq, 0, h->mk_tq_bytes) != hipSuccess || hipMemset(h->d_tkv, 0, h->mk_tkv_bytes) != hipSuccess ||
        hipMemset(h->d_tpart, 0, h->mk_tpart_bytes) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        set_err("persistent step kernel: device set-up failed");
        return -1;
    }
    a.layers = h->d_layers;
    a.bar = h->d_bar;
    a.tickets = h->d_mk_tickets;
    a.err = h->d_mk_err;
    a.am_v = h->d_amv;
    a.am_i = h->d_ami;
    const char *ab = getenv("FORWORD_GPU_ABORT_LAUNCH");
    if (ab) h->mk_abort_at = (uint32_t)strtoul(ab, nullptr, 10);
    const char *pt = getenv("FORWORD_GPU_PHASE_TIMES");
    if (pt && !strcmp(pt, "1")) {
        if (dalloc(h, (void **)&h->d_prof, (1 + (size_t)kMkStepsPerLaunch * (5 * L + 1)) * 8, "phase stamps")) return -1;
        a.prof = h->d_prof;
    }
    h->mk_tl = tl;
    h->mk_th = th;
    h->mk_tm = tm;
    h->mk_wg = (uint32_t)wg;
    h->mk_lds = lds;
    h->mk_epoch = 0;
    h->mk = true;
    return 0;
}

static void build_graph(forword_gpu_t *h)
{
    const char *env = getenv("FORWORD_GPU_GRAPH");
    if (env && !strcmp(env, "0")) return;
    if (hipStreamBeginCapture(h->stream, hipStreamCaptureModeThreadLocal) != hipSuccess) return;
    hipError_t e = enqueue_step(h);
    hipGraph_t g = nullptr;
    hipError_t e2 = hipStreamEndCapture(h->stream, &g);
    if (e != hipSuccess || e2 != hipSuccess || !g) {
        if (g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        fprintf(stderr, "forword_gpu: graph capture failed (%s); launching kernels directly\n",
                hipGetErrorString(e != hipSuccess ? e : e2));
        return;
    }
    if (hipGraphInstantiate(&h->exec, g, nullptr, nullptr, 0) != hipSuccess) {
        h->exec = nullptr;
        (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        fprintf(stderr, "forword_gpu: graph instantiation failed; launching kernels directly\n");
        return;
    }
    h->graph = g;
}

// ── model-level ABI ──────────────────────────────────────────────────────────

extern "C" void forword_gpu_free(forword_gpu_t *h)
{
    if (!h) return;
    if (h->stream) (void)hipStreamSynchronize(h->stream);
    if (h->exec) (void)hipGraphExecDestroy(h->exec);
    if (h->graph) (void)hipGraphDestroy(h->graph);
    for (void *p : h->allocs) (void)hipFree(p);
    if (h->h_logits) (void)hipHostFree(h->h_logits);
    if (h->h_u32) (void)hipHostFree(h->h_u32);
    if (h->stream) (void)hipStreamDestroy(h->stream);
    delete h;
}

extern "C" int forword_gpu_init(forword_gpu_t **out, const void *data, size_t data_size,
                                const forword_gpu_tensor_t *tensors, size_t n_tensors,
                                const forword_gpu_config_t *cfg, size_t max_ctx, const float *cos_tab,
                                const float *sin_tab)
{
    if (!out) { set_err("forword_gpu_init: out is NULL"); return -1; }
    *out = nullptr;
    if (!data || !data_size || !tensors || !cfg || !cos_tab || !sin_tab || !max_ctx) {
        set_err("forword_gpu_init: invalid arguments");
        return -1;
    }
    const forword_gpu_config_t &c = *cfg;
    if (!c.n_embd || !c.n_head || !c.n_layer || !c.n_vocab || !c.n_ff || !c.n_head_kv ||
        c.n_head % c.n_head_kv || c.head_dim * c.n_head != c.n_embd || c.n_embd % 32 || c.n_ff % 32) {
        set_err("forword_gpu_init: invalid model dimensions");
        return -1;
    }
    if ((c.norm_type != FORWORD_NORM_RMS && c.norm_type != FORWORD_NORM_LAYER) ||
        (c.rope_type != FORWORD_ROPE_NORMAL && c.rope_type != FORWORD_ROPE_NEOX && c.rope_type != FORWORD_ROPE_NONE) ||
        (c.arch == FORWORD_ARCH_GPT2 && c.n_head_kv != c.n_head)) {
        set_err("forword_gpu_init: unknown norm or RoPE type, or a GPT-2 model with grouped KV heads");
        return -1;
    }
    if (!attn_supported(c.head_dim, c.n_head / c.n_head_kv)) {
        set_err("forword_gpu_init: head_dim %u / GQA group %u not supported by the attention kernel",
                c.head_dim, c.n_head / c.n_head_kv);
        return -1;
    }
    if (max_ctx > c.n_ctx || max_ctx >= (1u << 31)) {
        set_err("forword_gpu_init: max_ctx %zu exceeds the model context %u", max_ctx, c.n_ctx);
        return -1;
    }

    forword_gpu_t *h = new forword_gpu_t();
    h->cfg = c;
    h->n_ctx = max_ctx;
    h->data_size = data_size;
    const uint32_t n = c.n_embd, hd = c.head_dim, kvd = c.n_head_kv * hd;
#define FAIL() do { forword_gpu_free(h); return -1; } while (0)
    if (hipStreamCreateWithFlags(&h->stream, hipStreamNonBlocking) != hipSuccess) {
        set_err("hipStreamCreate failed");
        FAIL();
    }
    if (dalloc(h, (void **)&h->d_data, data_size, "weights")) FAIL();
    if (hipMemcpy(h->d_data, data, data_size, hipMemcpyHostToDevice) != hipSuccess) {
        set_err("weight upload failed");
        FAIL();
    }

    // resolve every tensor once (tensor_find, tensor_data.c:8-23)
    const forword_gpu_tensor_t *te = find_t(tensors, n_tensors, "token_embd.weight");
    const forword_gpu_tensor_t *to = find_t(tensors, n_tensors, "output.weight");
    if (!to) to = find_t(tensors, n_tensors, "lm_head.weight");
    if (!to) to = te;                                                                   // transformer.c:310-316
    if (bind_lin(h, h->embd, te, "token_embd.weight", n, c.n_vocab)) FAIL();
    if (bind_lin(h, h->out, to, "output.weight", n, c.n_vocab)) FAIL();
    if (bind_vec(h, &h->out_norm, find_t(tensors, n_tensors, "output_norm.weight"), "output_norm.weight", n, false) ||
        bind_vec(h, &h->out_norm_b, find_t(tensors, n_tensors, "output_norm.bias"), "output_norm.bias", n, false))
        FAIL();
    h->L.resize(c.n_layer);
    for (uint32_t l = 0; l < c.n_layer; l++) {
        char nm[96];
        Layer &Ly = h->L[l];
#define LIN(f, sfx, in_, out_)                                                          \
        snprintf(nm, sizeof nm, "blk.%u." sfx, l);                                      \
        if (bind_lin(h, Ly.f, find_t(tensors, n_tensors, nm), nm, in_, out_)) FAIL();
        if (c.arch == FORWORD_ARCH_GPT2) {          // one [q | k | v] projection (attention.c:68-96)
            Lin qkv;
            LIN(q, "attn_qkv.weight", n, 3 * n);
            qkv = Ly.q;
            Ly.q.out = Ly.k.out = Ly.v.out = n;
            Ly.k = Ly.q; Ly.v = Ly.q;
            Ly.k.w = qkv.w + (size_t)n * qkv.row_bytes;
            Ly.v.w = qkv.w + 2 * (size_t)n * qkv.row_bytes;
        } else {
            LIN(q, "attn_q.weight", n, n);
            LIN(k, "attn_k.weight", n, kvd);
            LIN(v, "attn_v.weight", n, kvd);
        }
        LIN(o, "attn_output.weight", n, n);
        if (c.use_ffn_gate) {
            LIN(gate, "ffn_gate.weight", n, c.n_ff);
            LIN(up, "ffn_up.weight", n, c.n_ff);
            LIN(down, "ffn_down.weight", c.n_ff, n);
            if (Ly.gate.type != Ly.up.type) { set_err("layer %u: ffn_gate and ffn_up types differ", l); FAIL(); }
        } else {                                    // plain FFN (ffn.c:110-168), fc1/fc2 names too
            snprintf(nm, sizeof nm, "blk.%u.ffn_up.weight", l);
            const forword_gpu_tensor_t *tu = find_t(tensors, n_tensors, nm);
            if (!tu) { snprintf(nm, sizeof nm, "blk.%u.fc1.weight", l); tu = find_t(tensors, n_tensors, nm); }
            if (bind_lin(h, Ly.up, tu, nm, n, c.n_ff)) FAIL();
            snprintf(nm, sizeof nm, "blk.%u.fc2.weight", l);
            const forword_gpu_tensor_t *td = find_t(tensors, n_tensors, nm);
            if (!td) { snprintf(nm, sizeof nm, "blk.%u.ffn_down.weight", l); td = find_t(tensors, n_tensors, nm); }
            if (bind_lin(h, Ly.down, td, nm, c.n_ff, n)) FAIL();
            if (c.arch == FORWORD_ARCH_GPT2) {      // ffn.c:127-140 (required), :162-166 (fc2 has none)
                const bool fc2 = strstr(nm, "fc2") != nullptr;
                snprintf(nm, sizeof nm, "blk.%u.ffn_up.bias", l);
                if (bind_vec(h, &Ly.bu, find_t(tensors, n_tensors, nm), nm, c.n_ff, true)) FAIL();
                snprintf(nm, sizeof nm, "blk.%u.ffn_down.bias", l);
                if (bind_vec(h, &Ly.bd, find_t(tensors, n_tensors, nm), nm, n, true)) FAIL();
                if (fc2) Ly.bd = nullptr;
            }
        }
#undef LIN
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.weight", l);
        if (bind_vec(h, &Ly.attn_norm, find_t(tensors, n_tensors, nm), nm, n, true)) FAIL();
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.weight", l);                         // unused by a parallel block
        if (bind_vec(h, &Ly.ffn_norm, find_t(tensors, n_tensors, nm), nm, n, !c.parallel_res)) FAIL();
        snprintf(nm, sizeof nm, "blk.%u.attn_norm.bias", l);                          // transformer.c:212-230
        if (bind_vec(h, &Ly.attn_norm_b, find_t(tensors, n_tensors, nm), nm, n, false)) FAIL();
        snprintf(nm, sizeof nm, "blk.%u.ffn_norm.bias", l);
        if (bind_vec(h, &Ly.ffn_norm_b, find_t(tensors, n_tensors, nm), nm, n, false)) FAIL();
        snprintf(nm, sizeof nm, "blk.%u.attn_output.bias", l);                        // attention.c:106-107
        if (bind_vec(h, &Ly.bo, find_t(tensors, n_tensors, nm), nm, n, false)) FAIL();
        if (Ly.bo) h->generic = true;
    }
    if (c.norm_type != FORWORD_NORM_RMS || c.parallel_res || !c.use_ffn_gate || c.rope_type != FORWORD_ROPE_NORMAL)
        h->generic = true;
    if (c.arch == FORWORD_ARCH_GPT2) {                                                  // transformer.c:188-205
        const forword_gpu_tensor_t *tp = find_t(tensors, n_tensors, "position_embd.weight");
        if (bind_lin(h, h->pos_embd, tp, "position_embd.weight", n, tp && tp->n_dims > 1 ? tp->dims[1] : 0)) FAIL();
        if (h->pos_embd.out < max_ctx) {
            set_err("position_embd.weight has %u rows, fewer than the %zu positions", h->pos_embd.out, max_ctx);
            FAIL();
        }
    }
    if (c.parallel_res && dalloc(h, (void **)&h->d_ao, (size_t)n * 4, "attention output")) FAIL();
    if (c.arch == FORWORD_ARCH_GPT2) {
        // attention.c:78-90: attn_qkv.bias is already [q | k | v], used in place
        for (uint32_t l = 0; l < c.n_layer; l++) {
            char nm[96];
            snprintf(nm, sizeof nm, "blk.%u.attn_qkv.bias", l);
            if (bind_vec(h, &h->L[l].bqkv, find_t(tensors, n_tensors, nm), nm, 3 * (size_t)n, false)) FAIL();
        }
    } else if (c.use_qkv_bias) {
        // attention.c:114-122: the q/k/v biases of each layer, gathered into one
        // [n_embd | kv_dim | kv_dim] vector in the order the fused QKV rows use;
        // a missing one adds nothing (zeros).  linear.c:214-221 adds F32 biases only.
        const size_t per = (size_t)n + 2 * kvd;
        if (dalloc(h, (void **)&h->d_bias, c.n_layer * per * 4, "qkv bias") ||
            hipMemset(h->d_bias, 0, c.n_layer * per * 4) != hipSuccess)
            FAIL();
        static const char *const sfx[3] = { "attn_q.bias", "attn_k.bias", "attn_v.bias" };
        for (uint32_t l = 0; l < c.n_layer; l++) {
            float *dst = h->d_bias + l * per;
            const size_t off[3] = { 0, n, (size_t)n + kvd }, len[3] = { n, kvd, kvd };
            for (int r = 0; r < 3; r++) {
                char nm[96];
                snprintf(nm, sizeof nm, "blk.%u.%s", l, sfx[r]);
                const float *b = nullptr;
                if (bind_vec(h, &b, find_t(tensors, n_tensors, nm), nm, len[r], false)) FAIL();
                if (b && hipMemcpy(dst + off[r], b, len[r] * 4, hipMemcpyDeviceToDevice) != hipSuccess) {
                    set_err("qkv bias copy failed");
                    FAIL();
                }
            }
            h->L[l].bqkv = dst;
        }
    }

    const size_t kv_elems = (size_t)c.n_layer * max_ctx * kvd, half = hd / 2;
    h->n_splits = attn_splits((uint32_t)max_ctx, c.n_head_kv);
    h->am_blocks = argmax_blocks(c.n_vocab);
    if (dalloc(h, (void **)&h->d_k, kv_elems * 4, "K cache") || dalloc(h, (void **)&h->d_v, kv_elems * 4, "V cache") ||
        dalloc(h, (void **)&h->d_cos, max_ctx * half * 4, "RoPE cos") ||
        dalloc(h, (void **)&h->d_sin, max_ctx * half * 4, "RoPE sin") ||
        dalloc(h, (void **)&h->d_x, (size_t)n * 4, "x") || dalloc(h, (void **)&h->d_xn, (size_t)n * 4, "xn") ||
        dalloc(h, (void **)&h->d_q, (size_t)n * 4, "q") || dalloc(h, (void **)&h->d_att, (size_t)n * 4, "attn") ||
        dalloc(h, (void **)&h->d_h, (size_t)c.n_ff * 4, "ffn") ||
        dalloc(h, (void **)&h->d_logits, (size_t)c.n_vocab * 4, "logits") ||
        dalloc(h, (void **)&h->d_part, (size_t)c.n_head * h->n_splits * (hd + 2) * 4, "attention partials") ||
        dalloc(h, (void **)&h->d_trace, (size_t)2 * c.n_layer * n * 4, "trace") ||
        dalloc(h, (void **)&h->d_pv, h->am_blocks * 4, "argmax") || dalloc(h, (void **)&h->d_pi, h->am_blocks * 4, "argmax") ||
        dalloc(h, (void **)&h->d_counter, 4, "argmax") || dalloc(h, (void **)&h->d_argmax, 4, "argmax") ||
        dalloc(h, (void **)&h->d_prompt, max_ctx * 4, "prompt") || dalloc(h, (void **)&h->d_ids, (max_ctx + 1) * 4, "ids") ||
        dalloc(h, (void **)&h->d_state, sizeof(StepState), "state") ||
        dalloc(h, (void **)&h->d_pss, ((size_t)n / 16 + 64) * 4, "norm partials") ||
        dalloc(h, (void **)&h->d_scale, 64, "norm scale") || dalloc(h, (void **)&h->d_ticket, 64, "norm ticket"))
        FAIL();
    h->h_state = &h->host_state;
    if (hipHostMalloc((void **)&h->h_logits, (size_t)c.n_vocab * 4, 0) != hipSuccess ||
        hipHostMalloc((void **)&h->h_u32, 4 * 4, 0) != hipSuccess) {
        set_err("pinned host allocation failed");
        FAIL();
    }
    memset(h->h_state, 0, sizeof(StepState));
    if (hipMemset(h->d_k, 0, kv_elems * 4) != hipSuccess || hipMemset(h->d_v, 0, kv_elems * 4) != hipSuccess ||
        hipMemset(h->d_counter, 0, 4) != hipSuccess || hipMemset(h->d_state, 0, sizeof(StepState)) != hipSuccess ||
        hipMemset(h->d_ticket, 0, 64) != hipSuccess || hipMemset(h->d_scale, 0, 64) != hipSuccess ||
        hipMemset(h->d_trace, 0, (size_t)2 * c.n_layer * n * 4) != hipSuccess ||
        hipMemcpy(h->d_cos, cos_tab, max_ctx * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(h->d_sin, sin_tab, max_ctx * half * 4, hipMemcpyHostToDevice) != hipSuccess ||
        hipDeviceSynchronize() != hipSuccess) {
        set_err("device initialisation failed");
        FAIL();
    }
    if (setup_mk(h)) FAIL();
    if (!h->mk) build_graph(h);
#undef FAIL
    *out = h;
    return 0;
}

static int check_tok_pos(forword_gpu_t *h, uint32_t token, size_t pos)
{
    if (!h) { set_err("NULL handle"); return -1; }
    if (pos >= h->n_ctx) { set_err("position %zu exceeds KV cache (%zu)", pos, h->n_ctx); return -1; }
    if (token >= h->cfg.n_vocab) { set_err("token ID %u out of range", token); return -1; }
    return 0;
}

static int step_once(forword_gpu_t *h, uint32_t token, size_t pos)
{
    // a host-driven step ends any device-resident greedy loop
    h->h_state->token = token;
    h->h_state->pos = (uint32_t)pos;
    h->h_state->n_prompt = 0;
    h->h_state->greedy = 0;
    HIPCHK(launch_set_state(h->d_state, *h->h_state, h->stream), "state upload");
    if (run_steps(h, 1)) return -1;
    h->traced = true;
    return 0;
}

extern "C" float *forword_gpu_forward(forword_gpu_t *h, uint32_t token_id, size_t pos)
{
    if (check_tok_pos(h, token_id, pos) || step_once(h, token_id, pos)) return nullptr;
    if (hipMemcpyAsync(h->h_logits, h->d_logits, (size_t)h->cfg.n_vocab * 4, hipMemcpyDeviceToHost, h->stream) !=
            hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess) {
        set_err("forward: %s", hipGetErrorString(hipGetLastError()));
        return nullptr;
    }
    if (mk_check(h)) return nullptr;
    return h->h_logits;
}

extern "C" int forword_gpu_forward_argmax(forword_gpu_t *h, uint32_t token_id, size_t pos, uint32_t *next)
{
    if (!next) { set_err("forward_argmax: next is NULL"); return -1; }
    if (check_tok_pos(h, token_id, pos) || step_once(h, token_id, pos)) return -1;
    HIPCHK(hipMemcpyAsync(h->h_u32, h->d_argmax, 4, hipMemcpyDeviceToHost, h->stream), "argmax download");
    HIPCHK(hipStreamSynchronize(h->stream), "forward_argmax");
    if (mk_check(h)) return -1;
    *next = h->h_u32[0];
    return 0;
}

extern "C" int forword_gpu_generate_greedy(forword_gpu_t *h, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                                           uint32_t *out_ids)
{
    if (!h || !prompt || !n_prompt || (n_gen && !out_ids)) { set_err("generate_greedy: invalid arguments"); return -1; }
    const size_t n_fwd = n_gen ? n_prompt + n_gen - 1 : n_prompt;
    if (n_fwd > h->n_ctx) { set_err("generate_greedy: %zu forwards exceed the KV cache (%zu)", n_fwd, h->n_ctx); return -1; }
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= h->cfg.n_vocab) { set_err("generate_greedy: prompt token %u out of range", prompt[i]); return -1; }
    HIPCHK(hipMemcpyAsync(h->d_prompt, prompt, n_prompt * 4, hipMemcpyHostToDevice, h->stream), "prompt upload");
    h->h_state->token = prompt[0];
    h->h_state->pos = 0;
    h->h_state->n_prompt = (uint32_t)n_prompt;
    h->h_state->next = 0;
    h->h_state->greedy = 1;
    HIPCHK(launch_set_state(h->d_state, *h->h_state, h->stream), "state upload");
    if (run_steps(h, n_fwd)) return -1;
    if (n_gen) HIPCHK(hipMemcpyAsync(out_ids, h->d_ids, n_gen * 4, hipMemcpyDeviceToHost, h->stream), "ids download");
    HIPCHK(hipStreamSynchronize(h->stream), "generate_greedy");
    if (mk_check(h)) return -1;
    h->h_state->pos = (uint32_t)n_fwd;     // host mirror of the device state, for forword_gpu_decode
    h->traced = true;
    return 0;
}

extern "C" int forword_gpu_decode(forword_gpu_t *h, size_t n_steps, uint32_t *out_ids)
{
    if (!h) { set_err("decode: NULL handle"); return -1; }
    if (!h->h_state->greedy) { set_err("decode: no greedy loop to continue (call generate_greedy first)"); return -1; }
    const size_t pos = h->h_state->pos, n_prompt = h->h_state->n_prompt;
    if (pos + n_steps > h->n_ctx) { set_err("decode: %zu more forwards exceed the KV cache (%zu)", n_steps, h->n_ctx); return -1; }
    if (run_steps(h, n_steps)) return -1;
    h->h_state->pos = (uint32_t)(pos + n_steps);
    if (out_ids && n_steps) {
        // step at position p writes the token for position p+1 at ids[p + 1 - n_prompt]
        HIPCHK(hipMemcpyAsync(out_ids, h->d_ids + (pos + 1 - n_prompt), n_steps * 4, hipMemcpyDeviceToHost, h->stream),
               "ids download");
        HIPCHK(hipStreamSynchronize(h->stream), "decode");
        if (mk_check(h)) return -1;
    }
    return 0;
}

extern "C" int forword_gpu_decode_from(forword_gpu_t *h, uint32_t token, size_t pos, size_t n_steps,
                                       uint32_t *out_ids)
{
    if (!h || !n_steps) { set_err("decode_from: invalid arguments"); return -1; }
    if (check_tok_pos(h, token, pos)) return -1;
    if (pos + n_steps > h->n_ctx) { set_err("decode_from: %zu forwards from %zu exceed the KV cache (%zu)", n_steps, pos, h->n_ctx); return -1; }
    // n_prompt = pos + 1: no prefill step, ids[0] is the token for position pos + 1
    h->h_state->token = token;
    h->h_state->pos = (uint32_t)pos;
    h->h_state->n_prompt = (uint32_t)(pos + 1);
    h->h_state->next = 0;
    h->h_state->greedy = 1;
    HIPCHK(launch_set_state(h->d_state, *h->h_state, h->stream), "state upload");
    if (run_steps(h, n_steps)) return -1;
    h->h_state->pos = (uint32_t)(pos + n_steps);
    h->traced = true;
    if (out_ids) {
        HIPCHK(hipMemcpyAsync(out_ids, h->d_ids, n_steps * 4, hipMemcpyDeviceToHost, h->stream), "ids download");
        HIPCHK(hipStreamSynchronize(h->stream), "decode_from");
        if (mk_check(h)) return -1;
    }
    return 0;
}

// ── batched prefill ──────────────────────────────────────────────────────────

// Tokens per pass of the batched prefill: longer prompts run in passes, each
// attending to the cache rows the previous ones wrote.
static constexpr uint32_t kPrefillChunk = 512;

static bool prefill_type_ok(uint32_t t) { return t == kQ4_0 || t == kQ5_0 || t == kQ8_0 || t == kQ4_K || t == kQ6_K; }

// Queue the batched forward of tokens[0..n_tok) at positions pos0.. (KV rows
// written), the last token's logits into d_logits and their argmax into d_argmax.
static int prefill_run(forword_gpu_t *h, const uint32_t *tokens, size_t n_tok, size_t pos0)
{
    if (!h || !tokens || !n_tok) { set_err("prefill: invalid arguments"); return -1; }
    const forword_gpu_config_t &c = h->cfg;
    if (pos0 > h->n_ctx || n_tok > h->n_ctx - pos0) {
        set_err("prefill: positions [%zu, %zu) exceed the KV cache (%zu)", pos0, pos0 + n_tok, h->n_ctx);
        return -1;
    }
    for (size_t i = 0; i < n_tok; i++)
        if (tokens[i] >= c.n_vocab) { set_err("prefill: token %u out of range", tokens[i]); return -1; }
    const uint32_t n = c.n_embd, hd = c.head_dim, nq = c.n_head * hd, kvd = c.n_head_kv * hd, nff = c.n_ff;
    for (const Layer &Ly : h->L)
        for (const Lin *l : { &Ly.q, &Ly.k, &Ly.v, &Ly.o, &Ly.gate, &Ly.up, &Ly.down })
            if ((l != &Ly.gate || c.use_ffn_gate) && !prefill_type_ok(l->type)) {
                set_err("prefill: linear type %u not supported", l->type);
                return -1;
            }
    if (!attn_supported(hd, c.n_head / std::max<uint32_t>(c.n_head_kv, 1)) || c.n_head % c.n_head_kv || nq != n) {
        set_err("prefill: head layout not supported");
        return -1;
    }
    // per-token activations: x, xn [n] | q k v [nq + 2 kvd] | attention [nq] | gate, up [n_ff] | attn_out [n]
    const size_t ldqkv = (size_t)nq + 2 * kvd, per_tok = 3 * (size_t)n + ldqkv + nq + 2 * (size_t)nff;
    if (!h->d_pf && (dalloc(h, (void **)&h->d_pf, kPrefillChunk * per_tok * 4, "prefill activations") ||
                     dalloc(h, (void **)&h->d_pf_tok, kPrefillChunk * 4, "prefill tokens")))
        return -1;
    float *X = h->d_pf, *Xn = X + (size_t)kPrefillChunk * n, *QKV = Xn + (size_t)kPrefillChunk * n;
    float *Att = QKV + (size_t)kPrefillChunk * ldqkv, *G = Att + (size_t)kPrefillChunk * nq;
    float *U = G + (size_t)kPrefillChunk * nff, *AO = U + (size_t)kPrefillChunk * nff;
    const bool par = c.parallel_res != 0, neox = c.rope_type == FORWORD_ROPE_NEOX;
    hipStream_t s = h->stream;
#define TRY(x) do { hipError_t e_ = (x); if (e_ != hipSuccess) { set_err("prefill: %s (line %d)", hipGetErrorString(e_), __LINE__); return -1; } } while (0)
    uint32_t rows = 0;
    for (size_t c0 = 0; c0 < n_tok; c0 += kPrefillChunk) {
        rows = (uint32_t)std::min<size_t>(kPrefillChunk, n_tok - c0);
        const uint32_t p0 = (uint32_t)(pos0 + c0);
        TRY(hipMemcpyAsync(h->d_pf_tok, tokens + c0, (size_t)rows * 4, hipMemcpyHostToDevice, s));
        TRY(launch_embed_rows(h->embd.w, h->embd.type, n, h->d_pf_tok, rows, c.embd_scale, X, s));
        if (h->pos_embd.w)                                                              // transformer.c:188-205
            TRY(launch_pos_add(h->pos_embd.w, h->pos_embd.type, h->pos_embd.row_bytes, n, nullptr, p0, rows, X, s));
        for (uint32_t l = 0; l < c.n_layer; l++) {
            const Layer &Ly = h->L[l];
            float *kc = h->d_k + (size_t)l * h->n_ctx * kvd, *vc = h->d_v + (size_t)l * h->n_ctx * kvd;
            TRY(launch_block_norm(h, X, Ly.attn_norm, Ly.attn_norm_b, Xn, s, rows));          // transformer.c:234-261
            if (Ly.q.type == Ly.k.type && Ly.k.type == Ly.v.type) {                           // q | k | v rows
                GemmW g{};
                g.w[0] = Ly.q.w; g.w[1] = Ly.k.w; g.w[2] = Ly.v.w;
                g.rb[0] = Ly.q.row_bytes; g.rb[1] = Ly.k.row_bytes; g.rb[2] = Ly.v.row_bytes;
                g.end[0] = nq; g.end[1] = nq + kvd; g.end[2] = nq + 2 * kvd; g.n_seg = 3;
                TRY(launch_gemm_qs(Ly.q.type, Xn, n, g, QKV, ldqkv, rows, n, false, s));
            } else {
                TRY(launch_gemm_q(Ly.q.type, Xn, n, Ly.q.w, Ly.q.row_bytes, QKV, ldqkv, rows, nq, n, false, s));
                TRY(launch_gemm_q(Ly.k.type, Xn, n, Ly.k.w, Ly.k.row_bytes, QKV + nq, ldqkv, rows, kvd, n, false, s));
                TRY(launch_gemm_q(Ly.v.type, Xn, n, Ly.v.w, Ly.v.row_bytes, QKV + nq + kvd, ldqkv, rows, kvd, n, false,
                                  s));
            }
            TRY(launch_rope_append(QKV, Ly.bqkv, c.rope_type == FORWORD_ROPE_NONE ? 2 : neox ? 1 : 0, ldqkv, rows, c.n_head, c.n_head_kv, hd, p0, h->d_cos, h->d_sin, kc, vc, s));
            TRY(launch_attn_prefill(QKV, ldqkv, rows, kc, vc, Att, c.n_head, c.n_head_kv, hd, p0, s));
            const uint64_t cnt = (uint64_t)rows * n;
            if (par || Ly.bo) {                       // output projection kept apart: its bias, the parallel add
                TRY(launch_gemm_q(Ly.o.type, Att, nq, Ly.o.w, Ly.o.row_bytes, AO, n, rows, n, nq, false, s));
                if (!par) TRY(launch_resid_add(X, AO, Ly.bo, nullptr, cnt, n, s));         // :271-272
            } else {
                TRY(launch_gemm_q(Ly.o.type, Att, nq, Ly.o.w, Ly.o.row_bytes, X, n, rows, n, nq, true, s));   // :271-272
            }
            if (!par) TRY(launch_block_norm(h, X, Ly.ffn_norm, Ly.ffn_norm_b, Xn, s, rows));   // :275-280
            const float *H = G;
            if (c.use_ffn_gate) {                                                              // ffn.c:68-104
                TRY(launch_gemm_q(Ly.gate.type, Xn, n, Ly.gate.w, Ly.gate.row_bytes, G, nff, rows, nff, n, false, s));
                TRY(launch_gemm_q(Ly.up.type, Xn, n, Ly.up.w, Ly.up.row_bytes, U, nff, rows, nff, n, false, s));
                TRY(launch_act_mul(G, U, G, (uint64_t)rows * nff, ffn_act_code(c), s));
            } else {                                                                           // ffn.c:108-160
                TRY(launch_gemm_q(Ly.up.type, Xn, n, Ly.up.w, Ly.up.row_bytes, U, nff, rows, nff, n, false, s));
                TRY(launch_act(U, U, (uint64_t)rows * nff, plain_act_code(c), s, Ly.bu, nff));
                H = U;
            }
            if (par) {                                                                         // transformer.c:250-251
                TRY(launch_gemm_q(Ly.down.type, H, nff, Ly.down.w, Ly.down.row_bytes, Xn, n, rows, n, nff, false, s));
                TRY(launch_resid_add(X, AO, Ly.bo, Xn, cnt, n, s));
            } else if (Ly.bd) {                                                                // x += (W h + bd)
                TRY(launch_gemm_q(Ly.down.type, H, nff, Ly.down.w, Ly.down.row_bytes, AO, n, rows, n, nff, false, s));
                TRY(launch_resid_add(X, AO, Ly.bd, nullptr, cnt, n, s));
            } else {
                TRY(launch_gemm_q(Ly.down.type, H, nff, Ly.down.w, Ly.down.row_bytes, X, n, rows, n, nff, true, s));
            }
        }
    }
    // logits of the last token (transformer.c:293-323), then its argmax
    const float *xl = X + (size_t)(rows - 1) * n;
    if (h->out_norm) TRY(launch_block_norm(h, xl, h->out_norm, h->out_norm_b, h->d_xn, s));
    else TRY(hipMemcpyAsync(h->d_xn, xl, (size_t)n * 4, hipMemcpyDeviceToDevice, s));
    {
        QmvArgs a{};
        a.n_seg = 1; a.w[0] = h->out.w; a.rows[0] = h->out.out; a.n_cols = n; a.row_bytes = h->out.row_bytes;
        a.x = h->d_xn; a.out[0] = h->d_logits; a.state = h->d_state;
        qmv_plan(a, EPI_STORE);
        TRY(launch_qmv(h->out.type, EPI_STORE, a, s));
    }
    TRY(launch_argmax(h->d_logits, c.n_vocab, h->d_pv, h->d_pi, h->d_counter, h->d_argmax, nullptr, nullptr, nullptr,
                      h->am_blocks, s));
#undef TRY
    h->traced = false;                       // no per-layer trace of a batched pass
    return 0;
}

extern "C" float *forword_gpu_prefill(forword_gpu_t *h, const uint32_t *tokens, size_t n_tokens, size_t pos0)
{
    if (prefill_run(h, tokens, n_tokens, pos0)) return nullptr;
    if (hipMemcpyAsync(h->h_logits, h->d_logits, (size_t)h->cfg.n_vocab * 4, hipMemcpyDeviceToHost, h->stream) !=
            hipSuccess ||
        hipStreamSynchronize(h->stream) != hipSuccess) {
        set_err("prefill: %s", hipGetErrorString(hipGetLastError()));
        return nullptr;
    }
    return h->h_logits;
}

extern "C" int forword_gpu_prefill_argmax(forword_gpu_t *h, const uint32_t *tokens, size_t n_tokens, size_t pos0,
                                          uint32_t *next)
{
    if (!next) { set_err("prefill_argmax: next is NULL"); return -1; }
    if (prefill_run(h, tokens, n_tokens, pos0)) return -1;
    HIPCHK(hipMemcpyAsync(h->h_u32, h->d_argmax, 4, hipMemcpyDeviceToHost, h->stream), "argmax download");
    HIPCHK(hipStreamSynchronize(h->stream), "prefill_argmax");
    *next = h->h_u32[0];
    return 0;
}

// ── sampled generation ───────────────────────────────────────────────────────

static uint32_t next_pow2(uint32_t n)
{
    uint32_t p = 1;
    while (p < n) p <<= 1;
    return p;
}

// Candidates the top-p sort holds in LDS; more go to the global key buffer.
static constexpr uint32_t kSampleCap = 16384;

extern "C" int forword_gpu_generate(forword_gpu_t *h, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                                    float temperature, float top_p, float repetition_penalty, uint64_t seed,
                                    uint32_t *out_ids)
{
    if (!h || !prompt || !n_prompt || !n_gen || !out_ids) { set_err("generate: invalid arguments"); return -1; }
    const uint32_t nv = h->cfg.n_vocab;
    const size_t n_fwd = n_prompt + n_gen - 1;
    if (n_fwd > h->n_ctx) { set_err("generate: %zu forwards exceed the KV cache (%zu)", n_fwd, h->n_ctx); return -1; }
    for (size_t i = 0; i < n_prompt; i++)
        if (prompt[i] >= nv) { set_err("generate: prompt token %u out of range", prompt[i]); return -1; }
    if (!h->d_sbuf) {
        if (dalloc(h, (void **)&h->d_sbuf, (size_t)nv * 4, "sampler probabilities") ||
            dalloc(h, (void **)&h->d_spart, 512 * 4, "sampler partials") ||
            dalloc(h, (void **)&h->d_bsum, 1024 * 8, "sampler buckets") ||
            dalloc(h, (void **)&h->d_gkeys, (size_t)next_pow2(nv) * 8, "sampler keys") ||
            dalloc(h, (void **)&h->d_bcnt, 1024 * 4, "sampler buckets") ||
            dalloc(h, (void **)&h->d_counts, (size_t)nv * 4, "history counts") ||
            dalloc(h, (void **)&h->d_sids, (h->n_ctx + 1) * 4, "sampled ids") ||
            dalloc(h, (void **)&h->d_ss, sizeof(SampleState), "sampler state"))
            return -1;
        HIPCHK(hipMemset(h->d_bsum, 0, 1024 * 8), "sampler buckets");
        HIPCHK(hipMemset(h->d_bcnt, 0, 1024 * 4), "sampler buckets");
    }
    // history counts of the prompt (main.c:157-161) and the PRNG seed (main.c:98-99)
    std::vector<uint32_t> counts(nv, 0u);
    for (size_t i = 0; i < n_prompt; i++) counts[prompt[i]]++;
    SampleState ss{};
    ss.rng = seed ? seed : 12345u;
    HIPCHK(hipMemcpyAsync(h->d_counts, counts.data(), (size_t)nv * 4, hipMemcpyHostToDevice, h->stream), "counts upload");
    HIPCHK(hipMemcpyAsync(h->d_ss, &ss, sizeof ss, hipMemcpyHostToDevice, h->stream), "sampler state upload");
    // the prompt as generate_greedy feeds it (main.c:145-151); the last step leaves its logits
    HIPCHK(hipMemcpyAsync(h->d_prompt, prompt, n_prompt * 4, hipMemcpyHostToDevice, h->stream), "prompt upload");
    h->h_state->token = prompt[0];
    h->h_state->pos = 0;
    h->h_state->n_prompt = (uint32_t)n_prompt;
    h->h_state->next = 0;
    h->h_state->greedy = 1;
    HIPCHK(launch_set_state(h->d_state, *h->h_state, h->stream), "state upload");
    if (run_steps(h, n_prompt)) return -1;
    // main.c:173-217: sample from the logits on the device, forward the sample
    for (size_t g = 0; g < n_gen; g++) {
        HIPCHK(launch_sample(h->d_logits, nv, h->d_counts, temperature, top_p, repetition_penalty, h->d_sbuf,
                             h->d_spart, h->d_bcnt, h->d_bsum, h->d_gkeys, kSampleCap, h->d_ss, h->d_state, h->d_sids,
                             (uint32_t)g, h->d_counts, h->stream),
               "sampler launch");
        if (g + 1 < n_gen && run_steps(h, 1)) return -1;
    }
    HIPCHK(hipMemcpyAsync(out_ids, h->d_sids, n_gen * 4, hipMemcpyDeviceToHost, h->stream), "ids download");
    HIPCHK(hipMemcpyAsync(&ss, h->d_ss, sizeof ss, hipMemcpyDeviceToHost, h->stream), "sampler state download");
    HIPCHK(hipStreamSynchronize(h->stream), "generate");
    if (mk_check(h)) return -1;
    h->h_state->pos = (uint32_t)n_fwd;
    h->traced = true;
    if (ss.err) {
        set_err("generate: no finite probability to sample from (non-finite logits)");
        return -1;
    }
    return 0;
}

static int kv_args(forword_gpu_t *h, size_t layer, size_t pos0, size_t n_pos)
{
    if (!h) { set_err("NULL handle"); return -1; }
    if (layer >= h->cfg.n_layer || pos0 > h->n_ctx || n_pos > h->n_ctx - pos0) {
        set_err("kv: layer %zu / positions [%zu, %zu) out of range", layer, pos0, pos0 + n_pos);
        return -1;
    }
    return 0;
}

extern "C" int forword_gpu_kv_write(forword_gpu_t *h, size_t layer, size_t pos0, size_t n_pos, const float *k,
                                    const float *v)
{
    if (kv_args(h, layer, pos0, n_pos)) return -1;
    const size_t kvd = (size_t)h->cfg.n_head_kv * h->cfg.head_dim, off = (layer * h->n_ctx + pos0) * kvd;
    HIPCHK(hipStreamSynchronize(h->stream), "kv_write");
    if (k) HIPCHK(hipMemcpy(h->d_k + off, k, n_pos * kvd * 4, hipMemcpyHostToDevice), "kv_write K");
    if (v) HIPCHK(hipMemcpy(h->d_v + off, v, n_pos * kvd * 4, hipMemcpyHostToDevice), "kv_write V");
    return 0;
}

extern "C" int forword_gpu_kv_read(forword_gpu_t *h, size_t layer, size_t pos0, size_t n_pos, float *k, float *v)
{
    if (kv_args(h, layer, pos0, n_pos)) return -1;
    const size_t kvd = (size_t)h->cfg.n_head_kv * h->cfg.head_dim, off = (layer * h->n_ctx + pos0) * kvd;
    HIPCHK(hipStreamSynchronize(h->stream), "kv_read");
    if (k) HIPCHK(hipMemcpy(k, h->d_k + off, n_pos * kvd * 4, hipMemcpyDeviceToHost), "kv_read K");
    if (v) HIPCHK(hipMemcpy(v, h->d_v + off, n_pos * kvd * 4, hipMemcpyDeviceToHost), "kv_read V");
    return 0;
}

extern "C" int forword_gpu_layer_trace(forword_gpu_t *h, float *out)
{
    if (!h || !out) { set_err("layer_trace: invalid arguments"); return -1; }
    if (!h->traced) { set_err("layer_trace: no forward has run yet"); return -1; }
    HIPCHK(hipStreamSynchronize(h->stream), "layer_trace");
    HIPCHK(hipMemcpy(out, h->d_trace, (size_t)2 * h->cfg.n_layer * h->cfg.n_embd * 4, hipMemcpyDeviceToHost),
           "layer_trace");
    return 0;
}

extern "C" size_t forword_gpu_n_ctx(const forword_gpu_t *h) { return h ? h->n_ctx : 0; }
extern "C" void *forword_gpu_stream(const forword_gpu_t *h) { return h ? (void *)h->stream : nullptr; }
extern "C" int forword_gpu_step_impl(const forword_gpu_t *h) { return h && h->mk ? 1 : 0; }

extern "C" int forword_gpu_status(forword_gpu_t *h)
{
    if (!h) { set_err("status: NULL handle"); return -1; }
    HIPCHK(hipStreamSynchronize(h->stream), "status");
    return mk_check(h);
}

extern "C" int forword_gpu_phase_times(forword_gpu_t *h, double *us, size_t n)
{
    if (!h || !us) { set_err("phase_times: invalid arguments"); return -1; }
    if (!h->d_prof || !h->prof_steps) { set_err("phase_times: no stamped persistent launch"); return -1; }
    const size_t n_ops = 5 * (size_t)h->cfg.n_layer + 1, steps = h->prof_steps;
    std::vector<uint64_t> t(1 + steps * n_ops);
    int dev = 0, khz = 0;
    HIPCHK(hipStreamSynchronize(h->stream), "phase_times");
    HIPCHK(hipMemcpy(t.data(), h->d_prof, t.size() * 8, hipMemcpyDeviceToHost), "phase_times");
    HIPCHK(hipGetDevice(&dev), "phase_times");
    HIPCHK(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, dev), "phase_times");
    const size_t m = n < n_ops ? n : n_ops;
    for (size_t i = 0; i < m; i++) {
        double sum = 0;
        for (size_t st = 0; st < steps; st++) {
            const size_t k = 1 + st * n_ops + i;
            sum += (double)(t[k] - t[k - 1]);
        }
        us[i] = sum / steps * 1e3 / khz;
    }
    return (int)m;
}

// ── operator level ───────────────────────────────────────────────────────────

namespace {
// Scratch shared by operator-level calls on this device: argmax partials and
// attention partials.  Calls that overlap on different streams race on it.
std::mutex g_scratch_mu;
float *g_pv = nullptr;
uint32_t *g_pi = nullptr, *g_counter = nullptr;
float *g_part = nullptr;
size_t g_part_bytes = 0;

int op_scratch_argmax()
{
    if (g_counter) return 0;
    if (hipMalloc(&g_pv, 256 * 4) != hipSuccess || hipMalloc(&g_pi, 256 * 4) != hipSuccess ||
        hipMalloc(&g_counter, 4) != hipSuccess || hipMemset(g_counter, 0, 4) != hipSuccess) {
        set_err("argmax scratch allocation failed");
        return -1;
    }
    return 0;
}

int op_scratch_part(size_t bytes)
{
    if (g_part_bytes >= bytes) return 0;
    if (g_part) { (void)hipDeviceSynchronize(); (void)hipFree(g_part); g_part = nullptr; g_part_bytes = 0; }
    if (hipMalloc(&g_part, bytes) != hipSuccess) { set_err("attention scratch allocation failed"); return -1; }
    g_part_bytes = bytes;
    return 0;
}

int launched(hipError_t e, const char *what)
{
    if (e != hipSuccess) { set_err("%s: %s", what, hipGetErrorString(e)); return -1; }
    return 0;
}
} // namespace

extern "C" int forword_gpu_quant_matvec(const void *weights, size_t weights_size, uint32_t type, const float *input,
                                        float *output, size_t in, size_t out, void *stream)
{
    if (!weights || !input || !output || !in || !out) { set_err("quant_matvec: invalid arguments"); return -1; }
    uint64_t rb;
    if (type == kF32) rb = (uint64_t)in * 4;
    else if (type_block_values(type)) {
        if (in % type_block_values(type)) { set_err("quant_matvec: input size not a multiple of the block size"); return -1; }
        rb = type_row_bytes(type, in);
    } else { set_err("quant_matvec: unsupported ggml type %u", type); return -1; }
    if (in >= (1u << 31) || out >= (1u << 31) || out > SIZE_MAX / rb || weights_size < out * rb) {
        set_err("quant_matvec: weights buffer too small or sizes too large");
        return -1;
    }
    const hipError_t e = launch_gemv(type, (const uint8_t *)weights, rb, input, output, (uint32_t)out, (uint32_t)in,
                                     (hipStream_t)stream);
    if (e != hipErrorNotSupported) return launched(e, "quant_matvec");
    QmvArgs a{};
    a.n_seg = 1; a.w[0] = (const uint8_t *)weights; a.rows[0] = (uint32_t)out; a.n_cols = (uint32_t)in;
    a.row_bytes = rb; a.x = input; a.out[0] = output;
    qmv_plan(a, EPI_STORE);
    return launched(launch_qmv(type, EPI_STORE, a, (hipStream_t)stream), "quant_matvec");
}

extern "C" int forword_gpu_ffn_swiglu(const void *w_gate, const void *w_up, size_t weights_size, uint32_t type,
                                      const float *x, float *hout, size_t in, size_t n_ff, void *stream)
{
    if (!w_gate || !w_up || !x || !hout || !in || !n_ff) { set_err("ffn_swiglu: invalid arguments"); return -1; }
    if (!type_block_values(type) || in % type_block_values(type)) {
        set_err("ffn_swiglu: unsupported type or input size");
        return -1;
    }
    uint64_t rb = type_row_bytes(type, in);
    if (in >= (1u << 31) || n_ff >= (1u << 31) || weights_size < n_ff * rb) {
        set_err("ffn_swiglu: weights buffer too small or sizes too large");
        return -1;
    }
    QmvArgs a{};
    a.n_seg = 2; a.w[0] = (const uint8_t *)w_gate; a.w[1] = (const uint8_t *)w_up;
    a.rows[0] = a.rows[1] = (uint32_t)n_ff; a.n_cols = (uint32_t)in; a.row_bytes = rb; a.x = x; a.out[0] = hout;
    qmv_plan(a, EPI_SWIGLU);
    return launched(launch_qmv(type, EPI_SWIGLU, a, (hipStream_t)stream), "ffn_swiglu");
}

extern "C" int forword_gpu_tensor_matvec_f32(const float *weights, const float *x, float *y, size_t rows,
                                             size_t cols, void *stream)
{
    if (!weights || !x || !y || !rows || !cols) { set_err("tensor_matvec_f32: invalid arguments"); return -1; }
    return forword_gpu_quant_matvec(weights, rows * cols * 4, kF32, x, y, cols, rows, stream);
}

extern "C" int forword_gpu_dequant(const void *blocks, size_t size, uint32_t type, float *out, size_t count,
                                   void *stream)
{
    const uint32_t bv = type_block_values(type);
    const uint64_t bb = bv ? type_row_bytes(type, bv) : 0;
    if (!blocks || !out || type == kF32 || !bb || !size || size % bb || count % bv || size / bb != count / bv) {
        set_err("dequant: invalid arguments");
        return -1;
    }
    return launched(launch_dequant((const uint8_t *)blocks, type, size / bb, out, (hipStream_t)stream), "dequant");
}

extern "C" int forword_gpu_get_row(const void *w, size_t size, uint32_t type, size_t n_cols, size_t row, float *out,
                                   void *stream)
{
    if (!w || !out || !n_cols || n_cols >= (1u << 31) || row >= (1u << 31)) { set_err("get_row: invalid arguments"); return -1; }
    if (!type_block_values(type) || n_cols % type_block_values(type)) { set_err("get_row: unsupported type or shape"); return -1; }
    uint64_t rb = type_row_bytes(type, n_cols);
    if (rb == 0 || (row + 1) > size / rb) { set_err("get_row: row outside the tensor"); return -1; }
    return launched(launch_get_row((const uint8_t *)w, type, (uint32_t)n_cols, (uint32_t)row, out, (hipStream_t)stream),
                    "get_row");
}

extern "C" int forword_gpu_rms_norm(const float *x, const float *w, float *out, size_t n, float eps, void *stream)
{
    if (!x || !out || n >= (1u << 31)) { set_err("rms_norm: invalid arguments"); return -1; }
    if (!n) return 0;
    return launched(launch_rmsnorm(x, w, out, (uint32_t)n, eps, (hipStream_t)stream), "rms_norm");
}

extern "C" int forword_gpu_tensor_rms_norm(const float *x, const float *w, float *out, size_t n, float eps, void *stream)
{
    if (!x || !w || !out || !n || !isfinite(eps) || eps <= 0.0f) { set_err("tensor_rms_norm: invalid arguments"); return -1; }
    return forword_gpu_rms_norm(x, w, out, n, eps, stream);
}

extern "C" int forword_gpu_rope_apply(float *qk, size_t pos, size_t n_heads, size_t hd, const float *cos_tab,
                                      const float *sin_tab, int neox, void *stream)
{
    if (!qk || !cos_tab || !sin_tab || !hd || hd % 2 || n_heads * hd >= (1u << 31) || pos >= (1u << 31)) {
        set_err("rope_apply: invalid arguments");
        return -1;
    }
    if (!n_heads) return 0;
    return launched(launch_rope(qk, (uint32_t)pos, (uint32_t)n_heads, (uint32_t)hd, cos_tab, sin_tab, neox,
                                (hipStream_t)stream), "rope_apply");
}

extern "C" int forword_gpu_attention(const float *q, const float *kc, const float *vc, float *out, size_t n_head,
                                     size_t n_kv, size_t hd, size_t n_ctx, size_t pos, void *stream)
{
    if (!q || !kc || !vc || !out || !n_head || !n_kv || !hd || n_head % n_kv || pos >= n_ctx || n_ctx >= (1u << 31)) {
        set_err("attention: invalid head configuration or position");
        return -1;
    }
    if (!attn_supported((uint32_t)hd, (uint32_t)(n_head / n_kv))) {
        set_err("attention: head_dim %zu / GQA group %zu not supported", hd, n_head / n_kv);
        return -1;
    }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    const uint32_t ns = attn_splits((uint32_t)(pos + 1), (uint32_t)n_kv);
    if (op_scratch_part((size_t)n_head * ns * (hd + 2) * 4)) return -1;
    return launched(launch_attention(q, kc, vc, g_part, out, (uint32_t)n_head, (uint32_t)n_kv, (uint32_t)hd, ns, nullptr,
                                     (uint32_t)pos, (hipStream_t)stream), "attention");
}

// ── allocation-free attention ────────────────────────────────────────────────
// The split partials of forword_gpu_attention_noalloc live in `scratch`, one
// copy per device for the life of the process.  Host code never passes the
// symbol itself: its device address comes from hipGetSymbolAddress, looked up
// once per device on the first call made with that device current.  Every
// (head, split) entry a launch reads is written earlier in the same launch, so
// nothing is cleared between calls; calls that overlap on one device race.
namespace {
constexpr size_t kNoAllocScratchBytes = (size_t)8 << 20;
constexpr int kNoAllocMaxDevices = 64;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / 4];
std::mutex g_noalloc_mu;
float *g_noalloc_ptr[kNoAllocMaxDevices] = {};

float *noalloc_scratch()
{
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kNoAllocMaxDevices) {
        set_err("attention_noalloc: no usable current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (!g_noalloc_ptr[dev]) {
        void *p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            set_err("attention_noalloc: scratch address lookup failed: %s", hipGetErrorString(e));
            return nullptr;
        }
        g_noalloc_ptr[dev] = (float *)p;
    }
    return g_noalloc_ptr[dev];
}
} // namespace

extern "C" int forword_gpu_attention_noalloc(const float *q, const float *kc, const float *vc, float *out,
                                             size_t n_head, size_t n_kv, size_t hd, size_t n_ctx, size_t pos,
                                             void *stream)
{
    if (!q || !kc || !vc || !out || !n_head || !n_kv || !hd || n_head % n_kv || pos >= n_ctx || n_ctx >= (1u << 31)) {
        set_err("attention_noalloc: invalid head configuration or position");
        return -1;
    }
    if (!attn_supported((uint32_t)hd, (uint32_t)(n_head / n_kv))) {
        set_err("attention_noalloc: head_dim %zu / GQA group %zu not supported", hd, n_head / n_kv);
        return -1;
    }
    const uint32_t ns = attn_splits((uint32_t)(pos + 1), (uint32_t)n_kv);
    const size_t need = n_head * ns * (hd + 2) * 4;
    if (need > kNoAllocScratchBytes) {
        set_err("attention_noalloc: %zu heads x %u splits need %zu B of partials, above the %zu B scratch", n_head, ns,
                need, kNoAllocScratchBytes);
        return -1;
    }
    float *part = noalloc_scratch();
    if (!part) return -1;
    return launched(launch_attention(q, kc, vc, part, out, (uint32_t)n_head, (uint32_t)n_kv, (uint32_t)hd, ns, nullptr,
                                     (uint32_t)pos, (hipStream_t)stream), "attention_noalloc");
}

extern "C" int forword_gpu_silu_mul(const float *g, const float *u, float *out, size_t n, void *stream)
{
    if (!g || !u || !out) { set_err("silu_mul: invalid arguments"); return -1; }
    if (!n) return 0;
    return launched(launch_silu_mul(g, u, out, n, (hipStream_t)stream), "silu_mul");
}

extern "C" int forword_gpu_tensor_silu(const float *x, float *out, size_t n, void *stream)
{
    if (!x || !out || !n) { set_err("tensor_silu: invalid arguments"); return -1; }
    return launched(launch_silu(x, out, n, (hipStream_t)stream), "tensor_silu");
}

extern "C" int forword_gpu_tensor_add(const float *a, const float *b, float *out, size_t n, void *stream)
{
    if (!a || !b || !out || !n) { set_err("tensor_add: invalid arguments"); return -1; }
    return launched(launch_add(a, b, out, n, (hipStream_t)stream), "tensor_add");
}

extern "C" int forword_gpu_argmax(const float *logits, size_t n, uint32_t *out_index, void *stream)
{
    if (!logits || !out_index || n >= (1u << 31)) { set_err("argmax: invalid arguments"); return -1; }
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (op_scratch_argmax()) return -1;
    return launched(launch_argmax(logits, (uint32_t)n, g_pv, g_pi, g_counter, out_index, nullptr, nullptr, nullptr,
                                  argmax_blocks((uint32_t)n), (hipStream_t)stream), "argmax");
}

// ── device memory plumbing ───────────────────────────────────────────────────

extern "C" void *forword_gpu_dev_alloc(size_t bytes)
{
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 4) != hipSuccess) { set_err("hipMalloc(%zu) failed", bytes); return nullptr; }
    return p;
}

extern "C" int forword_gpu_dev_free(void *p)
{
    if (p) HIPCHK(hipFree(p), "hipFree");
    return 0;
}

extern "C" int forword_gpu_memcpy_h2d(void *dst, const void *src, size_t n)
{
    HIPCHK(hipMemcpy(dst, src, n, hipMemcpyHostToDevice), "memcpy_h2d");
    return 0;
}

extern "C" int forword_gpu_memcpy_d2h(void *dst, const void *src, size_t n)
{
    HIPCHK(hipMemcpy(dst, src, n, hipMemcpyDeviceToHost), "memcpy_d2h");
    return 0;
}

extern "C" int forword_gpu_memset(void *dst, int v, size_t n)
{
    HIPCHK(hipMemset(dst, v, n), "memset");
    return 0;
}

extern "C" int forword_gpu_synchronize(void *stream)
{
    if (stream) HIPCHK(hipStreamSynchronize((hipStream_t)stream), "synchronize");
    else HIPCHK(hipDeviceSynchronize(), "synchronize");
    return 0;
}
