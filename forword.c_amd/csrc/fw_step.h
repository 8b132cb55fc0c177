// Persistent token-step kernel: host-side interface (internal to libforword_gpu.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fw_kernels.h"

namespace fw {

// The matrices of one GEMV phase (built in registers): up to three
// row-concatenated matrices sharing one input vector (QKV), or two computed
// row by row together (FFN gate/up).
struct MkGemv {
    const uint8_t *w[3];
    uint32_t rows[3];
    uint32_t n_rows;         // rows of the phase (QKV: sum; FFN: rows of one matrix)
    uint32_t n_cols;
    uint64_t row_bytes;
    uint32_t qa;             // slice alignment of the phase's weight type (pairs per slice a multiple of it)
    uint32_t qmin;           // pairs per slice at least (up to the row's pairs and 64)
    uint32_t rlo, rhi;       // rows this GEMV computes (a QKV phase with a V of another type runs as two);
                             // workgroups still split all n_rows, so the partials of both share one layout
};

enum MkKind : uint32_t { MK_QKV = 0, MK_ATTN = 1, MK_WO = 2, MK_FFN = 3, MK_DOWN = 4, MK_HEAD = 5 };

// The weights of one layer (copied into LDS at kernel start; the phase
// descriptors are built from it in registers).
struct MkLayer {
    const uint8_t *wq, *wk, *wv, *wo, *wg, *wu, *wd;
    const float *attn_norm, *ffn_norm;
    uint32_t mix;            // MK_MIX_V / MK_MIX_DOWN: attn_v / ffn_down is of the kernel's second layer type
    uint32_t pad;
};
// Layers of Q4_K_M files: attn_v and ffn_down of some layers are Q6_K.
enum : uint32_t { MK_MIX_V = 1, MK_MIX_DOWN = 2 };

// A step is 5 phases per layer (QKV ATTN WO FFN DOWN) and the lm-head (HEAD).
struct MkArgs {
    const MkLayer *layers;
    uint32_t n_layer;
    uint64_t rb_embd;        // row bytes of a layer linear with n_embd columns
    uint64_t rb_ff;          // row bytes of ffn_down (n_ff columns)
    const uint8_t *head_w;   // lm-head [n_vocab rows][n_embd]
    uint64_t head_rb;
    const float *out_norm;   // may be null: logits of x itself
    const uint8_t *embd;
    uint32_t embd_type;
    uint64_t embd_row_bytes;
    float embd_scale;
    uint32_t n_embd, n_ff, n_head, n_kv, head_dim, n_vocab, n_ctx, n_splits;
    uint32_t act;            // FfnAct of the gated FFN
    // Attention units: the query heads of a KV head's group in sub-groups of
    // attn_gs (a power of two dividing the group), attn_units = n_kv * group / attn_gs.
    uint32_t attn_gs, attn_units;
    // Below position attn_long_pos: sub-groups of attn_gs_short heads (half of
    // attn_gs, at least 1), attn_units_short units, at most n_splits_short splits.
    uint32_t attn_gs_short, attn_units_short, n_splits_short, attn_long_pos;
    float eps;
    float *kc, *vc;
    const float *cos_tab, *sin_tab;
    const float *bqkv;       // [n_layer][n_embd + 2 kv_dim] attn_q|k|v.bias per layer, or null
    float *logits;
    // Activations passed between phases without a grid barrier, as {value,
    // epoch} words (see tagged()): residual stream x, attention output, q
    // (n_head * head_dim), the K/V row of the current position ([k | v],
    // 2 * n_kv * head_dim) and the attention partials
    // [n_head][n_splits][head_dim + 2] (o, then m and l).
    uint64_t *tx, *tatt, *tq, *tkv, *tpart;
    // The FFN activations h, n_ff floats per (step of the launch, layer): slot
    // (step * n_layer + layer), with one flag per workgroup (128 bytes apart)
    // raised to the phase's epoch once its rows are stored.
    float *hf;
    uint32_t *hflag;
    float *trace;            // [2 * n_layer][n_embd] residual stream after each residual add
    StepState *state;
    const uint32_t *prompt;
    uint32_t *ids, *argmax_out;
    uint32_t *bar;           // one barrier flag per workgroup, 128 bytes apart
    uint32_t *tickets;       // argmax ticket at [attn_units], zero between uses
    uint32_t *err;           // set when a barrier or tagged-value wait gives up
    float *am_v;
    uint32_t *am_i;
    uint64_t *prof;          // optional: wall-clock stamp at kernel start, then after every phase
    uint32_t epoch0, n_steps;
    uint32_t qa_lin, qa_head;  // slice alignment of the layer linears' and the lm-head's weight types
    uint64_t rb_mix_embd;    // row bytes of an attn_v of the second layer type (n_embd columns)
    uint64_t rb_mix_ff;      // row bytes of an ffn_down of the second layer type (n_ff columns)
};

// Threads of one workgroup, and how many of them poll barrier flags and load
// staged inputs (one flag each, so a launch has at most kMkPollers workgroups).
constexpr uint32_t kMkThreads = 512;
constexpr uint32_t kMkPollers = 256;

// Barriers one token step performs (the host advances its epoch by this much).
inline uint32_t mk_barriers_per_step(uint32_t n_layer) { return 5 * n_layer + 1; }
// Whether the persistent kernel supports this model (else the per-kernel path
// runs): layer linears of one type (Q4_0/Q5_0/Q8_0/Q4_K), except attn_v and
// ffn_down of some layers of mix_type (0 for none, kQ6_KR for Q6_K copies
// after launch_repack_q6k); lm-head of those types or kQ6_KR.
bool mk_supported(uint32_t n_embd, uint32_t n_ff, uint32_t head_dim, uint32_t group, uint32_t linear_type,
                  uint32_t head_type, uint32_t embd_type, uint32_t mix_type);
// Dynamic LDS of one workgroup (args fully set up, n_splits included), 0 if
// the staged input, the partials and weight rings of every phase do not fit.
size_t mk_lds_bytes(const MkArgs &a, uint32_t n_wg, uint32_t linear_type, uint32_t head_type, uint32_t mix_type);
// Workgroups of one cooperative launch (one per CU), 0 if it cannot launch.
int mk_max_workgroups(uint32_t linear_type, uint32_t head_type, uint32_t mix_type, size_t lds_bytes);
// Q6_K matrix [n_rows][n_sb super-blocks] (rows src_rb bytes apart) into
// kQ6_KR records at dst (n_rows * n_sb * 224 bytes, 4-byte aligned).
hipError_t launch_repack_q6k(const uint8_t *src, uint64_t src_rb, uint32_t n_rows, uint32_t n_sb, uint8_t *dst,
                             hipStream_t s);
// Slice alignment of a weight type in the persistent kernel (MkArgs::qa_lin, qa_head).
uint32_t mk_q_align(uint32_t type);
hipError_t mk_launch(const MkArgs &a, uint32_t linear_type, uint32_t head_type, uint32_t mix_type, uint32_t n_wg,
                     size_t lds_bytes, hipStream_t s);

} // namespace fw
