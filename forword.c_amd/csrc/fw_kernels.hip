// gfx950 kernels of the forword decode path.
//
// GEMV (quant_matvec.c:263-312 and the fused callers attention.c:124-166,
// ffn.c:82-106, transformer.c:271-288): one wave computes kRowsPerWave output
// rows; each lane walks the row in pairs of blocks (64 columns, a 4-byte
// aligned 36/44/68-byte chunk) with dword-aligned 128-bit loads, keeps the
// matching 64 activations in registers for all rows of the wave, and the
// partial sums meet in a cross-lane reduction.  Block scales are applied once
// per block; Q4_0/Q5_0 codes are unpacked two per instruction.  Epilogues fuse
// RoPE + KV append (QKV), the residual add (Wo, down) and SiLU(gate)*up.
//
// Attention (attention.c:142-164): split-K over positions ("flash decoding"),
// one workgroup per (KV head, split) serving all query heads of its GQA group
// from a single read of K/V, online softmax in the log2 domain, then a combine
// kernel per query head.
#include "fw_device.h"
#include "fw_kernels.h"

#include <math.h>

namespace fw {

// ── GEMV ─────────────────────────────────────────────────────────────────────

// Deterministic block sum (butterfly within waves, waves in order); result in thread 0.
__device__ __forceinline__ float block_sum_t0(float v, float *s_w)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) s_w[wave] = v;
    __syncthreads();
    float r = 0.f;
    if (threadIdx.x == 0)
        for (int w = 0; w < nw; w++) r += s_w[w];
    return r;
}

// Last-block ticket: every block publishes its partial sum of squares; the last
// block to arrive sums all partials in block order and publishes the RMSNorm
// scale 1.0f/sqrtf(ss/n + eps) (norm.c:8-9).  No agent-scope fences.
__device__ void publish_norm_scale(float part, float *pss, uint32_t *ticket, float *scale_out, uint32_t n,
                                   float eps)
{
    __shared__ float s_w[16];
    __shared__ bool s_last;
    float b = block_sum_t0(part, s_w);
    if (threadIdx.x == 0) {
        st_sys(pss + blockIdx.x, b);
        wait_mem();
        s_last = ticket_sys(ticket) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    float v = 0.f;
    for (uint32_t i = threadIdx.x; i < gridDim.x; i += blockDim.x) v += ld_sys(pss + i);
    float ss = block_sum_t0(v, s_w);
    if (threadIdx.x == 0) {
        st_sys(scale_out, 1.0f / sqrtf((ss / (float)n) + eps));
        st_sys(ticket, 0u);
    }
}

template <int N>
__device__ __forceinline__ void load_x(const float *xp, float *xv, bool vec4)
{
    if (vec4) {
#pragma unroll
        for (int i = 0; i < N / 4; i++) {
            float4 v = reinterpret_cast<const float4 *>(xp)[i];
            xv[4 * i] = v.x; xv[4 * i + 1] = v.y; xv[4 * i + 2] = v.z; xv[4 * i + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; i++) xv[i] = xp[i];
    }
}

// x (and the norm weights when the input RMSNorm is folded in) for N columns at c0.
template <int N>
__device__ __forceinline__ void load_input(const QmvArgs &a, size_t c0, float *xv, bool vec4, float scale)
{
    load_x<N>(a.x + c0, xv, vec4);
    if (a.norm_w) {
        float wv[N];
        load_x<N>(a.norm_w + c0, wv, vec4 && ((uintptr_t)a.norm_w & 15) == 0);
#pragma unroll
        for (int i = 0; i < N; i++) xv[i] = (xv[i] * wv[i]) * scale;     // simd_mul then simd_scale
    }
}

template <uint32_t T, int EPI, bool PAIR>
__global__ __launch_bounds__(256) void k_qmv(QmvArgs a)
{
    constexpr int R = kRowsPerWave;
    const int lane = threadIdx.x & 63;
    const uint32_t g = blockIdx.x * 4 + (threadIdx.x >> 6);
    const bool active = g < a.n_groups &&
        !(EPI == EPI_STORE && a.state && a.state->greedy && a.state->pos + 1 < a.state->n_prompt);
    // (greedy prefill: the logits of prompt positions before the last are never read)

    int seg = 0;
    if (EPI != EPI_SWIGLU)
        while (seg + 1 < (int)a.n_seg && g >= a.group_base[seg + 1]) seg++;
    const uint8_t *wr[R];
    bool ok[R];
    uint32_t row[R];
#pragma unroll
    for (int k = 0; k < R; k++) {
        int s = seg;
        if (EPI == EPI_SWIGLU) { s = k < R / 2 ? 0 : 1; row[k] = g * (R / 2) + (k % (R / 2)); }
        else row[k] = (g - a.group_base[seg]) * R + k;
        ok[k] = active && row[k] < a.rows[s];
        wr[k] = a.w[s] + (size_t)(ok[k] ? row[k] : 0) * a.row_bytes;
    }

    float acc[R];
#pragma unroll
    for (int k = 0; k < R; k++) acc[k] = 0.0f;
    const bool xv4 = ((uintptr_t)a.x & 15) == 0;
    const float nscale = (active && a.norm_w) ? ld_sys(a.norm_scale) : 1.0f;

    if (!active) {
        // idle wave: only takes part in the block-wide epilogue below
    } else if constexpr (T == kF32) {
        for (uint32_t c = lane; c < a.n_cols; c += 64) {
            float xc;
            load_input<1>(a, c, &xc, false, nscale);
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) acc[k] = __builtin_fmaf(reinterpret_cast<const float *>(wr[k])[c], xc, acc[k]);
        }
    } else if constexpr (PAIR && T != kQ4_K && T != kQ6_K) {
        constexpr int BB = Blk<T>::bytes, NDW = Blk<T>::pair_dw;
        const uint32_t n_pairs = a.n_cols / 64;
        for (uint32_t p = lane; p < n_pairs; p += 64) {
            uint32_t dw[R][NDW];
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) load_pair<T>(wr[k] + (size_t)p * (2 * BB), dw[k]);
            float xv[64];
            load_input<64>(a, 64 * (size_t)p, xv, xv4, nscale);
            float sx0 = 0.f, sx1 = 0.f;
            if constexpr (T != kQ8_0) {
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; s2 += xv[32 + i]; s3 += xv[33 + i]; }
                sx0 = s0 + s1;
                sx1 = s2 + s3;
            }
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) acc[k] += dot_pair<T>(dw[k], xv, sx0, sx1);
        }
    } else if constexpr (T == kQ4_K && PAIR) {
        // 64-value quarters of dword-aligned super-blocks, one per lane at a time:
        // groups 2p and 2p+1 share 32 code bytes (low and high nibbles), so each
        // byte is loaded once.  Per group (d·sc)·Σq·x − (dmin·m)·Σx (quant.c:111-126
        // factored; q in 1/512 units from the fp8 conversion, as for Q4_0).
        const uint32_t n_pairs = a.n_cols / 64;
        for (uint32_t u = lane; u < n_pairs; u += 64) {
            float xv[64];
            load_input<64>(a, 64 * (size_t)u, xv, xv4, nscale);
            float sx0, sx1;
            {
                float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; s2 += xv[32 + i]; s3 += xv[33 + i]; }
                sx0 = s0 + s1;
                sx1 = s2 + s3;
            }
            const uint32_t sb = u / 4, gp = u % 4;
#pragma unroll
            for (int k = 0; k < R; k++) {
                if (!ok[k]) continue;
                const FW_GLOBAL uint32_t *b32 = gptr(reinterpret_cast<const uint32_t *>(wr[k] + (size_t)sb * 144));
                const u32x4 hs = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(b32);   // d|dmin, scales 0..11
                const float d = h2f(hs.x), dmin = h2f(hs.x >> 16);
                const uint32_t sw[3] = { hs.y, hs.z, hs.w };
                auto sb8 = [&](uint32_t i) { return (sw[i / 4] >> (8 * (i % 4))) & 0xFFu; };
                float ds[2], dm[2];
#pragma unroll
                for (int h = 0; h < 2; h++) {
                    const uint32_t g = 2 * gp + h;
                    uint32_t sc, mn;
                    if (g < 4) { sc = sb8(g) & 63u; mn = sb8(g + 4) & 63u; }
                    else {
                        sc = (sb8(g + 4) & 15u) | ((sb8(g - 4) >> 6) << 4);
                        mn = (sb8(g + 4) >> 4) | ((sb8(g) >> 6) << 4);
                    }
                    ds[h] = d * (float)sc;
                    dm[h] = dmin * (float)mn;
                }
                const FW_GLOBAL uint32_t *q = b32 + 4 + gp * 8;
                const u32x4 q0 = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(q);
                const u32x4 q1 = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(q + 4);
                const uint32_t qw[8] = { q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w };
                float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint32_t lo = qw[i] & 0x0F0F0F0Fu, hi = (qw[i] >> 4) & 0x0F0F0F0Fu;
                    const float2v l01 = nib2<false>(lo), l23 = nib2<true>(lo);
                    const float2v h01 = nib2<false>(hi), h23 = nib2<true>(hi);
                    a0 = __builtin_fmaf(l01.x, xv[4 * i + 0], a0);
                    a1 = __builtin_fmaf(l01.y, xv[4 * i + 1], a1);
                    a0 = __builtin_fmaf(l23.x, xv[4 * i + 2], a0);
                    a1 = __builtin_fmaf(l23.y, xv[4 * i + 3], a1);
                    b0 = __builtin_fmaf(h01.x, xv[32 + 4 * i + 0], b0);
                    b1 = __builtin_fmaf(h01.y, xv[32 + 4 * i + 1], b1);
                    b0 = __builtin_fmaf(h23.x, xv[32 + 4 * i + 2], b0);
                    b1 = __builtin_fmaf(h23.y, xv[32 + 4 * i + 3], b1);
                }
                const float s0 = (a0 + a1) * 512.0f, s1 = (b0 + b1) * 512.0f;
                acc[k] += __builtin_fmaf(ds[0], s0, -dm[0] * sx0) + __builtin_fmaf(ds[1], s1, -dm[1] * sx1);
            }
        }
    } else if constexpr (T == kQ4_K || T == kQ6_K) {
        // 32-value groups of the 256-value super-blocks, one per lane at a time:
        // the group's values exactly as the reference decodes them, then FMAs.
        constexpr uint32_t SB = T == kQ4_K ? 144u : 210u;
        const uint32_t n_units = a.n_cols / 32;
        for (uint32_t u = lane; u < n_units; u += 64) {
            float xv[32];
            load_input<32>(a, 32 * (size_t)u, xv, xv4, nscale);
            const uint32_t sb = u / 8, g = u % 8;
#pragma unroll
            for (int k = 0; k < R; k++) {
                if (!ok[k]) continue;
                const uint8_t *blk = wr[k] + (size_t)sb * SB;
                float s = 0.f;
                if constexpr (T == kQ4_K && PAIR) {                   // dword-aligned super-blocks
                    const FW_GLOBAL uint32_t *b32 = gptr(reinterpret_cast<const uint32_t *>(blk));
                    const uint32_t h = b32[0];
                    const float d = h2f(h), dmin = h2f(h >> 16);
                    const u32x4 hs = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(b32);   // d|dmin, scales 0..11
                    const uint32_t sw[3] = { hs.y, hs.z, hs.w };
                    auto sb8 = [&](uint32_t i) { return (sw[i / 4] >> (8 * (i % 4))) & 0xFFu; };
                    uint32_t sc, mn;
                    if (g < 4) { sc = sb8(g) & 63u; mn = sb8(g + 4) & 63u; }
                    else {
                        sc = (sb8(g + 4) & 15u) | ((sb8(g - 4) >> 6) << 4);
                        mn = (sb8(g + 4) >> 4) | ((sb8(g) >> 6) << 4);
                    }
                    const float ds = d * (float)sc, dm = dmin * (float)mn;
                    const FW_GLOBAL uint32_t *q = b32 + 4 + (g / 2) * 8;
                    uint32_t qw[8];
#pragma unroll
                    for (int i = 0; i < 8; i += 4) {
                        const u32x4 v = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(q + i);
                        qw[i] = v.x; qw[i + 1] = v.y; qw[i + 2] = v.z; qw[i + 3] = v.w;
                    }
                    const uint32_t shift = (g & 1) ? 4u : 0u;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const uint32_t nb = (qw[i] >> shift) & 0x0F0F0F0Fu;
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            s = __builtin_fmaf(ds * (float)((nb >> (8 * e)) & 0xFFu) - dm, xv[4 * i + e], s);
                    }
                } else if constexpr (T == kQ4_K) {
                    const float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
                    const float dmin = h2f((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
                    uint32_t sc, mn;
                    scale_min_k4(g, blk + 4, sc, mn);
                    const float ds = d * (float)sc, dm = dmin * (float)mn;
                    const uint8_t *q = blk + 16 + (g / 2) * 32;
#pragma unroll
                    for (int i = 0; i < 32; i++) {
                        const uint32_t v = (g & 1) ? (uint32_t)(q[i] >> 4) : (uint32_t)(q[i] & 15);
                        s = __builtin_fmaf(ds * (float)v - dm, xv[i], s);
                    }
                } else {
                    // Q6_K (quant.c:160-183): 32 code bytes of ql (low or high nibbles) and
                    // 32 of qh (2 bits each) as dwords from the 2-byte-aligned block, four
                    // 6-bit codes per dword; per 16 values (d·sc)·(Σq·x − 32·Σx).
                    const uint32_t h = g / 4, kk = g % 4;
                    const float d = h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
                    const float s0 = d * (float)(int8_t)blk[192 + h * 8 + 2 * kk];
                    const float s1 = d * (float)(int8_t)blk[192 + h * 8 + 2 * kk + 1];
                    auto load8 = [](const uint8_t *p, uint32_t (&o)[8]) {      // 32 bytes at a 2-byte-aligned p
                        const uintptr_t ad = reinterpret_cast<uintptr_t>(p);
                        const uint32_t *w = reinterpret_cast<const uint32_t *>(ad & ~(uintptr_t)3);
                        uint32_t t[9];
#pragma unroll
                        for (int i = 0; i < 9; i++) t[i] = w[i];             // inside the 210-byte block
#pragma unroll
                        for (int i = 0; i < 8; i++) o[i] = (ad & 2) ? align16(t[i + 1], t[i]) : t[i];
                    };
                    if (reinterpret_cast<uintptr_t>(blk) & 1) {               // odd address: byte loads
                        const uint8_t *ql = blk + h * 64 + 32 * (kk & 1), *qh = blk + 128 + h * 32;
#pragma unroll
                        for (int l = 0; l < 32; l++) {
                            const int q = (int)(((kk >= 2) ? (ql[l] >> 4) : (ql[l] & 15)) |
                                                (((qh[l] >> (2 * kk)) & 3) << 4));
                            s = __builtin_fmaf((l < 16 ? s0 : s1) * (float)(q - 32), xv[l], s);
                        }
                        acc[k] += s;
                        continue;
                    }
                    uint32_t lw[8], hw[8];
                    load8(blk + h * 64 + 32 * (kk & 1), lw);
                    load8(blk + 128 + h * 32, hw);
                    float a0 = 0.f, a1 = 0.f, x0 = 0.f, x1 = 0.f;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const uint32_t nib = (kk >= 2 ? lw[i] >> 4 : lw[i]) & 0x0F0F0F0Fu;
                        const uint32_t q4 = nib | (((hw[i] >> (2 * kk)) & 0x03030303u) << 4);
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            const float q = (float)((q4 >> (8 * e)) & 0xFFu), xx = xv[4 * i + e];
                            if (i < 4) { a0 = __builtin_fmaf(q, xx, a0); x0 += xx; }
                            else { a1 = __builtin_fmaf(q, xx, a1); x1 += xx; }
                        }
                    }
                    s = s0 * __builtin_fmaf(-32.0f, x0, a0) + s1 * __builtin_fmaf(-32.0f, x1, a1);
                }
                acc[k] += s;
            }
        }
    } else {
        constexpr int BB = Blk<T>::bytes;
        const uint32_t n_blocks = a.n_cols / 32;
        for (uint32_t b = lane; b < n_blocks; b += 64) {
            float xv[32];
            load_input<32>(a, 32 * (size_t)b, xv, xv4, nscale);
            float sx = 0.f;
            if constexpr (T != kQ8_0) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; }
                sx = s0 + s1;
            }
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) acc[k] += dot_single<T>(wr[k] + (size_t)b * BB, xv, sx);
        }
    }

#pragma unroll
    for (int k = 0; k < R; k++) acc[k] = wave_sum(acc[k]);

    if constexpr (EPI == EPI_STORE) {
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) {
                    float v = a.bias[seg] ? acc[k] + a.bias[seg][row[k]] : acc[k];
                    if (a.store_act) v = ffn_act(v, a.store_act - 1);
                    a.out[seg][row[k]] = v;
                }
    } else if constexpr (EPI == EPI_RESID) {
        float ss = 0.f;
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) {
                    float y = acc[k];
                    if (a.bias[0]) y += a.bias[0][row[k]];          // linear.c:214-221
                    if (a.addend) y = a.addend[row[k]] + y;         // attn_out + ffn_out (transformer.c:250-251)
                    float v = a.out[0][row[k]] + y;                 // x[i] += y[i] (transformer.c:271-272)
                    a.out[0][row[k]] = v;
                    if (a.trace) a.trace[row[k]] = v;
                    if (a.trace2) a.trace2[row[k]] = v;
                    ss = __builtin_fmaf(v, v, ss);
                }
        if (a.scale_out) publish_norm_scale(ss, a.pss, a.ticket, a.scale_out, a.rows[0], a.norm_eps);
    } else if constexpr (EPI == EPI_SWIGLU) {
        if (lane == 0)
#pragma unroll
            for (int k = 0; k < R / 2; k++)
                if (ok[k]) a.out[0][row[k]] = ffn_act(acc[k], a.act) * acc[k + R / 2];   // ffn.c:88-104
    } else {   // EPI_QKV: bias (linear.c:214-221), RoPE on q and k rows (rope.c:37-43), q out / KV append at pos
        if (lane == 0 && active) {
            const uint32_t pos = a.state->pos, half = a.head_dim / 2;
            const uint32_t role = seg + a.role_base;
            const float *bias = a.bias[role];
            float v[R];
#pragma unroll
            for (int k = 0; k < R; k++) v[k] = bias && ok[k] ? acc[k] + bias[row[k]] : acc[k];
            if (role < 2 && a.cos_tab) {                         // no cos_tab: RoPE runs after (NEOX)
#pragma unroll
                for (int k = 0; k < R; k += 2) {
                    uint32_t i = (row[k] % a.head_dim) / 2;
                    float c = a.cos_tab[(size_t)pos * half + i], s = a.sin_tab[(size_t)pos * half + i];
                    float v0 = v[k], v1 = v[k + 1];
                    v[k] = v0 * c - v1 * s;
                    v[k + 1] = v0 * s + v1 * c;
                }
            }
            float *dst = role == 0 ? a.out[0] : a.out[role] + (size_t)pos * a.kv_dim;
#pragma unroll
            for (int k = 0; k < R; k++)
                if (ok[k]) dst[row[k]] = v[k];
        }
    }
}

void qmv_plan(QmvArgs &a, int epi)
{
    const uint32_t R = kRowsPerWave;
    if (epi == EPI_SWIGLU) {
        a.n_groups = (a.rows[0] + R / 2 - 1) / (R / 2);
        a.group_base[0] = 0;
        a.group_base[1] = a.n_groups;
        return;
    }
    uint32_t base = 0;
    for (uint32_t s = 0; s < a.n_seg; s++) {
        a.group_base[s] = base;
        base += (a.rows[s] + R - 1) / R;
    }
    a.group_base[a.n_seg] = base;
    a.n_groups = base;
}

bool qmv_pair_ok(uint32_t type, uint32_t n_cols, const void *base)
{
    if (type == kQ4_K) return ((uintptr_t)base & 3) == 0;          // 144-byte super-blocks stay aligned
    return (type == kQ4_0 || type == kQ5_0 || type == kQ8_0) && n_cols % 64 == 0 && ((uintptr_t)base & 3) == 0;
}

template <uint32_t T, int EPI>
static hipError_t launch_t(const QmvArgs &a, bool pair, hipStream_t s)
{
    dim3 grid((a.n_groups + 3) / 4), block(256);
    if (pair) hipLaunchKernelGGL((k_qmv<T, EPI, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_qmv<T, EPI, false>), grid, block, 0, s, a);
    return hipGetLastError();
}

template <int EPI>
static hipError_t launch_e(uint32_t type, const QmvArgs &a, hipStream_t s)
{
    bool pair = true;
    for (uint32_t i = 0; i < (EPI == EPI_SWIGLU ? 2u : a.n_seg); i++)
        pair = pair && qmv_pair_ok(type, a.n_cols, a.w[i]);
    switch (type) {
    case kQ4_0: return launch_t<kQ4_0, EPI>(a, pair, s);
    case kQ5_0: return launch_t<kQ5_0, EPI>(a, pair, s);
    case kQ8_0: return launch_t<kQ8_0, EPI>(a, pair, s);
    case kQ4_K: return launch_t<kQ4_K, EPI>(a, pair, s);     // pair: dword-aligned super-blocks
    case kQ6_K: return launch_t<kQ6_K, EPI>(a, false, s);
    case kF32: return launch_t<kF32, EPI>(a, false, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_qmv(uint32_t type, int epi, QmvArgs a, hipStream_t s)
{
    if (!a.n_groups) return hipSuccess;
    switch (epi) {
    case EPI_STORE: return launch_e<EPI_STORE>(type, a, s);
    case EPI_QKV: return launch_e<EPI_QKV>(type, a, s);
    case EPI_RESID: return launch_e<EPI_RESID>(type, a, s);
    case EPI_SWIGLU: return launch_e<EPI_SWIGLU>(type, a, s);
    default: return hipErrorInvalidValue;
    }
}

// ── RMSNorm (norm.c:7-16) with the reference's exact summation order ─────────
// ss = simd_sum_squares: 16 lane chains of FMAs over stride-16 elements, the
// two 8-lane halves added, one 8-wide FMA step, the 8->4->2->1 tree
// (simd.h:27-67), `0.0f + tree` and the scalar tail (simd.h:151-153); then
// scale = 1.0f/sqrtf(ss/n + eps) and out = (x*w)*scale, each product rounded.
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w,
                                                  float *__restrict__ out, uint32_t n, float eps)
{
    extern __shared__ float s_x[];                 // x staged once (n <= 16384), else read from global
    __shared__ float s_scale;
    x += (size_t)blockIdx.x * n;                   // one row per workgroup
    out += (size_t)blockIdx.x * n;
    const bool staged = n <= 16384;
    if (staged) {
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) s_x[i] = x[i];
        __syncthreads();
    }
    const float *xs = staged ? s_x : x;
    if (threadIdx.x < 64) {
        const int L = threadIdx.x;
        const uint32_t n16 = n / 16 * 16;
        float acc = 0.0f;
        if (L < 16) {
            uint32_t i = L;
            for (; i + 48 < n16; i += 64) {        // 4 loads in flight per step, same FMA order
                float a0 = xs[i], a1 = xs[i + 16], a2 = xs[i + 32], a3 = xs[i + 48];
                acc = __builtin_fmaf(a0, a0, acc);
                acc = __builtin_fmaf(a1, a1, acc);
                acc = __builtin_fmaf(a2, a2, acc);
                acc = __builtin_fmaf(a3, a3, acc);
            }
            for (; i < n16; i += 16) acc = __builtin_fmaf(xs[i], xs[i], acc);
        }
        float hi = __shfl_down(acc, 8, 64);
        if (L < 8) {
            acc = acc + hi;
            if (n16 + 8 <= n) acc = __builtin_fmaf(xs[n16 + L], xs[n16 + L], acc);
        }
        float a4 = __shfl_down(acc, 4, 64);
        float s = acc + a4;                       // lanes 0..3: lo128 + hi128
        float s2 = __shfl_down(s, 2, 64);
        float t = s + s2;                         // lanes 0,1: movehl step
        float t1 = __shfl_down(t, 1, 64);
        if (L == 0) {
            float sum = 0.0f + (t + t1);
            for (uint32_t i = n / 8 * 8; i < n; i++) sum = sum + xs[i] * xs[i];
            s_scale = 1.0f / sqrtf((sum / (float)n) + eps);
        }
    }
    __syncthreads();
    const float sc = s_scale;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        float v = w ? x[i] * w[i] : x[i];
        out[i] = v * sc;
    }
}

hipError_t launch_rmsnorm(const float *x, const float *w, float *out, uint32_t n, float eps, hipStream_t s)
{
    return launch_rmsnorm_rows(x, w, out, n, 1, eps, s);
}

hipError_t launch_rmsnorm_rows(const float *x, const float *w, float *out, uint32_t n, uint32_t rows, float eps,
                               hipStream_t s)
{
    size_t lds = n <= 16384 ? (size_t)n * 4 : 0;
    hipLaunchKernelGGL(k_rmsnorm, dim3(rows), dim3(256), lds, s, x, w, out, n, eps);
    return hipGetLastError();
}

// ── dequantisation: embedding row, get_row, bulk ─────────────────────────────

__global__ __launch_bounds__(1024) void k_row(const uint8_t *w, uint32_t type, uint32_t n_cols, uint32_t n_rows,
                                              const StepState *st, const uint32_t *tok_override, uint32_t row_fixed,
                                              float embd_scale, float *out, float *scale_out, float eps)
{
    __shared__ float s_w[16];
    uint32_t row = st ? st->token : (tok_override ? *tok_override : row_fixed);
    if (row >= n_rows) row = n_rows - 1;            // bounds were checked on the host
    float ss = 0.f;
    for (uint32_t j = blockIdx.x * blockDim.x + threadIdx.x; j < n_cols; j += gridDim.x * blockDim.x) {
        float v;
        if (type == kF32) v = reinterpret_cast<const float *>(w)[(size_t)row * n_cols + j];
        else {
            const uint32_t bb = block_bytes_dev(type), bv = block_values_dev(type);
            const uint8_t *blk = w + (size_t)row * (n_cols / bv) * bb + (size_t)(j / bv) * bb;
            v = dequant_one(blk, type, j % bv);
        }
        if (embd_scale != 1.0f) v *= embd_scale;               // transformer.c:179-182
        out[j] = v;
        ss = __builtin_fmaf(v, v, ss);
    }
    if (scale_out) {                                            // launched as one block
        float t = block_sum_t0(ss, s_w);
        if (threadIdx.x == 0) st_sys(scale_out, 1.0f / sqrtf((t / (float)n_cols) + eps));
    }
}

hipError_t launch_embed(const uint8_t *w, uint32_t type, uint32_t n_cols, uint32_t n_rows,
                        const StepState *st, const uint32_t *token_override, float embd_scale, float *x,
                        float *scale_out, float norm_eps, hipStream_t s)
{
    hipLaunchKernelGGL(k_row, dim3(1), dim3(1024), 0, s, w, type, n_cols, n_rows, st, token_override, 0u,
                       embd_scale, x, scale_out, norm_eps);
    return hipGetLastError();
}

hipError_t launch_get_row(const uint8_t *w, uint32_t type, uint32_t n_cols, uint32_t row, float *out,
                          hipStream_t s)
{
    uint32_t blocks = (n_cols + 255) / 256;
    hipLaunchKernelGGL(k_row, dim3(blocks), dim3(256), 0, s, w, type, n_cols, row + 1u,
                       (const StepState *)nullptr, (const uint32_t *)nullptr, row, 1.0f, out, (float *)nullptr, 0.f);
    return hipGetLastError();
}

__global__ void k_dequant(const uint8_t *blocks, uint32_t type, uint64_t n, float *out)
{
    const uint32_t bb = block_bytes_dev(type), bv = block_values_dev(type);
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n;
         i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = dequant_one(blocks + (i / bv) * bb, type, (uint32_t)(i % bv));
}

hipError_t launch_dequant(const uint8_t *blocks, uint32_t type, uint64_t n_blocks, float *out, hipStream_t s)
{
    uint64_t n = n_blocks * (type == kQ4_K || type == kQ6_K ? 256u : 32u);
    uint64_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    hipLaunchKernelGGL(k_dequant, dim3((uint32_t)g), dim3(256), 0, s, blocks, type, n, out);
    return hipGetLastError();
}

// ── attention ────────────────────────────────────────────────────────────────

// One workgroup: G query heads (of the group_total sharing KV head kvh; the
// group is walked in n_sub = group_total / G workgroups) over one split of the
// positions.
template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn(const float *__restrict__ q, const float *__restrict__ kc,
                                               const float *__restrict__ vc, float *__restrict__ part,
                                               uint32_t n_kv, uint32_t n_splits, const StepState *st,
                                               uint32_t pos_host, float scale_log2, uint32_t group_total)
{
    constexpr int HD = 16 * EPL;
    __shared__ float s_m[4][G], s_l[4][G], s_o[4][G][HD];
    const uint32_t pos = st ? st->pos : pos_host;
    const uint32_t n_sub = group_total / G, kvh = blockIdx.x % n_kv, rest = blockIdx.x / n_kv;
    const uint32_t sub = rest % n_sub, split = rest / n_sub, h0 = kvh * group_total + sub * G;
    const uint32_t n_pos = pos + 1, chunk = (n_pos + n_splits - 1) / n_splits;
    const uint32_t t0 = split * chunk, t1 = min(n_pos, t0 + chunk);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane >> 4, l16 = lane & 15;
    const size_t kvd = (size_t)n_kv * HD;

    float qv[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++)
#pragma unroll
        for (int e = 0; e < EPL; e++) qv[g][e] = q[(h0 + g) * HD + l16 * EPL + e];
    float m[G], l[G], o[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.f;
    }

    for (uint32_t t = t0 + wave * 4 + grp; t < t1; t += 16) {
        const float *kp = kc + (size_t)t * kvd + kvh * HD + l16 * EPL;
        const float *vp = vc + (size_t)t * kvd + kvh * HD + l16 * EPL;
        float kk[EPL], vv[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) { kk[e] = kp[e]; vv[e] = vp[e]; }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) d = __builtin_fmaf(qv[g][e], kk[e], d);
            d += __shfl_xor(d, 8, 64);
            d += __shfl_xor(d, 4, 64);
            d += __shfl_xor(d, 2, 64);
            d += __shfl_xor(d, 1, 64);
            float s = d * scale_log2;
            float mn = fmaxf(m[g], s);
            float c = exp2f(m[g] - mn), p = exp2f(s - mn);
            l[g] = __builtin_fmaf(l[g], c, p);
#pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] = __builtin_fmaf(o[g][e], c, p * vv[e]);
            m[g] = mn;
        }
    }

    // merge the four 16-lane groups of the wave
#pragma unroll
    for (int g = 0; g < G; g++) {
        float mw = fmaxf(m[g], __shfl_xor(m[g], 16, 64));
        mw = fmaxf(mw, __shfl_xor(mw, 32, 64));
        float c = mw == -INFINITY ? 0.f : exp2f(m[g] - mw);
        float lw = l[g] * c;
        lw += __shfl_xor(lw, 16, 64);
        lw += __shfl_xor(lw, 32, 64);
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            float ov = o[g][e] * c;
            ov += __shfl_xor(ov, 16, 64);
            ov += __shfl_xor(ov, 32, 64);
            o[g][e] = ov;
        }
        if (lane < 16) {
#pragma unroll
            for (int e = 0; e < EPL; e++) s_o[wave][g][l16 * EPL + e] = o[g][e];
            if (lane == 0) { s_m[wave][g] = mw; s_l[wave][g] = lw; }
        }
    }
    __syncthreads();
    // merge the four waves and write this split's partial
    for (int i = threadIdx.x; i < G * HD; i += 256) {
        const int g = i / HD, dd = i % HD;
        float M = fmaxf(fmaxf(s_m[0][g], s_m[1][g]), fmaxf(s_m[2][g], s_m[3][g]));
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < 4; w++) {
            float c = M == -INFINITY ? 0.f : exp2f(s_m[w][g] - M);
            L = __builtin_fmaf(s_l[w][g], c, L);
            O = __builtin_fmaf(s_o[w][g][dd], c, O);
        }
        float *pp = part + ((size_t)(h0 + g) * n_splits + split) * (HD + 2);
        pp[dd] = O;
        if (dd == 0) { pp[HD] = M; pp[HD + 1] = L; }
    }
}

__global__ __launch_bounds__(256) void k_attn_combine(const float *__restrict__ part, float *__restrict__ out,
                                                       uint32_t n_splits, uint32_t hd)
{
    __shared__ float s_wt[256], s_red[8];
    const uint32_t h = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const float *base = part + (size_t)h * n_splits * (hd + 2);
    // one split per thread (n_splits <= 256): its max and weight
    float ms = t < n_splits ? base[(size_t)t * (hd + 2) + hd] : -INFINITY;
    float M = wave_max(ms);
    if (lane == 0) s_red[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float wt = (t < n_splits && ms != -INFINITY) ? exp2f(ms - M) : 0.f;
    s_wt[t] = wt;
    float lw = t < n_splits ? base[(size_t)t * (hd + 2) + hd + 1] * wt : 0.f;
    lw = wave_sum(lw);
    __syncthreads();
    if (lane == 0) s_red[4 + wave] = lw;
    __syncthreads();
    const float inv = 1.0f / ((s_red[4] + s_red[5]) + (s_red[6] + s_red[7]));
    for (uint32_t d = t; d < hd; d += blockDim.x) {
        float O = 0.f;
        for (uint32_t s = 0; s < n_splits; s++) O = __builtin_fmaf(base[(size_t)s * (hd + 2) + d], s_wt[s], O);
        out[(size_t)h * hd + d] = O * inv;
    }
}

uint32_t attn_splits(uint32_t max_ctx, uint32_t n_kv)
{
    uint32_t a = (max_ctx + 15) / 16, b = (1024 + n_kv - 1) / n_kv;
    uint32_t s = a < b ? a : b;
    if (s < 1) s = 1;
    if (s > 256) s = 256;
    return s;
}

bool attn_supported(uint32_t hd, uint32_t group)
{
    return attn_epl(hd) && group >= 1 && group <= 256;
}

uint32_t attn_epl(uint32_t hd)
{
    switch (hd) {
    case 32: case 48: case 64: case 80: case 96: case 128: case 256: return hd / 16;
    default: return 0;
    }
}

uint32_t attn_sub_group(uint32_t hd, uint32_t group)
{
    for (uint32_t g = 8; g > 1; g >>= 1)
        if (group % g == 0 && g * (hd / 16) <= 64) return g;   // q and o of G heads stay in registers
    return 1;
}

template <int EPL>
static hipError_t attn_g(uint32_t group, uint32_t n_kv, uint32_t ns, hipStream_t s, const float *q,
                         const float *kc, const float *vc, float *part, const StepState *st, uint32_t pos, float sc)
{
    const uint32_t gs = attn_sub_group(16 * EPL, group);
    const dim3 grid(n_kv * (group / gs) * ns);
#define L(G) hipLaunchKernelGGL((k_attn<EPL, G>), grid, dim3(256), 0, s, q, kc, vc, part, n_kv, ns, st, pos, sc, group)
    switch (gs) {
    case 1: L(1); break;
    case 2: L(2); break;
    case 4: if constexpr (EPL <= 16) L(4); break;
    case 8: if constexpr (EPL <= 8) L(8); break;
    default: return hipErrorInvalidValue;
    }
#undef L
    return hipGetLastError();
}

hipError_t launch_attention(const float *q, const float *kc, const float *vc, float *part, float *out,
                            uint32_t n_head, uint32_t n_kv, uint32_t hd, uint32_t n_splits,
                            const StepState *st, uint32_t pos_host, hipStream_t s)
{
    if (!n_kv || n_head % n_kv) return hipErrorInvalidValue;
    const uint32_t group = n_head / n_kv;
    // scores are dot * (1/sqrtf(hd)) (attention.c:143,151-155), carried in log2 units
    const float sc = (1.0f / sqrtf((float)hd)) * 1.4426950408889634f;
    hipError_t e;
#define A(EPL) attn_g<EPL>(group, n_kv, n_splits, s, q, kc, vc, part, st, pos_host, sc)
    switch (hd) {
    case 32: e = A(2); break;
    case 48: e = A(3); break;
    case 64: e = A(4); break;
    case 80: e = A(5); break;
    case 96: e = A(6); break;
    case 128: e = A(8); break;
    case 256: e = A(16); break;
    default: return hipErrorInvalidValue;
    }
#undef A
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k_attn_combine, dim3(n_head), dim3(256), 0, s, part, out, n_splits, hd);
    return hipGetLastError();
}

// ── argmax (sampler_argmax, sampler.c:28-32) ─────────────────────────────────
// Lowest index of the maximum; NaN never wins, and a NaN at index 0 makes the
// answer 0 (the reference's strict '>' scan never leaves index 0 then).  One
// launch: per-block partials, the last block to finish reduces them in order
// and resets the ticket counter, so the kernel can be replayed in a graph.

__device__ __forceinline__ bool am_better(float v1, uint32_t i1, float v2, uint32_t i2)
{
    if (i1 == 0xffffffffu) return false;
    if (i2 == 0xffffffffu) return true;
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

__device__ void block_argmax(float &bv, uint32_t &bi)
{
    __shared__ float sv[4];
    __shared__ uint32_t si[4];
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        float ov = __shfl_xor(bv, m, 64);
        uint32_t oi = __shfl_xor(bi, m, 64);
        if (am_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { sv[wave] = bv; si[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < (int)(blockDim.x >> 6); w++)
            if (am_better(sv[w], si[w], bv, bi)) { bv = sv[w]; bi = si[w]; }
    }
}

__device__ void greedy_advance(StepState *st, const uint32_t *prompt, uint32_t *ids, uint32_t next)
{
    const uint32_t pos = st->pos;
    if (pos + 1 >= st->n_prompt) ids[pos + 1 - st->n_prompt] = next;
    st->token = pos + 1 < st->n_prompt ? prompt[pos + 1] : next;
    st->pos = pos + 1;
}

__global__ __launch_bounds__(256) void k_argmax(const float *__restrict__ x, uint32_t n, float *pv,
                                                 uint32_t *pi, uint32_t *counter, uint32_t *out, StepState *st,
                                                 const uint32_t *prompt, uint32_t *ids)
{
    __shared__ bool s_last;
    if (st && st->greedy && st->pos + 1 < st->n_prompt) {      // prefill step: logits unused
        if (blockIdx.x == 0 && threadIdx.x == 0) greedy_advance(st, prompt, ids, 0);
        return;
    }
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float v = x[i];
        if (!isnan(v) && (bi == 0xffffffffu || v > bv)) { bv = v; bi = i; }
    }
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        st_sys(pv + blockIdx.x, bv);
        st_sys(pi + blockIdx.x, bi);
        wait_mem();
        s_last = ticket_sys(counter) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    bv = -INFINITY;
    bi = 0xffffffffu;
    for (uint32_t b = threadIdx.x; b < gridDim.x; b += blockDim.x) {
        float v = ld_sys(pv + b);
        uint32_t i = ld_sys(pi + b);
        if (am_better(v, i, bv, bi)) { bv = v; bi = i; }
    }
    __syncthreads();
    block_argmax(bv, bi);
    if (threadIdx.x == 0) {
        uint32_t r = (bi == 0xffffffffu || isnan(x[0])) ? 0u : bi;
        *out = r;
        st_sys(counter, 0u);
        if (st) {
            st->next = r;
            if (st->greedy) greedy_advance(st, prompt, ids, r);
        }
    }
}

uint32_t argmax_blocks(uint32_t n)
{
    uint32_t b = (n + 2047) / 2048;
    return b < 1 ? 1 : (b > 256 ? 256 : b);
}

hipError_t launch_argmax(const float *x, uint32_t n, float *pv, uint32_t *pi, uint32_t *counter, uint32_t *out,
                         StepState *st, const uint32_t *prompt, uint32_t *ids, uint32_t n_blocks, hipStream_t s)
{
    hipLaunchKernelGGL(k_argmax, dim3(n_blocks), dim3(256), 0, s, x, n, pv, pi, counter, out, st, prompt, ids);
    return hipGetLastError();
}

// ── elementwise ──────────────────────────────────────────────────────────────

__global__ void k_rope(float *qk, uint32_t pos, uint32_t n_heads, uint32_t hd, const float *cos_tab,
                       const float *sin_tab, int neox)
{
    const uint32_t half = hd / 2;
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n_heads * half) return;
    const uint32_t h = i / half, p = i % half;
    float *v = qk + (size_t)h * hd;
    const uint32_t i0 = neox ? p : 2 * p, i1 = neox ? half + p : 2 * p + 1;
    const float c = cos_tab[(size_t)pos * half + p], s = sin_tab[(size_t)pos * half + p];
    const float v0 = v[i0], v1 = v[i1];
    v[i0] = v0 * c - v1 * s;                         // rope.c:37-43 / 44-51
    v[i1] = v0 * s + v1 * c;
}

hipError_t launch_rope(float *qk, uint32_t pos, uint32_t n_heads, uint32_t hd, const float *cos_tab,
                       const float *sin_tab, int neox, hipStream_t s)
{
    uint32_t n = n_heads * (hd / 2);
    hipLaunchKernelGGL(k_rope, dim3((n + 255) / 256), dim3(256), 0, s, qk, pos, n_heads, hd, cos_tab, sin_tab, neox);
    return hipGetLastError();
}

__global__ void k_silu_mul(const float *g, const float *u, float *out, uint64_t n)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = silu_ref(g[i]) * u[i];
}

__global__ void k_act_mul(const float *g, const float *u, float *out, uint64_t n, uint32_t act)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = ffn_act(g[i], act) * u[i];
}

__global__ void k_silu(const float *x, float *out, uint64_t n)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = silu_ref(x[i]);
}

__global__ void k_add(const float *a, const float *b, float *out, uint64_t n)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = a[i] + b[i];
}

static uint32_t ew_blocks(uint64_t n)
{
    uint64_t b = (n + 255) / 256;
    return (uint32_t)(b < 1 ? 1 : (b > 65536 ? 65536 : b));
}

// The step state as the host sets it, taken by value at launch: stream-ordered
// behind the work already queued, with no host buffer the host could change
// before a copy engine reads it.
__global__ void k_set_state(StepState *st, StepState v)
{
    if (threadIdx.x == 0) *st = v;
}

hipError_t launch_set_state(StepState *st, const StepState &v, hipStream_t s)
{
    hipLaunchKernelGGL(k_set_state, dim3(1), dim3(64), 0, s, st, v);
    return hipGetLastError();
}

hipError_t launch_silu_mul(const float *g, const float *u, float *out, uint64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_silu_mul, dim3(ew_blocks(n)), dim3(256), 0, s, g, u, out, n);
    return hipGetLastError();
}

__global__ void k_act(const float *x, float *out, uint64_t n, uint32_t act, const float *bias, uint32_t period)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x)
        out[i] = ffn_act(bias ? x[i] + bias[i % period] : x[i], act);
}

hipError_t launch_act(const float *x, float *out, uint64_t n, uint32_t act, hipStream_t s, const float *bias,
                      uint32_t period)
{
    hipLaunchKernelGGL(k_act, dim3(ew_blocks(n)), dim3(256), 0, s, x, out, n, act, bias, period);
    return hipGetLastError();
}

// x[r] += row (pos + r) of a position-embedding table (transformer.c:188-205),
// pos from the step state or p0; rows decoded exactly (linear_get_row).
__global__ void k_pos_add(const uint8_t *w, uint32_t type, uint64_t row_bytes, uint32_t n, const StepState *st,
                          uint32_t p0, float *x)
{
    const uint32_t r = blockIdx.y, row = (st ? st->pos : p0) + r;
    const uint8_t *wr = w + (size_t)row * row_bytes;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float v;
        if (type == kF32) v = reinterpret_cast<const float *>(wr)[i];
        else {
            const uint32_t bv = block_values_dev(type);
            v = dequant_one(wr + (size_t)(i / bv) * block_bytes_dev(type), type, i % bv);
        }
        x[(size_t)r * n + i] += v;
    }
}

hipError_t launch_pos_add(const uint8_t *w, uint32_t type, uint64_t row_bytes, uint32_t n, const StepState *st,
                          uint32_t p0, uint32_t rows, float *x, hipStream_t s)
{
    hipLaunchKernelGGL(k_pos_add, dim3((n + 255) / 256, rows), dim3(256), 0, s, w, type, row_bytes, n, st, p0, x);
    return hipGetLastError();
}

__device__ __forceinline__ double block_sum_d(double v, double *s)
{
    const uint32_t lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    __syncthreads();
    if (lane == 0) s[w] = v;
    __syncthreads();
    double r = 0.0;
    for (uint32_t i = 0; i < blockDim.x / 64; i++) r += s[i];
    return r;
}

// layer_norm (norm.c:18-40): one workgroup; mean and variance summed in double
// (the reference sums them in index order, here in a tree: the same doubles up
// to the last bits, the same floats after rounding but for ties).
__global__ __launch_bounds__(1024) void k_layernorm(const float *__restrict__ x, const float *__restrict__ w,
                                                    const float *__restrict__ b, float *__restrict__ out,
                                                    uint32_t n, float eps)
{
    __shared__ double s[16];
    const uint32_t t = threadIdx.x;
    x += (size_t)blockIdx.x * n;                  // one row per workgroup
    out += (size_t)blockIdx.x * n;
    double acc = 0.0;
    for (uint32_t i = t; i < n; i += blockDim.x) acc += x[i];
    const float mean = (float)(block_sum_d(acc, s) / (double)n);
    double var = 0.0;
    for (uint32_t i = t; i < n; i += blockDim.x) {
        const float d = x[i] - mean;
        var += (double)d * d;
    }
    const float scale = 1.0f / sqrtf((float)(block_sum_d(var, s) / (double)n) + eps);
    for (uint32_t i = t; i < n; i += blockDim.x) {
        float v = (x[i] - mean) * scale;
        if (w) v *= w[i];
        if (b) v += b[i];
        out[i] = v;
    }
}

hipError_t launch_layernorm(const float *x, const float *w, const float *b, float *out, uint32_t n, float eps,
                            hipStream_t s, uint32_t rows)
{
    hipLaunchKernelGGL(k_layernorm, dim3(rows), dim3(1024), 0, s, x, w, b, out, n, eps);
    return hipGetLastError();
}

// x[i] += (a[i] + bias[i % n]) + b2[i]: the residual add of a projection output
// kept apart (its bias, and for a parallel block the FFN output), in the
// reference's order (linear.c:214-221, transformer.c:250-251, 271-272).
__global__ void k_resid_add(float *x, const float *a, const float *bias, const float *b2, uint64_t count, uint32_t n)
{
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < count; i += (uint64_t)gridDim.x * blockDim.x) {
        float y = a[i];
        if (bias) y += bias[i % n];
        if (b2) y += b2[i];
        x[i] += y;
    }
}

hipError_t launch_resid_add(float *x, const float *a, const float *bias, const float *b2, uint64_t count, uint32_t n,
                            hipStream_t s)
{
    hipLaunchKernelGGL(k_resid_add, dim3(ew_blocks(count)), dim3(256), 0, s, x, a, bias, b2, count, n);
    return hipGetLastError();
}

// Pairs (v[i], v[half + i]) of every q head and of the K cache row at the
// step's position (rope.c:44-51).
__global__ void k_rope_neox_step(float *q, float *kc, uint32_t n_head, uint32_t n_kv, uint32_t hd,
                                 const float *cos_tab, const float *sin_tab, const StepState *st)
{
    const uint32_t half = hd / 2, i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (n_head + n_kv) * half) return;
    const uint32_t head = i / half, p = i % half, pos = st->pos;
    float *v = head < n_head ? q + (size_t)head * hd : kc + ((size_t)pos * n_kv + (head - n_head)) * hd;
    const float c = cos_tab[(size_t)pos * half + p], s = sin_tab[(size_t)pos * half + p];
    const float v0 = v[p], v1 = v[half + p];
    v[p] = v0 * c - v1 * s;
    v[half + p] = v0 * s + v1 * c;
}

hipError_t launch_rope_neox_step(float *q, float *kc_layer, uint32_t n_head, uint32_t n_kv, uint32_t hd,
                                 const float *cos_tab, const float *sin_tab, const StepState *st, hipStream_t s)
{
    const uint32_t n = (n_head + n_kv) * (hd / 2);
    hipLaunchKernelGGL(k_rope_neox_step, dim3((n + 255) / 256), dim3(256), 0, s, q, kc_layer, n_head, n_kv, hd,
                       cos_tab, sin_tab, st);
    return hipGetLastError();
}

hipError_t launch_act_mul(const float *g, const float *u, float *out, uint64_t n, uint32_t act, hipStream_t s)
{
    hipLaunchKernelGGL(k_act_mul, dim3(ew_blocks(n)), dim3(256), 0, s, g, u, out, n, act);
    return hipGetLastError();
}

hipError_t launch_silu(const float *x, float *out, uint64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_silu, dim3(ew_blocks(n)), dim3(256), 0, s, x, out, n);
    return hipGetLastError();
}

hipError_t launch_add(const float *a, const float *b, float *out, uint64_t n, hipStream_t s)
{
    hipLaunchKernelGGL(k_add, dim3(ew_blocks(n)), dim3(256), 0, s, a, b, out, n);
    return hipGetLastError();
}

} // namespace fw
