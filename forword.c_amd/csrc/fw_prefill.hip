// Batched prompt forward (prefill).  forword.c feeds a prompt one token at a
// time through transformer_forward (main.c:145-151), so every weight matrix is
// read once per prompt token.  Here the prompt's tokens go through each layer
// together: the linears are fp32 GEMMs on the matrix cores
// (v_mfma_f32_16x16x4_f32) with the quantised weights dequantised exactly into
// LDS, the rest are batched versions of the per-token kernels.  Same arithmetic
// as the reference per element except the order of the linears' sums (the
// matrix cores accumulate in their own order), so results agree within the
// floating-point tolerance, not bit for bit.
#include "fw_device.h"
#include "fw_kernels.h"

namespace fw {

typedef float floatx4 __attribute__((ext_vector_type(4)));

// ── GEMM: Y[t][r] = Σ_k X[t][k] · W[r][k] ───────────────────────────────────
//
// A workgroup computes a 64-token × 128-row tile; each of its 4 waves a 32×64
// part of it as 2×4 tiles of 16×16.  K advances one quantisation block (32
// columns) at a time: the 64×32 input tile and the 128 dequantised weight rows
// are staged in LDS (rows padded to 33 floats against bank conflicts).
// v_mfma_f32_16x16x4_f32 operands: lane l gives A[l%16][l/16] and B[l/16][l%16];
// the result tile holds D[4·(l/16)+i][l%16] in element i of lane l.
constexpr int PG_BM = 64, PG_BN = 128, PG_BK = 32, PG_THREADS = 256;

// Values j0..j0+15 (j0 a multiple of 16) of a K super-block, each exactly as
// dequant_q4_k / dequant_q6_k gives it, with the block's header decoded once
// (quant.c:111-126, 160-183).
template <uint32_t T>
__device__ __forceinline__ void deq16_k(const uint8_t *blk, uint32_t j0, float (&w)[16])
{
    if constexpr (T == kQ4_K) {
        const float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        const float dmin = h2f((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
        const uint32_t g = j0 / 32;
        uint32_t sc, mn;
        scale_min_k4(g, blk + 4, sc, mn);
        const float ds = d * (float)sc, dm = dmin * (float)mn;
        const uint8_t *q = blk + 16 + (g / 2) * 32 + j0 % 32;
#pragma unroll
        for (int i = 0; i < 16; i++) w[i] = ds * (float)((g & 1) ? (q[i] >> 4) : (q[i] & 15)) - dm;
    } else {
        const uint32_t h = j0 / 128, r = j0 % 128, k = r / 32, l0 = r % 32;
        const uint8_t *a = blk + h * 64 + l0 + 32 * (k & 1), *hb = blk + 128 + h * 32 + l0;
        const int8_t sc = (int8_t)blk[192 + h * 8 + l0 / 16 + 2 * k];
        const float ds = h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8)) * (float)sc;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int q = (int)(((k >= 2) ? (a[i] >> 4) : (a[i] & 15)) | (((hb[i] >> (2 * k)) & 3) << 4));
            w[i] = ds * (float)(q - 32);
        }
    }
}

template <uint32_t T>
__global__ __launch_bounds__(PG_THREADS) void k_gemm_q(const float *__restrict__ X, uint32_t ldx,
                                                       const uint8_t *__restrict__ W, uint64_t row_bytes,
                                                       float *__restrict__ Y, uint32_t ldy, uint32_t n_tok,
                                                       uint32_t n_out, uint32_t n_in, int accumulate)
{
    __shared__ float Xs[PG_BM][PG_BK + 1];
    __shared__ float Ws[PG_BN][PG_BK + 1];
    const uint32_t r0 = blockIdx.x * PG_BN, t0 = blockIdx.y * PG_BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    floatx4 acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    // this thread's share of the weight tile: row wr, columns 16·wh .. 16·wh+15
    const int wr = tid >> 1, wh = tid & 1;
    const uint32_t r = r0 + wr;
    const uint8_t *wrow = W + (size_t)min(r, n_out - 1) * row_bytes;
    for (uint32_t k0 = 0; k0 < n_in; k0 += PG_BK) {
#pragma unroll
        for (int i = 0; i < PG_BM * PG_BK / PG_THREADS; i++) {
            const int e = tid + i * PG_THREADS, m = e / PG_BK, k = e % PG_BK;
            const uint32_t t = t0 + m;
            Xs[m][k] = t < n_tok ? X[(size_t)t * ldx + k0 + k] : 0.f;
        }
        // K-quants: the 32 columns are one group of a 256-value super-block
        constexpr uint32_t BV = T == kQ4_K || T == kQ6_K ? 256u : 32u;
        constexpr uint32_t BBY = T == kQ4_K ? 144u : T == kQ6_K ? 210u : T == kQ4_0 ? 18u : T == kQ5_0 ? 22u : 34u;
        const uint8_t *blk = wrow + (size_t)(k0 / BV) * BBY;
        const uint32_t j0 = k0 % BV + 16 * wh;
        if constexpr (T == kQ4_K || T == kQ6_K) {
            float w[16];
            deq16_k<T>(blk, j0, w);                       // rows past n_out read row n_out-1 (wrow)
#pragma unroll
            for (int j = 0; j < 16; j++) Ws[wr][16 * wh + j] = r < n_out ? w[j] : 0.f;
        } else {
#pragma unroll
            for (int j = 0; j < 16; j++) Ws[wr][16 * wh + j] = r < n_out ? dequant_one(blk, T, j0 + j) : 0.f;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < PG_BK; kk += 4) {
            float a[2], b[4];
#pragma unroll
            for (int mi = 0; mi < 2; mi++) a[mi] = Xs[wm * 32 + mi * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int ni = 0; ni < 4; ni++) b[ni] = Ws[wn * 64 + ni * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int ni = 0; ni < 4; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = t0 + wm * 32 + mi * 16 + 4 * (lane >> 4) + i;
                const uint32_t rr = r0 + wn * 64 + ni * 16 + (lane & 15);
                if (t < n_tok && rr < n_out) {
                    float *p = Y + (size_t)t * ldy + rr;
                    *p = accumulate ? *p + acc[mi][ni][i] : acc[mi][ni][i];   // x[i] += y[i] (transformer.c:271-272)
                }
            }
}

// Block b (0 or 1) of a dword-aligned block pair as 32 floats, each rounded
// once as the reference dequantises it: d·(q − k) computed as fma(q, d, −k·d)
// (exact product and k·d, one rounding), quant.c:258, quant_matvec.c:204-212.
template <uint32_t T>
__device__ __forceinline__ void deq_pair_block(const uint32_t *dw, int b, float (&w)[32])
{
    if constexpr (T == kQ4_0) {
        const float d = h2f(b ? dw[4] >> 16 : dw[0]), m8 = -8.0f * d;
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = b ? dw[5 + k] : align16(dw[k + 1], dw[k]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                w[4 * k + e] = __builtin_fmaf((float)((lo >> (8 * e)) & 0xFFu), d, m8);
                w[16 + 4 * k + e] = __builtin_fmaf((float)((hi >> (8 * e)) & 0xFFu), d, m8);
            }
        }
    } else if constexpr (T == kQ5_0) {
        const float d = h2f(b ? dw[5] >> 16 : dw[0]), m16 = -16.0f * d;
        const uint32_t qh = b ? dw[6] : align16(dw[1], dw[0]);
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = b ? dw[7 + k] : align16(dw[k + 2], dw[k + 1]);
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const uint32_t lo = q[k] & 0x0F0F0F0Fu, hi = (q[k] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const int j = 4 * k + e;
                const uint32_t ql = ((lo >> (8 * e)) & 0xFFu) | (((qh >> j) & 1u) << 4);
                const uint32_t qu = ((hi >> (8 * e)) & 0xFFu) | (((qh >> (j + 16)) & 1u) << 4);
                w[j] = __builtin_fmaf((float)ql, d, m16);
                w[16 + j] = __builtin_fmaf((float)qu, d, m16);
            }
        }
    } else {
        const float d = h2f(b ? dw[8] >> 16 : dw[0]);
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const uint32_t v = b ? dw[9 + k] : align16(dw[k + 1], dw[k]);
#pragma unroll
            for (int e = 0; e < 4; e++) w[4 * k + e] = d * (float)((int32_t)(v << (24 - 8 * e)) >> 24);
        }
    }
}

// The same tile with K in block pairs (64 columns): the input tile moves as
// float4, each thread dequantises one block of a weight row from dword loads,
// and the next pair's loads are in flight while the matrix cores work on the
// current one.  Needs n_in % 64 == 0 (so rows are dword aligned).
constexpr int PP_BK = 64, PP_XS = PP_BK + 4;

// Dwords one thread pair loads per 64 columns: a block pair, or for Q4_K the
// super-block header (4 dwords) and the quarter's 32 code bytes (8 dwords).
template <uint32_t T> constexpr int pair_dwords()
{
    if constexpr (T == kQ4_K) return 12;
    else return Blk<T>::pair_dw;
}

// Group 2·gp + hb (hb = 0: low nibbles, 1: high) of a Q4_K super-block quarter
// loaded as header + code dwords, each value exactly as dequant_q4_k gives it.
__device__ __forceinline__ void deq_q4k_half(const uint32_t *wd, uint32_t gp, int hb, float (&w)[32])
{
    const float d = h2f(wd[0]), dmin = h2f(wd[0] >> 16);
    auto sb8 = [&](uint32_t i) { return (wd[1 + i / 4] >> (8 * (i % 4))) & 0xFFu; };
    const uint32_t g = 2 * gp + (uint32_t)hb;
    uint32_t sc, mn;
    if (g < 4) { sc = sb8(g) & 63u; mn = sb8(g + 4) & 63u; }
    else {
        sc = (sb8(g + 4) & 15u) | ((sb8(g - 4) >> 6) << 4);
        mn = (sb8(g + 4) >> 4) | ((sb8(g) >> 6) << 4);
    }
    const float ds = d * (float)sc, dm = dmin * (float)mn;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const uint32_t b = (wd[4 + i / 4] >> (8 * (i % 4))) & 0xFFu;
        w[i] = ds * (float)(hb ? (b >> 4) : (b & 15u)) - dm;
    }
}

template <uint32_t T>
__global__ __launch_bounds__(PG_THREADS) void k_gemm_qp(const float *__restrict__ X, uint32_t ldx, GemmW g,
                                                        float *__restrict__ Y, uint32_t ldy, uint32_t n_tok,
                                                        uint32_t n_in, int accumulate)
{
    constexpr int PDW = pair_dwords<T>(), XV = PG_BM * PP_BK / 4 / PG_THREADS;   // float4 of x per thread
    __shared__ __align__(16) float Xs[PG_BM][PP_XS];
    __shared__ __align__(16) float Ws[PG_BN][PP_XS];
    const uint32_t r0 = blockIdx.x * PG_BN, t0 = blockIdx.y * PG_BM;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    floatx4 acc[2][4];
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    // the matrix this tile's rows belong to (segments end on tile boundaries)
    const uint32_t n_out = g.end[g.n_seg - 1];
    const uint8_t *W = g.w[0];
    uint64_t row_bytes = g.rb[0];
    uint32_t base = 0;
    if (g.n_seg > 1 && r0 >= g.end[0]) {
        W = g.w[1]; row_bytes = g.rb[1]; base = g.end[0];
        if (g.n_seg > 2 && r0 >= g.end[1]) { W = g.w[2]; row_bytes = g.rb[2]; base = g.end[1]; }
    }
    const int wr = tid >> 1, wb = tid & 1;                 // weight row of the tile, block of the pair
    const uint32_t r = r0 + wr;
    const uint8_t *wrow = W + (size_t)(min(r, n_out - 1) - base) * row_bytes;
    float4 xr[XV];
    uint32_t wd[PDW];
    auto fetch = [&](uint32_t k0) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const int e = tid + i * PG_THREADS, m = e / (PP_BK / 4), c4 = e % (PP_BK / 4);
            const uint32_t t = t0 + m;
            xr[i] = t < n_tok ? *reinterpret_cast<const float4 *>(X + (size_t)t * ldx + k0 + 4 * c4)
                              : float4{0.f, 0.f, 0.f, 0.f};
        }
        if constexpr (T == kQ4_K) {
            const uint32_t c = k0 / 64;
            const uint32_t *b32 = reinterpret_cast<const uint32_t *>(wrow + (size_t)(c / 4) * 144);
#pragma unroll
            for (int i = 0; i < 4; i++) wd[i] = b32[i];
#pragma unroll
            for (int i = 0; i < 8; i++) wd[4 + i] = b32[4 + (c % 4) * 8 + i];
        } else {
            load_pair<T>(wrow + (size_t)(k0 / 64) * (2 * Blk<T>::bytes), wd);
        }
    };
    fetch(0);
    for (uint32_t k0 = 0; k0 < n_in; k0 += PP_BK) {
#pragma unroll
        for (int i = 0; i < XV; i++) {
            const int e = tid + i * PG_THREADS, m = e / (PP_BK / 4), c4 = e % (PP_BK / 4);
            *reinterpret_cast<float4 *>(&Xs[m][4 * c4]) = xr[i];
        }
        {
            float w[32];
            if constexpr (T == kQ4_K) deq_q4k_half(wd, (k0 / 64) % 4, wb, w);
            else deq_pair_block<T>(wd, wb, w);
#pragma unroll
            for (int j = 0; j < 32; j += 4)
                *reinterpret_cast<float4 *>(&Ws[wr][32 * wb + j]) =
                    r < n_out ? float4{w[j], w[j + 1], w[j + 2], w[j + 3]} : float4{0.f, 0.f, 0.f, 0.f};
        }
        __syncthreads();
        if (k0 + PP_BK < n_in) fetch(k0 + PP_BK);
#pragma unroll
        for (int kk = 0; kk < PP_BK; kk += 4) {
            float a[2], b[4];
#pragma unroll
            for (int mi = 0; mi < 2; mi++) a[mi] = Xs[wm * 32 + mi * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int ni = 0; ni < 4; ni++) b[ni] = Ws[wn * 64 + ni * 16 + (lane & 15)][kk + (lane >> 4)];
#pragma unroll
            for (int mi = 0; mi < 2; mi++)
#pragma unroll
                for (int ni = 0; ni < 4; ni++)
                    acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[mi], b[ni], acc[mi][ni], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int mi = 0; mi < 2; mi++)
#pragma unroll
        for (int ni = 0; ni < 4; ni++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t t = t0 + wm * 32 + mi * 16 + 4 * (lane >> 4) + i;
                const uint32_t rr = r0 + wn * 64 + ni * 16 + (lane & 15);
                if (t < n_tok && rr < n_out) {
                    float *p = Y + (size_t)t * ldy + rr;
                    *p = accumulate ? *p + acc[mi][ni][i] : acc[mi][ni][i];
                }
            }
}

hipError_t launch_gemm_q(uint32_t type, const float *x, uint32_t ldx, const uint8_t *w, uint64_t row_bytes, float *y,
                         uint32_t ldy, uint32_t n_tok, uint32_t n_out, uint32_t n_in, bool accumulate,
                         hipStream_t s)
{
    GemmW g{};
    g.w[0] = w; g.rb[0] = row_bytes; g.end[0] = n_out; g.n_seg = 1;
    return launch_gemm_qs(type, x, ldx, g, y, ldy, n_tok, n_in, accumulate, s);
}

hipError_t launch_gemm_qs(uint32_t type, const float *x, uint32_t ldx, const GemmW &g, float *y, uint32_t ldy,
                          uint32_t n_tok, uint32_t n_in, bool accumulate, hipStream_t s)
{
    if (!n_tok || !n_in || n_in % 32 || g.n_seg < 1 || g.n_seg > 3) return hipErrorInvalidValue;
    const uint32_t n_out = g.end[g.n_seg - 1];
    if (!n_out) return hipErrorInvalidValue;
    const int acc = accumulate ? 1 : 0;
    // block pairs when rows are whole pairs at dword-aligned addresses, x rows float4 aligned and
    // every matrix starts on a tile boundary; else one launch of the general kernel per matrix
    bool pairs = (type == kQ4_0 || type == kQ5_0 || type == kQ8_0 || type == kQ4_K) && n_in % 64 == 0 &&
                 ((uintptr_t)x & 15) == 0 && ldx % 4 == 0;
    for (uint32_t i = 0; i < g.n_seg; i++) pairs = pairs && g.rb[i] % 4 == 0;     // every row dword-aligned
    for (uint32_t i = 0; i < g.n_seg; i++) {
        pairs = pairs && ((uintptr_t)g.w[i] & 3) == 0;
        if (i + 1 < g.n_seg) pairs = pairs && g.end[i] % PG_BN == 0;
    }
    if (pairs) {
        const dim3 grid((n_out + PG_BN - 1) / PG_BN, (n_tok + PG_BM - 1) / PG_BM);
#define GEMM(TY) hipLaunchKernelGGL(k_gemm_qp<TY>, grid, dim3(PG_THREADS), 0, s, x, ldx, g, y, ldy, n_tok, n_in, acc)
        switch (type) {
        case kQ4_0: GEMM(kQ4_0); break;
        case kQ5_0: GEMM(kQ5_0); break;
        case kQ8_0: GEMM(kQ8_0); break;
        case kQ4_K: GEMM(kQ4_K); break;
        default: return hipErrorNotSupported;
        }
#undef GEMM
        return hipGetLastError();
    }
    for (uint32_t i = 0; i < g.n_seg; i++) {
        const uint32_t r0 = i ? g.end[i - 1] : 0u, rows = g.end[i] - r0;
        const dim3 grid((rows + PG_BN - 1) / PG_BN, (n_tok + PG_BM - 1) / PG_BM);
        float *yo = y + r0;
#define GEMM(TY) hipLaunchKernelGGL(k_gemm_q<TY>, grid, dim3(PG_THREADS), 0, s, x, ldx, g.w[i], g.rb[i], yo, ldy, n_tok, rows, n_in, acc)
        switch (type) {
        case kQ4_0: GEMM(kQ4_0); break;
        case kQ5_0: GEMM(kQ5_0); break;
        case kQ8_0: GEMM(kQ8_0); break;
        case kQ4_K: GEMM(kQ4_K); break;
        case kQ6_K: GEMM(kQ6_K); break;
        default: return hipErrorNotSupported;
        }
#undef GEMM
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    return hipSuccess;
}

// ── embedding rows, RMSNorm rows ────────────────────────────────────────────

// X[t] = row tokens[t] of the embedding (linear_get_row, linear.c:60-151), times
// embd_scale when it is not 1 (transformer.c:179-182).
__global__ __launch_bounds__(256) void k_embed_rows(const uint8_t *w, uint32_t type, uint32_t n_cols,
                                                    const uint32_t *tokens, float embd_scale, float *X)
{
    const uint32_t t = blockIdx.y, tok = tokens[t];
    const uint32_t j = blockIdx.x * 256 + threadIdx.x;
    if (j >= n_cols) return;
    float v;
    if (type == kF32) v = reinterpret_cast<const float *>(w)[(size_t)tok * n_cols + j];
    else {
        const uint32_t bb = block_bytes_dev(type), bv = block_values_dev(type);
        v = dequant_one(w + (size_t)tok * (n_cols / bv) * bb + (size_t)(j / bv) * bb, type, j % bv);
    }
    if (embd_scale != 1.0f) v *= embd_scale;
    X[(size_t)t * n_cols + j] = v;
}

hipError_t launch_embed_rows(const uint8_t *w, uint32_t type, uint32_t n_cols, const uint32_t *tokens,
                             uint32_t n_tok, float embd_scale, float *x, hipStream_t s)
{
    hipLaunchKernelGGL(k_embed_rows, dim3((n_cols + 255) / 256, n_tok), dim3(256), 0, s, w, type, n_cols, tokens,
                       embd_scale, x);
    return hipGetLastError();
}

// ── RoPE on q and k, K/V append ─────────────────────────────────────────────

// QKV[t] = [q (n_head·hd) | k (kvd) | v (kvd)] of token t at position pos0 + t:
// add the bias of the same layout when there is one (linear.c:214-221), rotate
// q in place and k (rope.c:37-43, interleaved pairs), append k and v to the
// cache rows (attention.c:129-140).
__global__ __launch_bounds__(256) void k_rope_append(float *qkv, const float *bias, int neox, uint32_t ld,
                                                     uint32_t n_head, uint32_t n_kv, uint32_t hd, uint32_t pos0,
                                                     const float *cos_tab, const float *sin_tab, float *kc, float *vc)
{
    const uint32_t t = blockIdx.y, half = hd / 2, pos = pos0 + t, kvd = n_kv * hd;
    float *row = qkv + (size_t)t * ld;
    const uint32_t i = blockIdx.x * 256 + threadIdx.x;
    const uint32_t n_pairs = (n_head + n_kv) * half;
    if (i < n_pairs) {
        const uint32_t p = i % half;
        // pair elements of q, then of k (contiguous): (2i, 2i+1), or NEOX (p, p + hd/2) of head i/half
        const uint32_t e0 = neox ? (i / half) * hd + p : 2 * i, e1 = neox ? e0 + half : e0 + 1;
        const float c = cos_tab[(size_t)pos * half + p], s = sin_tab[(size_t)pos * half + p];
        const float v0 = bias ? row[e0] + bias[e0] : row[e0], v1 = bias ? row[e1] + bias[e1] : row[e1];
        const bool rot = neox != 2;                  // 2: no RoPE (attention.c:129-133), bias and append only
        const float w0 = rot ? v0 * c - v1 * s : v0, w1 = rot ? v0 * s + v1 * c : v1;
        if (i < n_head * half) {
            row[e0] = w0;
            row[e1] = w1;
        } else {
            const uint32_t nq = n_head * hd;
            kc[(size_t)pos * kvd + e0 - nq] = w0;
            kc[(size_t)pos * kvd + e1 - nq] = w1;
        }
    } else if (i < n_pairs + kvd / 2) {
        const uint32_t e = 2 * (i - n_pairs);
        const size_t o = (size_t)n_head * hd + kvd + e;
        vc[(size_t)pos * kvd + e] = bias ? row[o] + bias[o] : row[o];
        vc[(size_t)pos * kvd + e + 1] = bias ? row[o + 1] + bias[o + 1] : row[o + 1];
    }
}

hipError_t launch_rope_append(float *qkv, const float *bias, int neox, uint32_t ld, uint32_t n_tok, uint32_t n_head,
                              uint32_t n_kv, uint32_t hd,
                              uint32_t pos0, const float *cos_tab, const float *sin_tab, float *kc_layer,
                              float *vc_layer, hipStream_t s)
{
    const uint32_t n = (n_head + n_kv) * (hd / 2) + n_kv * hd / 2;
    hipLaunchKernelGGL(k_rope_append, dim3((n + 255) / 256, n_tok), dim3(256), 0, s, qkv, bias, neox, ld, n_head, n_kv, hd, pos0,
                       cos_tab, sin_tab, kc_layer, vc_layer);
    return hipGetLastError();
}

// ── causal attention over the prompt ────────────────────────────────────────

// Token t (position pos0 + t) and KV head h: the G query heads of the group
// attend to cache rows 0..pos0+t (attention.c:142-164; softmax attention.c:18-33
// as an online softmax in the log2 domain).  16 lanes hold one position (EPL =
// hd/16 dimensions each), so a wave walks four positions at a time; the four
// groups of a wave, then the four waves, merge their running (m, l, o).
template <int EPL, int G>
__global__ __launch_bounds__(256) void k_attn_prefill(const float *__restrict__ qkv, uint32_t ld,
                                                      const float *__restrict__ kc, const float *__restrict__ vc,
                                                      float *__restrict__ out, uint32_t n_kv, uint32_t pos0,
                                                      uint32_t group_total)
{
    constexpr int HD = 16 * EPL, NW = 4;
    __shared__ float s_o[NW][G][HD];
    __shared__ float s_m[NW][G], s_l[NW][G];
    // G of the group_total query heads of KV head h (the group in n_sub workgroups)
    const uint32_t n_sub = group_total / G, h = blockIdx.y / n_sub, h0 = h * group_total + (blockIdx.y % n_sub) * G;
    const uint32_t t = blockIdx.x, n_pos = pos0 + t + 1, kvd = n_kv * HD;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = lane >> 4, l16 = lane & 15;
    const float sc = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;      // attention.c:143, log2 units
    const float *q = qkv + (size_t)t * ld + (size_t)h0 * HD;
    float qv[G][EPL], m[G], l[G], o[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            qv[g][e] = q[g * HD + l16 * EPL + e];
            o[g][e] = 0.f;
        }
    }
    for (uint32_t p = wave * 4 + grp; p < n_pos; p += 4 * NW) {
        const float *kr = kc + (size_t)p * kvd + h * HD + l16 * EPL;
        const float *vr = vc + (size_t)p * kvd + h * HD + l16 * EPL;
        float kk[EPL], vv[EPL];
#pragma unroll
        for (int e = 0; e < EPL; e++) { kk[e] = kr[e]; vv[e] = vr[e]; }
#pragma unroll
        for (int g = 0; g < G; g++) {
            float d = 0.f;
#pragma unroll
            for (int e = 0; e < EPL; e++) d = __builtin_fmaf(qv[g][e], kk[e], d);
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) d += __shfl_xor(d, off, 16);
            const float sg = d * sc, mx = fmaxf(m[g], sg);
            const float c = exp2f(m[g] - mx), pe = exp2f(sg - mx);
            l[g] = l[g] * c + pe;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] = __builtin_fmaf(pe, vv[e], o[g][e] * c);
            m[g] = mx;
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {                          // the wave's four position groups
#pragma unroll
        for (int off = 16; off <= 32; off <<= 1) {
            const float mw = fmaxf(m[g], __shfl_xor(m[g], off, 64));
            const float c = mw == -INFINITY ? 0.f : exp2f(m[g] - mw);
            float lw = l[g] * c;
            lw += __shfl_xor(lw, off, 64);
#pragma unroll
            for (int e = 0; e < EPL; e++) {
                float ov = o[g][e] * c;
                ov += __shfl_xor(ov, off, 64);
                o[g][e] = ov;
            }
            m[g] = mw;
            l[g] = lw;
        }
    }
    if (lane < 16) {
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) s_o[wave][g][l16 * EPL + e] = o[g][e];
            if (lane == 0) { s_m[wave][g] = m[g]; s_l[wave][g] = l[g]; }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * HD; i += 256) {       // merge the four waves
        const int g = i / HD, d = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; w++) M = fmaxf(M, s_m[w][g]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < NW; w++) {
            const float c = M == -INFINITY ? 0.f : exp2f(s_m[w][g] - M);
            L = __builtin_fmaf(s_l[w][g], c, L);
            O = __builtin_fmaf(s_o[w][g][d], c, O);
        }
        out[(size_t)t * (n_kv * group_total * HD) + ((size_t)h0 + g) * HD + d] = O / L;
    }
}

template <int EPL>
static hipError_t attn_prefill_g(uint32_t group, uint32_t n_tok, hipStream_t s, const float *qkv, uint32_t ld,
                                 const float *kc, const float *vc, float *out, uint32_t n_kv, uint32_t pos0)
{
    const uint32_t gs = attn_sub_group(16 * EPL, group);
    const dim3 grid(n_tok, n_kv * (group / gs));
#define L(G) hipLaunchKernelGGL((k_attn_prefill<EPL, G>), grid, dim3(256), 0, s, qkv, ld, kc, vc, out, n_kv, pos0, group)
    switch (gs) {
    case 1: L(1); break;
    case 2: L(2); break;
    case 4: if constexpr (EPL <= 16) L(4); break;
    case 8: if constexpr (EPL <= 8) L(8); break;
    default: return hipErrorNotSupported;
    }
#undef L
    return hipGetLastError();
}

hipError_t launch_attn_prefill(const float *qkv, uint32_t ld, uint32_t n_tok, const float *kc_layer,
                               const float *vc_layer, float *out, uint32_t n_head, uint32_t n_kv, uint32_t hd,
                               uint32_t pos0, hipStream_t s)
{
    if (!n_kv || n_head % n_kv) return hipErrorInvalidValue;
    const uint32_t g = n_head / n_kv;
#define A(EPL) attn_prefill_g<EPL>(g, n_tok, s, qkv, ld, kc_layer, vc_layer, out, n_kv, pos0)
    switch (hd) {
    case 32: return A(2);
    case 48: return A(3);
    case 64: return A(4);
    case 80: return A(5);
    case 96: return A(6);
    case 128: return A(8);
    case 256: return A(16);
    default: return hipErrorNotSupported;
    }
#undef A
}

} // namespace fw
