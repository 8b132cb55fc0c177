// Device-side building blocks shared by the gfx950 kernels of the decode path.
//
// GGUF blocks are read in place from the uploaded data section:
//   Q4_0 18 B = fp16 d | qs[16]          w_j = d*(q_j - 8), q_j = qs[j]&15, q_{j+16} = qs[j]>>4
//   Q5_0 22 B = fp16 d | qh u32 | qs[16]  5th bit of code j = bit j of qh, w_j = d*(q_j - 16)
//   Q8_0 34 B = fp16 d | int8 qs[32]      w_j = d*q_j
// (gguf.c:211-215; quant_matvec.c:192-229; quant.c:232-263).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fw_kernels.h"

namespace fw {

typedef float float2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// Vector types that only promise dword alignment: GGUF blocks are 18/22/34 B,
// so a pair of blocks starts on a 4-byte boundary but rarely on 16.
typedef u32x4 u32x4_a4 __attribute__((aligned(4)));
typedef u32x2 u32x2_a4 __attribute__((aligned(4)));

// Global-memory (address space 1) views of generic pointers.  Pointers that
// the kernels read out of memory (phase descriptors) are generic to the
// compiler, which then emits flat loads; those also count on lgkmcnt, so every
// LDS access would wait for all outstanding weight loads.
#define FW_GLOBAL __attribute__((address_space(1)))
template <typename T> __device__ __forceinline__ const FW_GLOBAL T *gptr(const T *p)
{
    return (const FW_GLOBAL T *)p;
}
template <typename T> __device__ __forceinline__ FW_GLOBAL T *gptr(T *p) { return (FW_GLOBAL T *)p; }

template <uint32_t T> struct Blk;
template <> struct Blk<kQ4_0> { static constexpr int bytes = 18, pair_dw = 9; };
template <> struct Blk<kQ5_0> { static constexpr int bytes = 22, pair_dw = 11; };
template <> struct Blk<kQ8_0> { static constexpr int bytes = 34, pair_dw = 17; };
// One 64-value quarter of a Q4_K super-block: its 8 code dwords, then the
// super-block's 4 header dwords (d|dmin, 12 scale bytes).
template <> struct Blk<kQ4_K> { static constexpr int bytes = 144, pair_dw = 12; };
// One 56-byte quarter record of a repacked Q6_K super-block (14 dwords).
template <> struct Blk<kQ6_KR> { static constexpr int bytes = 224, pair_dw = 14; };

// fp16 bits (low half of h) -> fp32, exact incl. subnormals (v_cvt_f32_f16 with
// fp16 denormals enabled, the gfx9 default).
__device__ __forceinline__ float h2f(uint32_t h)
{
    return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xffffu));
}

__device__ __forceinline__ uint32_t align16(uint32_t hi, uint32_t lo)
{
    return __builtin_amdgcn_alignbit(hi, lo, 16);
}

// Two codes q in 0..15, one per byte in the selected 16-bit half of v, to
// floats q/512: a byte holding 0..15 read as OCP e4m3 is exactly q * 2^-9.
template <bool HI_HALF>
__device__ __forceinline__ float2v nib2(uint32_t v)
{
    return __builtin_amdgcn_cvt_pk_f32_fp8((int)v, HI_HALF);
}

// d * sum_j (q_j - 8) x_j over one Q4_0 block; q[4] = the 16 code bytes, x[32].
__device__ __forceinline__ float dot_q4_0(float d, const uint32_t *q, const float *x, float sx)
{
    float a0 = 0.f, a1 = 0.f;                    // two chains: fewer adds to close than four
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t lo = q[w] & 0x0F0F0F0Fu, hi = (q[w] >> 4) & 0x0F0F0F0Fu;
        float2v l01 = nib2<false>(lo), l23 = nib2<true>(lo);
        float2v h01 = nib2<false>(hi), h23 = nib2<true>(hi);
        a0 = __builtin_fmaf(l01.x, x[4 * w + 0], a0);
        a1 = __builtin_fmaf(l01.y, x[4 * w + 1], a1);
        a0 = __builtin_fmaf(l23.x, x[4 * w + 2], a0);
        a1 = __builtin_fmaf(l23.y, x[4 * w + 3], a1);
        a0 = __builtin_fmaf(h01.x, x[16 + 4 * w + 0], a0);
        a1 = __builtin_fmaf(h01.y, x[16 + 4 * w + 1], a1);
        a0 = __builtin_fmaf(h23.x, x[16 + 4 * w + 2], a0);
        a1 = __builtin_fmaf(h23.y, x[16 + 4 * w + 3], a1);
    }
    float s = a0 + a1;                           // sum q_j x_j / 512
    return d * __builtin_fmaf(s, 512.0f, -8.0f * sx);
}

// d * sum_j (q_j - 16) x_j over one Q5_0 block.
__device__ __forceinline__ float dot_q5_0(float d, uint32_t qh, const uint32_t *q, const float *x,
                                          float sx)
{
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        uint32_t lo = q[w] & 0x0F0F0F0Fu, hi = (q[w] >> 4) & 0x0F0F0F0Fu;
        float2v l01 = nib2<false>(lo), l23 = nib2<true>(lo);
        float2v h01 = nib2<false>(hi), h23 = nib2<true>(hi);
        a0 = __builtin_fmaf(l01.x, x[4 * w + 0], a0);
        a1 = __builtin_fmaf(l01.y, x[4 * w + 1], a1);
        a0 = __builtin_fmaf(l23.x, x[4 * w + 2], a0);
        a1 = __builtin_fmaf(l23.y, x[4 * w + 3], a1);
        a0 = __builtin_fmaf(h01.x, x[16 + 4 * w + 0], a0);
        a1 = __builtin_fmaf(h01.y, x[16 + 4 * w + 1], a1);
        a0 = __builtin_fmaf(h23.x, x[16 + 4 * w + 2], a0);
        a1 = __builtin_fmaf(h23.y, x[16 + 4 * w + 3], a1);
    }
#pragma unroll
    for (int j = 0; j < 32; j += 2) {
        b0 = __builtin_fmaf((float)((qh >> j) & 1u), x[j], b0);
        b1 = __builtin_fmaf((float)((qh >> (j + 1)) & 1u), x[j + 1], b1);
    }
    float s = a0 + a1, hb = b0 + b1;               // sum lo_j x_j / 512, sum hb_j x_j
    return d * (__builtin_fmaf(s, 512.0f, __builtin_fmaf(hb, 16.0f, -16.0f * sx)));
}

// d * sum_j q_j x_j over one Q8_0 block; q[8] = the 32 code bytes.
__device__ __forceinline__ float dot_q8_0(float d, const uint32_t *q, const float *x)
{
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t v = q[k];
        a0 = __builtin_fmaf((float)((int32_t)(v << 24) >> 24), x[4 * k + 0], a0);
        a1 = __builtin_fmaf((float)((int32_t)(v << 16) >> 24), x[4 * k + 1], a1);
        a2 = __builtin_fmaf((float)((int32_t)(v << 8) >> 24), x[4 * k + 2], a2);
        a3 = __builtin_fmaf((float)((int32_t)v >> 24), x[4 * k + 3], a3);
    }
    return d * ((a0 + a1) + (a2 + a3));
}

// Dot of a 4-byte-aligned pair of blocks (2*32 columns) with x[64].
template <uint32_t T>
__device__ __forceinline__ float dot_pair(const uint32_t *dw, const float *x, float sx0, float sx1)
{
    if constexpr (T == kQ4_0) {
        uint32_t q0[4] = { align16(dw[1], dw[0]), align16(dw[2], dw[1]), align16(dw[3], dw[2]),
                           align16(dw[4], dw[3]) };
        uint32_t q1[4] = { dw[5], dw[6], dw[7], dw[8] };
        return dot_q4_0(h2f(dw[0]), q0, x, sx0) + dot_q4_0(h2f(dw[4] >> 16), q1, x + 32, sx1);
    } else if constexpr (T == kQ5_0) {
        uint32_t qh0 = align16(dw[1], dw[0]);
        uint32_t q0[4] = { align16(dw[2], dw[1]), align16(dw[3], dw[2]), align16(dw[4], dw[3]),
                           align16(dw[5], dw[4]) };
        uint32_t q1[4] = { dw[7], dw[8], dw[9], dw[10] };
        return dot_q5_0(h2f(dw[0]), qh0, q0, x, sx0) + dot_q5_0(h2f(dw[5] >> 16), dw[6], q1, x + 32, sx1);
    } else {
        uint32_t q0[8], q1[8];
#pragma unroll
        for (int k = 0; k < 8; k++) { q0[k] = align16(dw[k + 1], dw[k]); q1[k] = dw[9 + k]; }
        return dot_q8_0(h2f(dw[0]), q0, x) + dot_q8_0(h2f(dw[8] >> 16), q1, x + 32);
    }
}

// Σ over the two 32-value groups of a Q4_K quarter of (d·sc)·q·x − (dmin·m)·x
// (quant.c:111-126, factored per group): q[8] = the quarter's 32 code bytes,
// value i < 32 in the low nibble of byte i, value 32 + i in its high nibble.
// ds/dm are the groups' rounded products d·sc and dmin·m; sx0/sx1 the sums of
// x over the two groups.  Codes in 1/512 units from the fp8 conversion, as for Q4_0.
__device__ __forceinline__ float dot_q4k_quarter(const uint32_t *q, const float *x, float ds0, float dm0, float ds1,
                                                 float dm1, float sx0, float sx1)
{
    float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t lo = q[i] & 0x0F0F0F0Fu, hi = (q[i] >> 4) & 0x0F0F0F0Fu;
        const float2v l01 = nib2<false>(lo), l23 = nib2<true>(lo);
        const float2v h01 = nib2<false>(hi), h23 = nib2<true>(hi);
        a0 = __builtin_fmaf(l01.x, x[4 * i + 0], a0);
        a1 = __builtin_fmaf(l01.y, x[4 * i + 1], a1);
        a0 = __builtin_fmaf(l23.x, x[4 * i + 2], a0);
        a1 = __builtin_fmaf(l23.y, x[4 * i + 3], a1);
        b0 = __builtin_fmaf(h01.x, x[32 + 4 * i + 0], b0);
        b1 = __builtin_fmaf(h01.y, x[32 + 4 * i + 1], b1);
        b0 = __builtin_fmaf(h23.x, x[32 + 4 * i + 2], b0);
        b1 = __builtin_fmaf(h23.y, x[32 + 4 * i + 3], b1);
    }
    const float s0 = (a0 + a1) * 512.0f, s1 = (b0 + b1) * 512.0f;
    return __builtin_fmaf(ds0, s0, -dm0 * sx0) + __builtin_fmaf(ds1, s1, -dm1 * sx1);
}

// Q4_K quarter u (0..3) of a super-block whose header dwords are h[0..3]:
// scales and mins of its groups 2u and 2u+1 (get_scale_min_k4, quant.c:66-85).
// Groups j < 4 take bytes j and j+4 (6 low bits); groups 4 + j take the low
// or high nibble of byte 8 + j and the top two bits of bytes j and 4 + j.  The
// two groups of a quarter sit in adjacent bytes, so both come out of one
// shift and mask, sc in the low two bytes of *sc, mins likewise.
__device__ __forceinline__ void q4k_quarter_scales(const uint32_t *h, uint32_t u, uint32_t &sc, uint32_t &mn)
{
    const bool low = u < 2;
    const uint32_t sh = (u & 1) * 16;
    const uint32_t m1 = low ? 0x3F3Fu : 0x0F0Fu, m2 = low ? 0u : 0x3030u;
    const uint32_t xs = low ? h[1] : h[3], xm = low ? h[2] : h[3], shm = low ? sh : sh + 4;
    sc = ((xs >> sh) & m1) | ((h[1] >> (sh + 2)) & m2);
    mn = ((xm >> shm) & m1) | ((h[2] >> (sh + 2)) & m2);
}

// Quarter u of a Q4_K super-block held as in Blk<kQ4_K> (codes dw[0..7], header dw[8..11]).
__device__ __forceinline__ float dot_q4k_item(const uint32_t *dw, const float *x, float sx0, float sx1, uint32_t u)
{
    uint32_t sc, mn;
    q4k_quarter_scales(dw + 8, u, sc, mn);
    const float d = h2f(dw[8]), dmin = h2f(dw[8] >> 16);
    return dot_q4k_quarter(dw, x, d * (float)(sc & 0xFFu), dmin * (float)(mn & 0xFFu), d * (float)(sc >> 8),
                           dmin * (float)(mn >> 8), sx0, sx1);
}

// One quarter record of a repacked Q6_K super-block (14 dwords).  Values i of
// the quarter (0..63) are q_i = lo4_i | hi2_i << 4 (quant.c:160-183):
//   dw[k], k < 8:   byte b holds lo4 of value 4k+b (low nibble) and of value 32+4k+b (high);
//   dw[8 + k/2]:    byte b holds hi2 of those two values, at bits 4-5 and 6-7 for even k,
//                   at bits 0-1 and 2-3 for odd k;
//   dw[12]:         the int8 scales of values 0-15, 16-31, 32-47, 48-63;
//   dw[13]:         d (fp16) in the low half.
// Result: Σ_g (d·sc_g)·(Σ_{i in g} q_i x_i − 32 Σ_{i in g} x_i), sx[g] the sums of x over the groups.
__device__ __forceinline__ float dot_q6kr(const uint32_t *dw, const float *x, const float *sx)
{
    float a[4] = { 0.f, 0.f, 0.f, 0.f };
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t n = dw[k], h = dw[8 + k / 2];
        const uint32_t hl = (k & 1) ? h << 4 : h, hh = (k & 1) ? h << 2 : h >> 2;
        const uint32_t ql = (n & 0x0F0F0F0Fu) | (hl & 0x30303030u);
        const uint32_t qh = ((n >> 4) & 0x0F0F0F0Fu) | (hh & 0x30303030u);
        const int gl = k / 4, gh = 2 + k / 4;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            a[gl] = __builtin_fmaf((float)((ql >> (8 * b)) & 0xFFu), x[4 * k + b], a[gl]);
            a[gh] = __builtin_fmaf((float)((qh >> (8 * b)) & 0xFFu), x[32 + 4 * k + b], a[gh]);
        }
    }
    const float d = h2f(dw[13]);
    float r = 0.f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float ds = d * (float)(int8_t)(dw[12] >> (8 * g));
        r = __builtin_fmaf(ds, __builtin_fmaf(-32.0f, sx[g], a[g]), r);
    }
    return r;
}

// Load one pair of blocks (pair_dw dwords) from a dword-aligned address.
template <uint32_t T>
__device__ __forceinline__ void load_pair(const uint8_t *p, uint32_t *dw)
{
    const FW_GLOBAL uint32_t *w = gptr(reinterpret_cast<const uint32_t *>(p));
    if constexpr (T == kQ4_0) {                       // 36 B = 16 + 16 + 4
        u32x4 a = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(w);
        u32x4 b = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(w + 4);
        dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
        dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
        dw[8] = w[8];
    } else if constexpr (T == kQ5_0) {                // 44 B = 16 + 16 + 8 + 4
        u32x4 a = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(w);
        u32x4 b = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(w + 4);
        u32x2 c = *reinterpret_cast<const FW_GLOBAL u32x2_a4 *>(w + 8);
        dw[0] = a.x; dw[1] = a.y; dw[2] = a.z; dw[3] = a.w;
        dw[4] = b.x; dw[5] = b.y; dw[6] = b.z; dw[7] = b.w;
        dw[8] = c.x; dw[9] = c.y; dw[10] = w[10];
    } else {                                          // 68 B = 4*16 + 4
#pragma unroll
        for (int k = 0; k < 4; k++) {
            u32x4 a = *reinterpret_cast<const FW_GLOBAL u32x4_a4 *>(w + 4 * k);
            dw[4 * k] = a.x; dw[4 * k + 1] = a.y; dw[4 * k + 2] = a.z; dw[4 * k + 3] = a.w;
        }
        dw[16] = w[16];
    }
}

// One block from a 2-byte-aligned address (rows whose byte length is not a
// multiple of 4, e.g. 9 blocks of 34 B): 16-bit loads, reassembled.
template <uint32_t T>
__device__ __forceinline__ float dot_single(const uint8_t *p, const float *x, float sx)
{
    const uint16_t *h = reinterpret_cast<const uint16_t *>(p);
    if constexpr (T == kQ4_0) {
        uint32_t q[4];
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = (uint32_t)h[1 + 2 * k] | ((uint32_t)h[2 + 2 * k] << 16);
        return dot_q4_0(h2f(h[0]), q, x, sx);
    } else if constexpr (T == kQ5_0) {
        uint32_t q[4];
        uint32_t qh = (uint32_t)h[1] | ((uint32_t)h[2] << 16);
#pragma unroll
        for (int k = 0; k < 4; k++) q[k] = (uint32_t)h[3 + 2 * k] | ((uint32_t)h[4 + 2 * k] << 16);
        return dot_q5_0(h2f(h[0]), qh, q, x, sx);
    } else {
        uint32_t q[8];
#pragma unroll
        for (int k = 0; k < 8; k++) q[k] = (uint32_t)h[1 + 2 * k] | ((uint32_t)h[2 + 2 * k] << 16);
        return dot_q8_0(h2f(h[0]), q, x);
    }
}

// 6-bit scale and min of group j of a Q4_K super-block (get_scale_min_k4, quant.c:66-85).
__device__ __forceinline__ void scale_min_k4(uint32_t j, const uint8_t *q, uint32_t &sc, uint32_t &mn)
{
    if (j < 4) {
        sc = q[j] & 63u;
        mn = q[j + 4] & 63u;
    } else {
        sc = (q[j + 4] & 15u) | ((uint32_t)(q[j - 4] >> 6) << 4);
        mn = (uint32_t)(q[j + 4] >> 4) | ((uint32_t)(q[j] >> 6) << 4);
    }
}

// Value j (0..255) of a Q4_K super-block: (d*sc)*q - dmin*m, each product
// rounded, then the difference (quant.c:111-126).
__device__ __forceinline__ float dequant_q4_k(const uint8_t *blk, uint32_t j)
{
    const float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const float dmin = h2f((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
    const uint32_t g = j / 32, i = j % 32;
    uint32_t sc, mn;
    scale_min_k4(g, blk + 4, sc, mn);
    const uint8_t b = blk[16 + (g / 2) * 32 + i];
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    return ds * (float)((g & 1) ? (b >> 4) : (b & 15)) - dm;
}

// Value j (0..255) of a Q6_K super-block: (d*sc)*(q-32) (quant.c:160-183).
__device__ __forceinline__ float dequant_q6_k(const uint8_t *blk, uint32_t j)
{
    const uint32_t h = j / 128, r = j % 128, k = r / 32, l = r % 32;
    const uint8_t a = blk[h * 64 + l + 32 * (k & 1)], hb = blk[128 + h * 32 + l];
    const int q = (int)(((k >= 2) ? (a >> 4) : (a & 15)) | (((hb >> (2 * k)) & 3) << 4));
    const int8_t sc = (int8_t)blk[192 + h * 8 + l / 16 + 2 * k];
    const float d = h2f((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    return (d * (float)sc) * (float)(q - 32);
}

// Element j of one block (0..31; 0..255 for the K super-blocks), exactly as the
// reference dequantises it.
__device__ __forceinline__ float dequant_one(const uint8_t *blk, uint32_t type, uint32_t j)
{
    if (type == kQ4_K) return dequant_q4_k(blk, j);
    if (type == kQ6_K) return dequant_q6_k(blk, j);
    float d = h2f((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    if (type == kQ8_0) return d * (float)(int8_t)blk[2 + j];                    // quant.c:258
    if (type == kQ4_0) {
        uint32_t b = blk[2 + (j & 15)];
        int q = (int)(j < 16 ? (b & 15u) : (b >> 4));
        return d * (float)(q - 8);
    }
    uint32_t qh = (uint32_t)blk[2] | ((uint32_t)blk[3] << 8) | ((uint32_t)blk[4] << 16) |
                  ((uint32_t)blk[5] << 24);
    uint32_t b = blk[6 + (j & 15)];
    int q = (int)((j < 16 ? (b & 15u) : (b >> 4)) | (((qh >> j) & 1u) << 4));
    return d * (float)(q - 16);                                                 // quant_matvec.c:204-212
}

__device__ __forceinline__ uint32_t block_bytes_dev(uint32_t t)
{
    return t == kQ4_0 ? 18u : t == kQ5_0 ? 22u : t == kQ4_K ? 144u : t == kQ6_K ? 210u : 34u;
}

__device__ __forceinline__ uint32_t block_values_dev(uint32_t t)
{
    return t == kQ4_K || t == kQ6_K ? 256u : 32u;
}

// Sum over the 64 lanes of a wave; every lane receives the total.
__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// Cross-workgroup communication without cache maintenance.  The L2 of each of
// the eight XCDs is not coherent with the others, and an agent-scope release
// fence writes the whole L2 back (~10 us for 256 workgroups).  Values one
// workgroup publishes for another therefore go through system-scope relaxed
// atomics (sc0 sc1: written through / read past the L2), ordered by an
// explicit wait for this wave's outstanding memory operations.
__device__ __forceinline__ void st_sys(float *p, float v)
{
    __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ void st_sys(uint32_t *p, uint32_t v)
{
    __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ float ld_sys(const float *p)
{
    return __hip_atomic_load(gptr(const_cast<float *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t ld_sys(const uint32_t *p)
{
    return __hip_atomic_load(gptr(const_cast<uint32_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// Two floats at an 8-byte aligned address.  Atomic loads are not reordered by
// the compiler, so callers issue a batch of them before using any result.
__device__ __forceinline__ float2v ld_sys2(const float *p)
{
    const uint64_t v = __hip_atomic_load(gptr(reinterpret_cast<uint64_t *>(const_cast<float *>(p))), __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_SYSTEM);
    float2v r;
    r[0] = __builtin_bit_cast(float, (uint32_t)v);
    r[1] = __builtin_bit_cast(float, (uint32_t)(v >> 32));
    return r;
}
// A published value with the epoch it belongs to, stored and loaded as one
// 64-bit single-copy-atomic word: a reader that sees the tag sees the value.
__device__ __forceinline__ uint64_t tagged(float v, uint32_t tag)
{
    return (uint64_t)__builtin_bit_cast(uint32_t, v) | ((uint64_t)tag << 32);
}
__device__ __forceinline__ void st_sys64(uint64_t *p, uint64_t v)
{
    __hip_atomic_store(gptr(p), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ld_sys64(const uint64_t *p)
{
    return __hip_atomic_load(gptr(const_cast<uint64_t *>(p)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint32_t ticket_sys(uint32_t *p)
{
    return __hip_atomic_fetch_add(gptr(p), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// s_waitcnt vmcnt(0) expcnt(0) lgkmcnt(0): every memory operation this wave issued has completed.
__device__ __forceinline__ void wait_mem() { __builtin_amdgcn_s_waitcnt(0); }

// expf through double precision: the float result is the correctly rounded
// e^v except where the double lands within an ulp of a float rounding midpoint.
__device__ __forceinline__ float exp_f32(float v) { return (float)exp((double)v); }

// apply_silu (ffn.c:17-25): v * sigma(v) with the reference's two branches.
__device__ __forceinline__ float silu_ref(float v)
{
    float sig;
    if (v >= 0.0f) sig = 1.0f / (1.0f + exp_f32(-v));
    else { float e = exp_f32(v); sig = e / (1.0f + e); }
    return v * sig;
}

// The gated FFN's GELU forms: erf (ffn.c:27-31) and tanh (ffn.c:33-42).
__device__ __forceinline__ float gelu_erf(float v)
{
    return 0.5f * v * (1.0f + erff(v * 0.7071067811865476f));
}

__device__ __forceinline__ float gelu_tanh(float v)
{
    const float inner = 0.7978845608028654f * (v + 0.044715f * v * v * v);   // sqrt(2/pi) (v + 0.044715 v^3)
    return 0.5f * v * (1.0f + tanhf(inner));
}

__device__ __forceinline__ float ffn_act(float v, uint32_t act)
{
    return act == ACT_GELU        ? gelu_erf(v)
         : act == ACT_GELU_TANH ? gelu_tanh(v)
         : act == ACT_RELU      ? (v < 0.0f ? 0.0f : v)
                                : silu_ref(v);
}

} // namespace fw
