// Standalone block-quantised matrix-vector product y = W x (quant_matvec,
// quant_matvec.c:263-312) for Q4_0 / Q5_0 / Q8_0 rows of whole 64-value block
// pairs: the kernel behind forword_gpu_quant_matvec.
//
// At batch 1 the fp32 dequant-dot costs about 2.5 VALU instructions per weight
// (nibble/byte unpack, fp8 conversion, FMA), which at the HBM rate is most of
// the chip's vector issue rate: the kernel is as much an issue problem as a
// read stream, and the two only overlap if the loads are kept in flight while
// the products run.  So:
//   - lanes own block pairs (lane l of a wave: pair l of its rows; rows wider
//     than 64 pairs are split over KS waves of the workgroup), and a lane keeps
//     the 64 input values of its pair in registers for every row it visits;
//   - one workgroup of four waves per CU walks tasks of G*R rows (G = 4 / KS
//     row groups of R rows); each wave keeps the weights of its next two tasks
//     in flight in a ring of three register buffers, issued by inline asm and
//     waited for with explicit vmcnt counts (the compiler's own waits would
//     also wait for the prefetched tasks);
//   - row sums over the 64 lanes use DPP only (row sums, then row_bcast:15 and
//     row_bcast:31 into lane 63), and results wait in LDS until the loop ends:
//     a global store in the loop makes the compiler wait for every load in
//     flight before it may reuse the store's data register.
#include "fw_device.h"
#include "fw_kernels.h"

#include <algorithm>

namespace fw {

constexpr int kMvWaves = 4;
typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));

// Loads of one block pair per lane: Q4_0 36 B = 16 + 16 + 4, Q5_0 44 B =
// 16 + 16 + 12, Q8_0 68 B = 4 x 16 + 4 (dword-aligned pairs).
template <uint32_t T> struct MvPair;
template <> struct MvPair<kQ4_0> { static constexpr int loads = 3; u32x4 a, b; uint32_t t; };
template <> struct MvPair<kQ5_0> { static constexpr int loads = 3; u32x4 a, b; u32x3 t; };
template <> struct MvPair<kQ8_0> { static constexpr int loads = 5; u32x4 a, b, c, d; uint32_t t; };

#define FW_LD(OUT, INSN, OFF) asm volatile(INSN " %0, %1, off offset:" #OFF : "=v"(OUT) : "v"(p) : "memory")
template <uint32_t T>
__device__ __forceinline__ void mv_load(const uint8_t *src, MvPair<T> &q)
{
    const FW_GLOBAL uint8_t *p = gptr(src);
    if constexpr (T == kQ4_0) {
        FW_LD(q.a, "global_load_dwordx4", 0); FW_LD(q.b, "global_load_dwordx4", 16); FW_LD(q.t, "global_load_dword", 32);
    } else if constexpr (T == kQ5_0) {
        FW_LD(q.a, "global_load_dwordx4", 0); FW_LD(q.b, "global_load_dwordx4", 16); FW_LD(q.t, "global_load_dwordx3", 32);
    } else {
        FW_LD(q.a, "global_load_dwordx4", 0); FW_LD(q.b, "global_load_dwordx4", 16);
        FW_LD(q.c, "global_load_dwordx4", 32); FW_LD(q.d, "global_load_dwordx4", 48); FW_LD(q.t, "global_load_dword", 64);
    }
}
#undef FW_LD

// The pair's dwords once its loads have landed (the empty asm keeps the reads
// of the registers after the explicit wait).
template <uint32_t T>
__device__ __forceinline__ void mv_dwords(MvPair<T> &q, uint32_t (&dw)[Blk<T>::pair_dw])
{
    if constexpr (T == kQ8_0) {
        asm volatile("" : "+v"(q.a), "+v"(q.b), "+v"(q.c), "+v"(q.d), "+v"(q.t));
        const u32x4 v[4] = { q.a, q.b, q.c, q.d };
#pragma unroll
        for (int i = 0; i < 4; i++) { dw[4 * i] = v[i].x; dw[4 * i + 1] = v[i].y; dw[4 * i + 2] = v[i].z; dw[4 * i + 3] = v[i].w; }
        dw[16] = q.t;
    } else {
        asm volatile("" : "+v"(q.a), "+v"(q.b), "+v"(q.t));
        dw[0] = q.a.x; dw[1] = q.a.y; dw[2] = q.a.z; dw[3] = q.a.w;
        dw[4] = q.b.x; dw[5] = q.b.y; dw[6] = q.b.z; dw[7] = q.b.w;
        if constexpr (T == kQ4_0) dw[8] = q.t;
        else { dw[8] = q.t.x; dw[9] = q.t.y; dw[10] = q.t.z; }
    }
}

template <int N>
__device__ __forceinline__ void mv_vmwait()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most `ahead` tasks of D loads each are still in flight.
template <int D>
__device__ __forceinline__ void mv_wait_ahead(uint32_t ahead)
{
    if (ahead >= 2) mv_vmwait<2 * D>();
    else if (ahead == 1) mv_vmwait<D>();
    else mv_vmwait<0>();
}

template <int CTRL, int ROWS>
__device__ __forceinline__ float mv_dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROWS, 0xF, false));
}

// Sum over the wave's 64 lanes, complete in lane 63.
__device__ __forceinline__ float mv_sum_to63(float v)
{
    v += mv_dpp<0xB1, 0xF>(v);                     // quad_perm 1,0,3,2
    v += mv_dpp<0x4E, 0xF>(v);                     // quad_perm 2,3,0,1
    v += mv_dpp<0x141, 0xF>(v);                    // row_half_mirror
    v += mv_dpp<0x140, 0xF>(v);                    // row_mirror: every lane of a row holds its sum
    v += mv_dpp<0x142, 0xA>(v);                    // row_bcast:15 into rows 1 and 3
    v += mv_dpp<0x143, 0x8>(v);                    // row_bcast:31 into row 3
    return v;
}

template <uint32_t T, int R, int KS>
__global__ __launch_bounds__(64 * kMvWaves) void k_mv(const uint8_t *__restrict__ w, uint64_t row_bytes,
                                                      const float *__restrict__ x, float *__restrict__ y,
                                                      uint32_t n_rows, uint32_t n_pairs)
{
    constexpr int G = kMvWaves / KS, D = MvPair<T>::loads * R, NDW = Blk<T>::pair_dw;
    extern __shared__ float ybuf[];                               // [task][group][row][ks]
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6, grp = wave / KS, ks = wave % KS;
    const uint32_t per = (n_pairs + KS - 1) / KS, p0 = min(n_pairs, ks * per), p1 = min(n_pairs, p0 + per);
    const bool on = p0 + lane < p1;
    const uint32_t pc = on ? p0 + lane : 0u;                      // idle lanes read pair 0 and add nothing
    const uint32_t rpt = G * R, n_tasks = (n_rows + rpt - 1) / rpt;
    const uint32_t my = blockIdx.x < n_tasks ? (n_tasks - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;

    float xv[64];
    const FW_GLOBAL float4v *xp = reinterpret_cast<const FW_GLOBAL float4v *>(gptr(x) + 64 * (size_t)pc);
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4v v = xp[i];
        xv[4 * i] = v[0]; xv[4 * i + 1] = v[1]; xv[4 * i + 2] = v[2]; xv[4 * i + 3] = v[3];
    }
    float sx0 = 0.f, sx1 = 0.f;
    if constexpr (T != kQ8_0) {
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; s2 += xv[32 + i]; s3 += xv[33 + i]; }
        sx0 = s0 + s1;
        sx1 = s2 + s3;
    }
    asm volatile("" ::"v"(sx0), "v"(sx1));                        // x has landed before any weight load goes out

    MvPair<T> ring[3][R];
    auto issue = [&](uint32_t k, MvPair<T> (&q)[R]) {
        const uint32_t r0 = (blockIdx.x + k * gridDim.x) * rpt + grp * R;
#pragma unroll
        for (int r = 0; r < R; r++)
            mv_load<T>(w + (size_t)min(r0 + r, n_rows - 1) * row_bytes + (size_t)pc * (2 * Blk<T>::bytes), q[r]);
    };
    auto compute = [&](uint32_t k, MvPair<T> (&q)[R]) {
#pragma unroll
        for (int r = 0; r < R; r++) {
            uint32_t dw[NDW];
            mv_dwords<T>(q[r], dw);
            const float d = dot_pair<T>(dw, xv, sx0, sx1);
            const float s = mv_sum_to63(on ? d : 0.f);
            if (lane == 63) ybuf[((k * G + grp) * R + r) * KS + ks] = s;
        }
    };
    if (my > 0) issue(0, ring[0]);
    if (my > 1) issue(1, ring[1]);
    for (uint32_t k = 0; k < my; k += 3) {
        if (k + 2 < my) issue(k + 2, ring[2]);
        mv_wait_ahead<D>(min(my - 1 - k, 2u));
        compute(k, ring[0]);
        if (k + 1 >= my) break;
        if (k + 3 < my) issue(k + 3, ring[0]);
        mv_wait_ahead<D>(min(my - 2 - k, 2u));
        compute(k + 1, ring[1]);
        if (k + 2 >= my) break;
        if (k + 4 < my) issue(k + 4, ring[1]);
        mv_wait_ahead<D>(min(my - 3 - k, 2u));
        compute(k + 2, ring[2]);
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < my * rpt; i += 64 * kMvWaves) {
        const uint32_t row = (blockIdx.x + (i / rpt) * gridDim.x) * rpt + i % rpt;
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < KS; k++) s += ybuf[i * KS + k];
        if (row < n_rows) y[row] = s;
    }
}

template <uint32_t T, int R, int KS>
static hipError_t mv_launch(const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                            uint32_t n_pairs, hipStream_t s)
{
    static int cus = 0;
    if (!cus) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c < 1)
            return hipErrorNotSupported;
        cus = c;
    }
    const uint32_t rpt = R * (kMvWaves / KS), n_tasks = (n_rows + rpt - 1) / rpt;
    const uint32_t grid = std::min<uint32_t>(n_tasks, (uint32_t)cus);          // one workgroup per CU
    const size_t lds = (size_t)((n_tasks + grid - 1) / grid) * rpt * KS * 4;
    if (lds > 64 * 1024) return hipErrorNotSupported;
    hipLaunchKernelGGL((k_mv<T, R, KS>), dim3(grid), dim3(64 * kMvWaves), lds, s, w, row_bytes, x, y, n_rows, n_pairs);
    return hipGetLastError();
}

template <uint32_t T, int R>
static hipError_t mv_ks(const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                        uint32_t n_pairs, hipStream_t s)
{
    if (n_pairs <= 64) return mv_launch<T, R, 1>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (n_pairs <= 128) return mv_launch<T, R, 2>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (n_pairs <= 256) return mv_launch<T, R, 4>(w, row_bytes, x, y, n_rows, n_pairs, s);
    return hipErrorNotSupported;                                  // a lane would need more than one pair
}

hipError_t launch_gemv(uint32_t type, const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                       uint32_t n_cols, hipStream_t s)
{
    if ((type != kQ4_0 && type != kQ5_0 && type != kQ8_0) || n_cols % 64 || !n_rows || row_bytes % 4 ||
        ((uintptr_t)w & 3) || ((uintptr_t)x & 15))
        return hipErrorNotSupported;
    const uint32_t n_pairs = n_cols / 64;
    if (type == kQ4_0) return mv_ks<kQ4_0, 2>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (type == kQ5_0) return mv_ks<kQ5_0, 2>(w, row_bytes, x, y, n_rows, n_pairs, s);
    return mv_ks<kQ8_0, 1>(w, row_bytes, x, y, n_rows, n_pairs, s);
}

} // namespace fw
