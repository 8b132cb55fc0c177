// Standalone block-quantised matrix-vector product y = W x (quant_matvec,
// quant_matvec.c:263-312) for Q4_0 / Q5_0 / Q8_0 rows of whole 64-value block
// pairs: the kernel behind forword_gpu_quant_matvec.
//
// At batch 1 the fp32 dequant-dot costs about 2.3 VALU instructions per weight
// (nibble/byte unpack, fp8 conversion, FMA), which at the HBM rate is most of
// the chip's vector issue rate: the kernel is as much an issue problem as a
// read stream, and the two only overlap if loads stay in flight while the
// products run.  So:
//   - lanes own block pairs (lane l of a wave: pair l of its rows; rows wider
//     than 64 pairs are split over KS waves of the workgroup), and a lane keeps
//     the 64 input values of its pair in registers for every row it visits;
//   - x is staged once per workgroup in LDS (LDS-DMA, 16-byte chunks rotated
//     per pair so the lanes' reads are conflict free) instead of once per wave
//     through the vector memory pipe, and up to three workgroups of four waves
//     share a CU (three waves per SIMD: one computes while the others wait);
//   - each wave walks tasks of one row per row group, keeping the next task's
//     weights in flight in a second register buffer, issued by inline asm and
//     waited for with explicit vmcnt counts (the compiler's own waits would
//     also wait for the prefetched task); the first task's weights go out
//     right behind the x loads, so their latencies overlap;
//   - row sums over the 64 lanes use DPP only (row sums, then row_bcast:15 and
//     row_bcast:31 into lane 63), and results wait in LDS until the loop ends:
//     a global store in the loop makes the compiler wait for every load in
//     flight before it may reuse the store's data register.
// Measured choices (Llama-3-8B matrix shapes): three workgroups per CU beat one
// or two, and 8 or 12 waves per workgroup; one row per task beat two; a
// two-deep ring beat three to six (more loads in flight only lengthened their
// latency).
#include "fw_device.h"
#include "fw_kernels.h"

#include <algorithm>

namespace fw {

constexpr int kMvWaves = 4;                 // waves per workgroup
constexpr int kMvRows = 1;                  // rows per wave per task
constexpr int kMvRing = 2;                  // register ring depth (tasks in flight + 1)
constexpr int kMvWgPerCu = 3;               // workgroups per CU, as LDS allows
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

// Wait until at most `ahead` (< NB) tasks of D loads each are still in flight.
template <int D, int NB>
__device__ __forceinline__ void mv_wait_ahead(uint32_t ahead)
{
    static_assert((NB - 1) * D <= 63, "vmcnt range");
    switch (ahead) {
    case 1: mv_vmwait<D>(); break;
    case 2: mv_vmwait<(NB > 2 ? 2 : 0) * D>(); break;
    case 3: mv_vmwait<(NB > 3 ? 3 : 0) * D>(); break;
    case 4: mv_vmwait<(NB > 4 ? 4 : 0) * D>(); break;
    case 5: mv_vmwait<(NB > 5 ? 5 : 0) * D>(); break;
    default: mv_vmwait<0>(); break;
    }
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

typedef __attribute__((address_space(3))) void mv_lds_void;

// One LDS-DMA load of 16 bytes per lane: lane i's bytes land at LDS byte
// lds + 16 i (M0 saved and restored around the load that reads it).
__device__ __forceinline__ void mv_dma16(const FW_GLOBAL uint8_t *src, uint8_t *lds)
{
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(mv_lds_void *)lds);
    uint32_t keep;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\ts_mov_b32 m0, %0"
                 : "=&s"(keep)
                 : "v"(src), "s"(m)
                 : "memory");
}

// NW waves per workgroup, R rows per wave per task; NB: register ring depth
// (NB - 1 tasks in flight while one is summed).  x is staged once per
// workgroup in LDS, pair p's 16 chunks of 16 bytes rotated by p (chunk i at
// slot (i + p) & 15), so the lanes' reads of their pairs hit distinct banks.
template <uint32_t T, int R, int KS, int NB, int NW>
__global__ __launch_bounds__(64 * NW) void k_mv(const uint8_t *__restrict__ w, uint64_t row_bytes,
                                                const float *__restrict__ x, float *__restrict__ y,
                                                uint32_t n_rows, uint32_t n_pairs)
{
    constexpr int G = NW / KS, D = MvPair<T>::loads * R, NDW = Blk<T>::pair_dw;
    extern __shared__ __align__(16) float mv_lds[];
    const uint32_t x_slots = (n_pairs + 3) / 4;                   // 1 KB DMA slots of staged x
    uint8_t *xs = reinterpret_cast<uint8_t *>(mv_lds);
    float *ybuf = mv_lds + 256 * x_slots;                         // [task][group][row][ks]
    const uint32_t lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t grp = wave / KS, ks = wave % KS;
    const uint32_t per = (n_pairs + KS - 1) / KS, p0 = min(n_pairs, ks * per), p1 = min(n_pairs, p0 + per);
    const bool on = p0 + lane < p1;
    const uint32_t pc = on ? p0 + lane : 0u;                      // idle lanes read pair 0 and add nothing
    const uint32_t rpt = G * R, n_tasks = (n_rows + rpt - 1) / rpt;
    const uint32_t my = blockIdx.x < n_tasks ? (n_tasks - blockIdx.x + gridDim.x - 1) / gridDim.x : 0;

    // x into LDS: slot j holds chunks 64 j .. 64 j + 63; chunk q = 16 p + s holds
    // x's chunk 16 p + ((s - p) & 15).  Chunks past the input reload chunk 0.
    for (uint32_t j = wave; j < x_slots; j += NW) {
        const uint32_t q = 64 * j + lane, p = q >> 4, sl = q & 15;
        const uint32_t src = q < 16 * n_pairs ? 16 * p + ((sl - p) & 15) : 0u;
        mv_dma16(reinterpret_cast<const FW_GLOBAL uint8_t *>(gptr(x)) + 16 * (size_t)src, xs + 1024 * j);
    }
    MvPair<T> ring[NB][R];
    auto issue = [&](uint32_t k, MvPair<T> (&q)[R]) {
        const uint32_t r0 = (blockIdx.x + k * gridDim.x) * rpt + grp * R;
#pragma unroll
        for (int r = 0; r < R; r++)
            mv_load<T>(w + (size_t)min(r0 + r, n_rows - 1) * row_bytes + (size_t)pc * (2 * Blk<T>::bytes), q[r]);
    };
    // the first NB - 1 tasks' weights go out behind the x loads; vmcnt then says
    // when this wave's x slots have landed (loads complete in order)
    const uint32_t n_first = min(my, (uint32_t)(NB - 1));
#pragma unroll
    for (int j = 0; j < NB - 1; j++)
        if ((uint32_t)j < n_first) issue(j, ring[j]);
    mv_wait_ahead<D, NB>(n_first);
    __syncthreads();                                              // every wave's x slots are in LDS
    float xv[64];
    {
        const uint32_t base = (uint32_t)(uintptr_t)(mv_lds_void *)(xs + 256 * (size_t)pc);
        float4v r[16];
        uint32_t ad[16];
#pragma unroll
        for (int i = 0; i < 16; i++) ad[i] = base + (((i + pc) & 15u) << 4);
#pragma unroll
        for (int q = 0; q < 16; q += 4)
            asm volatile("ds_read_b128 %0, %4\n\tds_read_b128 %1, %5\n\tds_read_b128 %2, %6\n\tds_read_b128 %3, %7"
                         : "=&v"(r[q]), "=&v"(r[q + 1]), "=&v"(r[q + 2]), "=&v"(r[q + 3])
                         : "v"(ad[q]), "v"(ad[q + 1]), "v"(ad[q + 2]), "v"(ad[q + 3]));
        asm volatile("s_waitcnt lgkmcnt(0)"
                     : "+v"(r[0]), "+v"(r[1]), "+v"(r[2]), "+v"(r[3]), "+v"(r[4]), "+v"(r[5]), "+v"(r[6]), "+v"(r[7]),
                       "+v"(r[8]), "+v"(r[9]), "+v"(r[10]), "+v"(r[11]), "+v"(r[12]), "+v"(r[13]), "+v"(r[14]),
                       "+v"(r[15]));
#pragma unroll
        for (int i = 0; i < 16; i++) {
            xv[4 * i] = r[i][0]; xv[4 * i + 1] = r[i][1]; xv[4 * i + 2] = r[i][2]; xv[4 * i + 3] = r[i][3];
        }
    }
    float sx0 = 0.f, sx1 = 0.f;
    if constexpr (T != kQ8_0) {
        float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; s2 += xv[32 + i]; s3 += xv[33 + i]; }
        sx0 = s0 + s1;
        sx1 = s2 + s3;
    }

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
    // Task k sits in slot k % NB; before summing it, the wave issues task
    // k + NB - 1 into the slot of task k - 1 (already summed).
    for (uint32_t k = 0; k < my; k += NB) {
#pragma unroll
        for (int j = 0; j < NB; j++) {
            const uint32_t kk = k + j;
            if (kk >= my) break;
            if (kk + NB - 1 < my) issue(kk + NB - 1, ring[(j + NB - 1) % NB]);
            mv_wait_ahead<D, NB>(min(my - 1 - kk, (uint32_t)(NB - 1)));
            compute(kk, ring[j]);
        }
    }
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < my * rpt; i += 64 * NW) {
        const uint32_t row = (blockIdx.x + (i / rpt) * gridDim.x) * rpt + i % rpt;
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < KS; k++) s += ybuf[i * KS + k];
        if (row < n_rows) y[row] = s;
    }
}

template <uint32_t T, int KS>
static hipError_t mv_launch(const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                            uint32_t n_pairs, hipStream_t s)
{
    constexpr int R = kMvRows, NW = kMvWaves, NB = kMvRing;
    static int cus = 0;
    if (!cus) {
        int dev = 0, c = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            c < 1)
            return hipErrorNotSupported;
        cus = c;
    }
    const uint32_t rpt = R * (NW / KS), n_tasks = (n_rows + rpt - 1) / rpt;
    // workgroups per CU: up to kMvWgPerCu whose staged x (and results) fit the CU's 160 KB of LDS together
    const size_t x_lds = (size_t)1024 * ((n_pairs + 3) / 4);
    uint32_t wpc = kMvWgPerCu, grid = 0;
    size_t lds = 0;
    for (;; wpc--) {
        grid = std::min<uint32_t>(n_tasks, (uint32_t)cus * wpc);
        lds = x_lds + (size_t)((n_tasks + grid - 1) / grid) * rpt * KS * 4;
        if (wpc <= 1 || lds * wpc <= 160 * 1024) break;
    }
    if (lds > 64 * 1024) return hipErrorNotSupported;
    hipLaunchKernelGGL((k_mv<T, R, KS, NB, NW>), dim3(grid), dim3(64 * NW), lds, s, w, row_bytes, x, y, n_rows, n_pairs);
    return hipGetLastError();
}

template <uint32_t T>
static hipError_t mv_ks(const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                        uint32_t n_pairs, hipStream_t s)
{
    if (n_pairs <= 64) return mv_launch<T, 1>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (n_pairs <= 128) return mv_launch<T, 2>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (n_pairs <= 256) return mv_launch<T, 4>(w, row_bytes, x, y, n_rows, n_pairs, s);
    return hipErrorNotSupported;                                  // a lane would need more than one pair
}

hipError_t launch_gemv(uint32_t type, const uint8_t *w, uint64_t row_bytes, const float *x, float *y, uint32_t n_rows,
                       uint32_t n_cols, hipStream_t s)
{
    if ((type != kQ4_0 && type != kQ5_0 && type != kQ8_0) || n_cols % 64 || !n_rows || row_bytes % 4 ||
        ((uintptr_t)w & 3) || ((uintptr_t)x & 15))
        return hipErrorNotSupported;
    const uint32_t n_pairs = n_cols / 64;
    if (type == kQ4_0) return mv_ks<kQ4_0>(w, row_bytes, x, y, n_rows, n_pairs, s);
    if (type == kQ5_0) return mv_ks<kQ5_0>(w, row_bytes, x, y, n_rows, n_pairs, s);
    return mv_ks<kQ8_0>(w, row_bytes, x, y, n_rows, n_pairs, s);
}

} // namespace fw
