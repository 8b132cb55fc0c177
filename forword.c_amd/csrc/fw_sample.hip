// Device-resident sampling (sampler.c:12-101 as main.c:176-188 applies it): the
// repetition penalty, then greedy argmax (temperature <= 0) or temperature +
// softmax + top-p with the reference's xorshift64 stream, on the logits the
// step left in HBM, so a sampled generation loop never copies logits to the
// host.  Orders that decide the result are the reference's: the nucleus is
// walked in (probability descending, index ascending) order — glibc's stable
// qsort — with sequential float sums; only the softmax normaliser is a
// parallel sum, so a draw can differ from the reference's only when r lands
// within float rounding of a cumulative boundary.  Bucket weights (which only
// choose the candidates) are summed as integers, so no accumulation order can
// change a decision.
#include "fw_device.h"
#include "fw_kernels.h"

namespace fw {

constexpr uint32_t kSampBuckets = 1024;          // probability buckets: float bits >> 20 (p <= 1)
constexpr uint32_t kSampThreads = 256;
constexpr float kSampFix = 1099511627776.0f;     // bucket weights in units of 2^-40

__device__ __forceinline__ float block_reduce(float v, bool is_max)
{
    __shared__ float s[kSampThreads / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = __shfl_xor(v, m, 64);
        v = is_max ? fmaxf(v, o) : v + o;
    }
    __syncthreads();
    if (lane == 0) s[w] = v;
    __syncthreads();
    float r = s[0];
    for (int i = 1; i < (int)(kSampThreads / 64); i++) r = is_max ? fmaxf(r, s[i]) : r + s[i];
    return r;
}

// buf[i] = logit i after `counts[i]` applications of the repetition penalty
// (sampler.c:89-101: once per occurrence in the history), scaled by 1/temperature
// when scale (sampler.c:12-16); per-block maxima for the softmax.
__global__ __launch_bounds__(kSampThreads) void k_samp_prep(const float *__restrict__ logits,
                                                           const uint32_t *__restrict__ counts, uint32_t n, float pen,
                                                           float inv_t, int scale, float *__restrict__ buf,
                                                           float *__restrict__ pmax)
{
    float mx = -INFINITY;
    for (uint32_t i = blockIdx.x * kSampThreads + threadIdx.x; i < n; i += gridDim.x * kSampThreads) {
        float x = logits[i];
        if (pen != 1.0f)
            for (uint32_t k = counts[i]; k; k--) x = x > 0.0f ? x / pen : x * pen;
        if (scale) x *= inv_t;
        buf[i] = x;
        mx = fmaxf(mx, x);
    }
    mx = block_reduce(mx, true);
    if (threadIdx.x == 0) pmax[blockIdx.x] = mx;
}

// buf[i] = expf(buf[i] - max) (sampler.c:18-24); per-block sums.
__global__ __launch_bounds__(kSampThreads) void k_samp_exp(float *__restrict__ buf, uint32_t n,
                                                          const float *__restrict__ pmax, uint32_t nb,
                                                          float *__restrict__ psum)
{
    float mx = -INFINITY;
    for (uint32_t j = 0; j < nb; j++) mx = fmaxf(mx, pmax[j]);
    float s = 0.f;
    for (uint32_t i = blockIdx.x * kSampThreads + threadIdx.x; i < n; i += gridDim.x * kSampThreads) {
        const float e = exp_f32(buf[i] - mx);
        buf[i] = e;
        s += e;
    }
    s = block_reduce(s, false);
    if (threadIdx.x == 0) psum[blockIdx.x] = s;
}

// buf[i] *= 1/sum (sampler.c:25-26); count and weight (integer, 2^-40 units) of
// each probability bucket.
__global__ __launch_bounds__(kSampThreads) void k_samp_norm(float *__restrict__ buf, uint32_t n,
                                                           const float *__restrict__ psum, uint32_t nb,
                                                           uint32_t *__restrict__ bcnt,
                                                           unsigned long long *__restrict__ bsum)
{
    float sum = 0.f;
    for (uint32_t j = 0; j < nb; j++) sum += psum[j];
    const float inv = 1.0f / sum;
    for (uint32_t i = blockIdx.x * kSampThreads + threadIdx.x; i < n; i += gridDim.x * kSampThreads) {
        const float p = buf[i] * inv;
        buf[i] = p;
        const uint32_t b = min(__float_as_uint(p) >> 20, kSampBuckets - 1);
        atomicAdd(bcnt + b, 1u);
        atomicAdd(bsum + b, (unsigned long long)rintf(fminf(p, 1.0f) * kSampFix));
    }
}

__device__ __forceinline__ uint64_t xorshift64(uint64_t &s)
{
    s ^= s << 13;
    s ^= s >> 7;
    s ^= s << 17;
    return s;
}

// Ascending bitonic sort of keys[0..np2) (np2 a power of two) by the whole
// workgroup, in LDS or in global memory (a pass's pairs are disjoint, so each
// thread loads its pairs before it stores any).
__device__ void bitonic_sort(uint64_t *keys, uint32_t np2)
{
    const uint32_t t = threadIdx.x;
    for (uint32_t k = 2; k <= np2; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            for (uint32_t i0 = 0; i0 < np2; i0 += 8 * 1024) {
                uint64_t a[8], c[8];
                uint32_t ii[8];
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t p = i0 + u * 1024 + t;              // p-th pair of the pass
                    const uint32_t i = ((p & ~(j - 1)) << 1) | (p & (j - 1));   // its lower index (bit j clear)
                    ii[u] = i;
                    if (p < np2 / 2) { a[u] = keys[i]; c[u] = keys[i | j]; }
                }
#pragma unroll
                for (int u = 0; u < 8; u++) {
                    const uint32_t p = i0 + u * 1024 + t, i = ii[u];
                    if (p < np2 / 2 && (a[u] > c[u]) == ((i & k) == 0)) { keys[i] = c[u]; keys[i | j] = a[u]; }
                }
            }
            __syncthreads();
        }
}

// One workgroup: the decision.  Greedy: first maximum of the penalised logits
// (sampler.c:28-32).  Top-p: the buckets from the top whose weight reaches
// top_p, one bucket more as margin, are the candidates; they are sorted exactly
// by (probability descending, index ascending) — in LDS when at most `cap` of
// them, else in the global buffer gkeys (next power of two >= n keys) — then
// the nucleus, its normaliser and the draw follow sampler.c:65-86 in order,
// with the running sums taken sequentially in that order.  Writes the token to
// ids[g] and as the step state's next token, counts it in the history, clears
// the buckets.
__global__ __launch_bounds__(1024) void k_samp_pick(const float *__restrict__ buf, uint32_t n, float temperature,
                                                    float top_p, uint32_t cap, uint32_t *__restrict__ bcnt,
                                                    unsigned long long *__restrict__ bsum, uint64_t *__restrict__ gkeys,
                                                    SampleState *ss, StepState *st, uint32_t *__restrict__ ids,
                                                    uint32_t g, uint32_t *__restrict__ counts)
{
    extern __shared__ uint64_t lkeys[];
    __shared__ float s_v[16];
    __shared__ uint32_t s_i[16], s_sel, s_n, s_tok;
    const uint32_t t = threadIdx.x, lane = t & 63, w = t >> 6;
    if (temperature <= 0.0f) {
        float bv = -INFINITY;
        uint32_t bi = 0xffffffffu;
        for (uint32_t i = t; i < n; i += 1024) {
            const float v = buf[i];
            if (!isnan(v) && (bi == 0xffffffffu || v > bv)) { bv = v; bi = i; }
        }
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const float ov = __shfl_xor(bv, m, 64);
            const uint32_t oi = __shfl_xor(bi, m, 64);
            if (oi != 0xffffffffu && (bi == 0xffffffffu || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
        }
        if (lane == 0) { s_v[w] = bv; s_i[w] = bi; }
        __syncthreads();
        if (t == 0) {
            for (int k = 1; k < 16; k++)
                if (s_i[k] != 0xffffffffu && (bi == 0xffffffffu || s_v[k] > bv || (s_v[k] == bv && s_i[k] < bi))) {
                    bv = s_v[k];
                    bi = s_i[k];
                }
            s_tok = (bi == 0xffffffffu || isnan(buf[0])) ? 0u : bi;   // index 0 wins when it is NaN
        }
    } else {
        __shared__ float s_cum;
        __shared__ uint32_t s_nucleus, s_redo;
        if (t == 0) {
            double acc = 0.0;
            uint32_t b = kSampBuckets, cnt = 0;
            // at least the highest non-empty bucket: with top_p <= 0 the nucleus
            // is the single most probable token (sampler.c:71-76 stops at i = 0)
            do {
                b--;
                acc += (double)bsum[b] * (1.0 / 1099511627776.0);
                cnt += bcnt[b];
            } while (b > 0 && (acc < (double)top_p || cnt == 0));
            s_sel = b > 0 ? b - 1 : 0;                               // one bucket of margin
        }
        uint64_t *keys = lkeys;
        // A second pass with every token a candidate when the candidates' own
        // running sum stops short of top_p (the walk would go on into the buckets
        // left out).
        for (int attempt = 0; attempt < 2; attempt++) {
            if (t == 0) {
                if (attempt) s_sel = 0;
                s_n = 0;
            }
            __syncthreads();
            const uint32_t sel = s_sel;
            for (uint32_t i = t; i < n; i += 1024) {
                const uint32_t pb = __float_as_uint(buf[i]);
                if (min(pb >> 20, kSampBuckets - 1) >= sel) {
                    const uint32_t slot = atomicAdd(&s_n, 1u);
                    const uint64_t key = ((uint64_t)(~pb) << 32) | i;
                    if (slot < cap) lkeys[slot] = key;
                    gkeys[slot] = key;                               // slot < n always
                }
            }
            __syncthreads();
            const uint32_t m = s_n;
            uint32_t np2 = 1;
            while (np2 < m) np2 <<= 1;
            keys = m <= cap ? lkeys : gkeys;
            for (uint32_t i = m + t; i < np2; i += 1024) keys[i] = ~0ull;
            __syncthreads();
            bitonic_sort(keys, np2);
            // sampler.c:65-76 by wave 0: 64 keys loaded at a time, summed in order
            // by every lane (all lanes hold the same running sum)
            if (w == 0) {
                float cum = 0.f;
                uint32_t nucleus = 0;
                bool done = false;
                for (uint32_t base = 0; base < m && !done; base += 64) {
                    const uint64_t key = base + lane < m ? keys[base + lane] : ~0ull;
                    const uint32_t pbits = ~(uint32_t)(key >> 32), cnt = min(64u, m - base);
                    for (uint32_t l = 0; l < cnt; l++) {
                        cum += __uint_as_float(__builtin_amdgcn_readlane(pbits, l));
                        nucleus = base + l + 1;
                        if (cum >= top_p) { done = true; break; }
                    }
                }
                if (lane == 0) {
                    s_cum = cum;
                    s_nucleus = nucleus;
                    s_redo = !done && sel > 0;
                    if (m == 0) ss->err = 1;                         // no candidate: only non-finite logits
                }
            }
            __syncthreads();
            if (!s_redo) break;
        }
        // sampler.c:78-86: the draw, walking the nucleus again in order
        if (w == 0) {
            const float cum = s_cum;
            const uint32_t nucleus = s_nucleus;
            uint64_t rng = ss->rng;
            const float r = (float)(xorshift64(rng) >> 11) / (float)(0xFFFFFFFFFFFFFFFFull >> 11) * cum;
            uint32_t tok = nucleus ? (uint32_t)keys[nucleus - 1] : 0u;
            float c = 0.f;
            bool done = false;
            for (uint32_t base = 0; base < nucleus && !done; base += 64) {
                const uint64_t key = base + lane < nucleus ? keys[base + lane] : ~0ull;
                const uint32_t pbits = ~(uint32_t)(key >> 32), kidx = (uint32_t)key, cnt = min(64u, nucleus - base);
                for (uint32_t l = 0; l < cnt; l++) {
                    c += __uint_as_float(__builtin_amdgcn_readlane(pbits, l));
                    if (r <= c) { tok = __builtin_amdgcn_readlane(kidx, l); done = true; break; }
                }
            }
            if (lane == 0) {
                ss->rng = rng;
                s_tok = tok;
            }
        }
    }
    __syncthreads();
    for (uint32_t b = t; b < kSampBuckets; b += 1024) { bcnt[b] = 0; bsum[b] = 0ull; }
    if (t == 0) {
        const uint32_t tok = s_tok;
        ids[g] = tok;
        counts[tok] += 1;
        st->token = tok;                       // the next step forwards the sampled token
    }
}

uint32_t samp_blocks(uint32_t n)
{
    const uint32_t b = (n + kSampThreads * 8 - 1) / (kSampThreads * 8);
    return b < 1 ? 1 : b > 256 ? 256 : b;
}

hipError_t launch_sample(const float *logits, uint32_t n, const uint32_t *counts, float temperature, float top_p,
                         float penalty, float *buf, float *part, uint32_t *bcnt, unsigned long long *bsum,
                         uint64_t *gkeys, uint32_t cap, SampleState *ss, StepState *st, uint32_t *ids, uint32_t g,
                         uint32_t *counts_rw, hipStream_t s)
{
    const uint32_t nb = samp_blocks(n);
    const bool top = temperature > 0.0f;
    hipLaunchKernelGGL(k_samp_prep, dim3(nb), dim3(kSampThreads), 0, s, logits, counts, n, penalty,
                       top ? 1.0f / temperature : 1.0f, top && temperature != 1.0f ? 1 : 0, buf, part);
    if (top) {
        hipLaunchKernelGGL(k_samp_exp, dim3(nb), dim3(kSampThreads), 0, s, buf, n, part, nb, part + 256);
        hipLaunchKernelGGL(k_samp_norm, dim3(nb), dim3(kSampThreads), 0, s, buf, n, part + 256, nb, bcnt, bsum);
    }
    static bool attr = false;
    if (!attr) {
        (void)hipFuncSetAttribute((const void *)k_samp_pick, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)(cap * sizeof(uint64_t)));
        attr = true;
    }
    hipLaunchKernelGGL(k_samp_pick, dim3(1), dim3(1024), cap * sizeof(uint64_t), s, buf, n, temperature, top_p, cap,
                       bcnt, bsum, gkeys, ss, st, ids, g, counts_rw);
    return hipGetLastError();
}

} // namespace fw
