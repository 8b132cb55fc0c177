// Persistent token-step kernel: transformer_forward (transformer.c:149-326)
// plus the greedy pick (sampler.c:28-32) for one or more tokens in a single
// cooperative launch, one 512-thread workgroup (8 waves) per CU.
//
// Why: a decode step is ~4.6 GB of weight reads split over ~200 dependent
// matrix-vector products.  As separate kernels each pays launch ramp and a
// full memory round trip with HBM idle in between.  Here each CU keeps its
// share of every matrix streaming through LDS (global_load_lds), and a
// workgroup that arrives at a phase boundary has the first rows of its next
// phase in flight before it waits.  Two waves per SIMD: while one waits on
// LDS, a shuffle or its ring, the other computes.
//
// Phases per layer, each waiting only for its own inputs (tagged values or
// per-workgroup flags, described below):
//   QKV   input x, RMSNorm folded in; epilogue RoPE, KV append, q and the new
//         K/V row published as tagged words
//   ATTN  split-K over positions per KV head; the GQA group shares one read of
//         K/V; partials published as tagged words, which the workgroup of the
//         head's first split merges
//   WO    input: attention output; epilogue x += y (+ trace row)
//   FFN   input x, RMSNorm folded in; gate and up rows together -> silu(g)*u
//   DOWN  input h; epilogue x += y (+ trace row)
// then LM-HEAD (output RMSNorm folded in) with the argmax reduced by a ticket.
//
// GEMV mapping.  A phase's rows are split evenly (even counts, so RoPE pairs
// stay together) over the workgroups.  Columns are cut into slices of Q block
// pairs, Q = pairs / 8 rounded up but at least 32 (the whole row, up to 64
// pairs, for the lm-head); each wave owns a slice, its lanes are (row-in-group,
// pair) = (lane / P, lane % P) with P the power of two >= Q (lanes past Q only
// reload the slice's last pair), so one item of the wave's weight stream
// covers 64/P rows.  Wide slices give each item long contiguous runs of a row
// and the lm-head one partial per row.  A lane keeps the 64 input values of its pair in
// registers for the whole slice, so a wave reads only Q distinct 64-float
// blocks of the LDS-staged input (stored with a per-block rotation of its
// 16-byte chunks so those reads are bank-conflict free).  Per-row partial
// sums of the slices go through LDS and are added in slice order.
//
// Cross-workgroup data (activations, partials, tickets, flags, step state)
// moves through system-scope relaxed atomics: the L2s of the eight XCDs are not
// coherent with each other and an agent-scope release writes back a whole L2.
// K/V rows of earlier steps are read with plain loads: a row is written
// (write-through, ordered by the end-of-step barrier) before any workgroup of
// the launch reads it, and caches start clean at launch; the row of the
// current position is read only as tagged words in its own step.
// Grid barriers are per-workgroup epoch flags on separate cache lines, each
// polled by one thread of every workgroup; the spin is bounded and sets an
// error flag, after which every workgroup leaves the kernel.  The only grid
// barrier is at the end of a step; a workgroup raises its flag first and then
// issues the next step's first weight items, so the wait overlaps them.  x,
// q, the new K/V row, the attention partials and the attention output pass
// between phases as tagged {value, epoch} words (an attention item loads its
// older K/V rows before it polls q); the FFN activations h (14336 values on the
// 8B shape, read whole by every workgroup) pass as plain floats behind one
// such epoch flag per workgroup, read with 16-byte loads: one flag round trip
// and one load batch instead of three batches of tagged words.
#include "fw_device.h"
#include "fw_kernels.h"
#include "fw_step.h"

namespace fw {

constexpr int MK_WAVES = 8;                 // two waves per SIMD, 256 registers each
constexpr int MK_THREADS = MK_WAVES * 64;
static_assert(MK_THREADS == (int)kMkThreads, "workgroup size");
static_assert((int)kMkPollers <= MK_THREADS, "one barrier flag per polling thread");
// Items per wave issued before a barrier (or staging) for the phase after it:
// the wave's one ring slot.  A wave's own later loads (barrier polls, staged
// inputs) complete only after its earlier ones.
constexpr uint32_t MK_PF = 1;
constexpr int MK_SMAX = 8;                  // column slices per row at most (64 block pairs each)

// threadIdx.x through an opaque move.  Values derived from it are then formed
// where each phase uses them; otherwise the compiler hoists every phase's
// per-lane values out of the step loop and keeps them all live across every
// phase (256 registers and spills instead of under 200).
__device__ __forceinline__ uint32_t tid()
{
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

// Index of the calling wave in its workgroup, as a wave-uniform (scalar) value:
// what derives from it (slices, row ranges, trip counts) stays in SGPRs and
// the loops over it branch uniformly.
__device__ __forceinline__ uint32_t wave_id() { return __builtin_amdgcn_readfirstlane(tid() >> 6); }

// Position of input element j in the LDS staging area.
__device__ __forceinline__ uint32_t swz(uint32_t j)
{
    return (j & ~63u) | ((((j >> 2) + (j >> 6)) & 15u) << 2) | (j & 3u);
}

// ── grid barrier ─────────────────────────────────────────────────────────────

// Arrival: this workgroup's stores are complete (every wave waited for its own
// memory operations), then its flag carries the new epoch.
__device__ __forceinline__ void bar_arrive(const MkArgs &a, uint32_t epoch, uint32_t *s_fail)
{
    wait_mem();
    if (tid() == 0) *s_fail = 0;
    __syncthreads();
    if (tid() == 0) st_sys(a.bar + blockIdx.x * 32, epoch);
}

// Wait until every workgroup's flag has reached epoch: thread t polls the flag
// of workgroup t.  A wait that gives up (or sees another one give up) sets the
// error word; the caller then leaves the kernel.
__device__ __forceinline__ bool bar_wait(const MkArgs &a, uint32_t epoch, uint32_t *s_fail)
{
    if (tid() < gridDim.x) {
        uint32_t spins = 0;
        while ((int)(ld_sys(a.bar + tid() * 32) - epoch) < 0) {
            if (++spins > (1u << 22) || ld_sys(a.err) != 0) {
                atomicOr(a.err, 1u);
                *s_fail = 1;
                break;
            }
        }
    }
    __syncthreads();
    return *s_fail == 0;
}

// ── staging ──────────────────────────────────────────────────────────────────

// RMSNorm folded into the GEMV (rms_norm, norm.c:7-16): the staged input is
// x*w and the epilogue multiplies each row's sum by 1/sqrt(mean(x^2)+eps), so
// no pass over the staged values waits for the sum of squares.  Each wave
// stores its share of that sum in s_red (visible after the staging barrier);
// norm_scale adds the eight shares in wave order.
__device__ __forceinline__ void wave_ss(float ss, float *s_red)
{
    ss = wave_sum(ss);
    if ((tid() & 63) == 0) s_red[wave_id()] = ss;
}
__device__ __forceinline__ float norm_scale(const float *s_red, uint32_t n, float eps)
{
    float r = 0.f;
#pragma unroll
    for (int w = 0; w < MK_WAVES; w++) r += s_red[w];
    return 1.0f / sqrtf((r / (float)n) + eps);
}

// xs <- src: n values published by other workgroups as {value, tag} words,
// times the norm weights nw when given (the scale is folded into the
// epilogue, see norm_scale; each wave's sum of squares goes to s_red).  Every
// thread issues its loads at once and then calls issue() (this phase's first
// weight items, which queue behind them).  Values whose tag is not yet `tag`
// are loaded again, in batches with a back-off so early workgroups do not
// flood memory.  Returns false when a wait gives up or another workgroup has
// failed (the error word is then set); every thread returns the same.
constexpr int MK_TB_EMBD = 8;               // values per thread per batch (n_embd-wide inputs)

template <int MK_TB, typename F>
__device__ __forceinline__ bool stage(const MkArgs &a, float *xs, const uint64_t *src, uint32_t n, const float *nw,
                                      float eps, uint32_t tag, float *s_red, uint32_t *s_fail, F &&issue)
{
    const uint32_t t = tid();
    float ss = 0.f;
    bool ok = true;
    issue();
    for (uint32_t j0 = 0; j0 < n; j0 += MK_TB * MK_THREADS) {
        uint64_t v[MK_TB];
        float w[MK_TB];
#pragma unroll
        for (int b = 0; b < MK_TB; b++) {
            const uint32_t j = j0 + t + b * MK_THREADS;
            v[b] = (uint64_t)tag << 32;
            w[b] = 1.0f;
            if (j < n) {
                v[b] = ld_sys64(src + j);
                if (nw) w[b] = gptr(nw)[j];
            }
        }
        uint32_t stale = 0;
#pragma unroll
        for (int b = 0; b < MK_TB; b++)
            if ((uint32_t)(v[b] >> 32) != tag) stale |= 1u << b;
        for (uint32_t round = 0; stale && ok; round++) {
            __builtin_amdgcn_s_sleep(8);                           // ~512 cycles
            if (round > (1u << 16) || ((round & 15) == 15 && ld_sys(a.err) != 0)) {
                ok = false;
                break;
            }
#pragma unroll
            for (int b = 0; b < MK_TB; b++)
                if (stale & (1u << b)) v[b] = ld_sys64(src + j0 + t + b * MK_THREADS);
#pragma unroll
            for (int b = 0; b < MK_TB; b++)
                if ((stale & (1u << b)) && (uint32_t)(v[b] >> 32) == tag) stale &= ~(1u << b);
        }
#pragma unroll
        for (int b = 0; b < MK_TB; b++) {
            const uint32_t j = j0 + t + b * MK_THREADS;
            if (j < n) {
                const float x = __builtin_bit_cast(float, (uint32_t)v[b]);
                ss = __builtin_fmaf(x, x, ss);
                xs[swz(j)] = x * w[b];                             // (x * w), times the scale in the epilogue
            }
        }
    }
    if (!ok) *s_fail = 1;
    if (nw) wave_ss(ss, s_red);
    (void)eps;
    __syncthreads();
    if (*s_fail) {
        if (t == 0) atomicOr(a.err, 1u);
        return false;
    }
    return true;
}

// xs <- h (DOWN's input, n floats): every thread t below the workgroup count
// waits for workgroup t's flag to reach `tag` (bounded, like a barrier wait),
// then the workgroup loads h with 16-byte loads, up to 8 per thread at once.
// Half the bytes of tagged words, and one batch of loads where 14336 tagged
// words take three.  h has its own slot per (step, layer) of the launch, so
// no cache holds a line of it before every producer has stored (caches start
// clean at launch) and the loads may go through the L2: the first workgroup
// of an XCD fetches each line, the other 31 hit.  issue() goes out first, as
// in stage().
template <typename F>
__device__ __forceinline__ bool stage_h(const MkArgs &a, float *xs, uint32_t n, uint32_t tag, uint32_t *s_fail,
                                        F &&issue, const float *hrow)
{
    constexpr int NB = 8;
    const uint32_t t = tid();
    issue();
    if (t < gridDim.x) {
        uint32_t spins = 0;
        while ((int)(ld_sys(a.hflag + t * 32) - tag) < 0) {
            if (++spins > (1u << 22) || ((spins & 15) == 0 && ld_sys(a.err) != 0)) {
                atomicOr(a.err, 1u);
                *s_fail = 1;
                break;
            }
        }
    }
    __syncthreads();
    if (*s_fail) return false;
    for (uint32_t j0 = 0; j0 < n; j0 += 4 * NB * MK_THREADS) {
        float4v v[NB];
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t j = j0 + 4 * (t + b * MK_THREADS);
            if (j < n)
                asm volatile("global_load_dwordx4 %0, %1, off" : "=v"(v[b]) : "v"(gptr(hrow) + j) : "memory");
        }
        asm volatile("s_waitcnt vmcnt(0)"
                     : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]), "+v"(v[7]));
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const uint32_t j = j0 + 4 * (t + b * MK_THREADS);
            if (j < n) *reinterpret_cast<float4v *>(xs + swz(j)) = v[b];     // 4 consecutive values stay adjacent
        }
    }
    __syncthreads();
    return true;
}

// ── GEMV phase ───────────────────────────────────────────────────────────────

// Rows of a phase per workgroup: an even count, so RoPE pairs stay together.
__host__ __device__ inline uint32_t mk_rows_per_wg(uint32_t n_rows, uint32_t n_wg)
{
    const uint32_t per = (n_rows + n_wg - 1) / n_wg;
    return (per + 1) & ~1u;
}

// Block pairs per column slice: the pairs of a row spread evenly over the
// waves (at most 64 per slice), rounded up to a multiple of qa.  Q4_K slices
// hold whole super-blocks (qa = 4 quarters): the four lanes of a lane quad then
// share one super-block, whose header they fetch a dword each.
__host__ __device__ inline uint32_t slice_pairs(uint32_t n_pairs, uint32_t qa, uint32_t qmin)
{
    uint32_t q = (n_pairs + MK_WAVES - 1) / MK_WAVES;
    if (q < qmin) q = qmin < n_pairs ? qmin : n_pairs;
    q = q < 1 ? 1 : q > 64 ? 64 : q;
    return (q + qa - 1) / qa * qa;
}

// Slice alignment of a weight type (see slice_pairs).
__host__ __device__ constexpr uint32_t q_align(uint32_t t) { return t == kQ4_K ? 4u : 1u; }

// Lanes per row group: the power of two that holds a slice's pairs.
__host__ __device__ inline uint32_t lanes_per_row(uint32_t q)
{
    uint32_t p = 1;
    while (p < q) p <<= 1;
    return p;
}

// Column slices of a row of n_cols values.
__host__ __device__ inline uint32_t n_slices(uint32_t n_cols, uint32_t qa, uint32_t qmin)
{
    const uint32_t np = n_cols / 64, q = slice_pairs(np, qa, qmin);
    return (np + q - 1) / q;
}

struct Map {
    uint32_t base;            // first row of this workgroup's share (partials are indexed from it)
    uint32_t lo, hi;          // rows of the share this call computes (a sub-range of it)
    uint32_t Q, P, S, R;      // pairs per slice, lanes per row (power of two >= Q), slices, rows per group
    uint32_t ps, rs;          // this lane's pair in the slice, row in the group
    uint32_t n_pairs;         // pairs per row
    // This wave's items, (slice, row group) pairs: from (s0, g0) the group
    // advances by gstep and at gend wraps to gstart on slice s + sstep; n_items in all.
    uint32_t s0, g0, gstart, gstep, gend, sstep, n_items;
};

// Items of a wave.  Slices that divide the waves: each slice's waves split
// its row groups (interleaved).  More slices than waves: each wave walks
// slices wave, wave + 8, ...  Otherwise (3, 5, 6 or 7 slices, e.g. 8B's
// ffn_down in 7): each wave takes an equal run of the (slice, group) items in
// slice order, so no wave has more than one item above the mean.
__device__ __forceinline__ Map plan(const MkGemv &g)
{
    Map m;
    const uint32_t n_rows = g.n_rows, n_cols = g.n_cols, qa = g.qa;
    const uint32_t per = mk_rows_per_wg(n_rows, gridDim.x);
    m.base = min(n_rows, blockIdx.x * per);
    m.lo = max(m.base, g.rlo);
    m.hi = max(m.lo, min(min(n_rows, m.base + per), g.rhi));
    m.n_pairs = n_cols / 64;
    m.Q = slice_pairs(m.n_pairs, qa, g.qmin);
    m.P = lanes_per_row(m.Q);
    m.R = 64 / m.P;
    m.S = (m.n_pairs + m.Q - 1) / m.Q;
    const uint32_t wave = wave_id(), lane = tid() & 63;
    m.ps = lane & (m.P - 1);
    m.rs = lane / m.P;
    const uint32_t n_groups = (m.hi - m.lo + m.R - 1) / m.R;
    if (m.S > (uint32_t)MK_WAVES) {
        m.s0 = wave; m.g0 = 0; m.gstart = 0; m.gstep = 1; m.gend = n_groups; m.sstep = MK_WAVES;
        m.n_items = (m.S - wave + MK_WAVES - 1) / MK_WAVES * n_groups;
    } else if (MK_WAVES % m.S == 0) {
        const uint32_t wis = wave / m.S, nws = MK_WAVES / m.S;
        const uint32_t n_my = wis < n_groups ? (n_groups - wis + nws - 1) / nws : 0;
        m.s0 = wave % m.S; m.g0 = wis; m.gstart = wis; m.gstep = nws; m.gend = wis + n_my * nws; m.sstep = MK_SMAX;
        m.n_items = n_my;
    } else {
        const uint32_t n = m.S * n_groups, j0 = wave * n / MK_WAVES, j1 = (wave + 1) * n / MK_WAVES;
        m.s0 = n_groups ? j0 / n_groups : 0; m.g0 = n_groups ? j0 % n_groups : 0;
        m.gstart = 0; m.gstep = 1; m.gend = n_groups; m.sstep = 1;
        m.n_items = j1 - j0;
    }
    return m;
}

__device__ __forceinline__ uint32_t map_row(const Map &m, uint32_t grp)
{
    return m.lo + grp * m.R + m.rs;
}

template <int M>
__device__ __forceinline__ const uint8_t *row_ptr(const MkGemv &g, uint32_t r, int mat)
{
    if constexpr (M == 2) {
        return g.w[mat] + (size_t)r * g.row_bytes;
    } else {
        const uint8_t *w = g.w[0];                           // constant indices only: g stays in registers
        if (r >= g.rows[0]) {
            r -= g.rows[0];
            w = g.w[1];
            if (r >= g.rows[1]) { r -= g.rows[1]; w = g.w[2]; }
        }
        return w + (size_t)r * g.row_bytes;
    }
}

// ── weight stream ────────────────────────────────────────────────────────────
//
// A wave's share of a phase is a sequence of items, one row group each: M
// block pairs per lane (M = 2 for gate and up together).  Items travel from
// HBM straight into the wave's ring of NS slots in LDS (global_load_lds: no
// registers are held while they are in flight).  When the wave consumes an
// item it reads the slot into registers and refills it with the item NS
// places further on, so NS - 1 items stay in flight while it reads and one
// while it computes.  NS is 1: every phase, the lm-head included, measured
// fastest with a single slot per wave (one item landing while one is
// summed); deeper rings only queued more loads ahead of the latency-bound
// staging and publishing of the next phase.
// Vector memory loads complete in order, so the wave waits for an item with
// s_waitcnt vmcnt((NS - 1) * D), D being the DMA instructions per item.  The
// compiler does not track LDS written by these DMAs, so these waits are
// explicit.  The first items of the next phase are issued right after a
// workgroup arrives at a barrier and land during the barrier and the staging.
//
// A lane's share of an item (a block pair, a Q4_K quarter or a repacked Q6_K
// quarter record) is moved in 16-byte pieces and one or two tails: Q4_0 36 =
// 16+16+4, Q5_0 44 = 16+16+12, Q8_0 68 = 4*16+4; Q4_K the quarter's 32 code
// bytes (16+16) and one dword of its super-block's header (the lane quad
// fetches the four); Q6_K records 56 = 16+16+12+12.  A piece of s bytes puts
// lane l's bytes at l*s in LDS for s = 4 and 16 and at l*16 for s = 12.

__host__ __device__ constexpr uint32_t dma_n16(uint32_t t) { return t == kQ8_0 ? 4u : 2u; }
__host__ __device__ constexpr uint32_t dma_tail(uint32_t t) { return t == kQ5_0 || t == kQ6_KR ? 12u : 4u; }
__host__ __device__ constexpr uint32_t dma_tail2(uint32_t t) { return t == kQ6_KR ? 12u : 0u; }
__host__ __device__ constexpr uint32_t dma_count(uint32_t t) { return dma_n16(t) + 1u + (dma_tail2(t) ? 1u : 0u); }
__host__ __device__ constexpr uint32_t dma_pair_lds(uint32_t t)
{
    return 64u * (16u * dma_n16(t) + (dma_tail(t) == 4u ? 4u : 16u) + (dma_tail2(t) ? 16u : 0u));
}
__host__ __device__ constexpr uint32_t slot_bytes(uint32_t t, uint32_t M) { return M * dma_pair_lds(t); }

constexpr uint32_t MK_NS_MAX = 1;           // ring slots per wave at most (see the weight stream notes)
constexpr uint32_t MK_QMIN_LAYER = 32;      // block pairs per column slice at least: layer phases
constexpr uint32_t MK_QMIN_HEAD = 64;       // and the lm-head (a whole row of up to 64 pairs)
constexpr uint32_t MK_VMCNT_MAX = 63;       // largest s_waitcnt vmcnt

// Ring slots of a wave for items of type t with M matrices, given its bytes.
__host__ __device__ inline uint32_t ring_slots(uint32_t wave_bytes, uint32_t t, uint32_t M)
{
    uint32_t ns = wave_bytes / slot_bytes(t, M);
    const uint32_t cap = MK_VMCNT_MAX / (dma_count(t) * M) + 1;
    if (ns > cap) ns = cap;
    return ns < MK_NS_MAX ? ns : MK_NS_MAX;
}

// First byte of the rings of a phase whose input has n_in values: above the
// staged input and above the attention scratch (the rings of the phase after
// attention fill while it runs).
__host__ __device__ inline uint32_t ring_base(uint32_t n_in, uint32_t attn_bytes)
{
    const uint32_t b = (4 * n_in + 15) & ~15u;
    return b > attn_bytes ? b : attn_bytes;
}

// Bytes of LDS per wave for the rings between `base` and the fixed region.
__host__ __device__ inline uint32_t ring_wave_bytes(uint32_t fixed, uint32_t base)
{
    return base >= fixed ? 0u : ((fixed - base) / MK_WAVES) & ~15u;
}

struct Ring {
    uint8_t *base;            // this wave's slots
    uint32_t ns;              // slot count
};

template <uint32_t T, int M>
__device__ __forceinline__ Ring ring_of(uint8_t *lds, uint32_t fixed, uint32_t attn_bytes, uint32_t n_in)
{
    const uint32_t base = ring_base(n_in, attn_bytes), wb = ring_wave_bytes(fixed, base);
    Ring r;
    r.base = lds + base + wave_id() * wb;
    r.ns = ring_slots(wb, T, M);
    return r;
}

// Position of an item: slice index among the wave's slices, row group in the
// slice, ring slot.
struct Cur {
    uint32_t s, g, slot;      // slice, row group, ring slot of an item
};

__device__ __forceinline__ Cur cur0(const Map &m) { return Cur{m.s0, m.g0, 0}; }
__device__ __forceinline__ void advance(Cur &c, const Map &m, uint32_t ns)
{
    c.g += m.gstep;
    if (c.g >= m.gend) { c.g = m.gstart; c.s += m.sstep; }
    if (++c.slot == ns) c.slot = 0;
}

typedef __attribute__((address_space(3))) void lds_void;

// One LDS-DMA load of BYTES per lane (global_load_lds): lane i's bytes land at
// LDS byte lds + BYTES * i.  Issued through inline asm: the compiler treats
// the builtin's address registers as busy until the load completes and waits
// for every load in flight before reusing them, which serialises a ring fill.
// The ring's waits are explicit (wait_items), so nothing depends on the
// compiler's accounting.  M0 (reserved by the compiler) is saved and
// restored; it is written one instruction ahead of the load that reads it.
#define FW_DMA_LDS(INSN)                                                                                 \
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\t" INSN " %1, off\n\ts_mov_b32 m0, %0" \
                 : "=&s"(keep)                                                                            \
                 : "v"(src), "s"(m)                                                                       \
                 : "memory")
template <int BYTES>
__device__ __forceinline__ void dma_lds(const FW_GLOBAL uint8_t *src, uint8_t *lds)
{
    const uint32_t m = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds_void *)lds);
    uint32_t keep;
    if constexpr (BYTES == 16) FW_DMA_LDS("global_load_lds_dwordx4");
    else if constexpr (BYTES == 12) FW_DMA_LDS("global_load_lds_dwordx3");
    else FW_DMA_LDS("global_load_lds_dword");
}
#undef FW_DMA_LDS

// Lane's share of pair `pair` of a row into an item slot at dst.
template <uint32_t T>
__device__ __forceinline__ void dma_pair(const uint8_t *row, uint32_t pair, uint8_t *dst)
{
    if constexpr (T == kQ4_K) {
        // quarter pair & 3 of super-block pair / 4: codes at 16 + 32 * quarter, and
        // header dword (lane & 3): the quad's lanes hold one super-block's quarters
        const FW_GLOBAL uint8_t *sb = gptr(row) + (size_t)(pair >> 2) * 144;
        dma_lds<16>(sb + 16 + 32 * (pair & 3), dst);
        dma_lds<16>(sb + 32 + 32 * (pair & 3), dst + 1024);
        dma_lds<4>(sb + 4 * (tid() & 3), dst + 2048);
    } else if constexpr (T == kQ6_KR) {
        const FW_GLOBAL uint8_t *s = gptr(row) + (size_t)pair * 56;
        dma_lds<16>(s, dst);
        dma_lds<16>(s + 16, dst + 1024);
        dma_lds<12>(s + 32, dst + 2048);
        dma_lds<12>(s + 44, dst + 3072);
    } else {
        const FW_GLOBAL uint8_t *s = gptr(row) + (size_t)pair * (2 * Blk<T>::bytes);
#pragma unroll
        for (uint32_t i = 0; i < dma_n16(T); i++) dma_lds<16>(s + 16 * i, dst + 1024 * i);
        dma_lds<(int)dma_tail(T)>(s + 16 * dma_n16(T), dst + 1024 * dma_n16(T));
    }
}

// Issue item c.  Every load is issued: a row past the workgroup's last one and
// a pair past the row's end are clamped to the last valid one (results of
// such lanes are dropped), so every item counts D loads.
template <uint32_t T, int M>
__device__ __forceinline__ void dma_item(const MkGemv &g, const Map &m, const Cur &c, uint8_t *ring)
{
    const uint32_t pair = min(c.s * m.Q + min(m.ps, m.Q - 1), m.n_pairs - 1);   // lanes past Q reload the last
    const uint32_t r = min(map_row(m, c.g), m.hi - 1);
    uint8_t *slot = ring + c.slot * slot_bytes(T, M);
#pragma unroll
    for (int mat = 0; mat < M; mat++)
        dma_pair<T>(row_ptr<M>(g, r, mat), pair, slot + mat * dma_pair_lds(T));
}

template <uint32_t T, int M>
__device__ __forceinline__ void read_item(const uint8_t *slot, uint32_t (&dw)[M][Blk<T>::pair_dw])
{
    const uint32_t lane = tid() & 63;
#pragma unroll
    for (int mat = 0; mat < M; mat++) {
        const uint8_t *p = slot + mat * dma_pair_lds(T);
#pragma unroll
        for (uint32_t i = 0; i < dma_n16(T); i++) {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(p + 1024 * i + 16 * lane);
            dw[mat][4 * i] = v.x; dw[mat][4 * i + 1] = v.y; dw[mat][4 * i + 2] = v.z; dw[mat][4 * i + 3] = v.w;
        }
        const uint8_t *t = p + 1024 * dma_n16(T);
        if constexpr (T == kQ4_K) {
            // the quad's four header dwords, side by side
            const u32x4 v = *reinterpret_cast<const u32x4 *>(t + 16 * (lane >> 2));
            dw[mat][8] = v.x; dw[mat][9] = v.y; dw[mat][10] = v.z; dw[mat][11] = v.w;
        } else if constexpr (dma_tail(T) == 4) {
            dw[mat][4 * dma_n16(T)] = *reinterpret_cast<const uint32_t *>(t + 4 * lane);
        } else {
            const u32x4 v = *reinterpret_cast<const u32x4 *>(t + 16 * lane);
            dw[mat][8] = v.x; dw[mat][9] = v.y; dw[mat][10] = v.z;
            if constexpr (dma_tail2(T) != 0) {
                const u32x4 w = *reinterpret_cast<const u32x4 *>(t + 1024 + 16 * lane);
                dw[mat][11] = w.x; dw[mat][12] = w.y; dw[mat][13] = w.z;
            }
        }
    }
}

template <int N>
__device__ __forceinline__ void vmcnt_le()
{
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Wait until at most k items of D loads each are outstanding ((k * D) <= 63
// for every k the ring geometry allows; larger k wait for everything).
template <int D>
__device__ __forceinline__ void wait_items(uint32_t k)
{
#define MK_W(K) case K: vmcnt_le<((K) * D <= (int)MK_VMCNT_MAX ? (K) * D : 0)>(); break;
    switch (k) {
    MK_W(1) MK_W(2) MK_W(3) MK_W(4) MK_W(5) MK_W(6) MK_W(7) MK_W(8) MK_W(9) MK_W(10) MK_W(11)
    default: vmcnt_le<0>(); break;
    }
#undef MK_W
}

// The 64 input values of the lane's pair in slice sl (zero past the row) and,
// for the offset formats, their sums over the blocks (Q4_0, Q5_0) or scale
// groups (Q4_K: two of 32 values; Q6_K: four of 16).
template <uint32_t T>
__device__ __forceinline__ void load_x(const float *xs, const Map &m, uint32_t sl, float (&xv)[64], float (&sx)[4])
{
    const uint32_t pair = sl * m.Q + m.ps;
    sx[0] = sx[1] = sx[2] = sx[3] = 0.f;
    if (m.ps < m.Q && pair < m.n_pairs) {
        // Read through inline asm: for compiler-visible LDS reads the compiler
        // cannot tell xs from the weight rings and first waits for every DMA
        // in flight (the prefetched items of this phase).
        const uint32_t base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) float *)(xs + 64 * (size_t)pair);
        uint32_t ad[16];
#pragma unroll
        for (int i = 0; i < 16; i++) ad[i] = base + (((i + pair) & 15u) << 4);
        float4v r[16];
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
        if constexpr (T == kQ6_KR) {
#pragma unroll
            for (int g = 0; g < 4; g++) {
                float s0 = 0.f, s1 = 0.f;
#pragma unroll
                for (int i = 0; i < 16; i += 2) { s0 += xv[16 * g + i]; s1 += xv[16 * g + i + 1]; }
                sx[g] = s0 + s1;
            }
        } else if constexpr (T != kQ8_0) {
            float s0 = 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i += 2) { s0 += xv[i]; s1 += xv[i + 1]; s2 += xv[32 + i]; s3 += xv[33 + i]; }
            sx[0] = s0 + s1;
            sx[1] = s2 + s3;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 64; i++) xv[i] = 0.f;
    }
}

// Issue the first items of g into its ring (before the barrier that precedes
// the phase); returns how many were issued.
template <uint32_t T, int M>
__device__ __forceinline__ uint32_t prefetch(const MkGemv &g, uint8_t *lds, uint32_t fixed, uint32_t attn_bytes)
{
    const Map m = plan(g);
    const Ring rg = ring_of<T, M>(lds, fixed, attn_bytes, g.n_cols);
    const uint32_t n = min(min(rg.ns, MK_PF), m.n_items);
    Cur c = cur0(m);
    for (uint32_t i = 0; i < n; i++) {
        dma_item<T, M>(g, m, c, rg.base);
        advance(c, m, rg.ns);
    }
    return n;
}

// Dot of one item's dwords with the lane's 64 input values.
template <uint32_t T>
__device__ __forceinline__ float item_dot(const uint32_t *dw, const float (&xv)[64], const float (&sx)[4], uint32_t q)
{
    if constexpr (T == kQ4_K) return dot_q4k_item(dw, xv, sx[0], sx[1], q);
    else if constexpr (T == kQ6_KR) return dot_q6kr(dw, xv, sx);
    else return dot_pair<T>(dw, xv, sx[0], sx[1]);
}

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Sum over each aligned group of P lanes (P a power of two, wave-uniform); the
// group's first lane (at least) ends with the sum.  DPP quad permutes give
// the sums of 2 and 4 lanes; once the 4-lane groups hold equal values, adding
// the half-row mirror (lane 7 - i) and row mirror (lane 15 - i) gives those of
// 8 and 16; a swizzle and a permute give 32 and 64.
template <int M>
__device__ __forceinline__ void lane_sum(float (&v)[M], uint32_t P)
{
    if (P >= 2) {
#pragma unroll
        for (int i = 0; i < M; i++) v[i] += dpp<0xB1>(v[i]);                 // quad_perm 1,0,3,2
    }
    if (P >= 4) {
#pragma unroll
        for (int i = 0; i < M; i++) v[i] += dpp<0x4E>(v[i]);                 // quad_perm 2,3,0,1
    }
    if (P >= 8) {
#pragma unroll
        for (int i = 0; i < M; i++) v[i] += dpp<0x141>(v[i]);                // row_half_mirror
    }
    if (P >= 16) {
#pragma unroll
        for (int i = 0; i < M; i++) v[i] += dpp<0x140>(v[i]);                // row_mirror
    }
    if (P >= 32) {
#pragma unroll
        for (int i = 0; i < M; i++) {                                        // lane ^ 16: rows 0+1, 2+3
            const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i]), false, false);
            v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);             // (gfx950 permlane swap, no LDS)
        }
    }
    if (P >= 64) {
#pragma unroll
        for (int i = 0; i < M; i++) v[i] += __shfl_xor(v[i], 32, 64);
    }
}

// This workgroup's rows of g: part[(row_local*M + matrix)*S + slice].  The
// first n_pre items of this wave are in flight already.
template <uint32_t T, int M>
__device__ __forceinline__ void gemv(const MkGemv &g, const float *xs, float *part, uint8_t *lds, uint32_t fixed,
                                     uint32_t attn_bytes, uint32_t n_pre)
{
    constexpr int D = (int)dma_count(T) * M, NDW = Blk<T>::pair_dw;
    const Map m = plan(g);
    const Ring rg = ring_of<T, M>(lds, fixed, attn_bytes, g.n_cols);
    const uint32_t n_items = m.n_items;
    Cur is = cur0(m);
    for (uint32_t i = 0; i < n_pre; i++) advance(is, m, rg.ns);
    for (uint32_t i = n_pre; i < min(rg.ns, n_items); i++) {
        dma_item<T, M>(g, m, is, rg.base);
        advance(is, m, rg.ns);
    }
    uint32_t slot = 0, sl = ~0u;
    const uint32_t lane_q = tid() & 3;                           // Q4_K: the lane's quarter of its super-block
    float xv[64], sx[4];
    bool pair_on = false;
    Cur cc = cur0(m);
    for (uint32_t it = 0; it < n_items; it++) {
        if (cc.s != sl) {                                        // a new slice: its input values
            sl = cc.s;
            load_x<T>(xs, m, sl, xv, sx);
            pair_on = m.ps < m.Q && sl * m.Q + m.ps < m.n_pairs;
        }
        wait_items<D>(it + rg.ns <= n_items ? rg.ns - 1 : 0);
        uint32_t dw[M][NDW];
        read_item<T, M>(rg.base + slot * slot_bytes(T, M), dw);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");      // the slot is free again
        if (it + rg.ns < n_items) {
            dma_item<T, M>(g, m, is, rg.base);
            advance(is, m, rg.ns);
        }
        if (++slot == rg.ns) slot = 0;
        const uint32_t r = map_row(m, cc.g);
        const bool on = pair_on && r < m.hi;
        float acc[M];
#pragma unroll
        for (int mat = 0; mat < M; mat++) {
            acc[mat] = item_dot<T>(dw[mat], xv, sx, lane_q);
            if (!on) acc[mat] = 0.f;
        }
        lane_sum<M>(acc, m.P);
#pragma unroll
        for (int mat = 0; mat < M; mat++)
            if (m.ps == 0 && r < m.hi) part[((r - m.base) * M + mat) * m.S + sl] = acc[mat];
        advance(cc, m, 1);
    }
    __syncthreads();
}

template <int M>
__device__ __forceinline__ float row_sum(const float *part, uint32_t rl, int mat, uint32_t n_slices)
{
    float y = 0.f;
    for (uint32_t s = 0; s < n_slices; s++) y += part[(rl * M + mat) * n_slices + s];
    return y;
}

__device__ __forceinline__ void wg_rows(uint32_t n_rows, uint32_t &lo, uint32_t &hi)
{
    const uint32_t per = mk_rows_per_wg(n_rows, gridDim.x);
    lo = min(n_rows, blockIdx.x * per);
    hi = min(n_rows, lo + per);
}

// ── epilogues ────────────────────────────────────────────────────────────────

// Bias (linear.c:214-221; bias null when the model has none), RoPE on q/k rows
// (rope.c:37-43) with this position's cos/sin (rope[0..hd/2) and rope[hd/2..hd)
// in LDS), K/V append at pos (attention.c:129-140).  q and the new K/V row are
// also published as words tagged `tag` for this step's attention.
__device__ __forceinline__ void epi_qkv(const MkArgs &a, const MkGemv &g, const float *part, const float *rope,
                                        const float *bias, uint32_t layer, uint32_t pos, uint32_t tag, float nscale)
{
    uint32_t lo, hi;
    wg_rows(g.n_rows, lo, hi);
    const uint32_t ns = n_slices(g.n_cols, g.qa, g.qmin), hd = a.head_dim, half = hd / 2;
    const uint32_t kvd = a.n_kv * hd, nq = g.rows[0];
    for (uint32_t rl = 2 * tid(); rl < hi - lo; rl += 2 * MK_THREADS) {
        const uint32_t r = lo + rl;
        float v0 = row_sum<1>(part, rl, 0, ns) * nscale, v1 = row_sum<1>(part, rl + 1, 0, ns) * nscale;
        if (bias) {
            v0 += bias[r];
            v1 += bias[r + 1];
        }
        if (r < nq + kvd) {
            const uint32_t i = ((r < nq ? r : r - nq) % hd) / 2;
            const float c = rope[i], s = rope[half + i];
            const float w0 = v0 * c - v1 * s, w1 = v0 * s + v1 * c;
            v0 = w0;
            v1 = w1;
        }
        uint64_t *tdst;
        if (r < nq) {
            tdst = a.tq + r;
        } else {
            float *dst = r < nq + kvd ? a.kc + ((size_t)layer * a.n_ctx + pos) * kvd + (r - nq)
                                      : a.vc + ((size_t)layer * a.n_ctx + pos) * kvd + (r - nq - kvd);
            st_sys(dst, v0);
            st_sys(dst + 1, v1);
            tdst = a.tkv + (r - nq);
        }
        st_sys64(tdst, tagged(v0, tag));
        st_sys64(tdst + 1, tagged(v1, tag));
    }
}

// x[i] += y[i] (transformer.c:271-272, 287-288) on this workgroup's rows: the
// workgroup keeps its own rows of x in LDS (x_own), publishes the sums and
// records the trace row.
__device__ __forceinline__ void epi_resid(const MkArgs &a, const MkGemv &g, const float *part, float *x_own,
                                          float *trace_row, uint32_t tag)
{
    uint32_t lo, hi;
    wg_rows(g.n_rows, lo, hi);
    const uint32_t ns = n_slices(g.n_cols, g.qa, g.qmin);
    for (uint32_t rl = tid(); rl < hi - lo; rl += MK_THREADS) {
        const uint32_t r = lo + rl;
        const float v = x_own[rl] + row_sum<1>(part, rl, 0, ns);
        x_own[rl] = v;
        st_sys64(a.tx + r, tagged(v, tag));
        st_sys(trace_row + r, v);
    }
}

// apply_silu (ffn.c:17-25) with the reference's two branches, in float
// arithmetic (expf, within an ulp or two of the correctly rounded value).
__device__ __forceinline__ float silu_f(float v)
{
    float sig;
    if (v >= 0.0f) sig = 1.0f / (1.0f + expf(-v));
    else { const float e = expf(v); sig = e / (1.0f + e); }
    return v * sig;
}

// h = act(gate x) * (up x) (ffn.c:82-104): silu, or a GELU form.
__device__ __forceinline__ void epi_swiglu(const MkArgs &a, const MkGemv &g, const float *part, uint32_t tag,
                                           float nscale, float *hrow)
{
    uint32_t lo, hi;
    wg_rows(g.n_rows, lo, hi);
    const uint32_t ns = n_slices(g.n_cols, g.qa, g.qmin);
    for (uint32_t rl = tid(); rl < hi - lo; rl += MK_THREADS) {
        const float gv = row_sum<2>(part, rl, 0, ns) * nscale;
        const float av = a.act == ACT_SILU ? silu_f(gv) : a.act == ACT_GELU ? gelu_erf(gv) : gelu_tanh(gv);
        st_sys(hrow + lo + rl, av * (row_sum<2>(part, rl, 1, ns) * nscale));
    }
    wait_mem();                                   // this wave's rows are stored
    __syncthreads();
    if (tid() == 0) st_sys(a.hflag + blockIdx.x * 32, tag);
}

__device__ __forceinline__ bool am_better_mk(float v1, uint32_t i1, float v2, uint32_t i2)
{
    if (i1 == 0xffffffffu) return false;
    if (i2 == 0xffffffffu) return true;
    return v1 > v2 || (v1 == v2 && i1 < i2);
}

// Best (value, index) of the workgroup, valid in thread 0.
__device__ __forceinline__ void block_best(float &bv, uint32_t &bi, float *s_v, uint32_t *s_i)
{
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
        const float ov = __shfl_xor(bv, m, 64);
        const uint32_t oi = __shfl_xor(bi, m, 64);
        if (am_better_mk(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = tid() & 63, wave = wave_id();
    __syncthreads();
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (tid() == 0)
        for (int w = 1; w < MK_WAVES; w++)
            if (am_better_mk(s_v[w], s_i[w], bv, bi)) { bv = s_v[w]; bi = s_i[w]; }
}

// Logits of this workgroup's rows, their best candidate, and the winner picked
// by the last workgroup to arrive (sampler_argmax, sampler.c:28-32: the first
// maximum; NaN never wins; NaN at index 0 makes index 0 the answer), which also
// advances the device-resident greedy loop (main.c:173-217).
__device__ __forceinline__ void epi_head(const MkArgs &a, const MkGemv &g, const float *part, uint32_t pos,
                                         uint32_t greedy, uint32_t n_prompt, float nscale)
{
    __shared__ float s_v[MK_WAVES];
    __shared__ uint32_t s_i[MK_WAVES];
    __shared__ uint32_t s_last;
    uint32_t lo, hi;
    wg_rows(g.n_rows, lo, hi);
    const uint32_t ns = n_slices(g.n_cols, g.qa, g.qmin);
    float bv = -INFINITY;
    uint32_t bi = 0xffffffffu;
    for (uint32_t rl = tid(); rl < hi - lo; rl += MK_THREADS) {
        const float y = row_sum<1>(part, rl, 0, ns) * nscale;
        st_sys(a.logits + lo + rl, y);
        if (!isnan(y) && (bi == 0xffffffffu || y > bv)) { bv = y; bi = lo + rl; }
    }
    wait_mem();
    block_best(bv, bi, s_v, s_i);
    if (tid() == 0) {
        st_sys(a.am_v + blockIdx.x, bv);
        st_sys(a.am_i + blockIdx.x, bi);
        wait_mem();
        s_last = ticket_sys(a.tickets) == gridDim.x - 1;
    }
    __syncthreads();
    if (!s_last) return;
    bv = -INFINITY;
    bi = 0xffffffffu;
    for (uint32_t w = tid(); w < gridDim.x; w += MK_THREADS) {
        const float v = ld_sys(a.am_v + w);
        const uint32_t i = ld_sys(a.am_i + w);
        if (am_better_mk(v, i, bv, bi)) { bv = v; bi = i; }
    }
    block_best(bv, bi, s_v, s_i);
    if (tid() == 0) {
        const uint32_t r = (bi == 0xffffffffu || isnan(ld_sys(a.logits))) ? 0u : bi;
        st_sys(a.argmax_out, r);
        st_sys(&a.state->next, r);
        if (greedy) {
            if (pos + 1 >= n_prompt) st_sys(a.ids + (pos + 1 - n_prompt), r);
            st_sys(&a.state->token, pos + 1 < n_prompt ? a.prompt[pos + 1] : r);
            st_sys(&a.state->pos, pos + 1);
        }
        st_sys(a.tickets, 0u);
    }
}

// ── attention ────────────────────────────────────────────────────────────────

template <int EPL>
__device__ __forceinline__ void load_vec(const FW_GLOBAL float *p, float (&v)[EPL])
{
    if constexpr (EPL == 1) {
        v[0] = *p;
    } else if constexpr (EPL == 2) {
        const float2v t = *reinterpret_cast<const FW_GLOBAL float2v *>(p);
        v[0] = t[0]; v[1] = t[1];
    } else {
        const float4v t = *reinterpret_cast<const FW_GLOBAL float4v *>(p);
        v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
    }
}

// Splits of the positions 0..pos per KV head in this step: about one per 64
// positions, at most the n_splits the partial buffer holds.  Short contexts
// then have fewer, longer items and a cheaper combine.
// Query-head grouping of attention at position pos: half-size sub-groups
// (more, shorter items; each K/V row read by two units) while the K/V rows are
// few, the full sub-group (each row read once per KV head) from
// a.attn_long_pos on, where attention becomes bound by its K/V bytes.  Unit u
// is KV head u % n_kv, sub-group u / n_kv: the items of one KV head's units
// (item = split * units + u) are n_kv workgroups apart, on the same XCD when
// n_kv is a multiple of 8 (workgroups go to the eight XCDs round-robin), so
// the second unit's K/V reads can hit that XCD's L2.
struct AttnGrp {
    uint32_t gs, units, max_splits;
};
__device__ __forceinline__ AttnGrp attn_grp(const MkArgs &a, uint32_t pos)
{
    return pos < a.attn_long_pos ? AttnGrp{a.attn_gs_short, a.attn_units_short, a.n_splits_short}
                                 : AttnGrp{a.attn_gs, a.attn_units, a.n_splits};
}

__device__ __forceinline__ uint32_t attn_splits_at(const MkArgs &a, uint32_t pos)
{
    const uint32_t want = (pos + 64) / 64;
    const uint32_t cap = attn_grp(a, pos).max_splits;
    return want > cap ? cap : want;
}

// Waits until the tagged words w[k] (k with bit k of `valid`; the others are
// left as fresh) carry `tag`: all are loaded at once, the stale ones again in
// rounds with a back-off.  Returns false when the wait gives up or another
// workgroup has failed; the error word is then set.
template <int N, typename F>
__device__ __forceinline__ bool load_tagged(const MkArgs &a, uint64_t (&w)[N], uint64_t valid, uint32_t tag, F &&addr)
{
#pragma unroll
    for (int k = 0; k < N; k++) w[k] = (valid >> k) & 1u ? ld_sys64(addr(k)) : (uint64_t)tag << 32;
    static_assert(N <= 64, "one mask bit per word");
    uint64_t stale = 0;
#pragma unroll
    for (int k = 0; k < N; k++)
        if ((uint32_t)(w[k] >> 32) != tag) stale |= 1ull << k;
    for (uint32_t round = 0; stale; round++) {
        __builtin_amdgcn_s_sleep(8);                               // ~512 cycles
        if (round > (1u << 16) || ((round & 15) == 15 && ld_sys(a.err) != 0)) {
            atomicOr(a.err, 1u);
            return false;
        }
#pragma unroll
        for (int k = 0; k < N; k++)
            if ((stale >> k) & 1u) w[k] = ld_sys64(addr(k));
#pragma unroll
        for (int k = 0; k < N; k++)
            if (((stale >> k) & 1u) && (uint32_t)(w[k] >> 32) == tag) stale &= ~(1ull << k);
    }
    return true;
}

__device__ __forceinline__ float untag(uint64_t w) { return __builtin_bit_cast(float, (uint32_t)w); }

// 2^v by the hardware instruction (v_exp_f32): 2^-inf = 0; results below the
// normal range (weights under 2^-126 of the running maximum) may flush to 0.
__device__ __forceinline__ float ex2(float v) { return __builtin_amdgcn_exp2f(v); }

// One (KV head, split) item: online softmax (log2 domain) over the split's
// positions for the G query heads of the group (attention.c:142-164); partial
// (o[HD], m, l) per query head to a.tpart as words tagged `tag`.  A position
// is spread over 32 lanes (EPL = HD/32 dimensions each), so a wave walks two
// positions at a time, U per batch (positions past t1 reload the batch's
// first one and get no weight).
// The K/V rows below pos were written in earlier steps, so the first batch of
// them is loaded before the query; q and the K/V row of pos come from the QKV
// phase as words tagged `tin` and are polled.  Row pos is never read from the
// cache in this step: a plain load racing its write would leave a stale line
// in this XCD's L2 for later steps.
template <int EPL, int G, int U>
__device__ __forceinline__ bool attn_item(const MkArgs &a, uint32_t layer, uint32_t pos, uint32_t unit, uint32_t split,
                                          float *lds, uint32_t tin, uint32_t tag)
{
    constexpr uint32_t NG = 2 * MK_WAVES;                  // position streams of the workgroup
    constexpr int HD = 32 * EPL;
    const uint32_t kvh = unit % a.n_kv;                    // units: (sub-group, KV head), KV head fastest
    const uint32_t h0 = kvh * (a.n_head / a.n_kv) + (unit / a.n_kv) * G;    // first query head of the unit
    float (*s_o)[G][HD] = reinterpret_cast<float (*)[G][HD]>(lds);
    float (*s_m)[G] = reinterpret_cast<float (*)[G]>(lds + MK_WAVES * G * HD);
    float (*s_l)[G] = reinterpret_cast<float (*)[G]>(lds + MK_WAVES * G * HD + MK_WAVES * G);
    const uint32_t n_pos = pos + 1, ns = attn_splits_at(a, pos), chunk = (n_pos + ns - 1) / ns;
    const uint32_t t0 = split * chunk, t1 = min(n_pos, t0 + chunk);
    const bool has_pos = t1 == n_pos;                      // the split ends with the new position
    const int lane = tid() & 63, wave = wave_id(), l32 = lane & 31;
    const size_t kvd = (size_t)a.n_kv * HD;
    const FW_GLOBAL float *kc = gptr(a.kc) + (size_t)layer * a.n_ctx * kvd + kvh * HD + l32 * EPL;
    const FW_GLOBAL float *vc = gptr(a.vc) + (size_t)layer * a.n_ctx * kvd + kvh * HD + l32 * EPL;
    const float sc = (1.0f / sqrtf((float)HD)) * 1.4426950408889634f;     // attention.c:143, in log2 units
    // Each 32-lane group walks positions first, first + NG, ...
    const uint32_t first = t0 + wave * 2 + (lane >> 5);
    auto at = [&](uint32_t tb, int u) { return tb + u * NG < t1 ? tb + u * NG : tb; };
    float kk[U][EPL], vv[U][EPL];
    auto load = [&](uint32_t tb) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t t = at(tb, u);
            if (t != pos) {
                load_vec<EPL>(kc + (size_t)t * kvd, kk[u]);
                load_vec<EPL>(vc + (size_t)t * kvd, vv[u]);
            }
        }
    };
    if (first < t1) load(first);

    // q (G * HD words) and, for the split holding pos, its K then V row (HD
    // each) through LDS: every thread polls up to three words.
    float qv[G][EPL], kn[EPL], vn[EPL];
    bool ok;
    {
        constexpr uint32_t NQ = G * HD;
        const uint32_t nw = has_pos ? NQ + 2 * HD : NQ, t = tid();
        static_assert(NQ + 2 * HD <= 3 * MK_THREADS, "three words per thread");
        uint64_t w[3];
        auto word = [&](uint32_t j) {
            return j < NQ ? a.tq + (size_t)h0 * HD + j : a.tkv + (j - NQ >= HD ? kvd : 0) + kvh * HD + (j - NQ) % HD;
        };
        ok = load_tagged<3>(a, w, (t < nw ? 1u : 0u) | (t + MK_THREADS < nw ? 2u : 0u) | (t + 2 * MK_THREADS < nw ? 4u : 0u),
                            tin, [&](int k) { return word(t + k * MK_THREADS); });
#pragma unroll
        for (int k = 0; k < 3; k++)
            if (t + k * MK_THREADS < nw) lds[t + k * MK_THREADS] = untag(w[k]);
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; g++)
#pragma unroll
            for (int e = 0; e < EPL; e++) qv[g][e] = lds[g * HD + l32 * EPL + e];
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            kn[e] = has_pos ? lds[NQ + l32 * EPL + e] : 0.f;
            vn[e] = has_pos ? lds[NQ + HD + l32 * EPL + e] : 0.f;
        }
    }

    float m[G], l[G], o[G][EPL];
#pragma unroll
    for (int g = 0; g < G; g++) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < EPL; e++) o[g][e] = 0.f;
    }
    for (uint32_t tb = first; tb < t1; tb += U * NG) {
        if (tb != first) load(tb);
        if (has_pos) {
#pragma unroll
            for (int u = 0; u < U; u++)
                if (at(tb, u) == pos) {
#pragma unroll
                    for (int e = 0; e < EPL; e++) {
                        kk[u][e] = kn[e];
                        vv[u][e] = vn[e];
                    }
                }
        }
        float s[U][G];
#pragma unroll
        for (int u = 0; u < U; u++)
#pragma unroll
            for (int g = 0; g < G; g++) {
                float d = 0.f;
#pragma unroll
                for (int e = 0; e < EPL; e++) d = __builtin_fmaf(qv[g][e], kk[u][e], d);
                s[u][g] = d;
            }
#pragma unroll
        for (int u = 0; u < U; u++) lane_sum<G>(s[u], 32);          // every lane of the group gets the sum
#pragma unroll
        for (int g = 0; g < G; g++) {
            float mx = m[g];
#pragma unroll
            for (int u = 0; u < U; u++) {
                s[u][g] = tb + u * NG < t1 ? s[u][g] * sc : -INFINITY;
                mx = fmaxf(mx, s[u][g]);                     // finite: position tb is below t1
            }
            const float c = ex2(m[g] - mx);
            l[g] *= c;
#pragma unroll
            for (int e = 0; e < EPL; e++) o[g][e] *= c;
#pragma unroll
            for (int u = 0; u < U; u++) {
                const float pe = ex2(s[u][g] - mx);
                l[g] += pe;
#pragma unroll
                for (int e = 0; e < EPL; e++) o[g][e] = __builtin_fmaf(pe, vv[u][e], o[g][e]);
            }
            m[g] = mx;
        }
    }
#pragma unroll
    for (int g = 0; g < G; g++) {                          // merge the wave's two position groups
        const float mw = fmaxf(m[g], __shfl_xor(m[g], 32, 64));
        const float c = mw == -INFINITY ? 0.f : ex2(m[g] - mw);
        float lw = l[g] * c;
        lw += __shfl_xor(lw, 32, 64);
#pragma unroll
        for (int e = 0; e < EPL; e++) {
            float ov = o[g][e] * c;
            ov += __shfl_xor(ov, 32, 64);
            o[g][e] = ov;
        }
        m[g] = mw;
        l[g] = lw;
    }
    __syncthreads();                                       // LDS is free (q, previous item)
    if (lane < 32) {
#pragma unroll
        for (int g = 0; g < G; g++) {
#pragma unroll
            for (int e = 0; e < EPL; e++) s_o[wave][g][l32 * EPL + e] = o[g][e];
            if (lane == 0) { s_m[wave][g] = m[g]; s_l[wave][g] = l[g]; }
        }
    }
    __syncthreads();
    for (int i = tid(); i < G * HD; i += MK_THREADS) {   // merge the eight waves
        const int g = i / HD, dd = i % HD;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < MK_WAVES; w++) M = fmaxf(M, s_m[w][g]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < MK_WAVES; w++) {
            const float c = M == -INFINITY ? 0.f : ex2(s_m[w][g] - M);
            L = __builtin_fmaf(s_l[w][g], c, L);
            O = __builtin_fmaf(s_o[w][g][dd], c, O);
        }
        uint64_t *pp = a.tpart + ((size_t)(h0 + g) * ns + split) * (HD + 2);
        st_sys64(pp + dd, tagged(O, tag));
        if (dd == 0) {
            st_sys64(pp + HD, tagged(M, tag));
            st_sys64(pp + HD + 1, tagged(L, tag));
        }
    }
    __syncthreads();
    return ok;
}

// Merge the splits of a unit's G query heads into a.tatt (tagged): each thread
// polls the o values of its (head, dimension) for up to SB splits at once and
// the first G * ns threads also the (m, l) words, which go to LDS for the split
// weights; then O = sum over splits of o * w in split order, divided by the
// weighted sum of the l.
template <int EPL, int G>
__device__ __forceinline__ bool attn_combine(const MkArgs &a, uint32_t unit, float *lds, uint32_t tag, uint32_t pos)
{
    constexpr int HD = 32 * EPL, SB = 16;
    const uint32_t ns = attn_splits_at(a, pos);
    const uint32_t h0 = (unit % a.n_kv) * (a.n_head / a.n_kv) + (unit / a.n_kv) * G;
    float *s_w = lds;                                      // [G][ns] m, then the split weights
    float *s_l = lds + G * ns;                             // [G][ns] l
    float *s_inv = lds + 2 * G * ns;                       // [G] 1 / sum of weights
    const uint64_t *base = a.tpart + (size_t)h0 * ns * (HD + 2);  // (head h0+g, split s) at (g*ns + s)*(HD+2)
    const uint32_t t = tid(), nb = ns < (uint32_t)SB ? ns : (uint32_t)SB;
    uint64_t w[SB + 2];
    bool ok = true;
    {
        const uint32_t g = t / HD, d = t % HD;
        uint64_t valid = 0;
        if (t < (uint32_t)(G * HD)) valid |= (1ull << nb) - 1u;
        if (t < G * ns) valid |= 3ull << SB;
        ok = load_tagged<SB + 2>(a, w, valid, tag, [&](int k) {
            return k < SB ? base + ((size_t)g * ns + k) * (HD + 2) + d : base + (size_t)t * (HD + 2) + HD + (k - SB);
        });
        if (t < G * ns) {
            s_w[t] = untag(w[SB]);
            s_l[t] = untag(w[SB + 1]);
        }
        for (uint32_t j = t + MK_THREADS; j < G * ns; j += MK_THREADS) {     // more than one (m, l) per thread
            uint64_t ml[2];
            ok = load_tagged<2>(a, ml, 3ull, tag, [&](int k) { return base + (size_t)j * (HD + 2) + HD + k; }) && ok;
            s_w[j] = untag(ml[0]);
            s_l[j] = untag(ml[1]);
        }
    }
    __syncthreads();
    const int lane = t & 63;
    for (uint32_t g = wave_id(); g < (uint32_t)G; g += MK_WAVES) {
        float M = -INFINITY;
        for (uint32_t s = lane; s < ns; s += 64) M = fmaxf(M, s_w[g * ns + s]);
        M = wave_max(M);
        float L = 0.f;
        for (uint32_t s = lane; s < ns; s += 64) {
            const float ms = s_w[g * ns + s];
            const float wt = ms == -INFINITY ? 0.f : exp2f(ms - M);
            s_w[g * ns + s] = wt;
            L = __builtin_fmaf(s_l[g * ns + s], wt, L);
        }
        L = wave_sum(L);
        if (lane == 0) s_inv[g] = 1.0f / L;
    }
    __syncthreads();
    for (uint32_t i = t; i < (uint32_t)(G * HD); i += MK_THREADS) {
        const uint32_t g = i / HD, d = i % HD;
        const uint64_t *pp = base + (size_t)g * ns * (HD + 2) + d;
        const float *wt = s_w + g * ns;
        float O = 0.f;
        for (uint32_t s0 = 0; s0 < ns; s0 += SB) {
            if (i != t || s0) {                            // the first batch of the first element is here
                const uint32_t n = ns - s0 < (uint32_t)SB ? ns - s0 : (uint32_t)SB;
                ok = load_tagged<SB + 2>(a, w, (1ull << n) - 1u, tag,
                                         [&](int k) { return pp + (size_t)(s0 + k) * (HD + 2); }) && ok;
            }
#pragma unroll
            for (int k = 0; k < SB; k++)
                if (s0 + k < ns) O = __builtin_fmaf(untag(w[k]), wt[s0 + k], O);
        }
        st_sys64(a.tatt + (size_t)(h0 + g) * HD + d, tagged(O * s_inv[g], tag));
    }
    __syncthreads();
    return ok;
}

// Every (unit, split) item of this workgroup, then the combine of units
// blockIdx.x, blockIdx.x + gridDim.x, ... (after the items, so a workgroup
// never waits for an item of its own).  Returns false when a wait gave up.
template <int EPL, int G>
__device__ __forceinline__ bool attention_t(const MkArgs &a, uint32_t layer, uint32_t pos, float *lds, uint32_t tin,
                                            uint32_t tag, uint32_t *s_fail)
{
    const uint32_t units = attn_grp(a, pos).units, ns = attn_splits_at(a, pos), items = units * ns;
    const uint32_t per_group = ((pos + ns) / ns + 2 * MK_WAVES - 1) / (2 * MK_WAVES);   // positions per lane group
    bool ok = true;
    for (uint32_t it = blockIdx.x; it < items; it += gridDim.x) {
        const uint32_t unit = it % units, split = it / units;
        if (per_group <= 2) ok = attn_item<EPL, G, 2>(a, layer, pos, unit, split, lds, tin, tag) && ok;
        else ok = attn_item<EPL, G, EPL == 4 ? 4 : 8>(a, layer, pos, unit, split, lds, tin, tag) && ok;
    }
    for (uint32_t unit = blockIdx.x; unit < units; unit += gridDim.x)
        ok = attn_combine<EPL, G>(a, unit, lds, tag, pos) && ok;
    if (!ok) *s_fail = 1;
    __syncthreads();
    return *s_fail == 0;
}

template <int EPL>
__device__ __forceinline__ bool attention_e(const MkArgs &a, uint32_t layer, uint32_t pos, float *lds, uint32_t tin,
                                            uint32_t tag, uint32_t *s_fail)
{
    switch (attn_grp(a, pos).gs) {
    case 1: return attention_t<EPL, 1>(a, layer, pos, lds, tin, tag, s_fail);
    case 2: return attention_t<EPL, 2>(a, layer, pos, lds, tin, tag, s_fail);
    case 4: return attention_t<EPL, 4>(a, layer, pos, lds, tin, tag, s_fail);
    default: return attention_t<EPL, 8>(a, layer, pos, lds, tin, tag, s_fail);
    }
}

__device__ __forceinline__ bool attention(const MkArgs &a, uint32_t layer, uint32_t pos, float *lds, uint32_t tin,
                                          uint32_t tag, uint32_t *s_fail)
{
    switch (a.head_dim) {                                  // dimensions per lane: head_dim / 32
    case 32: return attention_e<1>(a, layer, pos, lds, tin, tag, s_fail);
    case 64: return attention_e<2>(a, layer, pos, lds, tin, tag, s_fail);
    default: return attention_e<4>(a, layer, pos, lds, tin, tag, s_fail);
    }
}

// ── the kernel ───────────────────────────────────────────────────────────────

// LDS of one workgroup (host and device agree on it).  Below byte `fixed`: the
// staged input of the current phase (floats from 0) or the attention scratch,
// and above them the waves' weight rings, so a phase with a short input has
// deep rings.  From `fixed`
// on, in floats: GEMV partials (or attention scratch), the layer table, this
// workgroup's rows of x, the RoPE factors of the current position.
constexpr uint32_t MK_LDS_BYTES = 159 * 1024;   // the static __shared__ variables take some of the rest

struct MkLds {
    uint32_t fixed, attn;                       // bytes: fixed region, attention scratch (from 0)
    uint32_t part, tab, x_own, rope, total;     // floats
};

__host__ __device__ inline uint32_t mk_fixed_floats(const MkArgs &a, uint32_t n_wg, uint32_t &part)
{
    const uint32_t kvd = a.n_kv * a.head_dim;
    const uint32_t ql = a.qa_lin, mq = MK_QMIN_LAYER;
    part = mk_rows_per_wg(a.n_vocab, n_wg) * n_slices(a.n_embd, a.qa_head, MK_QMIN_HEAD);      // lm-head
    const uint32_t c[] = { mk_rows_per_wg(a.n_embd + 2 * kvd, n_wg) * n_slices(a.n_embd, ql, mq),   // QKV
                           mk_rows_per_wg(a.n_ff, n_wg) * 2 * n_slices(a.n_embd, ql, mq),           // gate, up
                           mk_rows_per_wg(a.n_embd, n_wg) * n_slices(a.n_embd, ql, mq),             // WO
                           mk_rows_per_wg(a.n_embd, n_wg) * n_slices(a.n_ff, ql, mq) };             // down
    for (uint32_t v : c) part = v > part ? v : part;
    part = (part + 3) & ~3u;
    return part + a.n_layer * (uint32_t)(sizeof(MkLayer) / 4) + mk_rows_per_wg(a.n_embd, n_wg) + a.head_dim;
}

// Attention scratch (an item's per-wave partials, then the combine), from byte 0.
__host__ __device__ inline uint32_t mk_attn_bytes(const MkArgs &a)
{
    const uint32_t G = a.attn_gs;
    const uint32_t item = MK_WAVES * G * a.head_dim + 2 * MK_WAVES * G, comb = 2 * G * a.n_splits + G;
    return ((item > comb ? item : comb) * 4 + 15) & ~15u;
}

__host__ __device__ inline MkLds mk_layout(const MkArgs &a, uint32_t n_wg)
{
    uint32_t part;
    const uint32_t nf = mk_fixed_floats(a, n_wg, part);
    MkLds L;
    L.fixed = (MK_LDS_BYTES - 4 * nf) & ~15u;
    L.attn = mk_attn_bytes(a);
    L.part = L.fixed / 4;
    L.tab = L.part + part;
    L.x_own = L.tab + a.n_layer * (uint32_t)(sizeof(MkLayer) / 4);
    L.rope = L.x_own + mk_rows_per_wg(a.n_embd, n_wg);
    L.total = L.rope + a.head_dim;
    return L;
}

// A pointer read from LDS, made wave-uniform (scalar registers).
template <typename T> __device__ __forceinline__ T *uni(T *p)
{
    const uint64_t v = (uint64_t)p;
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v), hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
    return (T *)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ uint32_t layer_mix(const MkLayer &L) { return __builtin_amdgcn_readfirstlane(L.mix); }

// The matrices of phase `kind` of `layer`.
__device__ __forceinline__ MkGemv phase_gemv(const MkArgs &a, const MkLayer *tab, uint32_t kind, uint32_t layer)
{
    MkGemv g{};
    g.n_cols = a.n_embd;
    g.row_bytes = a.rb_embd;
    g.qa = a.qa_lin;
    g.qmin = MK_QMIN_LAYER;
    if (kind == MK_HEAD) {
        g.qa = a.qa_head;
        g.qmin = MK_QMIN_HEAD;
        g.w[0] = a.head_w;
        g.rows[0] = g.n_rows = a.n_vocab;
        g.row_bytes = a.head_rb;
        g.rhi = g.n_rows;
        return g;
    }
    const MkLayer &L = tab[layer];
    const uint32_t kvd = a.n_kv * a.head_dim, mix = layer_mix(L);
    if (kind == MK_QKV) {
        g.w[0] = uni(L.wq); g.w[1] = uni(L.wk); g.w[2] = uni(L.wv);
        g.rows[0] = a.n_embd; g.rows[1] = g.rows[2] = kvd;
        g.n_rows = a.n_embd + 2 * kvd;
    } else if (kind == MK_WO) {
        g.w[0] = uni(L.wo);
        g.rows[0] = g.n_rows = a.n_embd;
    } else if (kind == MK_FFN) {
        g.w[0] = uni(L.wg); g.w[1] = uni(L.wu);
        g.rows[0] = g.rows[1] = g.n_rows = a.n_ff;
    } else {
        g.w[0] = uni(L.wd);
        g.rows[0] = g.n_rows = a.n_embd;
        g.n_cols = a.n_ff;
        g.row_bytes = (mix & MK_MIX_DOWN) ? a.rb_mix_ff : a.rb_ff;
    }
    // a V of the second type: this descriptor covers the q and k rows, v_part the rest
    g.rhi = kind == MK_QKV && (mix & MK_MIX_V) ? a.n_embd + kvd : g.n_rows;
    return g;
}

// The v rows of a QKV phase whose attn_v is of the second layer type: same
// workgroup shares as the whole phase (n_rows unchanged), rows past q and k.
__device__ __forceinline__ MkGemv v_part(const MkArgs &a, const MkGemv &qkv, const MkLayer *tab, uint32_t layer)
{
    MkGemv g = qkv;
    const uint32_t kvd = a.n_kv * a.head_dim;
    g.w[1] = g.w[2] = uni(tab[layer].wv);
    g.rows[0] = a.n_embd + kvd;                // rows below are never read here
    g.rows[1] = kvd;
    g.rows[2] = 0;
    g.row_bytes = a.rb_mix_embd;
    g.rlo = a.n_embd + kvd;
    g.rhi = g.n_rows;
    return g;
}

__device__ __forceinline__ uint32_t phase_kind(const MkArgs &a, uint32_t i)
{
    return i == 5 * a.n_layer ? (uint32_t)MK_HEAD : i % 5;
}

// Embedding row (transformer.c:168-182) into the staging area, RMS-normalised
// for the first QKV; the workgroup's own rows also go to x_own.
__device__ __forceinline__ void embed(const MkArgs &a, float *xs, float *x_own, uint32_t tok, const float *nw,
                                      float *s_red)
{
    uint32_t lo, hi;
    wg_rows(a.n_embd, lo, hi);
    const uint8_t *row = a.embd + (size_t)tok * a.embd_row_bytes;
    const uint32_t bb = block_bytes_dev(a.embd_type), bv = block_values_dev(a.embd_type);
    float ss = 0.f;
    for (uint32_t j = tid(); j < a.n_embd; j += MK_THREADS) {
        float v = a.embd_type == kF32 ? reinterpret_cast<const float *>(row)[j]
                                      : dequant_one(row + (size_t)(j / bv) * bb, a.embd_type, j % bv);
        if (a.embd_scale != 1.0f) v *= a.embd_scale;
        xs[swz(j)] = v * gptr(nw)[j];                  // (x * w), times the scale in the epilogue
        ss = __builtin_fmaf(v, v, ss);
        if (j >= lo && j < hi) x_own[j - lo] = v;
    }
    wave_ss(ss, s_red);
    __syncthreads();
}

// Every workgroup walks the step's phases (5 per layer + the lm-head), each
// ending at a grid barrier.  Descriptors are built in registers from the layer
// table in LDS; the only state carried across a barrier in registers is the
// next matrix phase's first load batch.
// TL: type of the layers' linear weights; TH: type of the lm-head; TM: 0, or
// the type of the attn_v / ffn_down of layers flagged in MkLayer::mix.
template <uint32_t TL, uint32_t TH, uint32_t TM>
__global__ __launch_bounds__(MK_THREADS) void k_decode(MkArgs a)
{
    constexpr uint32_t TMX = TM ? TM : TL;
    extern __shared__ __align__(16) float lds[];
    __shared__ float s_red[MK_WAVES];
    __shared__ uint32_t s_fail;
    const MkLds lay = mk_layout(a, gridDim.x);
    uint8_t *lds8 = reinterpret_cast<uint8_t *>(lds);
    float *xs = lds, *part = lds + lay.part, *x_own = lds + lay.x_own, *rope = lds + lay.rope;
    MkLayer *tab = reinterpret_cast<MkLayer *>(lds + lay.tab);
    {
        const uint32_t *src = reinterpret_cast<const uint32_t *>(a.layers);
        uint32_t *dst = reinterpret_cast<uint32_t *>(tab);
        for (uint32_t j = tid(); j < a.n_layer * (uint32_t)(sizeof(MkLayer) / 4); j += MK_THREADS) dst[j] = src[j];
    }
    const uint32_t n_ops = 5 * a.n_layer + 1, half = a.head_dim / 2;
    uint32_t epoch = a.epoch0;
    uint32_t n_pre = 0;                       // items of this wave's next matrix phase in flight
    const bool stamp = a.prof && blockIdx.x == 0 && tid() == 0;
    if (tid() == 0) s_fail = 0;
    if (stamp) a.prof[0] = wall_clock64();
    __syncthreads();
    for (uint32_t step = 0; step < a.n_steps; step++) {
        const uint32_t tok = ld_sys(&a.state->token), pos = ld_sys(&a.state->pos);
        const uint32_t greedy = ld_sys(&a.state->greedy), n_prompt = ld_sys(&a.state->n_prompt);
        const bool skip_head = greedy && pos + 1 < n_prompt;   // prefill: logits never read
        for (uint32_t t = tid(); t < half; t += MK_THREADS) {
            rope[t] = a.cos_tab[(size_t)pos * half + t];
            rope[half + t] = a.sin_tab[(size_t)pos * half + t];
        }

        for (uint32_t i = 0; i < n_ops; i++) {
            const uint32_t kind = phase_kind(a, i), layer = i / 5;
            const uint32_t tag_out = epoch + 1;                // tag of the values this phase publishes
            if (kind == MK_ATTN) {
                if (!attention(a, layer, pos, lds, epoch, tag_out, &s_fail)) return;
            } else if (kind == MK_HEAD && skip_head) {
                if (blockIdx.x == 0 && tid() == 0) {
                    st_sys(&a.state->token, a.prompt[pos + 1]);
                    st_sys(&a.state->pos, pos + 1);
                }
            } else {
                // one call site per GEMV variant keeps the executed code small
                const uint64_t *src = kind == MK_WO ? a.tatt : a.tx;
                const uint32_t n_in = kind == MK_DOWN ? a.n_ff : a.n_embd;
                const float *nw = kind == MK_QKV ? uni(tab[layer].attn_norm)
                                : kind == MK_FFN ? uni(tab[layer].ffn_norm)
                                : kind == MK_HEAD ? a.out_norm : nullptr;
                const MkGemv g = phase_gemv(a, tab, kind, layer);
                float *hrow = a.hf + ((size_t)step * a.n_layer + layer) * a.n_ff;   // this step's, this layer's h
                const uint32_t mix = TM && kind != MK_HEAD ? layer_mix(tab[layer]) : 0u;
                const bool mixd = kind == MK_DOWN && (mix & MK_MIX_DOWN), mixv = kind == MK_QKV && (mix & MK_MIX_V);
                if (kind == MK_QKV && layer == 0) {
                    embed(a, xs, x_own, tok, nw, s_red);
                } else {
                    // the phase's first weight items go out right behind the input loads
                    auto issue = [&]() {
                        if (n_pre) return;
                        if (kind == MK_FFN) n_pre = prefetch<TL, 2>(g, lds8, lay.fixed, lay.attn);
                        else if (kind == MK_HEAD) n_pre = prefetch<TH, 1>(g, lds8, lay.fixed, lay.attn);
                        else if (mixd) n_pre = prefetch<TMX, 1>(g, lds8, lay.fixed, lay.attn);
                        else n_pre = prefetch<TL, 1>(g, lds8, lay.fixed, lay.attn);
                    };
                    const bool ok = kind == MK_DOWN
                                        ? stage_h(a, xs, n_in, epoch, &s_fail, issue, hrow)
                                        : stage<MK_TB_EMBD>(a, xs, src, n_in, nw, a.eps, epoch, s_red, &s_fail, issue);
                    if (!ok) return;
                }
                if (kind == MK_FFN) {
                    gemv<TL, 2>(g, xs, part, lds8, lay.fixed, lay.attn, n_pre);
                } else if (kind == MK_HEAD || mixd) {
                    if constexpr (TH == TMX) gemv<TH, 1>(g, xs, part, lds8, lay.fixed, lay.attn, n_pre);
                    else if (kind == MK_HEAD) gemv<TH, 1>(g, xs, part, lds8, lay.fixed, lay.attn, n_pre);
                    else gemv<TMX, 1>(g, xs, part, lds8, lay.fixed, lay.attn, n_pre);
                } else {
                    gemv<TL, 1>(g, xs, part, lds8, lay.fixed, lay.attn, n_pre);
                }
                if (mixv) gemv<TMX, 1>(v_part(a, g, tab, layer), xs, part, lds8, lay.fixed, lay.attn, 0);
                const float nscale = nw ? norm_scale(s_red, n_in, a.eps) : 1.0f;   // after gemv's barrier
                if (kind == MK_QKV)
                    epi_qkv(a, g, part, rope,
                            a.bqkv ? a.bqkv + (size_t)layer * (a.n_embd + 2 * a.n_kv * a.head_dim) : nullptr,
                            layer, pos, tag_out, nscale);
                else if (kind == MK_FFN) epi_swiglu(a, g, part, tag_out, nscale, hrow);
                else if (kind == MK_HEAD) epi_head(a, g, part, pos, greedy, n_prompt, nscale);
                else epi_resid(a, g, part, x_own, a.trace + (size_t)(2 * layer + (kind == MK_DOWN)) * a.n_embd, tag_out);
                n_pre = 0;
            }
            // A full grid barrier only at the end of a step (the next token);
            // every phase in between waits for its tagged or flagged inputs.
            // The next matrix phase's first items go out ahead of the wait: the
            // first QKV across the barrier, and WO across attention (not by a
            // workgroup with an attention item: its K/V loads would queue
            // behind these DMAs).
            if (i + 1 == n_ops) {
                bar_arrive(a, tag_out, &s_fail);
                if (step + 1 < a.n_steps) n_pre = prefetch<TL, 1>(phase_gemv(a, tab, MK_QKV, 0), lds8, lay.fixed, lay.attn);
                if (!bar_wait(a, tag_out, &s_fail)) return;
            } else if (kind == MK_QKV && blockIdx.x >= attn_grp(a, pos).units * attn_splits_at(a, pos)) {
                n_pre = prefetch<TL, 1>(phase_gemv(a, tab, MK_WO, layer), lds8, lay.fixed, lay.attn);
            }
            epoch = tag_out;
            if (stamp) a.prof[1 + step * n_ops + i] = wall_clock64();
        }
    }
}

// Q6_K rows into the persistent kernel's quarter records (one thread per
// record).  A Q6_K super-block is 210 bytes, so every other one starts at an
// odd halfword and cannot be moved by dword DMA; the records hold the same
// bits (quant.c:160-183), 4-byte aligned.  Quarter u of a super-block is its
// values 64u..64u+63: h = u / 2, kk = 2 (u & 1) for the first 32 values and
// kk + 1 for the next 32, l = the value's index within its 32.
__global__ __launch_bounds__(256) void k_repack_q6k(const uint8_t *src, uint64_t src_rb, uint32_t n_rows, uint32_t n_sb,
                                                    uint32_t *dst)
{
    const uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (uint64_t)n_rows * n_sb * 4) return;
    const uint32_t u = (uint32_t)(i & 3);
    const uint64_t sbi = i >> 2;
    const uint8_t *blk = src + (sbi / n_sb) * src_rb + (sbi % n_sb) * 210;
    const uint32_t h = u >> 1, k0 = 2 * (u & 1);
    uint32_t w[14];
#pragma unroll
    for (int k = 0; k < 14; k++) w[k] = 0;
    for (uint32_t l = 0; l < 32; l++) {
        uint32_t lo[2], hb[2];
        for (uint32_t e = 0; e < 2; e++) {
            const uint32_t kk = k0 + e;
            const uint32_t ql = blk[h * 64 + l + 32 * (kk & 1)];
            lo[e] = kk >= 2 ? ql >> 4 : ql & 15u;
            hb[e] = ((uint32_t)blk[128 + h * 32 + l] >> (2 * kk)) & 3u;
        }
        const uint32_t k = l / 4, b = 8 * (l % 4), sh = (k & 1) ? 0u : 4u;
        w[k] |= (lo[0] | lo[1] << 4) << b;
        w[8 + k / 2] |= (hb[0] << sh | hb[1] << (sh + 2)) << b;
    }
    const uint8_t *sc = blk + 192 + 4 * u;
    w[12] = (uint32_t)sc[0] | (uint32_t)sc[1] << 8 | (uint32_t)sc[2] << 16 | (uint32_t)sc[3] << 24;
    w[13] = (uint32_t)blk[208] | (uint32_t)blk[209] << 8;
    uint32_t *o = dst + (size_t)i * 14;
#pragma unroll
    for (int k = 0; k < 14; k++) o[k] = w[k];
}

hipError_t launch_repack_q6k(const uint8_t *src, uint64_t src_rb, uint32_t n_rows, uint32_t n_sb, uint8_t *dst,
                             hipStream_t s)
{
    const uint64_t n = (uint64_t)n_rows * n_sb * 4;
    if (n == 0) return hipSuccess;
    if (((uintptr_t)dst & 3) || (n + 255) / 256 > 0x7fffffffu) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_repack_q6k, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, src_rb, n_rows, n_sb,
                       reinterpret_cast<uint32_t *>(dst));
    return hipGetLastError();
}

// ── host side ───────────────────────────────────────────────────────────────

static bool mk_kernel_exists(uint32_t tl, uint32_t th, uint32_t tm);

static bool mk_small_type(uint32_t t) { return t == kQ4_0 || t == kQ5_0 || t == kQ8_0; }

bool mk_supported(uint32_t n_embd, uint32_t n_ff, uint32_t head_dim, uint32_t group, uint32_t linear_type,
                  uint32_t head_type, uint32_t embd_type, uint32_t mix_type)
{
    if (n_embd % 64 || n_ff % 64 || n_embd / 64 > 64 * MK_SMAX || n_ff / 64 > 64 * MK_SMAX) return false;
    if (head_dim != 32 && head_dim != 64 && head_dim != 128) return false;
    if (group < 1) return false;                    // any group, in units of mk_attn_gs query heads
    const bool lin_ok = mk_small_type(linear_type) || (linear_type == kQ4_K && n_embd % 256 == 0 && n_ff % 256 == 0);
    const bool head_ok = mk_small_type(head_type) || ((head_type == kQ4_K || head_type == kQ6_KR) && n_embd % 256 == 0);
    const bool embd_ok = mk_small_type(embd_type) || embd_type == kF32 || embd_type == kQ4_K || embd_type == kQ6_K;
    const bool mix_ok = mix_type == 0 || (mix_type == kQ6_KR && n_embd % 256 == 0 && n_ff % 256 == 0);
    return lin_ok && head_ok && embd_ok && mix_ok && mk_kernel_exists(linear_type, head_type, mix_type);
}

size_t mk_lds_bytes(const MkArgs &a, uint32_t n_wg, uint32_t linear_type, uint32_t head_type, uint32_t mix_type)
{
    uint32_t part;
    if ((size_t)4 * mk_fixed_floats(a, n_wg, part) + 16 > MK_LDS_BYTES) return 0;
    const MkLds L = mk_layout(a, n_wg);
    const uint32_t n_max = a.n_embd > a.n_ff ? a.n_embd : a.n_ff;
    if (4 * n_max > L.fixed || L.attn > L.fixed) return 0;           // staging, attention scratch
    const uint32_t re = ring_wave_bytes(L.fixed, ring_base(a.n_embd, L.attn));
    const uint32_t rf = ring_wave_bytes(L.fixed, ring_base(a.n_ff, L.attn));
    if (ring_slots(re, linear_type, 1) < 1 || ring_slots(re, linear_type, 2) < 1 ||
        ring_slots(rf, linear_type, 1) < 1 || ring_slots(re, head_type, 1) < 1 ||
        (mix_type && (ring_slots(re, mix_type, 1) < 1 || ring_slots(rf, mix_type, 1) < 1)))
        return 0;                                                    // a ring slot for every phase
    return MK_LDS_BYTES;
}

typedef void (*mk_kernel_t)(MkArgs);

// Instantiated (linear, lm-head, second layer) types: the Q4_0/Q5_0/Q8_0
// files' pairs, those with a Q6_K head (its repacked form), Q4_K layers with a
// Q4_K, Q6_K or Q8_0 head, and the Q4_K_M layout (Q4_K layers whose attn_v and
// ffn_down are Q6_K in some layers, Q6_K head).
static mk_kernel_t mk_kernel(uint32_t tl, uint32_t th, uint32_t tm)
{
#define K(A, B, C) if (tl == A && th == B && tm == C) return k_decode<A, B, C>;
    K(kQ4_0, kQ4_0, 0) K(kQ4_0, kQ5_0, 0) K(kQ4_0, kQ8_0, 0) K(kQ4_0, kQ6_KR, 0)
    K(kQ5_0, kQ4_0, 0) K(kQ5_0, kQ5_0, 0) K(kQ5_0, kQ8_0, 0) K(kQ5_0, kQ6_KR, 0)
    K(kQ8_0, kQ4_0, 0) K(kQ8_0, kQ5_0, 0) K(kQ8_0, kQ8_0, 0) K(kQ8_0, kQ6_KR, 0)
    K(kQ4_K, kQ4_K, 0) K(kQ4_K, kQ6_KR, 0) K(kQ4_K, kQ8_0, 0)
    K(kQ4_K, kQ6_KR, kQ6_KR)
#undef K
    return nullptr;
}

static bool mk_kernel_exists(uint32_t tl, uint32_t th, uint32_t tm) { return mk_kernel(tl, th, tm) != nullptr; }

uint32_t mk_q_align(uint32_t type) { return q_align(type); }

int mk_max_workgroups(uint32_t linear_type, uint32_t head_type, uint32_t mix_type, size_t lds_bytes)
{
    mk_kernel_t k = mk_kernel(linear_type, head_type, mix_type);
    int dev = 0, per_cu = 0;
    hipDeviceProp_t p;
    if (!k || lds_bytes > 160 * 1024) return 0;
    if (hipGetDevice(&dev) != hipSuccess || hipGetDeviceProperties(&p, dev) != hipSuccess || !p.cooperativeLaunch)
        return 0;
    if (hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds_bytes) != hipSuccess ||
        hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, k, MK_THREADS, lds_bytes) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    if (per_cu < 1) return 0;
    return p.multiProcessorCount;                                  // one workgroup per CU
}

hipError_t mk_launch(const MkArgs &a, uint32_t linear_type, uint32_t head_type, uint32_t mix_type, uint32_t n_wg,
                     size_t lds_bytes, hipStream_t s)
{
    mk_kernel_t k = mk_kernel(linear_type, head_type, mix_type);
    if (!k) return hipErrorInvalidValue;
    MkArgs arg = a;
    void *params[] = { &arg };
    return hipLaunchCooperativeKernel((const void *)k, dim3(n_wg), dim3(MK_THREADS), params, (unsigned)lds_bytes, s);
}

} // namespace fw
