// sample_core.h - device building blocks of the samplers (specification:
// sample.h): the per-row parameters, block-wide scans and radix helpers, the
// exact whole-row path, the top-k tail, and the streamed one-workgroup-per-row
// sampler (stream_sample_row). Used by the sampling kernels and by the fused
// decode step, whose sampling workgroups run stream_sample_row.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_sample_math.h"
#include "sample.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 32;
constexpr int kSplitLen = kThreads * kPerThread;  // 8,192 elements
constexpr int kCandCap = 1024;                    // candidates per split
// Stride of consecutive slices' candidate lists: 16 entries (128 bytes) past
// the capacity, so that the lists' starts, which every slice writes and every
// merge reads, fall on different memory channels instead of one 8 KiB period.
constexpr int kCandStride = kCandCap + 16;
constexpr int kMergeCap = 8192;                   // candidates per row in the merge
constexpr int kKeptCap = 1024;                    // kept (top-k with ties) per row

struct SplitStat {
    float max_x;     // slice max of x
    float sum_exp;   // sum exp(x - max_x) over the slice
    float arg_val;   // greedy: slice max of raw logits
    uint32_t arg_idx;
    uint32_t n_cand;  // candidates written (> kCandCap: overflow)
    uint32_t cand_lo; // every candidate key is >= this
    uint64_t draw;    // split 0 of a sampled row: the row's Philox draw
};

struct SampleParams {
    const float *logits;
    uint32_t rows, vocab, row_stride, splits;
    uint32_t greedy;
    const float *temperature;
    const uint32_t *top_k;
    const float *top_p;
    const uint64_t *seed;
    float temperature_all;
    uint32_t top_k_all;
    float top_p_all;
    uint64_t seed_all;
    uint64_t step;
    const uint64_t *steps;
    const uint32_t *draw_ids;  // [rows] third Philox counter word of each row, or NULL: the row index
    uint32_t *token_out;
    float *logprob_out;
    SplitStat *stats;       // [rows][splits]
    uint2 *cand;            // [rows][splits][kCandStride] (key, index)
};

// The kernel view of a call's arguments; the split/merge workspace (splits,
// stats, cand) is filled in by the caller that uses it.
inline SampleParams sample_params_of(const rl_sample_args_t *a)
{
    SampleParams p;
    p.logits = a->logits;
    p.rows = a->rows;
    p.vocab = a->vocab;
    p.row_stride = a->row_stride;
    p.splits = 0;
    p.greedy = a->greedy;
    p.temperature = a->temperature;
    p.top_k = a->top_k;
    p.top_p = a->top_p;
    p.seed = a->seed;
    p.temperature_all = a->temperature_all;
    p.top_k_all = a->top_k_all;
    p.top_p_all = a->top_p_all;
    p.seed_all = a->seed_all;
    p.step = a->step;
    p.steps = a->steps;
    p.draw_ids = a->draw_ids;
    p.token_out = a->token_out;
    p.logprob_out = a->logprob_out;
    p.stats = nullptr;
    p.cand = nullptr;
    return p;
}

__device__ __forceinline__ float row_temperature(const SampleParams &p, uint32_t row)
{
    return p.temperature ? p.temperature[row] : p.temperature_all;
}
__device__ __forceinline__ uint32_t row_topk(const SampleParams &p, uint32_t row)
{
    return p.top_k ? p.top_k[row] : p.top_k_all;
}
__device__ __forceinline__ float row_topp(const SampleParams &p, uint32_t row)
{
    return p.top_p ? p.top_p[row] : p.top_p_all;
}
__device__ __forceinline__ uint64_t row_step(const SampleParams &p, uint32_t row)
{
    return p.steps ? p.steps[row] : p.step;
}
__device__ __forceinline__ uint64_t row_seed(const SampleParams &p, uint32_t row)
{
    return p.seed ? p.seed[row] : p.seed_all;
}
// The third word of row `row`'s Philox counter: the caller's id for the
// sampling stream (a rollout id, say), so that the draw follows the stream
// wherever its row sits in the batch; the row index when none is given.
__device__ __forceinline__ uint32_t row_draw_id(const SampleParams &p, uint32_t row)
{
    return p.draw_ids ? p.draw_ids[row] : row;
}

// Effective top-k of a row (0 = no top-k) and whether it samples at all.
__device__ __forceinline__ uint32_t effective_k(uint32_t k, uint32_t vocab)
{
    if (k == 0 || k >= vocab)
        return 0;
    return k < RL_SAMPLE_TOPK_MAX ? k : RL_SAMPLE_TOPK_MAX;
}

__device__ __forceinline__ float readlane_f(float v, int lane)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// wave-uniform max / sum: DPP inside each row of 16, then the four row results
__device__ __forceinline__ float wave_max(float v)
{
    v = rl_row_max(v);
    return fmaxf(fmaxf(readlane_f(v, 0), readlane_f(v, 16)), fmaxf(readlane_f(v, 32), readlane_f(v, 48)));
}

__device__ __forceinline__ float wave_sum(float v)
{
    v = rl_row_sum(v);
    return (readlane_f(v, 0) + readlane_f(v, 16)) + (readlane_f(v, 32) + readlane_f(v, 48));
}

// (value desc, index asc) argmax across the wave.
__device__ __forceinline__ void wave_argmax(float &v, uint32_t &i)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float ov = __shfl_xor(v, off);
        const uint32_t oi = __shfl_xor(i, off);
        if (ov > v || (ov == v && oi < i)) {
            v = ov;
            i = oi;
        }
    }
}

// The kw-th largest key held by the 64 lanes (kw in [1, 64]) among keys that
// equal `prefix` above bit top, exact: MSB-first radix select on ballot counts
// over bits top .. 0 (smaller keys never count).
__device__ __forceinline__ uint32_t wave_kth_largest_key_from(uint32_t key, uint32_t kw, uint32_t prefix, int top)
{
    for (int bit = top; bit >= 0; bit--) {
        const uint32_t cand = prefix | (1u << bit);
        const uint64_t ge = __ballot(key >= cand);
        if ((uint32_t)__popcll(ge) >= kw)
            prefix = cand;
    }
    return prefix;
}

// The kw-th largest key held by the 64 lanes (kw in [1, 64]), exact: MSB-first
// radix select on ballot counts.
__device__ __forceinline__ uint32_t wave_kth_largest_key(uint32_t key, uint32_t kw)
{
    uint32_t prefix = 0;
#pragma unroll
    for (int bit = 31; bit >= 0; bit--) {
        const uint32_t cand = prefix | (1u << bit);
        const uint64_t ge = __ballot(key >= cand);
        if ((uint32_t)__popcll(ge) >= kw)
            prefix = cand;
    }
    return prefix;
}

// ---- block-wide helpers of the merge (512 threads = 8 waves) ----------------

constexpr int kMergeThreads = 512;  // 8 waves: two per SIMD hide each other's latency
constexpr int kMergeWaves = kMergeThreads / 64;

__device__ __forceinline__ uint64_t wave_inclusive_scan_u64(uint64_t v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint64_t o = __shfl_up(v, off);
        if (lane >= off)
            v += o;
    }
    return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
        v = min(v, __shfl_xor(v, off));
    return v;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
        v = max(v, __shfl_xor(v, off));
    return v;
}

struct BlockShared {
    unsigned long long w64[kMergeWaves];
    uint32_t w32[kMergeWaves];
    unsigned long long sel64;
    uint32_t n;
    unsigned long long res64[2];  // results published by one thread (whole-row path)
    uint32_t cnt[2];              // LDS list counters (whole-row path)
};

// Exclusive prefix over the block in thread order; `total` gets the block sum.
__device__ __forceinline__ uint64_t block_excl_scan_u64_inl(uint64_t v, uint64_t &total, BlockShared &bs)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint64_t incl = wave_inclusive_scan_u64(v);
    if (lane == 63)
        bs.w64[wave] = incl;
    __syncthreads();
    uint64_t base = 0, t = 0;
#pragma unroll
    for (int w = 0; w < kMergeWaves; w++) {
        const uint64_t x = bs.w64[w];
        base += w < wave ? x : 0ull;
        t += x;
    }
    __syncthreads();
    total = t;
    return base + incl - v;
}

// (the merge kernel calls it; the row kernel inlines it, a call there would
// save and restore the registers that hold the row)
__device__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t &total, BlockShared &bs)
{
    return block_excl_scan_u64_inl(v, total, bs);
}

__device__ uint64_t block_sum_u64(uint64_t v, BlockShared &bs)
{
    uint64_t total;
    (void)block_excl_scan_u64(v, total, bs);
    return total;
}

__device__ uint32_t block_min_u32(uint32_t v, BlockShared &bs)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_min_u32(v);
    if (lane == 0)
        bs.w32[wave] = v;
    __syncthreads();
    uint32_t r = bs.w32[0];
#pragma unroll
    for (int w = 1; w < kMergeWaves; w++)
        r = min(r, bs.w32[w]);
    __syncthreads();
    return r;
}

__device__ uint32_t block_max_u32(uint32_t v, BlockShared &bs)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max_u32(v);
    if (lane == 0)
        bs.w32[wave] = v;
    __syncthreads();
    uint32_t r = bs.w32[0];
#pragma unroll
    for (int w = 1; w < kMergeWaves; w++)
        r = max(r, bs.w32[w]);
    __syncthreads();
    return r;
}

// One digit of an MSB-first radix search over a 256-bin histogram (thread t
// < 256 passes bin 255 - t, the others 0): the highest digit d in [1, 255]
// for which above + sum(bins >= d) reaches need, else 0. `acc` receives
// above + sum(bins > d), the amount ranked strictly above the chosen digit.
__device__ uint32_t block_pick_digit(uint64_t h, uint64_t above, uint64_t need, uint64_t &acc, BlockShared &bs)
{
    const bool has_bin = threadIdx.x < 256u;
    const uint32_t r = has_bin ? 255u - threadIdx.x : 0u;
    uint64_t total;
    const uint64_t S = block_excl_scan_u64(h, total, bs);  // bins > r
    const bool cross = has_bin && r >= 1u && above + S < need && above + S + h >= need;
    const uint32_t d = block_max_u32(cross ? r : 0u, bs);
    if (has_bin && r == d)
        bs.sel64 = above + S;
    __syncthreads();
    acc = bs.sel64;
    __syncthreads();
    return d;
}

// ---- exact full-row path -----------------------------------------------------
// Used for rows without top-k (whole-vocabulary nucleus) and for rows whose
// top-k candidates overflow the slice buffers (massive ties). Streams the row
// (L2-resident after the split kernel) twice. Wave w takes the rounds
// r = w, w + 8, ... of 256 consecutive elements, lane l the 4 elements
// [256 r + 4 l, 256 r + 4 l + 4), so every load instruction reads 1 KiB of
// consecutive logits; each wave keeps kRoundBatch rounds' loads in flight and
// the per-element code is branch-free (rl_sample_weight_nb).
//   cutoff  top-k only: radix select of the k-th largest float key.
//   pass A  integer weights w = rl_sample_weight(x - max) of the kept
//           elements, summed (W_K) and, for a nucleus, summed per bin of
//           d = max - x (4096 bins over [0, 17): a monotone map, so the bins
//           hold contiguous runs of the (x desc, index asc) order; weights
//           vanish below d = 16.7).
//   bin     the first bin where the cumulative weight reaches
//           thr = ceil(p W_K) holds the nucleus boundary.
//   pass B  each round's weight in the bins wholly inside the nucleus, and
//           the boundary bin's elements (composite key (float key, ~index),
//           weight) gathered into LDS.
//   tau     the boundary bin is split into 4096 sub-bins (again monotone);
//           the elements of the sub-bin where thr is reached are compared
//           pairwise: the boundary element is the one whose strictly-higher
//           weight plus the weight above its sub-bin is below thr while
//           adding its own reaches it. The boundary bin's members join
//           their rounds' weights.
//   walk    the round where the cumulative weight first exceeds the draw u,
//           then the element inside it, with one wave scan.
// More than kBinCap elements in the boundary bin or kSubCap in its sub-bin
// (massive ties) take the radix fallback: an exact 64-bit radix search on
// weight histograms.
constexpr int kBins = 4096;
constexpr float kBinSpan = 17.0f;               // d in [0, 17): w(d) = 0 beyond 16.7
constexpr int kBinCap = 1024;
constexpr int kSubCap = 240;
constexpr int kMaxRounds = 64 * kSplitLen / 256;  // rounds of the largest vocabulary

struct RowScratch {
    unsigned long long hist[kBins];       // bin weights, then the boundary bin's sub-bin weights
    unsigned long long rounds[kMaxRounds];
    unsigned long long bkey[kBinCap];     // the boundary bin: composite keys and weights
    uint32_t bw[kBinCap];
    unsigned long long skey[kSubCap];     // the boundary sub-bin
    uint32_t sw[kSubCap];
};

__device__ __forceinline__ uint64_t composite_key(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ __forceinline__ float dist_t(float m, float x)
{
    return (m - x) * ((float)kBins / kBinSpan);
}

__device__ __forceinline__ uint32_t dist_bin(float m, float x)
{
    const float b = dist_t(m, x);
    return b < (float)(kBins - 1) ? (uint32_t)b : (uint32_t)(kBins - 1);
}

// Sub-bin (1/kBins of a bin) of an element of bin b: monotone in x like the
// bin itself, since t - b and the scaling by a power of two are monotone.
__device__ __forceinline__ uint32_t dist_sub(float m, float x, uint32_t b)
{
    const float f = (dist_t(m, x) - (float)b) * (float)kBins;
    return f < (float)(kBins - 1) ? (uint32_t)f : (uint32_t)(kBins - 1);
}

// Appends (key, w) to an LDS list for every lane with `take`, one atomic per
// wave; returns the list position of this lane's entry.
__device__ __forceinline__ uint32_t wave_append(bool take, uint32_t *counter)
{
    const uint64_t bal = __ballot(take);
    if (!bal)
        return 0;
    const int first = (int)__ffsll((long long)bal) - 1;
    uint32_t base = 0;
    if ((int)(threadIdx.x & 63) == first)
        base = atomicAdd(counter, (uint32_t)__popcll(bal));
    base = (uint32_t)__builtin_amdgcn_readlane((int)base, first);
    return base + __builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0u));
}

// 4 consecutive logits from index i (i % 4 == 0), -inf past the end. The
// load itself is unconditional - past the end it re-reads the row's last
// quad, inside the row since row_stride % 4 == 0 - so a batch of them can
// be in flight together.
__device__ __forceinline__ rl_f32x4 load_quad(const float *l, uint32_t i, uint32_t V)
{
    const rl_f32x4 r = *(const RL_GLOBAL rl_f32x4 *)(l + min(i, (V - 1) & ~3u));
    rl_f32x4 v;
    v.x = i < V ? r.x : -INFINITY;
    v.y = i + 1 < V ? r.y : -INFINITY;
    v.z = i + 2 < V ? r.z : -INFINITY;
    v.w = i + 3 < V ? r.w : -INFINITY;
    return v;
}

__device__ __forceinline__ float quad_at(const rl_f32x4 &v, int e)
{
    return e == 0 ? v.x : e == 1 ? v.y : e == 2 ? v.z : v.w;
}

// Calls f(r, i0, quad) for this wave's rounds r (i0 = 256 r + 4 lane, the
// lane's first index), with the loads of kRoundBatch rounds issued before
// any of them is used: one row pass has that many loads in flight per wave.
constexpr int kRoundBatch = 8;

template <class F>
__device__ __forceinline__ void for_rounds(const float *l, uint32_t V, uint32_t R, int wave, int lane, F &&f)
{
    for (uint32_t r0 = wave; r0 < R; r0 += kMergeWaves * kRoundBatch) {
        rl_f32x4 v[kRoundBatch];
#pragma unroll
        for (int j = 0; j < kRoundBatch; j++)
            v[j] = load_quad(l, (r0 + j * kMergeWaves) * 256 + lane * 4, V);
#pragma unroll
        for (int j = 0; j < kRoundBatch; j++) {
            const uint32_t r = r0 + j * kMergeWaves;
            if (r < R)
                f(r, r * 256 + lane * 4, v[j]);
        }
    }
}

// k_eff-th largest finite x (multiplicity counted) as a float key; 0 keeps all.
__device__ uint32_t row_topk_cutoff(const float *l, uint32_t V, float inv_t, uint32_t k_eff, uint32_t *s_hist,
                                    BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    uint32_t prefix = 0, mask = 0;
    uint64_t need = k_eff;
    for (int pass = 3; pass >= 0; pass--) {
        const int shift = pass * 8;
        if (tid < 256)
            s_hist[tid] = 0;
        __syncthreads();
        for (uint32_t i = tid; i < V; i += kMergeThreads) {
            const float x = l[i] * inv_t;
            const uint32_t key = rl_float_key(x);
            if (x != -INFINITY && (key & mask) == prefix)
                atomicAdd(&s_hist[(key >> shift) & 0xFFu], 1u);
        }
        __syncthreads();
        uint64_t acc;
        const uint32_t d = block_pick_digit(tid < 256 ? s_hist[255 - tid] : 0u, 0, need, acc, bs);
        prefix |= d << shift;
        mask |= 0xFFu << shift;
        need -= acc;
    }
    return prefix;
}

// The radix fallback: nucleus boundary tau as the largest composite key whose
// suffix weight reaches thr (8 passes of 8-bit digits), then W_P and the
// ascending-index walk in chunks of 256 threads x 8 elements.
__device__ __forceinline__ uint32_t radix_row_sample(uint64_t seed, uint64_t step, uint32_t draw_id, uint32_t V,
                                                     const float *l, float inv_t, uint32_t cutoff, float topp, float m,
                                                     uint64_t wk, unsigned long long *s_whist, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    uint64_t tau = 0;
    if (topp > 0.f && topp < 1.f) {
        const uint64_t thr = rl_topp_threshold(topp, wk);
        uint64_t prefix = 0, mask = 0, above = 0;
        for (int pass = 7; pass >= 0; pass--) {
            const int shift = pass * 8;
            if (tid < 256)
                s_whist[tid] = 0;
            __syncthreads();
            for (uint32_t i = tid; i < V; i += kMergeThreads) {
                const float x = l[i] * inv_t;
                const uint32_t key = rl_float_key(x);
                if (x == -INFINITY || key < cutoff)
                    continue;
                const uint64_t ck = composite_key(key, i);
                if ((ck & mask) == prefix)
                    atomicAdd(&s_whist[(ck >> shift) & 0xFFu], (unsigned long long)rl_sample_weight(x - m));
            }
            __syncthreads();
            // (thr >= 1 whenever K is non-empty: the row maximum weighs 2^24)
            uint64_t acc;
            const uint32_t d = block_pick_digit(tid < 256 ? s_whist[255 - tid] : 0ull, above, thr, acc, bs);
            prefix |= (uint64_t)d << shift;
            mask |= 0xFFull << shift;
            above = acc;
        }
        tau = prefix;
    }

    uint64_t wp_own = 0;
    uint32_t lowest = 0xFFFFFFFFu;
    for (uint32_t i = tid; i < V; i += kMergeThreads) {
        const float x = l[i] * inv_t;
        const uint32_t key = rl_float_key(x);
        if (x != -INFINITY && key >= cutoff && composite_key(key, i) >= tau) {
            wp_own += rl_sample_weight(x - m);
            lowest = min(lowest, i);
        }
    }
    const uint64_t wp = block_sum_u64(wp_own, bs);
    lowest = block_min_u32(lowest, bs);

    const uint64_t u = rl_mulhi_u64(rl_sample_draw64(seed, step, draw_id), wp);
    uint64_t carry = 0;
    uint32_t tok = 0xFFFFFFFFu;
    for (uint32_t base = 0; base < V && tok == 0xFFFFFFFFu; base += kMergeThreads * 8) {
        uint64_t w8[8], own = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t i = base + tid * 8 + e;
            w8[e] = 0;
            if (i < V) {
                const float x = l[i] * inv_t;
                const uint32_t key = rl_float_key(x);
                if (x != -INFINITY && key >= cutoff && composite_key(key, i) >= tau)
                    w8[e] = rl_sample_weight(x - m);
            }
            own += w8[e];
        }
        uint64_t total;
        const uint64_t excl = block_excl_scan_u64(own, total, bs);
        if (carry + total > u) {
            uint64_t c = carry + excl;
            uint32_t cand = 0xFFFFFFFFu;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                c += w8[e];
                if (cand == 0xFFFFFFFFu && c > u)
                    cand = base + tid * 8 + e;
            }
            tok = block_min_u32(cand, bs);
        }
        carry += total;
    }
    if (tok == 0xFFFFFFFFu)
        tok = lowest;        // zero total weight: lowest index of P
    if (tok >= V)
        tok = 0;             // every logit -inf
    return tok;
}

__device__ __forceinline__ uint32_t exact_row_sample(const SampleParams &p, uint32_t row, float inv_t, uint32_t k_eff,
                                                     float topp, float m, RowScratch &rs, uint32_t *s_hist,
                                                     unsigned long long *s_whist, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const float *l = p.logits + (size_t)row * p.row_stride;
    const uint32_t V = p.vocab;
    const uint32_t R = (V + 255) / 256;  // rounds
    const bool trunc = topp > 0.f && topp < 1.f;

    const uint32_t cutoff = k_eff ? row_topk_cutoff(l, V, inv_t, k_eff, s_hist, bs) : 0u;

    // ---- pass A: W_K and the per-bin weights --------------------------------
    if (trunc)
        for (uint32_t b = tid; b < (uint32_t)kBins; b += kMergeThreads)
            rs.hist[b] = 0;
    __syncthreads();
    uint64_t wk_own = 0;
    for_rounds(l, V, R, wave, lane, [&](uint32_t, uint32_t, const rl_f32x4 &v) {
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x = quad_at(v, e) * inv_t;  // -inf weighs 0
            const uint32_t wx = rl_sample_weight_nb(x - m);
            const uint32_t w = rl_float_key(x) >= cutoff ? wx : 0u;
            wk_own += w;
            if (trunc && w)
                atomicAdd(&rs.hist[dist_bin(m, x)], (unsigned long long)w);
        }
    });
    const uint64_t wk = block_sum_u64(wk_own, bs);  // (synchronises: the histogram is complete)
    if (wk == 0)
        return 0;  // no finite logit at or above the cutoff: token 0

    // ---- nucleus boundary bin --------------------------------------------------
    uint32_t bstar = kBins;   // bins below bstar are wholly in P; kBins: no truncation
    uint64_t thr = 0, above = 0;
    constexpr int per = kBins / kMergeThreads;
    if (trunc) {
        thr = rl_topp_threshold(topp, wk);
        uint64_t own = 0;
#pragma unroll
        for (int j = 0; j < per; j++)
            own += rs.hist[tid * per + j];
        uint64_t total;
        const uint64_t excl = block_excl_scan_u64(own, total, bs);
        if (excl < thr && excl + own >= thr) {  // exactly one thread
            uint64_t c = excl;
            uint32_t b = tid * per;
            while (c + rs.hist[b] < thr) {
                c += rs.hist[b];
                b++;
            }
            bs.n = b;
            bs.sel64 = c;
        }
        if (tid == 0) {
            bs.cnt[0] = 0;
            bs.cnt[1] = 0;
        }
        __syncthreads();
        bstar = bs.n;
        above = bs.sel64;
        for (uint32_t b = tid; b < (uint32_t)kBins; b += kMergeThreads)
            rs.hist[b] = 0;  // reused for the sub-bins
    }

    // ---- pass B: each round's weight in the bins wholly in P; the boundary
    // bin's elements, gathered with their indices --------------------------------
    for_rounds(l, V, R, wave, lane, [&](uint32_t r, uint32_t i0, const rl_f32x4 &v) {
        uint32_t s = 0;  // at most 4 x 2^24
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x = quad_at(v, e) * inv_t;  // -inf weighs 0
            const uint32_t key = rl_float_key(x);
            const uint32_t b = trunc ? dist_bin(m, x) : 0u;
            const uint32_t w = rl_sample_weight_nb(x - m);
            const bool ok = key >= cutoff;
            s += ok && b < bstar ? w : 0u;
            const bool edge = ok && b == bstar && w != 0;
            const uint32_t pos = wave_append(edge, &bs.cnt[0]);
            if (edge && pos < (uint32_t)kBinCap) {
                rs.bkey[pos] = composite_key(key, i0 + e);
                rs.bw[pos] = w;
            }
        }
        // the wave sum can reach 2^32: two DPP sums of 24-bit and 8-bit parts
        const uint32_t hi = rl_wave_sum_u32(s >> 8), lo = rl_wave_sum_u32(s & 0xFFu);
        if (lane == 0)
            rs.rounds[r] = ((uint64_t)hi << 8) + lo;
    });
    __syncthreads();

    uint64_t tau = 0, wp = wk;
    if (trunc) {
        const uint32_t nb = bs.cnt[0];
        if (nb > (uint32_t)kBinCap)
            return radix_row_sample(row_seed(p, row), row_step(p, row), row_draw_id(p, row), V, l, inv_t, cutoff, topp, m, wk, s_whist,
                                    bs);

        // ---- the boundary bin's sub-bins: the one where thr is reached ----------
        for (uint32_t e = tid; e < nb; e += kMergeThreads) {
            const float x = rl_key_float((uint32_t)(rs.bkey[e] >> 32));
            atomicAdd(&rs.hist[dist_sub(m, x, bstar)], (unsigned long long)rs.bw[e]);
        }
        __syncthreads();
        uint64_t sub_above = 0;
        uint32_t sb = 0;
        {
            uint64_t own2 = 0;
#pragma unroll
            for (int j = 0; j < per; j++)
                own2 += rs.hist[tid * per + j];
            uint64_t total2;
            const uint64_t excl2 = block_excl_scan_u64(own2, total2, bs);
            if (above + excl2 < thr && above + excl2 + own2 >= thr) {  // exactly one thread
                uint64_t c = above + excl2;
                uint32_t b = tid * per;
                while (c + rs.hist[b] < thr) {
                    c += rs.hist[b];
                    b++;
                }
                bs.res64[0] = c;
                bs.n = b;
            }
            __syncthreads();
            sub_above = bs.res64[0];
            sb = bs.n;
        }
        // ---- its elements, compared pairwise (exact ties of x share a sub-bin) ---
        for (uint32_t e0 = 0; e0 < nb; e0 += kMergeThreads) {
            const uint32_t e = e0 + tid;
            bool take = false;
            if (e < nb)
                take = dist_sub(m, rl_key_float((uint32_t)(rs.bkey[e] >> 32)), bstar) == sb;
            const uint32_t pos = wave_append(take, &bs.cnt[1]);
            if (take && pos < (uint32_t)kSubCap) {
                rs.skey[pos] = rs.bkey[e];
                rs.sw[pos] = rs.bw[e];
            }
        }
        __syncthreads();
        const uint32_t ns = bs.cnt[1];
        if (ns > (uint32_t)kSubCap)
            return radix_row_sample(row_seed(p, row), row_step(p, row), row_draw_id(p, row), V, l, inv_t, cutoff, topp, m, wk, s_whist,
                                    bs);
        if (tid < ns) {
            const uint64_t ck = rs.skey[tid];
            uint64_t s = 0;  // sub-bin weight strictly above this element
            for (uint32_t j = 0; j < ns; j++)
                s += rs.skey[j] > ck ? (uint64_t)rs.sw[j] : 0ull;
            if (sub_above + s < thr && sub_above + s + rs.sw[tid] >= thr) {  // exactly one element
                bs.res64[0] = ck;
                bs.res64[1] = sub_above + s + rs.sw[tid];
            }
        }
        __syncthreads();
        tau = bs.res64[0];
        wp = bs.res64[1];
        // the boundary bin's members of P join their rounds
        for (uint32_t e = tid; e < nb; e += kMergeThreads) {
            const uint64_t ck = rs.bkey[e];
            if (ck >= tau)
                atomicAdd(&rs.rounds[(0xFFFFFFFFu - (uint32_t)ck) / 256u], (unsigned long long)rs.bw[e]);
        }
        __syncthreads();
    }

    // ---- the draw and the round where the cumulative weight first exceeds it -----
    const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), row_step(p, row), row_draw_id(p, row)), wp);
    {
        const uint32_t per = (R + kMergeThreads - 1) / kMergeThreads;
        const uint32_t r0 = min(R, tid * per), r1 = min(R, r0 + per);
        uint64_t own = 0;
        for (uint32_t r = r0; r < r1; r++)
            own += rs.rounds[r];
        uint64_t total;
        const uint64_t excl = block_excl_scan_u64(own, total, bs);
        if (excl <= u && u < excl + own) {  // exactly one thread: u < W_P = total
            uint64_t c = excl;
            uint32_t r = r0;
            while (c + rs.rounds[r] <= u) {
                c += rs.rounds[r];
                r++;
            }
            bs.n = r;
            bs.sel64 = c;
        }
        __syncthreads();
    }
    const uint32_t rstar = bs.n;
    const uint64_t before = bs.sel64;
    uint32_t tok = 0;
    if (wave == 0) {
        const uint32_t i0 = rstar * 256 + lane * 4;
        const rl_f32x4 v = load_quad(l, i0, V);
        uint32_t w4[4], own = 0;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const float x = quad_at(v, e) * inv_t;
            const uint32_t key = rl_float_key(x);
            const uint32_t b = trunc ? dist_bin(m, x) : 0u;
            const uint32_t at_tau = (uint32_t)(b == bstar) & (uint32_t)(composite_key(key, i0 + e) >= tau);
            const uint32_t in = (uint32_t)(key >= cutoff) & ((uint32_t)(b < bstar) | at_tau);
            const uint32_t w = rl_sample_weight_nb(x - m);  // -inf weighs 0
            w4[e] = w & (0u - in);  // (a mask: no short-circuit branches)
            own += w4[e];
        }
        uint64_t c = before + wave_inclusive_scan_u64(own) - own;
        uint32_t cand = 0xFFFFFFFFu;
#pragma unroll
        for (int e = 0; e < 4; e++) {
            c += w4[e];
            if (cand == 0xFFFFFFFFu && c > u)
                cand = i0 + e;
        }
        tok = rl_wave_min_u32(cand);
        if (tok >= V)
            tok = 0;
    }
    return tok;
}

// ---- one-wave top-k pick -------------------------------------------------------
// Lane j holds the j-th kept composite key in (x desc, index asc) order (j <
// nk <= 64): integer weights, the nucleus prefix, the draw and the smallest
// index whose ascending-index cumulative weight exceeds it. With at most 64
// weights of at most 2^24 every prefix fits in 32 bits. Every lane of the
// wave returns the token; xtok / xknown: its x from the kept key.
__device__ __forceinline__ void wave_draw_sorted(uint64_t cs, uint32_t nk, float m, float topp, uint64_t draw,
                                                 uint32_t vocab, uint32_t &tok, float &xtok, bool &xknown)
{
    const int lane = threadIdx.x & 63;
    const bool valid = (uint32_t)lane < nk;
    const uint32_t idx = 0xFFFFFFFFu - (uint32_t)cs;
    const uint32_t w = valid ? rl_sample_weight(rl_key_float((uint32_t)(cs >> 32)) - m) : 0u;
    const uint32_t c = rl_wave_incl_scan_u32(w);
    const uint32_t wk = rl_readlane(c, 63);
    uint32_t np = nk;
    if (topp > 0.f && topp < 1.f) {
        const uint64_t thr = rl_topp_threshold(topp, wk);
        const uint64_t hit = __ballot(valid && (uint64_t)c >= thr);
        np = hit ? (uint32_t)__ffsll((long long)hit) : nk;  // first reaching lane + 1
    }
    const uint32_t wp = np ? rl_readlane(c, (int)np - 1) : 0u;
    const uint64_t u = rl_mulhi_u64(draw, wp);
    const bool in_p = (uint32_t)lane < np;
    // ascending-index prefix weight at my index (lane j holds sorted element j)
    uint32_t s_le = 0;
    for (uint32_t j = 0; j < np; j++)
        s_le += rl_readlane(idx, (int)j) <= idx ? rl_readlane(w, (int)j) : 0u;
    tok = rl_wave_min_u32(in_p && (uint64_t)s_le > u ? idx : 0xFFFFFFFFu);
    if (tok == 0xFFFFFFFFu)  // zero total weight: lowest index of P
        tok = rl_wave_min_u32(in_p ? idx : 0xFFFFFFFFu);
    if (tok >= vocab)        // empty kept set (every logit -inf): token 0
        tok = 0;
    const uint64_t own = __ballot(valid && idx == tok);
    if (own) {
        const int src = (int)__ffsll((long long)own) - 1;
        xtok = rl_key_float(rl_readlane((uint32_t)(cs >> 32), src));
        xknown = true;
    }
}

// ---- the top-k tail shared by the merge and the stream kernels ---------------
// Input: the candidates s_cand[0, nf), among them every key of the row's
// k_eff largest (every candidate key lies in [key_lo, key_hi], key_hi the
// key of the row max m); s_h2[0] holding the histogram of the first radix
// digit, bits hb .. hb - 7 (bits 7 .. 0 when hb < 7), of the candidate keys
// equal to prefix0 above bit hb (hb < 0: every candidate key equals key_hi);
// bs.cnt[1] and bs.n zero; all of it visible to the block. Returns the
// sampled token, or overflow when the kept set exceeds kKeptCap (the caller
// then takes the exact whole-row path).
struct TopkPick {
    uint32_t tok;
    float xtok;    // the token's x when the path that chose it holds it
    bool xknown;
    bool overflow;
};

__device__ __forceinline__ TopkPick topk_pick(uint32_t nf, uint32_t k_eff, int hb, uint32_t key_hi, uint32_t prefix0,
                                              float m, float topp, uint64_t draw, uint32_t vocab, uint2 *s_cand,
                                              uint32_t (*s_h2)[256], uint64_t *s_keep, uint64_t *s_sort,
                                              uint32_t *s_w, uint32_t *s_idx, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;
    uint32_t tok = 0;
    float xtok = 0.f;
    bool xknown = false, exact = false;
    // ---- exact k_eff-th largest key --------------------------------------
    // Each pass's histogram (after the first) is filled while the other one
    // is cleared; every wave then finds the digit itself: lane l holds
    // bins 255-4l .. 252-4l, a DPP scan gives the count in higher bins,
    // and the digit is the bin where that count reaches need. Once the
    // chosen bin holds at most 64 keys, they are copied out and one wave
    // finishes the selection with a ballot radix select. With fewer than
    // k_eff candidates the row has fewer than k_eff finite logits, and
    // every finite one is kept.
    uint32_t cutoff = 0;
    if (nf >= k_eff) {
        if (hb < 0) {
            cutoff = key_hi;
        } else {
            uint32_t prefix = prefix0;
            uint32_t need = k_eff;
            int pass = 0;
            for (int top = hb; top >= 0; top -= 8, pass++) {
                const int shift = top >= 7 ? top - 7 : 0;
                const uint32_t above = top >= 31 ? 0u : ~((2u << top) - 1u);
                uint32_t *H = s_h2[pass & 1];
                if (pass > 0) {
                    for (uint32_t i = tid; i < nf; i += kMergeThreads) {
                        const uint32_t key = s_cand[i].x;
                        if ((key & above) == prefix)
                            atomicAdd(&H[(key >> shift) & 0xFFu], 1u);
                    }
                    __syncthreads();
                }
                if (tid < 256)
                    s_h2[(pass & 1) ^ 1][tid] = 0;
                uint32_t h[4], own = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    h[j] = H[255 - 4 * lane - j];
                    own += h[j];
                }
                uint32_t acc = rl_wave_incl_scan_u32(own) - own;
                int found = -1;
                uint32_t rem = 0, hcnt = 0;
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    if (found < 0 && acc < need && acc + h[j] >= need) {
                        found = 255 - 4 * lane - j;
                        rem = need - acc;
                        hcnt = h[j];
                    }
                    acc += h[j];
                }
                const uint64_t hit = __ballot(found >= 0);  // never empty: need <= matching keys
                const int src = hit ? (int)__ffsll((long long)hit) - 1 : 0;
                prefix |= (uint32_t)__builtin_amdgcn_readlane(found, src) << shift;
                need = rl_readlane(rem, src);
                const uint32_t bin_cnt = rl_readlane(hcnt, src);
                __syncthreads();
                if (shift > 0 && bin_cnt <= 64u) {
                    // the keys sharing every bit fixed so far (bits >= shift)
                    const uint32_t above_s = ~((1u << shift) - 1u);
                    uint32_t *lst = s_h2[pass & 1];  // H is read by no one after the barrier
                    for (uint32_t i = tid; i < nf; i += kMergeThreads) {
                        const uint32_t key = s_cand[i].x;
                        if ((key & above_s) == prefix)
                            lst[atomicAdd(&bs.cnt[1], 1u)] = key;  // bin_cnt <= 64 of them
                    }
                    __syncthreads();
                    if (tid < 64) {
                        const uint32_t key = (uint32_t)lane < bin_cnt ? lst[lane] : 0u;
                        const uint32_t c = wave_kth_largest_key_from(key, need, prefix, shift - 1);
                        if (tid == 0)
                            bs.w32[0] = c;
                    }
                    __syncthreads();
                    prefix = bs.w32[0];
                    break;
                }
            }
            cutoff = prefix;
        }
    }

    // ---- kept set K = {key >= cutoff} ------------------------------------
    for (uint32_t i = tid; i < nf; i += kMergeThreads) {
        const uint2 c = s_cand[i];
        if (c.x >= cutoff) {
            const uint32_t pos = atomicAdd(&bs.n, 1u);
            if (pos < (uint32_t)kKeptCap)
                s_keep[pos] = composite_key(c.x, c.y);
        }
    }
    __syncthreads();
    const uint32_t nk = bs.n;
    __syncthreads();
    if (nk > (uint32_t)kKeptCap) {
        exact = true;
    } else if (nk <= 64u) {
        // ---- one wave: lane i holds sorted element i; with at most 64
        // weights of at most 2^24 every prefix fits in 32 bits ------------
        tok = 0;
        // rank of kept key i = kept keys above it; thread (i, b) counts
        // over keys 8b .. 8b + 7 (s_h2 is free after the cutoff)
        {
            const uint32_t i = tid & 63u, b = tid >> 6;
            const uint64_t cki = i < nk ? s_keep[i] : 0ull;
            uint32_t part = 0;
#pragma unroll
            for (uint32_t jj = 0; jj < 8; jj++) {
                const uint32_t j = b * 8 + jj;
                part += (j < nk && s_keep[j] > cki) ? 1u : 0u;
            }
            s_h2[b >> 2][(b & 3) * 64 + i] = part;
        }
        __syncthreads();
        if (tid < 64) {
            const bool valid = (uint32_t)lane < nk;
            const uint64_t ck = valid ? s_keep[lane] : 0ull;  // real keys are > 0
            uint32_t rank = 0;
#pragma unroll
            for (uint32_t b = 0; b < 8; b++)
                rank += s_h2[b >> 2][(b & 3) * 64 + lane];
            if (valid)
                s_sort[rank] = ck;
            rl_wave_lds_fence();
            wave_draw_sorted(valid ? s_sort[lane] : 0ull, nk, m, topp, draw, vocab, tok, xtok, xknown);
        }
    } else {
        // ---- rank sort by (x desc, index asc): composite keys are distinct
        for (uint32_t i = tid; i < nk; i += kMergeThreads) {
            const uint64_t ck = s_keep[i];
            uint32_t rank = 0;
            for (uint32_t j = 0; j < nk; j++)
                rank += s_keep[j] > ck ? 1u : 0u;
            s_sort[rank] = ck;
        }
        __syncthreads();
        for (uint32_t i = tid; i < nk; i += kMergeThreads) {
            const uint64_t ck = s_sort[i];
            s_w[i] = rl_sample_weight(rl_key_float((uint32_t)(ck >> 32)) - m);
            s_idx[i] = 0xFFFFFFFFu - (uint32_t)ck;
        }
        __syncthreads();

        // ---- nucleus prefix over the sorted order -----------------------
        // thread t owns the contiguous sorted positions [t*per, (t+1)*per)
        const uint32_t per = (nk + kMergeThreads - 1) / kMergeThreads;
        const uint32_t i0 = min(nk, tid * per), i1 = min(nk, (tid + 1) * per);
        uint64_t own = 0;
        for (uint32_t i = i0; i < i1; i++)
            own += s_w[i];
        uint64_t wk;
        const uint64_t excl = block_excl_scan_u64(own, wk, bs);
        uint32_t np = nk;
        if (topp > 0.f && topp < 1.f) {
            const uint64_t thr = rl_topp_threshold(topp, wk);
            // first sorted position whose inclusive prefix reaches thr
            uint32_t first = 0xFFFFFFFFu;
            uint64_t c = excl;
            for (uint32_t i = i0; i < i1; i++) {
                c += s_w[i];
                if (c >= thr) {
                    first = i;
                    break;
                }
            }
            first = block_min_u32(first, bs);
            np = (first == 0xFFFFFFFFu) ? nk : first + 1;
        }
        uint64_t wp_own = 0;
        for (uint32_t i = i0; i < min(i1, np); i++)
            wp_own += s_w[i];
        const uint64_t wp = block_sum_u64(wp_own, bs);

        // ---- draw; smallest index whose ascending-index prefix weight exceeds u
        const uint64_t u = rl_mulhi_u64(draw, wp);
        uint32_t cand = 0xFFFFFFFFu, lowest = 0xFFFFFFFFu;
        for (uint32_t i = tid; i < np; i += kMergeThreads) {
            const uint32_t idx_i = s_idx[i];
            lowest = min(lowest, idx_i);
            uint64_t s_le = 0;
            for (uint32_t j = 0; j < np; j++)
                s_le += s_idx[j] <= idx_i ? (uint64_t)s_w[j] : 0ull;
            if (s_le > u)
                cand = min(cand, idx_i);
        }
        tok = block_min_u32(cand, bs);
        lowest = block_min_u32(lowest, bs);
        if (tok == 0xFFFFFFFFu)  // zero total weight: lowest index of P
            tok = lowest;
        if (tok >= vocab)      // empty kept set (every logit -inf): token 0
            tok = 0;
    }
    return TopkPick{tok, xtok, xknown, exact};
}

// ---- split: one slice of a row per workgroup (sample_split_kernel) -----------
// LDS of one slice's workgroup: per-wave maxima, argmax indexes, exp sums,
// candidate bounds and candidate counts.
struct SplitLds {
    float s_red[4];
    uint32_t s_red_i[4];
    float s_z[4];
    uint32_t s_key[4];
    uint32_t s_wtot[4];
};

// One slice of the split kernel: slice `split` of row `row`, by the calling
// workgroup of kThreads threads (every thread calls it); L in LDS.
__device__ __forceinline__ void split_slice(const SampleParams &p, uint32_t split, uint32_t row, SplitLds &L)
{
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    float *s_red = L.s_red;
    uint32_t *s_red_i = L.s_red_i;
    float *s_z = L.s_z;
    uint32_t *s_key = L.s_key;
    uint32_t *s_wtot = L.s_wtot;

    const float *lrow = p.logits + (size_t)row * p.row_stride;
    const uint32_t c0 = split * kSplitLen;
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);
    const float inv_t = greedy ? 1.0f : 1.0f / row_temperature(p, row);

    // Stream the slice: element (k, e) of thread tid is column c0 + (k*256 + tid)*4 + e.
    // Every load is issued unconditionally (a quad past the end re-reads the
    // row's last quad, which row_stride % 4 == 0 keeps inside the row) and
    // masked afterwards, so all eight are in flight together. Only the last
    // slice of a row can reach past the vocabulary (a workgroup-uniform test).
    float x[kPerThread];
    const uint32_t last_quad = (p.vocab - 1) & ~3u;
    rl_f32x4 raw[kPerThread / 4];
#pragma unroll
    for (int k = 0; k < kPerThread / 4; k++) {
        const uint32_t col = c0 + (uint32_t)(k * kThreads + tid) * 4u;
        raw[k] = __builtin_nontemporal_load((const rl_f32x4 *)(lrow + min(col, last_quad)));
    }
    // the row's Philox draw, for the merge (computed while the loads are in flight)
    uint64_t draw = 0;
    if (split == 0 && !greedy && wave == 0)
        draw = rl_sample_draw64(row_seed(p, row), row_step(p, row), row_draw_id(p, row));
    if (c0 + (uint32_t)kSplitLen <= p.vocab) {
#pragma unroll
        for (int k = 0; k < kPerThread / 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                x[k * 4 + e] = raw[k][e];
    } else {
#pragma unroll
        for (int k = 0; k < kPerThread / 4; k++) {
            const uint32_t col = c0 + (uint32_t)(k * kThreads + tid) * 4u;
#pragma unroll
            for (int e = 0; e < 4; e++)
                x[k * 4 + e] = col + (uint32_t)e < p.vocab ? raw[k][e] : -INFINITY;
        }
    }

    SplitStat *st = p.stats + (size_t)row * p.splits + split;

    if (greedy) {
        float best = -INFINITY;
        uint32_t bidx = 0xFFFFFFFFu;
#pragma unroll
        for (int k = 0; k < kPerThread / 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = x[k * 4 + e];
                if (v > best) {
                    best = v;
                    bidx = c0 + (uint32_t)(k * kThreads + tid) * 4u + e;
                }
            }
        wave_argmax(best, bidx);
        if (lane == 0) {
            s_red[wave] = best;
            s_red_i[wave] = bidx;
        }
        __syncthreads();
        float m = s_red[0];
        uint32_t mi = s_red_i[0];
#pragma unroll
        for (int w = 1; w < 4; w++)
            if (s_red[w] > m || (s_red[w] == m && s_red_i[w] < mi)) {
                m = s_red[w];
                mi = s_red_i[w];
            }
        float z = 0.f;
        if (m != -INFINITY) {
            const float ml = m * 1.4426950408889634f;
#pragma unroll
            for (int i = 0; i < kPerThread; i++)
                z += __builtin_amdgcn_exp2f(fmaf(x[i], 1.4426950408889634f, -ml));
        }
        z = wave_sum(z);
        if (lane == 0)
            s_z[wave] = z;
        __syncthreads();
        if (tid == 0) {
            st->max_x = m;
            st->sum_exp = s_z[0] + s_z[1] + s_z[2] + s_z[3];
            st->arg_val = m;
            st->arg_idx = mi;
            st->n_cand = 0;
        }
        return;
    }

    // ---- sampling: x = l * inv_t, slice max, sum exp, candidates -------------
    // Two barriers: (1) wave maxima and k-th bounds, (2) wave sums and
    // candidate counts; the candidates are then written at their offsets.
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPerThread; i++) {
        x[i] = x[i] * inv_t;
        tmax = fmaxf(tmax, x[i]);
    }
    const float wmax = wave_max(tmax);
    const uint32_t k_eff = effective_k(row_topk(p, row), p.vocab);
    if (k_eff != 0) {
        const uint32_t kw = (k_eff + 3) / 4;
        const uint32_t ck = wave_kth_largest_key(rl_float_key(tmax), kw);
        if (lane == 0)
            s_key[wave] = ck;
    }
    if (lane == 0)
        s_red[wave] = wmax;
    __syncthreads();
    const float m = fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
    float z = 0.f;
    if (m != -INFINITY) {
        const float ml = m * 1.4426950408889634f;
#pragma unroll
        for (int i = 0; i < kPerThread; i++)
            z += __builtin_amdgcn_exp2f(fmaf(x[i], 1.4426950408889634f, -ml));
    }
    z = wave_sum(z);
    if (lane == 0)
        s_z[wave] = z;

    // Candidates: key(x) >= clb and x != -inf. For x not NaN that is x >= t
    // with t = the float of clb (the key order is the float order with -0 =
    // +0), t raised to -FLT_MAX when clb is the key of -inf; a NaN x has a key
    // above every non-NaN key, and !(x < t) keeps it too.
    uint32_t cand_lo = 0, cnt = 0, incl = 0;
    float t = 0.f;
    if (k_eff != 0) {
        const uint32_t clb = min(min(s_key[0], s_key[1]), min(s_key[2], s_key[3]));
        cand_lo = clb;
        t = clb == rl_float_key(-INFINITY) ? -__FLT_MAX__ : rl_key_float(clb);
#pragma unroll
        for (int i = 0; i < kPerThread; i++)
            cnt += !(x[i] < t) ? 1u : 0u;
        incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(incl, off);
            if (lane >= off)
                incl += o;
        }
        if (lane == 63)
            s_wtot[wave] = incl;
    }
    __syncthreads();
    if (k_eff != 0 && cnt) {
        uint32_t base = incl - cnt;
        for (int w = 0; w < wave; w++)
            base += s_wtot[w];
        uint2 *cand = p.cand + ((size_t)row * p.splits + split) * kCandStride;
#pragma unroll
        for (int k = 0; k < kPerThread / 4; k++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float v = x[k * 4 + e];
                if (!(v < t)) {
                    if (base < (uint32_t)kCandCap)
                        cand[base] = make_uint2(rl_float_key(v), c0 + (uint32_t)(k * kThreads + tid) * 4u + e);
                    base++;
                }
            }
    }
    if (tid == 0) {
        st->max_x = m;
        st->sum_exp = s_z[0] + s_z[1] + s_z[2] + s_z[3];
        st->arg_val = m;
        st->arg_idx = 0;
        st->n_cand = k_eff != 0 ? s_wtot[0] + s_wtot[1] + s_wtot[2] + s_wtot[3] : 0u;
        st->cand_lo = cand_lo;
        st->draw = draw;
    }
}

// The merge of a greedy row split into p.splits slices (at most 64), by one
// wave: the row's log-sum-exp from the slices' (max, exp-sum) and the lowest
// index holding the row's maximum; lane 0 writes the token and logprob when
// `writer` is set.
__device__ __forceinline__ void greedy_merge_row(const SampleParams &p, uint32_t row, int lane, bool writer)
{
    const SplitStat *st = p.stats + (size_t)row * p.splits;
    float mx = -INFINITY, zs = 0.f;
    float av = -INFINITY;
    uint32_t ai = 0xFFFFFFFFu;
    if ((uint32_t)lane < p.splits) {
        mx = st[lane].max_x;
        zs = st[lane].sum_exp;
        av = st[lane].arg_val;
        ai = st[lane].arg_idx;
    }
    const float m = wave_max(mx);
    const float zterm = (mx == -INFINITY) ? 0.f : zs * exp2f((mx - m) * 1.4426950408889634f);
    const float lse = m + logf(wave_sum(zterm));
    wave_argmax(av, ai);
    if (writer && lane == 0) {
        const uint32_t i = ai >= p.vocab ? 0u : ai;  // all -inf: lowest index
        p.token_out[row] = i;
        // av is the logit at i (for a row of -inf, logit 0 is -inf too): no reload
        p.logprob_out[row] = av - lse;
    }
}

// ---- one workgroup per row, the row streamed in chunks (rows with top-k) -----
// Thread t's quad j of chunk c holds the logits from 2,048 Q c + (512 j + t)
// * 4 (Q quads per thread per chunk), so each wave's load instruction reads
// 1 KiB of consecutive logits
// and each thread's elements ascend in (c, j, e). Two register buffers of
// kStreamQuads quads alternate: the next chunk's loads are in flight while the
// current chunk is processed, so the vector-ALU work overlaps the stream, and
// no slice statistics or candidate lists go through memory. Per chunk:
//   max     x = l * inv_t (masked past the row's end), the quad maxima and the
//           thread's running max;
//   bound   (the chunks of the first kStreamRefreshQuads * 2,048 logits)
//           the minimum over the waves of each wave's ceil(k/8)-th largest
//           running lane max. At least k
//           elements seen so far lie at or above it, so it is a lower bound
//           of the row's k-th largest key, and it only grows. Only the first
//           chunk waits for every wave's entry; later refreshes read whatever
//           entries are there, and the final bound is the largest of the
//           waves' own;
//   sum     sum exp(x - running max) in four partial sums, rescaled when the
//           max grows (the log-sum-exp of the logprob). A NaN or +inf logit
//           turns the sum NaN;
//   append  the elements at or above the bound (a quad is tested by its max
//           first) into the thread's own LDS list of kStreamList entries, so
//           appends need no atomics. An element below the bound in force at
//           its chunk is below the final bound too, hence outside the top k.
// After the last chunk: the block max and log-sum-exp; the lists compacted
// into the candidate buffer, keeping the keys at or above the final bound and
// filling the first radix histogram on the way; then the top-k tail shared
// with the merge kernel. A list overflow, a NaN sum, a kept set beyond
// kKeptCap and rows without top-k take the exact whole-row path. Greedy rows
// keep the (value desc, index asc) argmax instead of candidates.
// Quads per thread per chunk: 16,384 logits (64 KiB) per chunk. At 256 rows of
// 128,256 logits this streams a row ~2.5 us sooner than chunks of 16 quads
// (the last chunk's processing, exposed after the stream, is half as long);
// chunks of 4 quads, or three buffers in flight, were no faster.
constexpr int kStreamQuads = 8;
// Quads per thread over which the bound is raised (four 8-quad chunks). A
// bound raised over 16 quads only lets so many candidates through that the
// lists overflow into the exact path.
constexpr uint32_t kStreamRefreshQuads = 32;
constexpr uint32_t kStreamList = 8;                                       // list entries per thread
// Long rows (above 32,768 logits) take the stream kernel from this many rows
// on: at 128,256 logits, 144 rows (9/16 of the 256 compute units) is where
// one row per compute unit overtakes split and merge.
constexpr uint32_t kStreamMinRows = 144;
constexpr float kLog2e = 1.4426950408889634f;
// Third dword of a gfx9 buffer descriptor for raw (unswizzled) 32-bit data,
// and the load's cache-policy operand for a nontemporal load.
constexpr int kBufferWord3 = 0x00020000;
constexpr int kBufferNontemporal = 2;

// What one thread holds after streaming its part of a row.
struct StreamOut {
    bool greedy;
    float inv_t;
    uint32_t k_eff;
    uint64_t draw;    // the row's Philox draw (when asked for and sampled)
    float mt, zt;     // running max of x and sum exp(x - mt)
    float bv;         // greedy: the running (value desc, index asc) argmax
    uint32_t bi;
    uint32_t nt;      // list entries appended (> kStreamList: overflow)
    uint32_t bound;   // key lower bound of the k_eff-th largest of what was streamed
};

// The streaming part of the stream kernel: nch chunks of Q quads per thread
// from column col0 (see the stream kernel's description), the candidates into
// s_list, the wave bounds through s_bound. Called by every thread of the
// workgroup.
template <int Q>
__device__ __forceinline__ StreamOut stream_row(const SampleParams &p, uint32_t row, uint32_t col0, uint32_t nch,
                                                bool want_draw, uint2 (*s_list)[kMergeThreads], uint32_t *s_bound)
{
    constexpr uint32_t chunk = (uint32_t)kMergeThreads * 4u * Q;
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const float *lrow = p.logits + (size_t)row * p.row_stride;
    const uint32_t V = p.vocab;

    // Buffer loads over the row's stride: the per-load offset is one scalar
    // and the thread's offset one register, so the loads of two chunks fit
    // beside the data; quads past the stride (the chunk after the last one,
    // which the pipeline below also loads) read as 0 without a memory access,
    // and everything past the vocabulary is masked before use.
    const __amdgpu_buffer_rsrc_t rsrc =
        __builtin_amdgcn_make_buffer_rsrc((void *)lrow, (short)0, (int)(p.row_stride * 4u), kBufferWord3);
    const uint32_t voff = tid * 16u;
    auto load = [&](rl_f32x4 (&v)[Q], uint32_t c) {
#pragma unroll
        for (int j = 0; j < Q; j++)
            v[j] = __builtin_bit_cast(rl_f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                    rsrc, (int)voff, (int)((col0 + c * chunk) * 4u + j * kMergeThreads * 16u),
                                                    kBufferNontemporal));
    };

    StreamOut o;
    rl_f32x4 A[Q], B[Q];
    load(A, 0);
    // the row's parameters and Philox draw, while the first loads are in flight
    o.greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);
    o.inv_t = o.greedy ? 1.0f : 1.0f / row_temperature(p, row);
    o.k_eff = o.greedy ? 0u : effective_k(row_topk(p, row), V);
    o.draw = (o.greedy || !want_draw) ? 0ull : rl_sample_draw64(row_seed(p, row), row_step(p, row), row_draw_id(p, row));
    const bool greedy = o.greedy;
    const float inv_t = o.inv_t;
    const uint32_t k_eff = o.k_eff;

    float mt = -INFINITY, zt = 0.f;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    uint32_t nt = 0;
    uint32_t bound = 0;
    float t = INFINITY;  // candidates: !(x < t)

    auto process = [&](rl_f32x4 (&v)[Q], uint32_t c) {
        const uint32_t c0 = col0 + c * chunk;
        if (c0 + chunk > V) {  // workgroup-uniform: the chunk reaches past the row
#pragma unroll
            for (int j = 0; j < Q; j++) {
                const uint32_t col = c0 + (uint32_t)(j * kMergeThreads + tid) * 4u;
#pragma unroll
                for (int e = 0; e < 4; e++)
                    v[j][e] = col + (uint32_t)e < V ? v[j][e] : -INFINITY;
            }
        }
        float qm[Q];
#pragma unroll
        for (int j = 0; j < Q; j++) {
#pragma unroll
            for (int e = 0; e < 4; e++)
                v[j][e] = v[j][e] * inv_t;
            qm[j] = fmaxf(fmaxf(v[j][0], v[j][1]), fmaxf(v[j][2], v[j][3]));
        }
        float m4[Q / 4];
#pragma unroll
        for (int a = 0; a < Q / 4; a++)
            m4[a] = fmaxf(fmaxf(qm[4 * a], qm[4 * a + 1]), fmaxf(qm[4 * a + 2], qm[4 * a + 3]));
        float cm = m4[0];
#pragma unroll
        for (int a = 1; a < Q / 4; a++)
            cm = fmaxf(cm, m4[a]);
        const float mnew = fmaxf(mt, cm);

        if (greedy) {
#pragma unroll
            for (int j = 0; j < Q; j++) {
                if (qm[j] > bv) {  // the quad's lowest index holding its max
                    const uint32_t col = c0 + (uint32_t)(j * kMergeThreads + tid) * 4u;
                    bi = col + (v[j][0] == qm[j] ? 0u : v[j][1] == qm[j] ? 1u : v[j][2] == qm[j] ? 2u : 3u);
                    bv = qm[j];
                }
            }
        } else if (k_eff != 0 && c < kStreamRefreshQuads / Q) {
            // Each wave's entry certifies kw elements of that wave at or above
            // it, so the minimum over the entries bounds the k_eff-th largest
            // from below. After the first chunk's barrier the waves refresh
            // without one: entries only grow, and any mix of older and newer
            // entries still certifies 8 kw >= k_eff elements.
            const uint32_t kw = (k_eff + kMergeWaves - 1) / kMergeWaves;
            const uint32_t ck = wave_kth_largest_key(rl_float_key(mnew), kw);
            if (lane == 0)
                __hip_atomic_store(&s_bound[wave], ck, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            if (c == 0)
                __syncthreads();
            uint32_t b = ck;
#pragma unroll
            for (int w = 0; w < kMergeWaves; w++)
                if (w != wave)
                    b = min(b, __hip_atomic_load(&s_bound[w], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
            b = max(bound, b);
            bound = b;
            // x >= t selects the keys >= bound (the key order is the float
            // order with -0 = +0); the key of -inf admits every finite x
            t = b == rl_float_key(-INFINITY) ? -__FLT_MAX__ : rl_key_float(b);
        }

        // sum exp(x - mt): ml = 0 while every element so far is -inf (or
        // NaN), so that a NaN still reaches the sum
        const float sc = mt == mnew ? 1.0f : __builtin_amdgcn_exp2f((mt - mnew) * kLog2e);
        zt *= sc;
        mt = mnew;
        const float ml = mt == -INFINITY ? 0.f : mt * kLog2e;
        float z4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < Q; j++)
#pragma unroll
            for (int e = 0; e < 4; e++)
                z4[e] += __builtin_amdgcn_exp2f(fmaf(v[j][e], kLog2e, -ml));
        zt += (z4[0] + z4[1]) + (z4[2] + z4[3]);

        if (k_eff != 0) {
#pragma unroll
            for (int j = 0; j < Q; j++) {
                if (!(qm[j] < t)) {
                    const uint32_t col = c0 + (uint32_t)(j * kMergeThreads + tid) * 4u;
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float x = v[j][e];
                        if (!(x < t)) {
                            if (nt < kStreamList)
                                s_list[nt][tid] = make_uint2(rl_float_key(x), col + (uint32_t)e);
                            nt++;
                        }
                    }
                }
            }
        }
    };

    for (uint32_t c = 0; c < nch; c += 2) {
        load(B, c + 1);
        process(A, c);
        load(A, c + 2);
        if (c + 1 < nch)
            process(B, c + 1);
    }
    o.mt = mt;
    o.zt = zt;
    o.bv = bv;
    o.bi = bi;
    o.nt = nt;
    o.bound = bound;
    return o;
}

// The workgroup's max, exp-sum relative to it, flags (1: a NaN sum, 2: a list
// overflow), largest wave bound and (greedy) argmax, through one barrier.
struct StreamTotals {
    float m, zs, av;
    uint32_t ai, flags, key_lo;
};

__device__ __forceinline__ StreamTotals stream_totals(const StreamOut &o, float *s_wm, float *s_wz, float *s_wv,
                                                      uint32_t *s_wi, uint32_t *s_wflag, uint32_t *s_wb)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const float wm = wave_max(o.mt);
    const float wz = wave_sum(o.mt == -INFINITY ? 0.f : o.zt * exp2f((o.mt - wm) * kLog2e));
    const uint32_t wflag = (__ballot(o.zt != o.zt) ? 1u : 0u) | (__ballot(o.nt > kStreamList) ? 2u : 0u);
    float bv = o.bv;
    uint32_t bi = o.bi;
    if (o.greedy)
        wave_argmax(bv, bi);
    if (lane == 0) {
        s_wm[wave] = wm;
        s_wz[wave] = wz;
        s_wflag[wave] = wflag;
        s_wv[wave] = bv;
        s_wi[wave] = bi;
        s_wb[wave] = o.bound;
    }
    __syncthreads();
    StreamTotals r;
    r.m = s_wm[0];
    r.flags = s_wflag[0];
    r.key_lo = s_wb[0];  // the largest of the waves' bounds, each a valid one
    r.av = s_wv[0];
    r.ai = s_wi[0];
#pragma unroll
    for (int w = 1; w < kMergeWaves; w++) {
        r.m = fmaxf(r.m, s_wm[w]);
        r.flags |= s_wflag[w];
        r.key_lo = max(r.key_lo, s_wb[w]);
        if (s_wv[w] > r.av || (s_wv[w] == r.av && s_wi[w] < r.ai)) {
            r.av = s_wv[w];
            r.ai = s_wi[w];
        }
    }
    r.zs = 0.f;
#pragma unroll
    for (int w = 0; w < kMergeWaves; w++)
        r.zs += s_wm[w] == -INFINITY ? 0.f : s_wz[w] * exp2f((s_wm[w] - r.m) * kLog2e);
    return r;
}

// LDS of one streamed row (kMergeThreads threads): the candidate buffer
// (reused by the whole-row path as RowScratch), the per-thread lists, the
// radix histograms, the kept set and the per-wave totals.
struct StreamLds {
    uint2 s_cand[kMergeCap];
    uint2 s_list[kStreamList][kMergeThreads];  // thread t's entries: column t
    uint32_t s_hist[256];
    uint32_t s_h2[2][256];
    unsigned long long s_whist[256];
    uint64_t s_keep[kKeptCap];
    uint64_t s_sort[kKeptCap];
    uint32_t s_w[kKeptCap];
    uint32_t s_idx[kKeptCap];
    BlockShared bs;
    uint32_t s_bound[kMergeWaves];  // each wave's latest candidate bound
    float s_wm[kMergeWaves], s_wz[kMergeWaves], s_wv[kMergeWaves];
    uint32_t s_wi[kMergeWaves], s_wflag[kMergeWaves], s_wb[kMergeWaves];
};
static_assert(sizeof(RowScratch) <= sizeof(StreamLds::s_cand), "row scratch fits the candidate buffer");

// One row sampled by the whole workgroup (kMergeThreads threads, every one of
// them calls it): the row streamed in chunks of Q quads per thread, then the block totals, the
// candidates compacted and the top-k tail (or the exact whole-row path), the
// token and logprob written. L must be LDS; it is free again on return.
template <int Q = kStreamQuads>
__device__ __forceinline__ void stream_sample_row(const SampleParams &p, uint32_t row, StreamLds &L)
{
    const uint32_t tid = threadIdx.x;
    RowScratch &rs = *reinterpret_cast<RowScratch *>(L.s_cand);

    constexpr uint32_t chunk = (uint32_t)kMergeThreads * 4u * Q;  // 16,384 logits at Q = 8
    const uint32_t V = p.vocab;
    const StreamOut so = stream_row<Q>(p, row, 0u, (V + chunk - 1) / chunk, true, L.s_list, L.s_bound);
    const StreamTotals tt = stream_totals(so, L.s_wm, L.s_wz, L.s_wv, L.s_wi, L.s_wflag, L.s_wb);
    const float m = tt.m;
    const float lse = m + logf(tt.zs);

    if (so.greedy) {
        if (tid == 0) {
            p.token_out[row] = tt.ai >= V ? 0u : tt.ai;  // all -inf: lowest index
            p.logprob_out[row] = tt.av - lse;
        }
        return;
    }

    const uint32_t k_eff = so.k_eff;
    const float topp = row_topp(p, row);
    uint32_t tok = 0;
    float xtok = 0.f;
    bool xknown = false;
    bool exact = k_eff == 0 || tt.flags != 0;
    if (!exact) {
        // ---- compact the lists: keys at or above the final bound ------------
        // (every wave's elements at or above it were tested against a bound
        // no higher, so they are all listed)
        const uint32_t key_lo = tt.key_lo;
        const uint32_t key_hi = rl_float_key(m);
        const uint32_t diff = key_lo ^ key_hi;
        const int hb = diff ? 31 - __builtin_clz(diff) : -1;
        const int shift0 = hb >= 7 ? hb - 7 : 0;
        const uint32_t above0 = (hb < 0 || hb >= 31) ? 0u : ~((2u << hb) - 1u);
        const uint32_t prefix0 = key_hi & above0;
        if (tid == 0) {
            L.bs.cnt[1] = 0;
            L.bs.n = 0;
        }
        if (tid < 256)
            L.s_h2[0][tid] = 0;
        const uint32_t nt = so.nt;
        uint32_t own = 0;
#pragma unroll
        for (uint32_t e = 0; e < kStreamList; e++)
            own += (e < nt && L.s_list[e][tid].x >= key_lo) ? 1u : 0u;
        uint64_t total;
        uint32_t pos = (uint32_t)block_excl_scan_u64_inl(own, total, L.bs);  // (synchronises)
        const uint32_t nf = (uint32_t)total;                           // <= kMergeThreads * kStreamList
#pragma unroll
        for (uint32_t e = 0; e < kStreamList; e++) {
            if (e < nt) {
                const uint2 cd = L.s_list[e][tid];
                if (cd.x >= key_lo) {
                    L.s_cand[pos++] = cd;
                    if (hb >= 0 && (cd.x & above0) == prefix0)
                        atomicAdd(&L.s_h2[0][(cd.x >> shift0) & 0xFFu], 1u);
                }
            }
        }
        __syncthreads();
        const TopkPick pk = topk_pick(nf, k_eff, hb, key_hi, prefix0, m, topp, so.draw, V, L.s_cand, L.s_h2, L.s_keep,
                                      L.s_sort, L.s_w, L.s_idx, L.bs);
        tok = pk.tok;
        xtok = pk.xtok;
        xknown = pk.xknown;
        exact = pk.overflow;
    }
    if (exact)
        tok = exact_row_sample(p, row, so.inv_t, k_eff, topp, m, rs, L.s_hist, L.s_whist, L.bs);
    if (tid == 0) {
        p.token_out[row] = tok;
        const float x = xknown ? xtok : p.logits[(size_t)row * p.row_stride + tok] * so.inv_t;
        p.logprob_out[row] = x - lse;
    }
}

}  // namespace
