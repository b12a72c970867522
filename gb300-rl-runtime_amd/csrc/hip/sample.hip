// sample.hip - on-device token sampling for gfx950 (specification: sample.h).
//
// Replaces the reference's serial sample_token (cu/sample.cu:41-123: one
// thread, O(V*k) insertion top-k, xoshiro256** draw, float CDF walk) with a
// two-kernel, HBM-streaming design:
//
//  split  grid (split, row): each 256-thread workgroup streams an 8,192-
//         element slice of one row (32 fp32 per thread, 16-byte loads) and
//         emits: the slice max of x = l * inv_t and sum exp(x - max) (for the
//         log-sum-exp), the slice argmax (greedy), and for top-k the slice's
//         candidates: every element >= a lower bound of the slice's k-th
//         largest value. The bound is the minimum over the four waves of each
//         wave's ceil(k/4)-th largest lane maximum (found with a 32-step ballot
//         radix select), so at least k distinct elements lie above it.
//  merge  grid (row): one 256-thread workgroup merges the slices: global max
//         and log-sum-exp, exact k-th largest among the candidates (4-pass
//         8-bit radix select on LDS histograms, each wave finding the digit
//         with DPP scans), rank sort of the kept set by (x desc, index asc),
//         24-bit integer weights rl_sample_weight(x - max), nucleus prefix,
//         Philox4x32-10 draw and the ascending-index integer CDF walk - in one
//         wave when at most 64 elements are kept.
// Integer weights make every sum exact, so the token is bit-identical to the
// host restatement whatever the reduction order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"
#include "rl_sample_math.h"
#include "sample.h"

namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = 32;
constexpr int kSplitLen = kThreads * kPerThread;  // 8,192 elements
constexpr int kCandCap = 1024;                    // candidates per split
constexpr int kMergeCap = 8192;                   // candidates per row in the merge
constexpr int kKeptCap = 1024;                    // kept (top-k with ties) per row

struct SplitStat {
    float max_x;     // slice max of x
    float sum_exp;   // sum exp(x - max_x) over the slice
    float arg_val;   // greedy: slice max of raw logits
    uint32_t arg_idx;
    uint32_t n_cand;  // candidates written (> kCandCap: overflow)
    uint32_t cand_lo; // every candidate key is >= this
    uint32_t pad[2];
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
    uint32_t *token_out;
    float *logprob_out;
    SplitStat *stats;       // [rows][splits]
    uint2 *cand;            // [rows][splits][kCandCap] (key, index)
};

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

__global__ __launch_bounds__(kThreads) void sample_split_kernel(SampleParams p)
{
    const uint32_t split = blockIdx.x;
    const uint32_t row = blockIdx.y;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    __shared__ float s_red[4];
    __shared__ uint32_t s_red_i[4];
    __shared__ uint32_t s_key[4];
    __shared__ uint32_t s_wtot[4];
    __shared__ uint32_t s_ncand;

    const float *lrow = p.logits + (size_t)row * p.row_stride;
    const uint32_t c0 = split * kSplitLen;
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);
    const float inv_t = greedy ? 1.0f : 1.0f / row_temperature(p, row);

    // Stream the slice: element (k, e) of thread tid is column c0 + (k*256 + tid)*4 + e.
    float x[kPerThread];
#pragma unroll
    for (int k = 0; k < kPerThread / 4; k++) {
        const uint32_t col = c0 + (uint32_t)(k * kThreads + tid) * 4u;
        if (col + 3 < p.vocab) {
            const rl_f32x4 v = __builtin_nontemporal_load((const rl_f32x4 *)(lrow + col));
            x[k * 4 + 0] = v.x;
            x[k * 4 + 1] = v.y;
            x[k * 4 + 2] = v.z;
            x[k * 4 + 3] = v.w;
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++)
                x[k * 4 + e] = (col + e < p.vocab) ? lrow[col + e] : -INFINITY;
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
        __syncthreads();
        if (lane == 0)
            s_red[wave] = z;
        __syncthreads();
        if (tid == 0) {
            st->max_x = m;
            st->sum_exp = s_red[0] + s_red[1] + s_red[2] + s_red[3];
            st->arg_val = m;
            st->arg_idx = mi;
            st->n_cand = 0;
        }
        return;
    }

    // ---- sampling: x = l * inv_t, slice max, sum exp, candidates -------------
    float tmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPerThread; i++) {
        x[i] = x[i] * inv_t;
        tmax = fmaxf(tmax, x[i]);
    }
    const float wmax = wave_max(tmax);
    const uint32_t k_eff = effective_k(row_topk(p, row), p.vocab);
    uint32_t cand_lo = 0;
    if (k_eff != 0) {
        const uint32_t kw = (k_eff + 3) / 4;
        const uint32_t ck = wave_kth_largest_key(rl_float_key(tmax), kw);
        if (lane == 0)
            s_key[wave] = ck;
    }
    if (lane == 0)
        s_red[wave] = wmax;
    if (tid == 0)
        s_ncand = 0;
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

    if (k_eff != 0) {
        const uint32_t clb = min(min(s_key[0], s_key[1]), min(s_key[2], s_key[3]));
        cand_lo = clb;
        // count, block-wide exclusive scan, then write: no per-element ballots
        uint32_t cnt = 0;
#pragma unroll
        for (int i = 0; i < kPerThread; i++)
            cnt += (rl_float_key(x[i]) >= clb && x[i] != -INFINITY) ? 1u : 0u;
        uint32_t incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const uint32_t o = __shfl_up(incl, off);
            if (lane >= off)
                incl += o;
        }
        if (lane == 63)
            s_wtot[wave] = incl;
        __syncthreads();
        uint32_t base = incl - cnt;
        for (int w = 0; w < wave; w++)
            base += s_wtot[w];
        if (tid == 0)
            s_ncand = s_wtot[0] + s_wtot[1] + s_wtot[2] + s_wtot[3];
        uint2 *cand = p.cand + ((size_t)row * p.splits + split) * kCandCap;
        if (cnt) {
#pragma unroll
            for (int k = 0; k < kPerThread / 4; k++)
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float v = x[k * 4 + e];
                    const uint32_t key = rl_float_key(v);
                    if (key >= clb && v != -INFINITY) {
                        if (base < (uint32_t)kCandCap)
                            cand[base] = make_uint2(key, c0 + (uint32_t)(k * kThreads + tid) * 4u + e);
                        base++;
                    }
                }
        }
    }
    __syncthreads();
    if (lane == 0)
        s_red[wave] = z;
    __syncthreads();
    if (tid == 0) {
        st->max_x = m;
        st->sum_exp = s_red[0] + s_red[1] + s_red[2] + s_red[3];
        st->arg_val = m;
        st->arg_idx = 0;
        st->n_cand = s_ncand;
        st->cand_lo = cand_lo;
    }
}

// ---- block-wide helpers of the merge (256 threads = 4 waves) ----------------

constexpr int kMergeThreads = 256;
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
};

// Exclusive prefix over the block in thread order; `total` gets the block sum.
__device__ uint64_t block_excl_scan_u64(uint64_t v, uint64_t &total, BlockShared &bs)
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
// passes bin 255 - t): the highest digit d in [1, 255] for which
// above + sum(bins >= d) reaches need, else 0. `acc` receives
// above + sum(bins > d), the amount ranked strictly above the chosen digit.
__device__ uint32_t block_pick_digit(uint64_t h, uint64_t above, uint64_t need, uint64_t &acc, BlockShared &bs)
{
    const uint32_t r = 255u - threadIdx.x;
    uint64_t total;
    const uint64_t S = block_excl_scan_u64(h, total, bs);  // bins > r
    const bool cross = r >= 1u && above + S < need && above + S + h >= need;
    const uint32_t d = block_max_u32(cross ? r : 0u, bs);
    if (r == d)
        bs.sel64 = above + S;
    __syncthreads();
    acc = bs.sel64;
    __syncthreads();
    return d;
}

// ---- exact full-row path -----------------------------------------------------
// Used for rows without top-k (whole-vocabulary nucleus) and for rows whose
// top-k candidates overflow the slice buffers (massive ties). Streams the row
// from global memory (L2-resident after the first pass) several times:
// radix select of the top-k cutoff on the float keys; the kept weight W_K; the
// nucleus boundary as an exact 64-bit composite key (float key, ~index) found
// by MSB-first radix search on weight histograms; W_P; the ascending-index
// integer CDF walk.
__device__ __forceinline__ uint64_t composite_key(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | (uint64_t)(0xFFFFFFFFu - idx);
}

__device__ uint32_t exact_row_sample(const SampleParams &p, uint32_t row, float inv_t, uint32_t k_eff, float topp,
                                     float m, uint32_t *s_hist, unsigned long long *s_whist, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    const float *l = p.logits + (size_t)row * p.row_stride;
    const uint32_t V = p.vocab;

    // (1) cutoff key: k_eff-th largest finite x (multiplicity counted); 0 keeps all.
    uint32_t cutoff = 0;
    if (k_eff) {
        uint32_t prefix = 0, mask = 0;
        uint64_t need = k_eff;
        for (int pass = 3; pass >= 0; pass--) {
            const int shift = pass * 8;
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
            const uint32_t d = block_pick_digit(s_hist[255 - tid], 0, need, acc, bs);
            prefix |= d << shift;
            mask |= 0xFFu << shift;
            need -= acc;
        }
        cutoff = prefix;
    }

    // (2) W_K
    uint64_t wk_own = 0;
    for (uint32_t i = tid; i < V; i += kMergeThreads) {
        const float x = l[i] * inv_t;
        if (x != -INFINITY && rl_float_key(x) >= cutoff)
            wk_own += rl_sample_weight(x - m);
    }
    const uint64_t wk = block_sum_u64(wk_own, bs);

    // (3) nucleus boundary tau: the largest composite key whose suffix weight reaches thr.
    uint64_t tau = 0;
    if (topp > 0.f && topp < 1.f) {
        const uint64_t thr = rl_topp_threshold(topp, wk);
        uint64_t prefix = 0, mask = 0, above = 0;
        for (int pass = 7; pass >= 0; pass--) {
            const int shift = pass * 8;
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
            const uint32_t d = block_pick_digit(s_whist[255 - tid], above, thr, acc, bs);
            prefix |= (uint64_t)d << shift;
            mask |= 0xFFull << shift;
            above = acc;
        }
        tau = prefix;
    }

    // (4) W_P and the lowest index of P
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

    // (5) ascending-index walk: chunks of 256 threads x 8 contiguous elements
    const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), row_step(p, row), row), wp);
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

// One workgroup of 256 threads per row.
__global__ __launch_bounds__(kMergeThreads) void sample_merge_kernel(SampleParams p)
{
    const uint32_t row = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;

    __shared__ uint2 s_cand[kMergeCap];
    __shared__ uint32_t s_hist[256];
    __shared__ uint32_t s_h2[2][256];
    __shared__ unsigned long long s_whist[256];
    __shared__ uint64_t s_keep[kKeptCap];   // kept composite keys, unordered
    __shared__ uint64_t s_sort[kKeptCap];   // ... sorted descending
    __shared__ uint32_t s_w[kKeptCap];      // weights in sorted order
    __shared__ uint32_t s_idx[kKeptCap];    // token index in sorted order
    __shared__ BlockShared bs;

    const SplitStat *st = p.stats + (size_t)row * p.splits;
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);

    // Global max and log-sum-exp over the slices (splits <= 64: one per lane;
    // every wave computes the same values).
    float mx = -INFINITY, zs = 0.f;
    uint32_t ncand = 0;
    float av = -INFINITY;
    uint32_t ai = 0xFFFFFFFFu, clo = 0xFFFFFFFFu;
    if ((uint32_t)lane < p.splits) {
        mx = st[lane].max_x;
        zs = st[lane].sum_exp;
        ncand = st[lane].n_cand;
        av = st[lane].arg_val;
        ai = st[lane].arg_idx;
        clo = st[lane].n_cand ? st[lane].cand_lo : 0xFFFFFFFFu;
    }
    const float m = wave_max(mx);
    const float zterm = (mx == -INFINITY) ? 0.f : zs * exp2f((mx - m) * 1.4426950408889634f);
    const float lse = m + logf(wave_sum(zterm));

    if (greedy) {
        wave_argmax(av, ai);
        if (tid == 0) {
            const uint32_t i = ai >= p.vocab ? 0u : ai;  // all -inf: lowest index
            p.token_out[row] = i;
            p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + i] - lse;
        }
        return;
    }

    const float inv_t = 1.0f / row_temperature(p, row);
    const uint32_t k_eff = effective_k(row_topk(p, row), p.vocab);
    const float topp = row_topp(p, row);
    const bool split_over = __ballot(ncand > (uint32_t)kCandCap) != 0;
    const uint64_t cum = wave_inclusive_scan_u64(ncand);
    const uint32_t n = (uint32_t)__shfl(cum, 63);
    uint32_t tok;
    if (k_eff == 0 || split_over || n > (uint32_t)kMergeCap) {
        tok = exact_row_sample(p, row, inv_t, k_eff, topp, m, s_hist, s_whist, bs);
    } else {
        // ---- gather the slices' candidates ----------------------------------
        // Flat slot f belongs to the split whose inclusive count first exceeds
        // it; each thread issues all its loads before storing any.
        constexpr int kGather = 8;
        const uint2 *rbase = p.cand + (size_t)row * p.splits * kCandCap;
        for (uint32_t base = 0; base < n; base += kMergeThreads * kGather) {
            uint32_t sp[kGather], excl[kGather];
#pragma unroll
            for (int r = 0; r < kGather; r++)
                sp[r] = excl[r] = 0;
            for (uint32_t t = 0; t < p.splits; t++) {
                const uint32_t inc = rl_readlane((uint32_t)cum, (int)t);
#pragma unroll
                for (int r = 0; r < kGather; r++) {
                    const uint32_t f = base + tid + (uint32_t)r * kMergeThreads;
                    if (inc <= f) {
                        sp[r] = t + 1;
                        excl[r] = inc;
                    }
                }
            }
            uint2 v[kGather];
#pragma unroll
            for (int r = 0; r < kGather; r++) {
                const uint32_t f = base + tid + (uint32_t)r * kMergeThreads;
                v[r] = f < n ? rbase[(size_t)sp[r] * kCandCap + (f - excl[r])] : make_uint2(0u, 0u);
            }
#pragma unroll
            for (int r = 0; r < kGather; r++) {
                const uint32_t f = base + tid + (uint32_t)r * kMergeThreads;
                if (f < n)
                    s_cand[f] = v[r];
            }
        }
        if (tid == 0)
            bs.n = 0;
        s_h2[0][tid] = 0;
        __syncthreads();

        // ---- exact k_eff-th largest key --------------------------------------
        // Every candidate key lies in [key_lo, key_hi] (the slices' bounds and
        // the row max), so the MSB-first radix select starts at the highest bit
        // where those differ: 8-bit digits, and the first pass already spreads
        // the candidates over many bins. The pass's histogram is filled while
        // the other one is cleared; every wave then finds the digit itself:
        // lane l holds bins 255-4l .. 252-4l, a DPP scan gives the count in
        // higher bins, and the digit is the bin where that count reaches need.
        // With fewer than k_eff candidates the row has fewer than k_eff finite
        // logits, and every finite one is kept.
        uint32_t cutoff = 0;
        if (n >= k_eff) {
            const uint32_t key_lo = rl_wave_min_u32(clo);
            const uint32_t key_hi = rl_float_key(m);
            const uint32_t diff = key_lo ^ key_hi;
            if (diff == 0) {
                cutoff = key_hi;
            } else {
                const int hb = 31 - __builtin_clz(diff);
                uint32_t prefix = key_hi & ~((2u << hb) - 1u);
                uint32_t need = k_eff;
                int pass = 0;
                for (int top = hb; top >= 0; top -= 8, pass++) {
                    const int shift = top >= 7 ? top - 7 : 0;
                    const uint32_t above = top >= 31 ? 0u : ~((2u << top) - 1u);
                    uint32_t *H = s_h2[pass & 1];
                    for (uint32_t i = tid; i < n; i += kMergeThreads) {
                        const uint32_t key = s_cand[i].x;
                        if ((key & above) == prefix)
                            atomicAdd(&H[(key >> shift) & 0xFFu], 1u);
                    }
                    __syncthreads();
                    s_h2[(pass & 1) ^ 1][tid] = 0;
                    uint32_t h[4], own = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        h[j] = H[255 - 4 * lane - j];
                        own += h[j];
                    }
                    uint32_t acc = rl_wave_incl_scan_u32(own) - own;
                    int found = -1;
                    uint32_t rem = 0;
#pragma unroll
                    for (int j = 0; j < 4; j++) {
                        if (found < 0 && acc < need && acc + h[j] >= need) {
                            found = 255 - 4 * lane - j;
                            rem = need - acc;
                        }
                        acc += h[j];
                    }
                    const uint64_t hit = __ballot(found >= 0);  // never empty: need <= matching keys
                    const int src = hit ? (int)__ffsll((long long)hit) - 1 : 0;
                    prefix |= (uint32_t)__builtin_amdgcn_readlane(found, src) << shift;
                    need = rl_readlane(rem, src);
                    __syncthreads();
                }
                cutoff = prefix;
            }
        }

        // ---- kept set K = {key >= cutoff} ------------------------------------
        for (uint32_t i = tid; i < n; i += kMergeThreads) {
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
            tok = exact_row_sample(p, row, inv_t, k_eff, topp, m, s_hist, s_whist, bs);
        } else if (nk <= 64u) {
            // ---- one wave: lane i holds sorted element i; with at most 64
            // weights of at most 2^24 every prefix fits in 32 bits ------------
            tok = 0;
            if (tid < 64) {
                const bool valid = (uint32_t)lane < nk;
                const uint64_t ck = valid ? s_keep[lane] : 0ull;  // real keys are > 0
                // rank = kept keys above mine (broadcast LDS reads, independent)
                uint32_t rank = 0;
                for (uint32_t j = 0; j < nk; j++)
                    rank += s_keep[j] > ck ? 1u : 0u;
                if (valid)
                    s_sort[rank] = ck;
                rl_wave_lds_fence();
                const uint64_t cs = valid ? s_sort[lane] : 0ull;
                const uint32_t idx = 0xFFFFFFFFu - (uint32_t)cs;
                const uint32_t w = valid ? rl_sample_weight(rl_key_float((uint32_t)(cs >> 32)) - m) : 0u;
                s_idx[lane] = idx;
                s_w[lane] = w;
                const uint32_t c = rl_wave_incl_scan_u32(w);
                const uint32_t wk = rl_readlane(c, 63);
                uint32_t np = nk;
                if (topp > 0.f && topp < 1.f) {
                    const uint64_t thr = rl_topp_threshold(topp, wk);
                    const uint64_t hit = __ballot(valid && (uint64_t)c >= thr);
                    np = hit ? (uint32_t)__ffsll((long long)hit) : nk;  // first reaching lane + 1
                }
                const uint32_t wp = np ? rl_readlane(c, (int)np - 1) : 0u;
                const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), row_step(p, row), row), wp);
                const bool in_p = (uint32_t)lane < np;
                rl_wave_lds_fence();
                uint32_t s_le = 0;
                for (uint32_t j = 0; j < np; j++)
                    s_le += s_idx[j] <= idx ? s_w[j] : 0u;
                tok = rl_wave_min_u32(in_p && (uint64_t)s_le > u ? idx : 0xFFFFFFFFu);
                if (tok == 0xFFFFFFFFu)  // zero total weight: lowest index of P
                    tok = rl_wave_min_u32(in_p ? idx : 0xFFFFFFFFu);
                if (tok >= p.vocab)      // empty kept set (every logit -inf): token 0
                    tok = 0;
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
            const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), row_step(p, row), row), wp);
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
            if (tok >= p.vocab)      // empty kept set (every logit -inf): token 0
                tok = 0;
        }
    }
    if (tid == 0) {
        p.token_out[row] = tok;
        p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + tok] * inv_t - lse;
    }
}

uint32_t splits_for(uint32_t vocab) { return (vocab + kSplitLen - 1) / kSplitLen; }

struct WsLayout {
    size_t stats_off, cand_off, total;
};

WsLayout ws_layout(const rl_sample_args_t *a)
{
    const size_t splits = splits_for(a->vocab);
    WsLayout w;
    w.stats_off = 0;
    w.cand_off = ((a->rows * splits * sizeof(SplitStat) + 255) / 256) * 256;
    w.total = w.cand_off + (size_t)a->rows * splits * kCandCap * sizeof(uint2);
    return w;
}

int validate(const rl_sample_args_t *a)
{
    if (!a) {
        rl_set_error("rl_hip_sample: NULL args");
        return -1;
    }
    if (!a->logits || !a->token_out || !a->logprob_out) {
        rl_set_error("rl_hip_sample: NULL device pointer");
        return -1;
    }
    if (a->rows == 0 || a->rows > 65535 || a->vocab == 0 || a->row_stride < a->vocab || a->row_stride % 4 != 0) {
        rl_set_error("rl_hip_sample: rows %u vocab %u row_stride %u invalid", a->rows, a->vocab, a->row_stride);
        return -1;
    }
    if (splits_for(a->vocab) > 64) {
        rl_set_error("rl_hip_sample: vocab %u exceeds %d elements", a->vocab, 64 * kSplitLen);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" size_t rl_hip_sample_workspace(const rl_sample_args_t *a)
{
    if (validate(a))
        return 0;
    return ws_layout(a).total;
}

extern "C" int rl_hip_sample(const rl_sample_args_t *a)
{
    if (rl_require_open("rl_hip_sample") || validate(a))
        return -1;
    const WsLayout w = ws_layout(a);
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_sample: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    SampleParams p;
    p.logits = a->logits;
    p.rows = a->rows;
    p.vocab = a->vocab;
    p.row_stride = a->row_stride;
    p.splits = splits_for(a->vocab);
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
    p.token_out = a->token_out;
    p.logprob_out = a->logprob_out;
    uint8_t *ws = (uint8_t *)a->workspace;
    p.stats = (SplitStat *)(ws + w.stats_off);
    p.cand = (uint2 *)(ws + w.cand_off);

    hipLaunchKernelGGL(sample_split_kernel, dim3(p.splits, a->rows), dim3(kThreads), 0, rl_stream(), p);
    if (rl_check_launch("sample_split_kernel launch"))
        return -1;
    hipLaunchKernelGGL(sample_merge_kernel, dim3(a->rows), dim3(kMergeThreads), 0, rl_stream(), p);
    return rl_check_launch("sample_merge_kernel launch");
}
