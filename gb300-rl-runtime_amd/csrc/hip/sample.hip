// sample.hip - on-device token sampling for gfx950 (specification: sample.h).
//
// Replaces the reference's serial sample_token (cu/sample.cu:41-123: one
// thread, O(V*k) insertion top-k, xoshiro256** draw, float CDF walk) with a
// two-kernel, HBM-streaming design:
//
//  split  grid (split, row): each 256-thread workgroup streams a 16,384-
//         element slice of one row (64 fp32 per thread, 16-byte loads) and
//         emits: the slice max of x = l * inv_t and sum exp(x - max) (for the
//         log-sum-exp), the slice argmax (greedy), and for top-k the slice's
//         candidates: every element >= a lower bound of the slice's k-th
//         largest value. The bound is the minimum over the four waves of each
//         wave's ceil(k/4)-th largest lane maximum (found with a 32-step ballot
//         radix select), so at least k distinct elements lie above it.
//  merge  grid (row): one workgroup merges the slices: global max and
//         log-sum-exp, exact k-th largest among the candidates (4-pass 8-bit
//         radix select in LDS), sort of the kept set by (x desc, index asc),
//         24-bit integer weights rl_sample_weight(x - max), nucleus prefix,
//         Philox4x32-10 draw and the ascending-index integer CDF walk.
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
constexpr int kPerThread = 64;
constexpr int kSplitLen = kThreads * kPerThread;  // 16,384 elements
constexpr int kCandCap = 1024;                    // candidates per split
constexpr int kMergeCap = 8192;                   // candidates per row in the merge
constexpr int kKeptCap = 1024;                    // kept (top-k with ties) per row
constexpr int kRegCand = 16;                      // merge fast path: candidates per lane

struct SplitStat {
    float max_x;     // slice max of x
    float sum_exp;   // sum exp(x - max_x) over the slice
    float arg_val;   // greedy: slice max of raw logits
    uint32_t arg_idx;
    uint32_t n_cand;  // candidates written (> kCandCap: overflow)
    uint32_t pad[3];
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

__device__ __forceinline__ float wave_max(float v)
{
    v = rl_row_max(v);
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
    v = rl_row_sum(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
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
                z += exp2f(fmaf(x[i], 1.4426950408889634f, -ml));
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
            z += exp2f(fmaf(x[i], 1.4426950408889634f, -ml));
    }
    z = wave_sum(z);

    if (k_eff != 0) {
        const uint32_t clb = min(min(s_key[0], s_key[1]), min(s_key[2], s_key[3]));
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
    }
}

// ---- single-wave merge helpers ---------------------------------------------

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

__device__ __forceinline__ uint32_t wave_sum_u32(uint32_t v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
        v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
#pragma unroll
    for (int off = 1; off < 64; off <<= 1)
        v = min(v, __shfl_xor(v, off));
    return v;
}


// One wave per row: every barrier below is a single-wave s_barrier.
constexpr int kMergeThreads = 64;

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
                                     float m, uint32_t *s_hist, unsigned long long *s_whist)
{
    const int lane = threadIdx.x;
    const float *l = p.logits + (size_t)row * p.row_stride;
    const uint32_t V = p.vocab;

    // (1) cutoff key: k_eff-th largest finite x (multiplicity counted); 0 keeps all.
    uint32_t cutoff = 0;
    if (k_eff) {
        uint32_t prefix = 0, mask = 0, need = k_eff;
        for (int pass = 3; pass >= 0; pass--) {
            const int shift = pass * 8;
#pragma unroll
            for (int b = 0; b < 4; b++)
                s_hist[lane * 4 + b] = 0;
            __syncthreads();
            for (uint32_t i = lane; i < V; i += kMergeThreads) {
                const float x = l[i] * inv_t;
                const uint32_t key = rl_float_key(x);
                if (x != -INFINITY && (key & mask) == prefix)
                    atomicAdd(&s_hist[(key >> shift) & 0xFFu], 1u);
            }
            __syncthreads();
            if (lane == 0) {
                uint32_t acc = 0;
                int d = 255;
                for (; d > 0; d--) {
                    if (acc + s_hist[d] >= need)
                        break;
                    acc += s_hist[d];
                }
                s_hist[256] = (uint32_t)d;
                s_hist[257] = need - acc;
            }
            __syncthreads();
            prefix |= s_hist[256] << shift;
            mask |= 0xFFu << shift;
            need = s_hist[257];
            __syncthreads();
        }
        cutoff = prefix;
    }

    // (2) W_K
    uint64_t wk_own = 0;
    for (uint32_t i = lane; i < V; i += kMergeThreads) {
        const float x = l[i] * inv_t;
        if (x != -INFINITY && rl_float_key(x) >= cutoff)
            wk_own += rl_sample_weight(x - m);
    }
    const uint64_t wk = __shfl(wave_inclusive_scan_u64(wk_own), 63);

    // (3) nucleus boundary tau: the largest composite key whose suffix weight reaches thr.
    uint64_t tau = 0;
    if (topp > 0.f && topp < 1.f) {
        const uint64_t thr = rl_topp_threshold(topp, wk);
        uint64_t prefix = 0, mask = 0, above = 0;
        for (int pass = 7; pass >= 0; pass--) {
            const int shift = pass * 8;
#pragma unroll
            for (int b = 0; b < 4; b++)
                s_whist[lane * 4 + b] = 0;
            __syncthreads();
            for (uint32_t i = lane; i < V; i += kMergeThreads) {
                const float x = l[i] * inv_t;
                const uint32_t key = rl_float_key(x);
                if (x == -INFINITY || key < cutoff)
                    continue;
                const uint64_t ck = composite_key(key, i);
                if ((ck & mask) == prefix)
                    atomicAdd(&s_whist[(ck >> shift) & 0xFFu], (unsigned long long)rl_sample_weight(x - m));
            }
            __syncthreads();
            if (lane == 0) {
                // Highest digit whose cumulative weight from the top reaches thr
                // (thr >= 1 whenever K is non-empty: the row maximum weighs 2^24).
                uint64_t acc = above;
                int d = 255;
                for (; d > 0; d--) {
                    if (acc + s_whist[d] >= thr)
                        break;
                    acc += s_whist[d];
                }
                s_whist[256] = (unsigned long long)d;
                s_whist[257] = acc;
            }
            __syncthreads();
            prefix |= (uint64_t)s_whist[256] << shift;
            mask |= 0xFFull << shift;
            above = s_whist[257];
            __syncthreads();
        }
        tau = prefix;
    }

    // (4) W_P and the lowest index of P
    uint64_t wp_own = 0;
    uint32_t lowest = 0xFFFFFFFFu;
    for (uint32_t i = lane; i < V; i += kMergeThreads) {
        const float x = l[i] * inv_t;
        const uint32_t key = rl_float_key(x);
        if (x != -INFINITY && key >= cutoff && composite_key(key, i) >= tau) {
            wp_own += rl_sample_weight(x - m);
            lowest = min(lowest, i);
        }
    }
    const uint64_t wp = __shfl(wave_inclusive_scan_u64(wp_own), 63);
    lowest = wave_min_u32(lowest);

    // (5) ascending-index walk: chunks of 64 lanes x 8 contiguous elements
    const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), p.step, row), wp);
    uint64_t carry = 0;
    uint32_t tok = 0xFFFFFFFFu;
    for (uint32_t base = 0; base < V && tok == 0xFFFFFFFFu; base += kMergeThreads * 8) {
        uint64_t w8[8], own = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const uint32_t i = base + lane * 8 + e;
            w8[e] = 0;
            if (i < V) {
                const float x = l[i] * inv_t;
                const uint32_t key = rl_float_key(x);
                if (x != -INFINITY && key >= cutoff && composite_key(key, i) >= tau)
                    w8[e] = rl_sample_weight(x - m);
            }
            own += w8[e];
        }
        const uint64_t incl = wave_inclusive_scan_u64(own);
        const uint64_t total = __shfl(incl, 63);
        if (carry + total > u) {
            uint64_t c = carry + incl - own;
            uint32_t cand = 0xFFFFFFFFu;
#pragma unroll
            for (int e = 0; e < 8; e++) {
                c += w8[e];
                if (cand == 0xFFFFFFFFu && c > u)
                    cand = base + lane * 8 + e;
            }
            tok = wave_min_u32(cand);
        }
        carry += total;
    }
    if (tok == 0xFFFFFFFFu)
        tok = lowest;        // zero total weight: lowest index of P
    if (tok >= V)
        tok = 0;             // every logit -inf
    return tok;
}

__global__ __launch_bounds__(kMergeThreads) void sample_merge_kernel(SampleParams p)
{
    const uint32_t row = blockIdx.x;
    const int lane = threadIdx.x;

    __shared__ uint2 s_cand[kMergeCap];
    __shared__ uint32_t s_hist[258];
    __shared__ unsigned long long s_whist[258];
    __shared__ uint64_t s_sort[kKeptCap];
    __shared__ uint32_t s_w[kKeptCap];
    __shared__ uint32_t s_nk;

    const SplitStat *st = p.stats + (size_t)row * p.splits;
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);

    // Global max and log-sum-exp over the slices (splits <= 64: one per lane).
    float mx = -INFINITY, zs = 0.f;
    uint32_t ncand = 0;
    float av = -INFINITY;
    uint32_t ai = 0xFFFFFFFFu;
    if ((uint32_t)lane < p.splits) {
        mx = st[lane].max_x;
        zs = st[lane].sum_exp;
        ncand = st[lane].n_cand;
        av = st[lane].arg_val;
        ai = st[lane].arg_idx;
    }
    const float m = wave_max(mx);
    const float zterm = (mx == -INFINITY) ? 0.f : zs * exp2f((mx - m) * 1.4426950408889634f);
    const float lse = m + logf(wave_sum(zterm));

    if (greedy) {
        wave_argmax(av, ai);
        if (lane == 0) {
            const uint32_t i = ai >= p.vocab ? 0u : ai;  // all -inf: lowest index
            p.token_out[row] = i;
            p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + i] - lse;
        }
        return;
    }

    const float inv_t = 1.0f / row_temperature(p, row);
    const uint32_t k_eff = effective_k(row_topk(p, row), p.vocab);
    const float topp = row_topp(p, row);
    // ---- gather the slices' candidates --------------------------------------
    const bool split_over = __ballot(ncand > (uint32_t)kCandCap) != 0;
    const uint64_t cum = wave_inclusive_scan_u64(ncand);
    const uint32_t n = (uint32_t)__shfl(cum, 63);
    if (k_eff == 0 || split_over || n > (uint32_t)kMergeCap) {
        const uint32_t tok = exact_row_sample(p, row, inv_t, k_eff, topp, m, s_hist, s_whist);
        if (lane == 0) {
            p.token_out[row] = tok;
            p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + tok] * inv_t - lse;
        }
        return;
    }
    for (uint32_t s = 0; s < p.splits; s++) {
        const uint32_t cnt = __shfl(ncand, s);
        const uint32_t off = (uint32_t)__shfl(cum, s) - cnt;
        const uint2 *src = p.cand + ((size_t)row * p.splits + s) * kCandCap;
        for (uint32_t i = lane; i < cnt; i += kMergeThreads)
            s_cand[off + i] = src[i];
    }
    __syncthreads();

    // ---- fast path: candidates in registers, kept set of at most 64 ---------
    if (n <= (uint32_t)(kMergeThreads * kRegCand)) {
        uint32_t key[kRegCand], idx[kRegCand];
#pragma unroll
        for (int j = 0; j < kRegCand; j++) {
            const uint32_t f = (uint32_t)(j * kMergeThreads + lane);
            const uint2 c = f < n ? s_cand[f] : make_uint2(0u, 0u);  // key 0: below every real key
            key[j] = c.x;
            idx[j] = c.y;
        }
        // exact k_eff-th largest key: MSB-first, counting keys >= candidate
        uint32_t cutoff = 0;
        for (int bit = 31; bit >= 0; bit--) {
            const uint32_t cand = cutoff | (1u << bit);
            uint32_t cnt = 0;
#pragma unroll
            for (int j = 0; j < kRegCand; j++)
                cnt += key[j] >= cand ? 1u : 0u;
            if (wave_sum_u32(cnt) >= k_eff)
                cutoff = cand;
        }
        // (padding slots hold key 0, below every finite key, and are never kept;
        // cutoff itself stays 0 only when the row has fewer than k finite logits)
        uint32_t kept = 0;
#pragma unroll
        for (int j = 0; j < kRegCand; j++)
            kept += (key[j] >= cutoff && key[j] != 0u) ? 1u : 0u;
        const uint32_t nk = wave_sum_u32(kept);
        if (nk <= 64u) {
            // compact the kept set to one element per lane
            uint32_t pos = 0;
            {
                uint32_t incl = kept;
#pragma unroll
                for (int off = 1; off < 64; off <<= 1) {
                    const uint32_t o = __shfl_up(incl, off);
                    if (lane >= off)
                        incl += o;
                }
                pos = incl - kept;
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < kRegCand; j++)
                if (key[j] >= cutoff && key[j] != 0u)
                    s_sort[pos++] = ((uint64_t)key[j] << 32) | (uint64_t)(0xFFFFFFFFu - idx[j]);
            __syncthreads();
            uint64_t mine = (uint32_t)lane < nk ? s_sort[lane] : 0ull;
            // bitonic sort of 64 lanes, descending by (key, ~index)
#pragma unroll
            for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
                for (int stride = size >> 1; stride > 0; stride >>= 1) {
                    const uint64_t other = __shfl_xor(mine, stride);
                    const bool lower = (lane & stride) == 0;
                    const bool desc = (lane & size) == 0;
                    const uint64_t hi = mine > other ? mine : other;
                    const uint64_t lo = mine > other ? other : mine;
                    mine = (lower == desc) ? hi : lo;
                }
            }
            const bool valid = (uint32_t)lane < nk;
            const uint32_t my_idx = 0xFFFFFFFFu - (uint32_t)mine;
            const uint64_t w = valid ? rl_sample_weight(rl_key_float((uint32_t)(mine >> 32)) - m) : 0ull;
            const uint64_t cw = wave_inclusive_scan_u64(w);
            const uint64_t wk = __shfl(cw, 63);
            uint32_t np = nk;
            if (topp > 0.f && topp < 1.f) {
                const uint64_t thr = rl_topp_threshold(topp, wk);
                const uint64_t hit = __ballot(valid && cw >= thr);
                np = hit ? (uint32_t)__ffsll((long long)hit) : nk;  // first reaching lane + 1
            }
            const uint64_t wp = np ? __shfl(cw, np - 1) : 0ull;
            const uint64_t u = rl_mulhi_u64(rl_sample_draw64(row_seed(p, row), p.step, row), wp);
            const bool in_p = (uint32_t)lane < np;
            uint64_t s_le = 0;
            for (uint32_t j = 0; j < np; j++) {
                const uint32_t idx_j = (uint32_t)__shfl((int)my_idx, (int)j);
                const uint64_t w_j = __shfl(w, (int)j);
                if (idx_j <= my_idx)
                    s_le += w_j;
            }
            uint32_t tok = wave_min_u32(in_p && s_le > u ? my_idx : 0xFFFFFFFFu);
            if (tok == 0xFFFFFFFFu)
                tok = wave_min_u32(in_p ? my_idx : 0xFFFFFFFFu);
            if (tok >= p.vocab)
                tok = 0;
            if (lane == 0) {
                p.token_out[row] = tok;
                p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + tok] * inv_t - lse;
            }
            return;
        }
    }

    // ---- exact k_eff-th largest key: 4 passes of 8-bit radix select ----------
    uint32_t prefix = 0, prefix_mask = 0, need = k_eff;
    for (int pass = 3; pass >= 0; pass--) {
        const int shift = pass * 8;
#pragma unroll
        for (int b = 0; b < 4; b++)
            s_hist[lane * 4 + b] = 0;
        __syncthreads();
        for (uint32_t i = lane; i < n; i += kMergeThreads) {
            const uint32_t key = s_cand[i].x;
            if ((key & prefix_mask) == prefix)
                atomicAdd(&s_hist[(key >> shift) & 0xFFu], 1u);
        }
        __syncthreads();
        // Lane l owns digits 4l..4l+3; above = count of digits > 4l+3.
        uint32_t h[4], own = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            h[b] = s_hist[lane * 4 + b];
            own += h[b];
        }
        uint32_t above = 0;  // suffix sum over lanes > lane
        {
            uint32_t v = own;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const uint32_t o = __shfl_down(v, off);
                if (lane + off < 64)
                    v += o;
            }
            above = v - own;
        }
        int found = -1;
        uint32_t rem = 0;
        uint32_t acc = above;
#pragma unroll
        for (int b = 3; b >= 0; b--) {
            if (found < 0 && acc < need && acc + h[b] >= need) {
                found = lane * 4 + b;
                rem = need - acc;
            }
            acc += h[b];
        }
        const uint64_t hit = __ballot(found >= 0);
        const int src = hit ? (int)__ffsll((long long)hit) - 1 : 0;
        const uint32_t digit = hit ? (uint32_t)__shfl(found, src) : 0u;
        need = hit ? __shfl(rem, src) : need;
        prefix |= digit << shift;
        prefix_mask |= 0xFFu << shift;
        __syncthreads();
    }
    const uint32_t cutoff = prefix;

    // ---- kept set K = {key >= cutoff}, sorted by (x desc, index asc) ---------
    if (lane == 0)
        s_nk = 0;
    __syncthreads();
    for (uint32_t i = lane; i < n; i += kMergeThreads) {
        const uint2 c = s_cand[i];
        if (c.x >= cutoff) {
            const uint32_t pos = atomicAdd(&s_nk, 1u);
            if (pos < kKeptCap)
                s_sort[pos] = ((uint64_t)c.x << 32) | (uint64_t)(0xFFFFFFFFu - c.y);
        }
    }
    __syncthreads();
    const uint32_t nk = s_nk;
    if (nk > (uint32_t)kKeptCap) {
        const uint32_t tok = exact_row_sample(p, row, inv_t, k_eff, topp, m, s_hist, s_whist);
        if (lane == 0) {
            p.token_out[row] = tok;
            p.logprob_out[row] = p.logits[(size_t)row * p.row_stride + tok] * inv_t - lse;
        }
        return;
    }
    uint32_t np2 = 1;
    while (np2 < nk)
        np2 <<= 1;
    for (uint32_t i = nk + lane; i < np2; i += kMergeThreads)
        s_sort[i] = 0;  // sorts last in descending order
    __syncthreads();
    for (uint32_t size = 2; size <= np2; size <<= 1) {
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
            for (uint32_t i = lane; i < np2 / 2; i += kMergeThreads) {
                const uint32_t lo = 2 * i - (i & (stride - 1));
                const uint32_t hi = lo + stride;
                const bool desc = (lo & size) == 0;
                const uint64_t a = s_sort[lo], b = s_sort[hi];
                if ((a < b) == desc) {
                    s_sort[lo] = b;
                    s_sort[hi] = a;
                }
            }
            __syncthreads();
        }
    }

    // ---- integer weights; nucleus prefix over the sorted order ----------------
    for (uint32_t i = lane; i < nk; i += kMergeThreads)
        s_w[i] = rl_sample_weight(rl_key_float((uint32_t)(s_sort[i] >> 32)) - m);
    __syncthreads();
    // Lane l owns the contiguous sorted positions [l*per, (l+1)*per).
    const uint32_t per = (nk + kMergeThreads - 1) / kMergeThreads;
    uint64_t own = 0;
    for (uint32_t i = lane * per; i < min(nk, (lane + 1) * per); i++)
        own += s_w[i];
    const uint64_t incl = wave_inclusive_scan_u64(own);
    const uint64_t wk = __shfl(incl, 63);
    uint32_t np = nk;
    if (topp > 0.f && topp < 1.f) {
        const uint64_t thr = rl_topp_threshold(topp, wk);
        // First position whose inclusive prefix reaches thr.
        uint32_t first = 0xFFFFFFFFu;
        uint64_t c = incl - own;
        for (uint32_t i = lane * per; i < min(nk, (lane + 1) * per); i++) {
            c += s_w[i];
            if (c >= thr) {
                first = i;
                break;
            }
        }
        first = wave_min_u32(first);
        np = (first == 0xFFFFFFFFu) ? nk : first + 1;
    }
    uint64_t wp_own = 0;
    for (uint32_t i = lane * per; i < min(np, (lane + 1) * per); i++)
        wp_own += s_w[i];
    const uint64_t wp = __shfl(wave_inclusive_scan_u64(wp_own), 63);

    // ---- draw; smallest index whose ascending-index prefix weight exceeds u ---
    const uint64_t r = rl_sample_draw64(row_seed(p, row), p.step, row);
    const uint64_t u = rl_mulhi_u64(r, wp);
    uint32_t tok = 0xFFFFFFFFu, lowest = 0xFFFFFFFFu;
    for (uint32_t i = lane; i < np; i += kMergeThreads) {
        const uint32_t idx_i = 0xFFFFFFFFu - (uint32_t)s_sort[i];
        lowest = min(lowest, idx_i);
        uint64_t s_le = 0;
        for (uint32_t j = 0; j < np; j++) {
            const uint32_t idx_j = 0xFFFFFFFFu - (uint32_t)s_sort[j];
            if (idx_j <= idx_i)
                s_le += s_w[j];
        }
        if (s_le > u)
            tok = min(tok, idx_i);
    }
    tok = wave_min_u32(tok);
    lowest = wave_min_u32(lowest);
    if (tok == 0xFFFFFFFFu)  // zero total weight: lowest index of P
        tok = lowest;
    if (tok >= p.vocab)      // empty kept set (every logit -inf): token 0
        tok = 0;
    if (lane == 0) {
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
