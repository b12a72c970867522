// sample.hip - on-device token sampling for gfx950 (specification: sample.h).
//
// Replaces the reference's serial sample_token (cu/sample.cu:41-123: one
// thread, O(V*k) insertion top-k, xoshiro256** draw, float CDF walk) with
// HBM-streaming kernels. Batches with top-k take one workgroup per row that
// streams the row in chunks (sample_stream_kernel, below) when the rows are at
// most 32,768 logits or number at least kStreamMinRows, and split + merge when
// fewer long rows would leave most compute units idle. Vocabularies above
// 32,768 without top-k (or greedy) take split + merge too; the others
// (whole-vocabulary nucleus, greedy) one workgroup per row holding the row in
// registers (sample_row_kernel, below).
//
//  split  grid (split, row): each 256-thread workgroup streams an 8,192-
//         element slice of one row (32 fp32 per thread, 16-byte loads) and
//         emits: the slice max of x = l * inv_t and sum exp(x - max) (for the
//         log-sum-exp), the slice argmax (greedy), and for top-k the slice's
//         candidates: every element >= a lower bound of the slice's k-th
//         largest value. The bound is the minimum over the four waves of each
//         wave's ceil(k/4)-th largest lane maximum (found with a 32-step ballot
//         radix select), so at least k distinct elements lie above it. The
//         kernel is VALU-bound once its loads land, so the per-element work is
//         kept small: masking only in a row's last slice, one float compare as
//         the candidate test, two barriers. Slice 0 of each row also computes
//         the row's Philox draw while its loads are in flight.
//  merge  grid (row): one 512-thread workgroup (8 waves) merges the slices:
//         the global max (the log-sum-exp only at the end, for the logprob);
//         the candidates gathered into LDS - wave w takes the lists of slices
//         w and w + 8, their first 256 entries loaded at kernel entry with the
//         slice records, one LDS atomic per wave for eight groups of 64 -
//         keeping only keys at or above the largest slice bound (every slice's
//         bound is below the row's k-th largest key); the exact k-th largest
//         among them by an MSB-first 8-bit radix select on LDS histograms from
//         the highest bit where the candidate keys differ (the first
//         histogram filled during the gather, each wave finding the digit
//         with DPP scans), finished by one wave's ballot select once the
//         chosen bin holds at most 64 keys; rank sort of the kept set by
//         (x desc, index asc); 24-bit integer weights rl_sample_weight(x -
//         max), nucleus prefix and the ascending-index integer CDF walk - in
//         one wave when at most 64 elements are kept. Rows without top-k (a
//         whole-vocabulary nucleus) or whose candidates overflow take the
//         exact full-row path below.
// Integer weights make every sum exact, so the token is bit-identical to the
// host restatement whatever the reduction order.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"
#include "rl_sample_math.h"
#include "sample.h"
#include "sample_core.h"

namespace {

__global__ __launch_bounds__(kThreads) void sample_split_kernel(SampleParams p)
{
    __shared__ SplitLds L;
    split_slice(p, blockIdx.x, blockIdx.y, L);
}

// One workgroup of kMergeThreads threads per row.
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
    // the whole-row path's scratch reuses the candidate buffer
    static_assert(sizeof(RowScratch) <= sizeof(s_cand), "row scratch fits the candidate buffer");
    RowScratch &rs = *reinterpret_cast<RowScratch *>(s_cand);

    const SplitStat *st = p.stats + (size_t)row * p.splits;
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);
    const uint32_t wave = tid >> 6;
    if (greedy) {
        greedy_merge_row(p, row, lane, tid == 0);
        return;
    }

    // Issued before the slice statistics are known, so that the latencies
    // overlap: this wave's first 256 candidates of the lists of splits w and
    // w + 8 (in bounds whatever the split wrote; masked by the counts later),
    // and the row's Philox draw (computed by the row's first split).
    const uint2 *rbase = p.cand + (size_t)row * p.splits * kCandStride;
    uint2 pv[8];
    const uint64_t draw = st[0].draw;
    {
        const uint2 *pf1 = rbase + (size_t)min(wave, p.splits - 1) * kCandStride;
        const uint2 *pf2 = rbase + (size_t)min(wave + kMergeWaves, p.splits - 1) * kCandStride;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            pv[r] = pf1[r * 64 + lane];
            pv[4 + r] = pf2[r * 64 + lane];
        }
    }

    // Global max and log-sum-exp over the slices (splits <= 64: one per lane;
    // every wave computes the same values).
    float mx = -INFINITY, zs = 0.f;
    uint32_t ncand = 0;
    uint32_t clo = 0xFFFFFFFFu;
    if ((uint32_t)lane < p.splits) {
        mx = st[lane].max_x;
        zs = st[lane].sum_exp;
        ncand = st[lane].n_cand;
        clo = st[lane].cand_lo;
    }
    const float m = wave_max(mx);
    // the row's log-sum-exp, needed only for the logprob written at the end
    auto row_lse = [&]() {
        const float zterm = (mx == -INFINITY) ? 0.f : zs * exp2f((mx - m) * 1.4426950408889634f);
        return m + logf(wave_sum(zterm));
    };

    const float inv_t = 1.0f / row_temperature(p, row);
    const uint32_t k_eff = effective_k(row_topk(p, row), p.vocab);
    const float topp = row_topp(p, row);
    const bool split_over = __ballot(ncand > (uint32_t)kCandCap) != 0;
    const uint64_t cum = wave_inclusive_scan_u64(ncand);
    const uint32_t n = (uint32_t)__shfl(cum, 63);
    uint32_t tok = 0;
    // the sampled token's x when the path that chose it holds it (its key is
    // the float l * inv_t itself), so the logprob needs no reload of the logit
    float xtok = 0.f;
    bool xknown = false;
    // the exact whole-row path (one call site, so it is inlined and its
    // pointers stay in their address spaces): no top-k, or too many candidates
    bool exact = k_eff == 0 || split_over || n > (uint32_t)kMergeCap;
    if (!exact) {
        // ---- gather the slices' candidates ----------------------------------
        // Every slice's bound is below its own k-th largest key, hence below
        // the row's: the largest bound is a lower bound of the cutoff, and
        // only candidates at or above it are kept. Wave w copies the lists of
        // splits w, w + 8, ..., four loads per lane in flight, and appends
        // the kept ones (order is irrelevant below).
        const uint32_t key_lo = rl_wave_max_u32(ncand ? clo : 0u);
        // Every kept candidate key lies in [key_lo, key_hi] (the slices' bounds
        // and the row max), so the MSB-first radix select below starts at the
        // highest bit hb where those differ, 8-bit digits. Its first histogram
        // is filled during the gather.
        const uint32_t key_hi = rl_float_key(m);
        const uint32_t diff = key_lo ^ key_hi;
        const int hb = diff ? 31 - __builtin_clz(diff) : -1;
        const int shift0 = hb >= 7 ? hb - 7 : 0;
        const uint32_t above0 = (hb < 0 || hb >= 31) ? 0u : ~((2u << hb) - 1u);
        const uint32_t prefix0 = key_hi & above0;
        if (tid == 0) {
            bs.cnt[0] = 0;
            bs.cnt[1] = 0;
            bs.n = 0;
        }
        if (tid < 256) {
            s_h2[0][tid] = 0;
            s_h2[1][tid] = 0;
        }
        __syncthreads();
        // Wave w copies the lists of splits w and w + 8 (then w + 16 and
        // w + 24, ...): both lists' loads in flight together, one LDS atomic
        // per wave for the eight groups of 64, keeping only keys at or above
        // key_lo (order is irrelevant below).
        for (uint32_t t = wave; t < p.splits; t += 2 * kMergeWaves) {
            const uint32_t t2 = t + kMergeWaves;
            const bool has2 = t2 < p.splits;
            const uint32_t cnt1 = rl_readlane(ncand, (int)t);
            const uint32_t cnt2 = has2 ? rl_readlane(ncand, (int)min(t2, 63u)) : 0u;
            const uint2 *src1 = rbase + (size_t)t * kCandStride;
            const uint2 *src2 = has2 ? rbase + (size_t)t2 * kCandStride : src1;
            const uint32_t last1 = cnt1 ? cnt1 - 1 : 0u, last2 = cnt2 ? cnt2 - 1 : 0u;
            for (uint32_t j0 = 0; j0 < max(cnt1, cnt2); j0 += 256) {
                uint2 v[8];
                if (t == wave && j0 == 0) {
#pragma unroll
                    for (int g = 0; g < 8; g++)
                        v[g] = pv[g];
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        v[r] = src1[min(j0 + (uint32_t)(r * 64 + lane), last1)];
                        v[4 + r] = src2[min(j0 + (uint32_t)(r * 64 + lane), last2)];
                    }
                }
                bool tk[8];
                uint64_t bal[8];
                uint32_t off[8], tot = 0;
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    const uint32_t j = j0 + (uint32_t)((g & 3) * 64 + lane);
                    tk[g] = j < (g < 4 ? cnt1 : cnt2) && v[g].x >= key_lo;
                    bal[g] = __ballot(tk[g]);
                    off[g] = tot;
                    tot += (uint32_t)__popcll(bal[g]);
                }
                uint32_t base = 0;
                if (lane == 0 && tot)
                    base = atomicAdd(&bs.cnt[0], tot);
                base = (uint32_t)__builtin_amdgcn_readfirstlane((int)base);
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    if (tk[g]) {
                        const uint32_t below = __builtin_amdgcn_mbcnt_hi(
                            (uint32_t)(bal[g] >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal[g], 0u));
                        s_cand[base + off[g] + below] = v[g];  // < n <= kMergeCap
                        if (hb >= 0 && (v[g].x & above0) == prefix0)
                            atomicAdd(&s_h2[0][(v[g].x >> shift0) & 0xFFu], 1u);
                    }
                }
            }
        }
        __syncthreads();
        const uint32_t nf = bs.cnt[0];

        const TopkPick pk = topk_pick(nf, k_eff, hb, key_hi, prefix0, m, topp, draw, p.vocab, s_cand, s_h2, s_keep,
                                      s_sort, s_w, s_idx, bs);
        tok = pk.tok;
        xtok = pk.xtok;
        xknown = pk.xknown;
        exact = pk.overflow;
    }
    if (exact)
        tok = exact_row_sample(p, row, inv_t, k_eff, topp, m, rs, s_hist, s_whist, bs);
    if (tid < 64) {
        const float lse = row_lse();
        if (tid == 0) {
            p.token_out[row] = tok;
            const float x = xknown ? xtok : p.logits[(size_t)row * p.row_stride + tok] * inv_t;
            p.logprob_out[row] = x - lse;
        }
    }
}

__global__ __launch_bounds__(kMergeThreads) void sample_stream_kernel(SampleParams p)
{
    __shared__ StreamLds L;
    stream_sample_row(p, blockIdx.x, L);
}

// ---- one workgroup per row, the whole row in registers (vocab <= 32,768) ----
// Wave w holds the 4,096 consecutive logits from 4,096 w in 16 rounds of 256:
// lane l of round j holds the quad at 4,096 w + 256 j + 4 l, so each load
// instruction reads 1 KiB of consecutive logits and each thread's elements
// ascend with (j, e). Rows without top-k only (whole-vocabulary nucleus and
// greedy rows); the host sends batches with top-k to the split and merge
// kernels. With one row per compute unit the kernel is bound by vector-ALU
// issue (a wave64 instruction every 4 cycles per SIMD), so the element loops
// are kept to two passes over the registers:
//   weights  d = x - m, w = floor(e^d 2^24) (rl_sample_weight_f), the float
//            e^d 2^24 summed for the log-sum-exp, and the weight histogram
//            by bin of d
//   gather   per round, the weight in the bins above the nucleus boundary
//            bin, and that bin's members appended to an LDS list
// then, on LDS: the boundary member (members ranked pairwise), the per-round
// nucleus weights (the lanes' round sums reduced through LDS, plus the
// boundary bin's members in the nucleus), the round where the cumulative
// weight first exceeds the draw (one wave), and the element inside it (one
// wave scan).
// Bins: the bin coordinate t = (x - m)(-s) >= 0, s = kRowBins / span, span =
// min(m - min x, 17) (w = 0 beyond 16.64), is a monotone function of x (two
// correctly rounded steps); bin = min(t, kRowBins - 1) truncated. Both passes
// compute t the same way, and the gather tests t against the boundary bin
// as a float. u32 weight sums: a bin that wraps shows as a histogram total
// below W and sends the row to the exact path. The nucleus boundary is the
// composite key tau (x desc, index asc) at which the weights ranked above tau
// sum to less than thr = ceil(p W) and with tau to at least thr: the bin
// where the cumulative weight reaches thr, then its members. A boundary bin
// with more than kRowList members (massive ties) sends the row to the exact
// whole-row path above, which reads it again from memory.
constexpr int kRowRounds = 16;
constexpr uint32_t kRowVocab = (uint32_t)kMergeWaves * kRowRounds * 256u;  // 32,768
constexpr int kRowBins = 8192;
constexpr int kRowPer = kRowBins / kMergeThreads;  // bins per thread in the scan
constexpr int kRowList = 256;

struct RowEntry {
    unsigned long long ck;  // composite key
    uint32_t val;
    uint32_t pad;
};

struct RowLds {
    union {
        uint32_t hist[kRowBins];
        uint32_t lane_rs[kMergeWaves][kRowRounds][64];  // per-lane round sums
    };
    RowEntry list[kRowList];
    unsigned long long rsum[kMergeWaves * kRowRounds];
    float f0[kMergeWaves], f1[kMergeWaves];
    uint32_t u0[kMergeWaves];
    unsigned long long u1[kMergeWaves];
};

// Redefines every element as far as the compiler knows (no instruction is
// emitted): values derived from the elements before this point are computed
// again after it instead of being held in registers across the phases of the
// row kernel, whose elements already take 128 registers per lane.
template <class T>
__device__ __forceinline__ void row_fence(T (&a)[kRowRounds][4])
{
#pragma unroll
    for (int j = 0; j < kRowRounds; j++)
#pragma unroll
        for (int e = 0; e < 4; e++)
            asm volatile("" : "+v"(a[j][e]));
}

// Bin coordinate of x (ns = -s): 0 at the maximum, never negative; +inf for
// -inf (s > 0).
__device__ __forceinline__ float row_t(float x, float m, float ns) { return (x - m) * ns; }

__device__ __forceinline__ uint32_t row_bin(float t)
{
    return (uint32_t)fminf(t, (float)(kRowBins - 1));  // (NaN: the last bin)
}

__device__ __forceinline__ void row_clear_hist(RowLds &L)
{
    for (uint32_t b = threadIdx.x; b < (uint32_t)kRowBins / 4u; b += kMergeThreads)
        reinterpret_cast<uint4 *>(L.hist)[b] = make_uint4(0u, 0u, 0u, 0u);
}

// Block max of a and min of b (every thread gets both).
__device__ __forceinline__ void row_max_min(float &a, float &b, RowLds &L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    a = wave_max(a);
    b = -wave_max(-b);
    if (lane == 0) {
        L.f0[wave] = a;
        L.f1[wave] = b;
    }
    __syncthreads();
    a = L.f0[0];
    b = L.f1[0];
#pragma unroll
    for (int w = 1; w < kMergeWaves; w++) {
        a = fmaxf(a, L.f0[w]);
        b = fminf(b, L.f1[w]);
    }
    __syncthreads();
}

// Block sums of a float and of a per-thread u32 below 2^31 (exact, in 64 bits).
__device__ __forceinline__ void row_sum_f_u(float &f, uint32_t v, uint64_t &total, RowLds &L)
{
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    f = wave_sum(f);
    const uint64_t ws = ((uint64_t)rl_wave_sum_u32(v >> 8) << 8) + rl_wave_sum_u32(v & 0xFFu);
    if (lane == 0) {
        L.f0[wave] = f;
        L.u1[wave] = ws;
    }
    __syncthreads();
    f = 0.f;
    total = 0;
#pragma unroll
    for (int w = 0; w < kMergeWaves; w++) {
        f += L.f0[w];
        total += L.u1[w];
    }
    __syncthreads();
}

// Inclusive scan of a u32 below 2^26 over the wave, exact in 64 bits: two DPP
// scans of its high and low parts.
__device__ __forceinline__ uint64_t row_wave_scan26(uint32_t v)
{
    return ((uint64_t)rl_wave_incl_scan_u32(v >> 8) << 8) + rl_wave_incl_scan_u32(v & 0xFFu);
}

// The bin where the cumulative histogram value (bins in order) reaches need,
// and the value in the bins before it; need in [1, total]. Returns false when
// the histogram total is not W (a bin wrapped). Also clears the list counter.
// (Thread t reads bins 16 t .. 16 t + 15 as four 16-byte reads.)
__device__ __forceinline__ bool row_hist_scan(uint64_t need, uint64_t W, uint32_t &bstar, uint64_t &above,
                                              RowLds &L, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    uint32_t h[kRowPer];
    uint64_t own = 0;
#pragma unroll
    for (int k = 0; k < kRowPer; k += 4) {
        const uint4 v = reinterpret_cast<const uint4 *>(L.hist)[(tid * kRowPer + k) / 4];
        h[k] = v.x;
        h[k + 1] = v.y;
        h[k + 2] = v.z;
        h[k + 3] = v.w;
        own += (uint64_t)v.x + v.y + v.z + v.w;
    }
    uint64_t total;
    const uint64_t excl = block_excl_scan_u64_inl(own, total, bs);
    if (excl < need && excl + own >= need) {  // exactly one thread (when no bin wrapped)
        uint64_t c = excl;
        uint32_t b = 0;
#pragma unroll
        for (int k = 0; k < kRowPer; k++)
            if (c + h[k] < need && b == (uint32_t)k) {
                c += h[k];
                b++;
            }
        bs.n = tid * kRowPer + b;
        bs.sel64 = c;
    }
    if (tid == 0)
        bs.cnt[0] = 0;
    __syncthreads();
    bstar = bs.n;
    above = bs.sel64;
    __syncthreads();
    return total == W;
}

// Appends this lane's element to the LDS list when `take`: one LDS atomic per
// wave and round for the four elements of the round.
__device__ __forceinline__ void row_append4(const bool (&take)[4], const float (&x4)[4], const uint32_t (&v4)[4],
                                            uint32_t idx0, RowLds &L, BlockShared &bs)
{
    uint64_t bal[4];
    uint32_t off[4], tot = 0;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        bal[e] = __ballot(take[e]);
        off[e] = tot;
        tot += (uint32_t)__popcll(bal[e]);
    }
    if (tot == 0)
        return;
    uint32_t pos0 = 0;
    if ((threadIdx.x & 63) == 0)
        pos0 = atomicAdd(&bs.cnt[0], tot);
    pos0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)pos0);
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const uint32_t pos = pos0 + off[e] +
                             __builtin_amdgcn_mbcnt_hi((uint32_t)(bal[e] >> 32),
                                                       __builtin_amdgcn_mbcnt_lo((uint32_t)bal[e], 0u));
        if (take[e] && pos < (uint32_t)kRowList)
            L.list[pos] = RowEntry{composite_key(rl_float_key(x4[e]), idx0 + e), v4[e], 0u};
    }
}

// Member tid of the list (tid < n): publishes (tau, above + value ranked
// above tau + tau's value) when it is the boundary. The caller synchronises.
__device__ __forceinline__ void row_rank(uint32_t n, uint64_t above, uint64_t need, RowLds &L, BlockShared &bs)
{
    const uint32_t tid = threadIdx.x;
    if (tid < n) {
        const RowEntry me = L.list[tid];
        uint64_t s = 0;  // value of the members ranked above me
        // four entries per step, their LDS reads in flight together (the
        // entries past n, read in bounds, count nothing)
        for (uint32_t k = 0; k < n; k += 4) {
            RowEntry o[4];
#pragma unroll
            for (int i = 0; i < 4; i++)
                o[i] = L.list[min(k + i, (uint32_t)kRowList - 1u)];
#pragma unroll
            for (int i = 0; i < 4; i++)
                s += (k + i < n && o[i].ck > me.ck) ? (uint64_t)o[i].val : 0ull;
        }
        if (above + s < need && above + s + me.val >= need) {  // exactly one member
            bs.res64[0] = me.ck;
            bs.res64[1] = above + s + me.val;
        }
    }
}

__global__ __launch_bounds__(kMergeThreads) void sample_row_kernel(SampleParams p)
{
    const uint32_t row = blockIdx.x;
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    __shared__ union {
        RowLds r;
        RowScratch x;  // the exact whole-row path
    } lds;
    __shared__ uint32_t s_hist[256];
    __shared__ unsigned long long s_whist[256];
    __shared__ BlockShared bs;
    RowLds &L = lds.r;

    const float *l = p.logits + (size_t)row * p.row_stride;
    const uint32_t V = p.vocab;
    const uint32_t wave_base = (uint32_t)wave * (kRowRounds * 256u);
    // (base is redefined, as far as the compiler knows, at every phase, so
    // that the 64 element indices are formed again where used, not held)
    uint32_t base = wave_base + (uint32_t)lane * 4u;
    const uint32_t last_quad = (V - 1) & ~3u;
    rl_f32x4 raw[kRowRounds];
#pragma unroll
    for (int j = 0; j < kRowRounds; j++)
        raw[j] = __builtin_nontemporal_load((const rl_f32x4 *)(l + min(base + 256u * j, last_quad)));
    const bool greedy = p.greedy != 0 || !(row_temperature(p, row) > 0.f);
    const float inv_t = greedy ? 1.0f : 1.0f / row_temperature(p, row);
    const uint64_t draw = greedy ? 0ull : rl_sample_draw64(row_seed(p, row), row_step(p, row), row_draw_id(p, row));
    const float topp = row_topp(p, row);
    const bool trunc = !greedy && topp > 0.f && topp < 1.f;
    if (trunc)
        row_clear_hist(L);  // ordered before the atomics by the barriers of the max
    constexpr float kLog2e = 1.4426950408889634f;

    float x[kRowRounds][4];
    float m = -INFINITY, xmin = INFINITY;  // (xmin: -inf when the row holds a -inf logit)
#pragma unroll
    for (int j = 0; j < kRowRounds; j++) {
        if (wave_base + 256u * j + 256u <= V) {  // a round inside the vocabulary (wave-uniform)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                x[j][e] = raw[j][e] * inv_t;
                xmin = fminf(xmin, x[j][e]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const bool in = base + 256u * j + e < V;
                x[j][e] = in ? raw[j][e] * inv_t : -INFINITY;
                xmin = fminf(xmin, in ? x[j][e] : INFINITY);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; e++)
            m = fmaxf(m, x[j][e]);
    }
    row_max_min(m, xmin, L);
    row_fence(x);
    asm volatile("" : "+v"(base));

    if (greedy) {  // the lowest index holding the maximum (0 for a row of -inf)
        uint32_t bi = 0xFFFFFFFFu;
        float z = 0.f;
        const float ml = m * kLog2e;
#pragma unroll
        for (int j = kRowRounds - 1; j >= 0; j--)
#pragma unroll
            for (int e = 3; e >= 0; e--) {
                bi = x[j][e] == m ? base + 256u * j + e : bi;
                z += m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(fmaf(x[j][e], kLog2e, -ml));
            }
        uint64_t unused;
        row_sum_f_u(z, 0u, unused, L);
        bi = rl_wave_min_u32(bi);
        if (lane == 0)
            L.u0[wave] = bi;
        __syncthreads();
        if (tid == 0) {
#pragma unroll
            for (int w = 1; w < kMergeWaves; w++)
                bi = min(bi, L.u0[w]);
            p.token_out[row] = bi;
            p.logprob_out[row] = m - (m + logf(z));
        }
        return;
    }

    // bins over d in [0, span): the row's spread, at most 17
    const float span = fminf(m - xmin, kBinSpan);
    const float sc = span > 0.f ? (float)kRowBins / span : 0.f;
    const float ns = -sc;

    // ---- weights, log-sum-exp terms, the histogram ------------------------------
    uint32_t w[kRowRounds][4];
    float zf = 0.f;
    uint32_t own = 0;  // the weight sum (< 2^31)
    if (trunc) {
#pragma unroll
        for (int j = 0; j < kRowRounds; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float f;
                w[j][e] = rl_sample_weight_f(x[j][e] - m, &f);
                zf += f;
                own += w[j][e];
                atomicAdd(&L.hist[row_bin(row_t(x[j][e], m, ns))], w[j][e]);
            }
    } else {
#pragma unroll
        for (int j = 0; j < kRowRounds; j++)
#pragma unroll
            for (int e = 0; e < 4; e++) {
                float f;
                w[j][e] = rl_sample_weight_f(x[j][e] - m, &f);
                zf += f;
                own += w[j][e];
            }
    }
    uint64_t total;
    row_sum_f_u(zf, own, total, L);  // (synchronises: the histogram is complete)
    // log of the sum of e^(x - m) 2^24, less 24 ln 2
    const float lse = m + (logf(zf) - 16.635532333438686f);

    uint32_t tok = 0;
    float xtok = 0.f;
    bool found = false;  // this lane holds the token
    bool ok = true;
    if (m == -INFINITY) {  // every logit -inf: token 0
        found = tid == 0;
        xtok = x[0][0];
    } else {
        const uint64_t wk = total;
        // ---- the nucleus boundary bin, then one pass: the round weights above
        // it and its members -----------------------------------------------------
        uint32_t bstar = kRowBins;  // every bin below: no truncation
        uint64_t above = 0;
        const uint64_t thr = trunc ? rl_topp_threshold(topp, wk) : 0ull;
        if (trunc)
            ok = row_hist_scan(thr, wk, bstar, above, L, bs);
        // t < lo: a bin below bstar (every t without truncation); lo <= t <
        // hi: bin bstar (the last bin takes every t above it)
        const float lo = bstar >= (uint32_t)kRowBins ? INFINITY : (float)bstar;
        const float hi = bstar >= (uint32_t)(kRowBins - 1) ? INFINITY : (float)(bstar + 1u);
        row_fence(x);
        row_fence(w);
        asm volatile("" : "+v"(base));
#pragma unroll
        for (int j = 0; j < kRowRounds; j++) {
            bool take[4];
            float x4[4];
            uint32_t w4[4], s = 0;  // < 2^26
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const float t = row_t(x[j][e], m, ns);
                const bool below = t < lo;
                s += below ? w[j][e] : 0u;
                take[e] = !below && t < hi;
                x4[e] = x[j][e];
                w4[e] = w[j][e];
            }
            if (trunc)
                row_append4(take, x4, w4, base + 256u * j, L, bs);
            L.lane_rs[wave][j][lane] = s;  // (the histogram is no longer read)
        }
        __syncthreads();
        const uint32_t n = trunc ? bs.cnt[0] : 0u;
        ok = ok && n <= (uint32_t)kRowList;
        if (ok) {
            // round r = 16 wave + j (index order): threads 4r .. 4r + 3 add 16
            // lanes each
            {
                const uint32_t r = tid >> 2, q = tid & 3u;
                const uint32_t *src = &L.lane_rs[r / kRowRounds][r % kRowRounds][q * 16u];
                uint32_t part = 0;  // < 2^30
#pragma unroll
                for (int k = 0; k < 16; k += 4) {
                    const uint4 v = *reinterpret_cast<const uint4 *>(src + k);
                    part += (v.x + v.y) + (v.z + v.w);
                }
                uint64_t rs = part;
                rs += __shfl_xor(rs, 1);
                rs += __shfl_xor(rs, 2);
                if (q == 0)
                    L.rsum[r] = rs;
            }
            if (trunc)
                row_rank(n, above, thr, L, bs);
            __syncthreads();
            uint64_t tau = 0, wp = wk;
            if (trunc) {
                tau = bs.res64[0];
                wp = bs.res64[1];
                // the boundary bin's members in the nucleus join their rounds
                if (tid < n) {
                    const RowEntry me = L.list[tid];
                    if (me.ck >= tau)
                        atomicAdd(&L.rsum[(0xFFFFFFFFu - (uint32_t)me.ck) >> 8], (unsigned long long)me.val);
                }
                __syncthreads();
            }
            // ---- the walk: the round where the cumulative weight first exceeds
            // the draw (wave 0: rounds 2 l and 2 l + 1 on lane l), then the
            // element in it ----------------------------------------------------
            const uint64_t u = rl_mulhi_u64(draw, wp);
            if (wave == 0) {
                const uint64_t r0 = L.rsum[2 * lane], r1 = L.rsum[2 * lane + 1];
                const uint64_t ex = wave_inclusive_scan_u64(r0 + r1) - (r0 + r1);
                if (ex <= u && u < ex + r0) {  // exactly one lane and round: u < W_P
                    bs.n = 2 * lane;
                    bs.sel64 = ex;
                } else if (ex + r0 <= u && u < ex + r0 + r1) {
                    bs.n = 2 * lane + 1;
                    bs.sel64 = ex + r0;
                }
            }
            __syncthreads();
            const uint32_t rstar = bs.n;
            const uint64_t before = bs.sel64;
            row_fence(x);
            row_fence(w);
            asm volatile("" : "+v"(base));
            if ((uint32_t)wave == rstar / kRowRounds) {
                const uint32_t jstar = rstar % kRowRounds;
                uint32_t w4[4] = {0u, 0u, 0u, 0u};
                float x4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < kRowRounds; j++)
                    if ((uint32_t)j == jstar)
#pragma unroll
                        for (int e = 0; e < 4; e++) {
                            w4[e] = w[j][e];
                            x4[e] = x[j][e];
                        }
                const uint32_t i0 = base + 256u * jstar;
                // Nucleus membership as a bit mask: written with || and &&,
                // the short-circuit became divergent branches that cleared w
                // also for the boundary bin's members inside the nucleus.
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    const float t = row_t(x4[e], m, ns);
                    const uint64_t ck = composite_key(rl_float_key(x4[e]), i0 + e);
                    const uint32_t in = (uint32_t)(t < lo) | ((uint32_t)(t >= lo && t < hi) & (uint32_t)(ck >= tau));
                    w4[e] &= 0u - in;
                }
                const uint32_t mine = (w4[0] + w4[1]) + (w4[2] + w4[3]);
                uint64_t c = before + row_wave_scan26(mine) - mine;
                uint32_t cand = 0xFFFFFFFFu;
                float xc = 0.f;
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    c += w4[e];
                    if (cand == 0xFFFFFFFFu && c > u) {
                        cand = i0 + e;
                        xc = x4[e];
                    }
                }
                tok = rl_wave_min_u32(cand);
                found = cand == tok && cand != 0xFFFFFFFFu;
                xtok = xc;
            }
        }
    }
    if (!ok) {  // boundary bin too full: the exact path (uniform: ok comes from LDS)
        __syncthreads();
        tok = exact_row_sample(p, row, inv_t, 0u, topp, m, lds.x, s_hist, s_whist, bs);
        found = tid == 0;
        xtok = l[tok] * inv_t;
    }
    if (found) {
        p.token_out[row] = tok;
        p.logprob_out[row] = xtok - lse;
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
    w.total = w.cand_off + (size_t)a->rows * splits * kCandStride * sizeof(uint2);
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
    if (((uintptr_t)a->logits & 15u) != 0) {
        rl_set_error("rl_hip_sample: logits must be 16-byte aligned");
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

int rl_sample_check(const rl_sample_args_t *a)
{
    return validate(a);
}

int rl_sample_greedy_split(const rl_sample_args_t *a, uint32_t *splits, size_t *cand_off)
{
    if (validate(a))
        return -1;
    const WsLayout w = ws_layout(a);
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_sample: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    // rl_hip_sample's choice: greedy batches of rows above kRowVocab logits
    // take split + merge
    if (!a->greedy || a->vocab <= kRowVocab)
        return 0;
    *splits = splits_for(a->vocab);
    *cand_off = w.cand_off;
    return 1;
}

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
    SampleParams p = sample_params_of(a);
    p.splits = splits_for(a->vocab);
    uint8_t *ws = (uint8_t *)a->workspace;
    p.stats = (SplitStat *)(ws + w.stats_off);
    p.cand = (uint2 *)(ws + w.cand_off);

    // Rows without top-k whose whole row fits one workgroup's registers: the
    // row kernel. Batches with top-k: the stream kernel when the rows are
    // short or fill most of the device (one row per compute unit, so fewer
    // long rows leave it idle), else split and merge. Everything else: split
    // and merge.
    const bool no_topk = !a->top_k && (a->top_k_all == 0 || a->top_k_all >= a->vocab);
    if (a->vocab <= kRowVocab && (no_topk || a->greedy)) {
        hipLaunchKernelGGL(sample_row_kernel, dim3(a->rows), dim3(kMergeThreads), 0, rl_stream(), p);
        return rl_check_launch("sample_row_kernel launch");
    }
    if (!no_topk && !a->greedy && (a->vocab <= kRowVocab || a->rows >= kStreamMinRows)) {
        hipLaunchKernelGGL(sample_stream_kernel, dim3(a->rows), dim3(kMergeThreads), 0, rl_stream(), p);
        return rl_check_launch("sample_stream_kernel launch");
    }
    hipLaunchKernelGGL(sample_split_kernel, dim3(p.splits, a->rows),
                       dim3(kThreads), 0, rl_stream(), p);
    if (rl_check_launch("sample_split_kernel launch"))
        return -1;
    hipLaunchKernelGGL(sample_merge_kernel, dim3(a->rows), dim3(kMergeThreads), 0, rl_stream(), p);
    return rl_check_launch("sample_merge_kernel launch");
}
