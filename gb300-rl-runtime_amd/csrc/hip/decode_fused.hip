// decode_fused.hip - one decode step of a micro-batch and the sampling of
// another micro-batch's logits in one persistent gfx950 launch, then the
// log-sum-exp merge of split rows with the KV append.
//
// In a rollout loop that keeps two micro-batches of rollouts in flight, step
// t runs the attention of micro-batch t % 2 while the tokens of the other
// micro-batch are drawn from the logits its previous step produced (the
// projection runs between the two). Both halves are HBM streams with no data
// dependence between them, so one launch runs them side by side:
//
//  grid     one 512-thread workgroup (8 waves) per compute unit. Workgroup w
//           runs on XCD w % 8.
//  sample   workgroups 0 .. sample_wgs - 1 (a multiple of 8, so each XCD
//           gets the same number) each sample rows w, w + sample_wgs, ...
//           with the streamed one-workgroup-per-row sampler
//           (stream_sample_row, sample_core.h), then stream attention tiles.
//  attend   the tile sequence of the attention (rows (b, g) in order, 16-token
//           tiles, as in attn_decode.hip) is cut into 8 contiguous XCD ranges
//           and each range into one piece per wave of that XCD, weighted: a
//           sampling wave's piece is smaller by the time its workgroup spends
//           sampling, so that both kinds of wave end together. Tiles stream
//           through LDS exactly as in attn_decode.hip (attn_stream,
//           attn_core.h); a row split between pieces leaves one fp32 partial
//           per piece at slot piece + row. The pieces depend only on the
//           step's tile count, so results do not depend on which compute unit
//           streams what.
//  merge    merge_pieces_kernel: the split rows' partials combined by the
//           same log-sum-exp as attn_merge_kernel, and the step's K/V token
//           appended.
//  pipeline rl_hip_decode_pipeline_step launches the fused kernel alone: its
//           sampling waves first merge the previous step's split rows (one
//           wave per row, merge_row_wave) and append that step's K/V token,
//           so a step costs one launch. The lanes (two session streams) let
//           the launch of step t + 1 start on the compute units that step t's
//           last pieces leave idle: the end of a launch is uneven across the
//           XCDs, and on one stream each launch waits for the previous one to
//           finish.
//  loop     ring_loop_kernel: the ring-driven batched step (ring_core.h's
//           turn, then these steps over the rows the turn admitted) as one
//           self-scheduled persistent launch; described where it is defined.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_hip.h"
#include "rl_hip_internal.h"
#include "attn_core.h"
#include "kv_append_core.h"
#include "kv_layout.h"
#include "rl_dev_common.h"
#include "ring_core.h"
#include "sample_core.h"

namespace {

constexpr uint32_t kXcds = 8;                  // MI355X: workgroup w runs on XCD w % 8
constexpr int kFWaves = 8;                     // waves per workgroup
constexpr int kFThreads = kFWaves * 64;
constexpr int kFStages = 2;                    // tile stages per wave (as attn_decode_kernel)
constexpr uint32_t kFusedMaxBatch = 1024;      // rollouts whose tile prefix fits the LDS
static_assert(kFThreads == kMergeThreads, "the sampling role runs the stream sampler's workgroup shape");
// Quads per thread of the sampling role's chunks (16,384 logits, as the stream
// kernel's): the two register buffers beside the attention role's state stay
// within the 256 VGPRs of two waves per SIMD (16 quads spilled).
constexpr int kFusedQuads = 8;

// ---- the split of the tiles among the waves ------------------------------------
// What the split follows from, identically in both kernels once the step's
// tile count U is known.
struct SplitIn {
    uint32_t wgs, sample_wgs;   // workgroups, of which sampling first (multiples of 8)
    uint32_t tile_bytes;        // K and V bytes of one tile
    uint32_t merge_rounds;      // rows of the previous step each sampling wave merges first
    uint64_t sample_bytes;      // logits bytes one sampling workgroup streams
    float sample_cost;          // its time per byte over an attention workgroup's
};

// A sampling workgroup streams its logits slower than an attention workgroup
// streams the same bytes of KV: the top-k tail and the per-chunk processing
// sit on one compute unit. Measured on the 64 x 128,256 (top-k 50, top-p 0.9)
// batch beside the 64-rollout attention: 36-40 us per row, the attention
// workgroups' tiles at about 2.7 us per wave; a factor of 1.8 ended both kinds
// of wave together best (1.0, 1.4, 1.8 and 2.2 tried).
constexpr float kSampleCost = 1.8f;
// A wave's merge of one row of the previous step (pipelined calls) costs
// about as long as an attention workgroup takes to stream this many bytes:
// one round trip for the partials (about 4 us) at a workgroup's share of HBM.
constexpr uint64_t kMergeRoundBytes = 96u * 1024u;

// The pieces of one XCD's N tiles, one per wave of the XCD: the Aa attention
// waves' first (weight 256 each), then the As sampling waves' (weight ws).
// Piece k is [floor(N c_k / W), floor(N c_{k+1} / W)), c_k the weight of the
// pieces before k, W the total. With fewer than 4 tiles per wave the weights
// are equal and only min(waves, N) pieces exist (waves past them idle), so no
// piece is empty.
struct Sched {
    uint32_t N, np, Aw, ws;  // tiles, pieces, pieces of weight 256, weight of the others
    uint64_t W;
};

__host__ __device__ inline Sched sched_of(uint32_t N, uint32_t Aa, uint32_t As, uint32_t ws)
{
    Sched s;
    s.N = N;
    const uint32_t n = Aa + As;
    if (n > 0 && N >= 4u * n) {
        s.np = n;
        s.Aw = Aa;
        s.ws = ws;
    } else {
        s.np = n < N ? n : N;
        s.Aw = s.np;
        s.ws = 256u;
    }
    s.W = 256ull * s.Aw + (uint64_t)s.ws * (s.np - s.Aw);
    return s;
}

__host__ __device__ inline uint32_t piece_start(const Sched &s, uint32_t k)
{
    const uint64_t c = 256ull * (k < s.Aw ? k : s.Aw) + (uint64_t)s.ws * (k > s.Aw ? k - s.Aw : 0u);
    return (uint32_t)(((uint64_t)s.N * c) / s.W);
}

// The piece holding offset o (o < N): the largest k with start(k) <= o, i.e.
// N c_k < (o + 1) W.
__host__ __device__ inline uint32_t piece_at(const Sched &s, uint32_t o)
{
    const uint64_t t = ((uint64_t)o + 1) * s.W;
    if (o < piece_start(s, s.Aw))
        return (uint32_t)((t - 1) / (256ull * s.N));
    return s.Aw + (uint32_t)((t - 256ull * s.Aw * s.N - 1) / ((uint64_t)s.ws * s.N));
}

// XCD x's range of the U tiles: [floor(x U / 8), floor((x + 1) U / 8)).
__host__ __device__ inline uint32_t xcd_start(uint32_t x, uint32_t U)
{
    return (uint32_t)(((uint64_t)x * U) / kXcds);
}

// The schedule of XCD x: a sampling wave's weight is 1 - (sample_cost x its
// workgroup's logits bytes + its merge rounds' equivalent bytes) / a
// workgroup's share of all bytes, at least 1/4.
__host__ __device__ inline Sched sched_x(uint32_t x, uint32_t U, const SplitIn &in)
{
    const uint32_t Aa = (in.wgs - in.sample_wgs) / kXcds * kFWaves;
    const uint32_t As = in.sample_wgs / kXcds * kFWaves;
    const double fair = ((double)U * in.tile_bytes + (double)in.sample_bytes * in.sample_wgs) / in.wgs;
    const double pre = (double)in.sample_cost * (double)in.sample_bytes + (double)in.merge_rounds * kMergeRoundBytes;
    double w = fair > 0.0 ? 1.0 - pre / fair : 1.0;
    w = w < 0.25 ? 0.25 : (w > 1.0 ? 1.0 : w);
    return sched_of(xcd_start(x + 1, U) - xcd_start(x, U), Aa, As, (uint32_t)(w * 256.0 + 0.5));
}

// Global index of the first piece of XCD x: pieces are numbered XCD by XCD,
// so the index grows with the tile position.
__device__ inline uint32_t xcd_base(uint32_t x, uint32_t U, const SplitIn &in)
{
    uint32_t base = 0;
    for (uint32_t y = 0; y < x; y++)
        base += sched_x(y, U, in).np;
    return base;
}

// Global index of the piece holding tile t (t < U).
__device__ inline uint32_t global_piece_of(uint32_t t, uint32_t U, const SplitIn &in)
{
    const uint32_t x = (uint32_t)((((uint64_t)t + 1) * kXcds - 1) / U);
    return xcd_base(x, U, in) + piece_at(sched_x(x, U, in), t - xcd_start(x, U));
}

// ---- the kernels ---------------------------------------------------------------------

struct FusedParams {
    AttnParams p;          // p.part: partials at (piece + row); p.cum: [batch + 1] (written by workgroup 0)
    SampleParams sp;       // the sampled micro-batch
    SplitIn si;
    SplitIn *si_out;       // the workspace's record of si (workgroup 0 writes it)
    // the previous step of a pipeline: its rows merged and its K/V appended
    // by the sampling waves before they sample (has_prev 0: none)
    uint32_t has_prev;
    AttnParams pp;         // its attention, partials and prefix in its workspace
    AppendParams pap;
    const SplitIn *psi;    // its split, recorded by its own call
};

template <int D, int G, int DT, int TPB>
struct FusedLayout {
    using C = Cfg<D, G, DT, TPB>;
    static constexpr int ST_BYTES = kFStages * kFWaves * C::STAGE;
    static constexpr int Q_OFF = ST_BYTES;
    static constexpr int Q_BYTES = kFWaves * kFStages * C::QSLOT;
    static constexpr int CUM_OFF = Q_OFF + Q_BYTES;
    static constexpr int ATTN_END = CUM_OFF + (int)((kFusedMaxBatch + 1) * 4);
    static constexpr int TOTAL = ATTN_END > (int)sizeof(StreamLds) ? ATTN_END : (int)sizeof(StreamLds);
    static constexpr bool FITS = TOTAL <= 160 * 1024;
};

// Largest b < batch with cum[b] <= s (the rollout holding tile s < U; rollouts
// without tiles share their successor's prefix and are skipped).
__device__ __forceinline__ uint32_t rollout_of(RL_LDS const uint32_t *cum, uint32_t batch, uint32_t s)
{
    uint32_t lo = 0, hi = batch;
    while (hi - lo > 1) {
        const uint32_t mid = (lo + hi) >> 1;
        if (cum[mid] <= s)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

// The previous step's split rows merged and its K/V token appended, one row
// per wave: rows w0, w0 + nw, ... of pp (its partials and tile prefix in its
// workspace, its split psi). LIVE: the prefix was written by this launch.
template <int D, int G, int DT, bool LIVE = false>
__device__ __forceinline__ void merge_rows_waves(const AttnParams &pp, const AppendParams &pap, const SplitIn &psi,
                                                 uint32_t w0, uint32_t nw, int lane)
{
    const uint32_t rows = pp.batch * pp.kv_heads;
    const uint32_t Up = LIVE ? rl_live_u32(pp.cum + pp.batch) : rl_sload(pp.cum + pp.batch);
    for (uint32_t r = w0; r < rows; r += nw) {
        const uint32_t b = r / pp.kv_heads, g = r % pp.kv_heads;
        const uint32_t cin = pp.ctx[b];
        const bool bad = cin > pp.max_ctx;
        const uint32_t nu = tiles_of(pp, cin);
        if (nu == 0) {
            empty_row<D, G, DT, G>(pp, b, g, 0, bad, (uint32_t)lane, 64);
        } else {
            const uint32_t R0 = pp.cum[b] + g * nu;
            merge_row_wave<D, G, DT>(pp, b, g, global_piece_of(R0, Up, psi), global_piece_of(R0 + nu - 1, Up, psi),
                                     bad, lane);
        }
        if (pap.arena)
            append_row(pap, b, g, (uint32_t)lane, 64);
    }
}

// The sampling role of a fused step, for workgroups wg < f.si.sample_wgs:
// rows wg, wg + sample_wgs, ... streamed by the whole workgroup.
template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void fused_sample_part(const FusedParams &f, uint8_t *lds, uint32_t wg)
{
    if (wg < f.si.sample_wgs) {
        StreamLds &L = *reinterpret_cast<StreamLds *>(lds);
        for (uint32_t row = wg; row < f.sp.rows; row += f.si.sample_wgs) {
            stream_sample_row<kFusedQuads>(f.sp, row, L);
            __syncthreads();  // L is rewritten by the next row or by the attention below
        }
    }
}

// The attention role of a fused step by workgroup wg of the step's grid
// (f.si.wgs workgroups, workgroup w on XCD w % 8), every thread of it: the
// tile prefix, then each wave's piece. lds is its LDS of FusedLayout::TOTAL
// bytes. LIVE: the contexts and the row map were written by this launch (a
// persistent kernel's turn), so the prefix pass copies them into lctx / lrow
// (LDS, batch entries each) and the attention reads them there, never
// through the scalar cache.
template <int D, int G, int DT, int TPB, bool LIVE = false>
__device__ __forceinline__ void fused_attn_part(const FusedParams &f, uint8_t *lds, uint32_t wg,
                                                RL_LDS uint32_t *lctx = nullptr, RL_LDS uint32_t *lrow = nullptr)
{
    using C = Cfg<D, G, DT, TPB>;
    using LY = FusedLayout<D, G, DT, TPB>;
    const AttnParams &p = f.p;
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)(tid >> 6));
    const bool sampler = wg < f.si.sample_wgs;

    if (wg == 0 && tid == 0)
        *f.si_out = f.si;  // read by the merge kernel, or by the next call of a pipeline
    // ---- tile prefix over the rollouts, in LDS -----------------------------------
    RL_LDS uint32_t *cum = (RL_LDS uint32_t *)(lds + LY::CUM_OFF);
    RL_LDS uint32_t *wtot = (RL_LDS uint32_t *)(lds + LY::Q_OFF);  // q slots as scratch until the copies start
    {
        const uint32_t per = (p.batch + kFThreads - 1) / kFThreads;
        const uint32_t b0 = min(tid * per, p.batch), b1 = min(b0 + per, p.batch);
        uint32_t S = 0;
        for (uint32_t bb = b0; bb < b1; bb++) {
            const uint32_t cb = p.ctx[bb];
            if constexpr (LIVE) {
                lctx[bb] = cb;
                lrow[bb] = p.row_map ? p.row_map[bb] : bb;
            }
            S += tiles_of(p, cb) * p.kv_heads;
        }
        const uint32_t inc = rl_wave_incl_scan_u32(S);
        if (lane == 63)
            wtot[wave] = inc;
        __syncthreads();
        uint32_t before = 0, U = 0;
#pragma unroll
        for (int v = 0; v < kFWaves; v++) {
            const uint32_t t = wtot[v];
            before += v < wave ? t : 0u;
            U += t;
        }
        uint32_t c = before + inc - S;
        for (uint32_t bb = b0; bb < b1; bb++) {
            cum[bb] = c;
            if (wg == 0)
                p.cum[bb] = c;
            c += tiles_of(p, LIVE ? lctx[bb] : p.ctx[bb]) * p.kv_heads;
        }
        if (tid == 0) {
            cum[p.batch] = U;
            if (wg == 0)
                p.cum[p.batch] = U;
        }
        __syncthreads();  // prefix and scratch reads done before any copy lands in the q slots
    }

    // ---- attention role: this wave's piece ---------------------------------------
    const uint32_t U = cum[p.batch];
    if (U == 0)
        return;
    const uint32_t x = wg % kXcds;
    const uint32_t Aa = (f.si.wgs - f.si.sample_wgs) / kXcds * kFWaves;
    const uint32_t k = sampler ? Aa + (wg / kXcds) * kFWaves + (uint32_t)wave
                               : ((wg - f.si.sample_wgs) / kXcds) * kFWaves + (uint32_t)wave;
    const Sched s = sched_x(x, U, f.si);
    if (k >= s.np)
        return;
    const uint32_t x0 = xcd_start(x, U);
    const uint32_t s_begin = x0 + piece_start(s, k);
    const uint32_t s_end = x0 + piece_start(s, k + 1);
    const uint32_t b = rollout_of(cum, p.batch, s_begin);
    RL_LDS uint8_t *st = (RL_LDS uint8_t *)lds + wave * C::STAGE;
    RL_LDS uint8_t *qs = (RL_LDS uint8_t *)lds + LY::Q_OFF + wave * kFStages * C::QSLOT;
    if constexpr (LIVE)
        attn_stream<D, G, DT, TPB, kFStages>(p, CtxLds{lctx, lrow}, xcd_base(x, U, f.si) + k, s_begin, s_end, b,
                                             cum[b], st, kFWaves * C::STAGE, qs, lane);
    else
        attn_stream<D, G, DT, TPB, kFStages>(p, CtxFromArray{p.ctx}, xcd_base(x, U, f.si) + k, s_begin, s_end, b,
                                             cum[b], st, kFWaves * C::STAGE, qs, lane);
}


// One fused step by workgroup wg: the previous pipeline step's rows merged
// (sampling waves, when f.has_prev), the sampling, the attention.
template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void fused_step_body(const FusedParams &f, uint8_t *lds, uint32_t wg)
{
    const int wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    if (wg < f.si.sample_wgs && f.has_prev)
        merge_rows_waves<D, G, DT>(f.pp, f.pap, *f.psi, wg * kFWaves + (uint32_t)wave, f.si.sample_wgs * kFWaves,
                                   (int)(threadIdx.x & 63));
    fused_sample_part<D, G, DT, TPB>(f, lds, wg);
    fused_attn_part<D, G, DT, TPB>(f, lds, wg);
}

template <int D, int G, int DT, int TPB>
__global__ __launch_bounds__(kFThreads) void decode_fused_kernel(FusedParams f)
{
    using LY = FusedLayout<D, G, DT, TPB>;
    static_assert(LY::FITS, "fused step LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LY::TOTAL];
    fused_step_body<D, G, DT, TPB>(f, lds, blockIdx.x);
}

// Combines the partials of every row split across pieces (merge_span), writes
// rows without tiles and appends the step's K/V token (the row's first
// workgroup). HS workgroups of G / HS heads per row, as attn_merge_kernel.
template <int D, int G, int DT, int HS>
__global__ __launch_bounds__(256) void merge_pieces_kernel(AttnParams p, AppendParams ap, const SplitIn *psi)
{
    constexpr int GH = G / HS;
    __shared__ float s_f[kMergeLds * G];
    __shared__ float s_L[G];
    const uint32_t g = blockIdx.x / HS;
    const uint32_t h0 = (blockIdx.x % HS) * GH;
    const uint32_t b = blockIdx.y;
    const uint32_t cin = rl_sload(p.ctx + b);
    const uint32_t U = rl_sload(p.cum + p.batch);
    const uint32_t cum_b = rl_sload(p.cum + b);
    if (ap.arena && h0 == 0 && threadIdx.x >= 192)
        append_row(ap, b, g, threadIdx.x - 192, 64);
    const bool bad = cin > p.max_ctx;
    const uint32_t nu = tiles_of(p, cin);
    if (nu == 0) {
        empty_row<D, G, DT, GH>(p, b, g, h0, bad, threadIdx.x, 256);
        return;
    }
    const SplitIn si = *psi;
    const uint32_t R0 = cum_b + g * nu;
    const uint32_t wf = global_piece_of(R0, U, si);
    const uint32_t wl = global_piece_of(R0 + nu - 1, U, si);
    merge_span<D, G, DT, 256, GH>(p, b, g, h0, wf, wl, bad, threadIdx.x, s_f, s_L);
}

// ---- launcher ----------------------------------------------------------------------

// ---- the self-scheduled ring loop ----------------------------------------------
// One cooperative launch of one workgroup per compute unit runs the
// ring-driven batched step for as many steps as the rings call for, with no
// launch between steps. Three roles:
//  turn   wave 0 of workgroup 0, beside the steps: turn t (ring_core.h)
//         publishes step t - 1 (the hw_worker_sim rule does not depend on
//         the token, so it runs while step t - 1 is still streaming) and
//         admits descriptors for step t into argument set t % 3, once step
//         t - 3's merges have released that set and step workspace t % 3.
//         It releases step t (the go word) as soon as step t - 1's K/V
//         appends are done. Step t - 1's completions become visible once
//         its merges are done: the turn keeps them pending and stores the
//         completion ring's tail when it finds those merges finished (before
//         a later turn, or waiting for them at the end). A turn that has to
//         wait for the host with every row free has the append waves merge
//         the step just published first, so that its completions are
//         visible while it waits.
//  steps  workgroups kLoopService.. (the same number on each XCD; the other
//         workgroups of the first kLoopService, one per XCD, keep the turn
//         off the steps' compute units): step t over argument set and step
//         workspace t % 3 and step t's slots. A workgroup starts step t as
//         soon as it is released, while others may still finish step t - 1
//         (or t - 2). The sampling workgroups merge step t - 1's split rows
//         (one row per wave) once every workgroup has finished that step -
//         before sampling the step's logits if it already has, else after;
//         then every workgroup streams its attention pieces, split rows left
//         as partials for the next step's merges. When the loop ends, the
//         sampling workgroups merge the last step's rows.
//  appends the other waves of the first kLoopService workgroups: once step
//         t is released, its K/V tokens, four (row, kv head) pairs at a time
//         per wave (the attention masks positions past the context, the
//         appended one among them); between steps, the turn's early merges.
// Hand-offs are monotonic counters in the workspace: a release fence and an
// atomic add by the producer, a bounded wait and an acquire fence by the
// consumer. Workgroups may run step t + 2 while others finish step t (never
// t + 3: that needs step t's merges), so the counts of finished steps and of
// merges are kept per step modulo 3. A wait that runs out sets an error word
// that ends every role's loop at its next wait. Cooperative launch keeps
// every workgroup resident, so no wait is for a workgroup that cannot run.
// Step t's merges write output slot t % output_slots while steps t + 1 and
// t + 2 run, so output_slots is at least 3.
constexpr uint32_t kLoopService = kXcds;  // workgroups kept off the steps: the turn's, one per XCD
constexpr uint32_t kLoopAppenders = kLoopService * kFWaves - 1;  // their waves less the turn's
// A merge wave's cost in the loop's split, in the pipelined step's merge
// rounds. The sampling workgroups set the loop's pace (every step they also
// wait for the previous one to finish everywhere before merging it): at 4
// they spent about 73 us sampling and merging and 78 us on attention a step
// against 125 us for an attention workgroup; 9 gives them about a third less
// attention.
constexpr uint32_t kLoopMergeWeight = 9;

struct LoopParams {
    RingParams rp;            // the turn's arguments over argument set 0
    FusedParams f;            // the step over input / output slot 0, argument set 0, step workspace 0
    AppendParams ap;          // the append over input slot 0, argument set 0
    // argument sets and step workspaces 1 and 2 (set 0 is in rp, f and ap)
    struct Set {
        uint32_t *ctx, *pos, *rmap;
        uint64_t *rseed, *rstep;
        uint32_t *cum;
        float *part;
        SplitIn *si_out;
    } set[2];
    size_t q_slot, out_slot;  // bytes per input slot of q, per output slot of the 16-bit outputs
    size_t out32_slot;        // floats per output slot of the fp32 outputs
    size_t logits_slot;       // floats per input slot of the logits
    size_t tok_slot;          // entries per output slot of tokens and logprobs
    size_t kv_slot;           // bytes per input slot of the new K (and V) rows
    uint32_t *row_rollout;    // [output_slots][batch] or nullptr
    uint32_t *steps_run;      // steps the loop ran, written at its end (or nullptr)
    uint32_t input_slots, output_slots;
    uint64_t first_step;
    uint32_t max_steps;
    uint32_t *sync;           // device [kLoopSyncWords], zeroed: see kSync*
    uint64_t go_ticks;        // longest wait for a turn, in 100 MHz clock ticks
    uint64_t bar_ticks;       // longest wait for a step's workgroups or merges
};

enum : uint32_t { kLoopSyncTimeout = 5 };  // stats[3] when a wait of the loop ran out
// The words at LoopParams::sync: the turn's go word; step workgroups done
// with steps 0, 1, 2 modulo 3; sampling workgroups done with the merges of
// steps 0, 1, 2 modulo 3; append waves done with the appends of all steps;
// the error word.
// Then the turn's requests for an early merge (the count of requests, the
// step of the last one) and the append waves' count of merges done for them.
enum : uint32_t { kSyncGo = 0, kSyncSteps = 1, kSyncMerges = 4, kSyncAppends = 7, kSyncError = 8 };
enum : uint32_t { kSyncFlushReq = 9, kSyncFlushStep = 10, kSyncFlushDone = 11 };
constexpr uint32_t kLoopSyncWords = 16;

// Counter of step u modulo 3 among the three at c, and its value once all n
// producers are done with step u.
__device__ __forceinline__ uint32_t par_ctr(uint32_t c, uint32_t u) { return c + u % 3u; }
__device__ __forceinline__ uint32_t par_target(uint32_t u, uint32_t n) { return (u / 3u + 1) * n; }

// The loop's arguments, read from the kernel-argument segment through a
// pointer the optimizer cannot see through: each phase reloads (scalar loads
// of memory that never changes) the fields it uses, instead of every phase's
// fields being hoisted out of the loop and held in registers across all of
// it, which spills. Only the kernel itself has the segment's address
// (a called function gets it as an argument: loop_args_at).
__device__ __forceinline__ const RL_CONST LoopParams &loop_args_at(uint64_t a)
{
    asm volatile("" : "+s"(a));
    return *(const RL_CONST LoopParams *)a;
}

__device__ __forceinline__ const RL_CONST LoopParams &loop_args()
{
    return loop_args_at((uint64_t)__builtin_amdgcn_kernarg_segment_ptr());
}

template <class T>
__device__ __forceinline__ T kcopy(const RL_CONST T &x)
{
    T v;
    __builtin_memcpy(&v, (const void *)&x, sizeof(T));
    return v;
}

__device__ __forceinline__ uint32_t sync_load(const uint32_t *w)
{
    return __hip_atomic_load(const_cast<uint32_t *>(w), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The pause between two polls of a sync word: short at first, then longer
// (hundreds of waves may wait on one word while the steps stream, and each
// poll is a load from the device-coherent copy of that line).
__device__ __forceinline__ void loop_backoff(uint32_t polls)
{
    if (polls < 16)
        __builtin_amdgcn_s_sleep(2);
    else if (polls < 64)
        __builtin_amdgcn_s_sleep(16);
    else
        __builtin_amdgcn_s_sleep(64);
}

// Bounded wait (acquire) until counter sync[c] reaches target. False when
// the wait ran out or another wait did (the error word, then set).
__device__ __forceinline__ bool loop_wait(uint32_t *sync, uint32_t c, uint32_t target, uint64_t limit_ticks)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t polls = 0; sync_load(&sync[c]) < target; polls++) {
        if (sync_load(&sync[kSyncError]) != 0 || __builtin_amdgcn_s_memrealtime() - t0 > limit_ticks) {
            __hip_atomic_store(&sync[kSyncError], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        loop_backoff(polls);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");  // the producers' writes are visible here
    return true;
}

// Bounded wait (acquire) for the turn's word on step t: true to run step t,
// false when the loop ends before it (or a wait ran out). The word is the
// number of steps released, with bit 31 set once no further step will be.
__device__ __forceinline__ bool loop_go(uint32_t *sync, uint32_t t, uint64_t limit_ticks)
{
    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
    for (uint32_t polls = 0;; polls++) {
        const uint32_t v = sync_load(&sync[kSyncGo]);
        if ((v & 0x7FFFFFFFu) > t)
            break;
        if (v >> 31)
            return false;
        if (sync_load(&sync[kSyncError]) != 0 || __builtin_amdgcn_s_memrealtime() - t0 > limit_ticks) {
            __hip_atomic_store(&sync[kSyncError], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            return false;
        }
        loop_backoff(polls);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    return true;
}

// One count for the calling workgroup, after its writes are released
// device-wide. Every thread of the workgroup calls it. Each wave waits for
// its own stores to reach the L2 (the barrier does not wait for other
// waves' stores); then one release - an L2 write-back, which every wave
// doing its own would repeat while other workgroups still stream - covers
// them all.
__device__ __forceinline__ void loop_signal_wg(uint32_t *sync, uint32_t c)
{
    rl_wait_vmcnt<0>();
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        rl_wait_vmcnt<0>();  // the write-back done before the count
        atomicAdd(&sync[c], 1u);
    }
}

// Thread 0 waits (bounded) for counter c to reach target; the workgroup
// follows. False when the wait ran out.
__device__ __forceinline__ bool loop_wait_wg(uint32_t *sync, uint32_t c, uint32_t target, uint64_t limit,
                                             uint32_t *s_flag)
{
    if (threadIdx.x == 0)
        *s_flag = loop_wait(sync, c, target, limit) ? 1u : 0u;
    __syncthreads();
    return *s_flag != 0;
}

// The turn's admission may wait for the host only after the completions
// written so far are visible, step u's (the step just published) among them.
// Earlier steps are merged by the sampling waves of steps already released
// (n sampling workgroups); step u's merges would come with step u + 1, which
// this turn has not released yet, so the append waves merge step u now (the
// sampling waves merge it again later, to the same results).
struct MergedBy {
    static constexpr bool kDefer = true;
    uint32_t *sync;
    uint32_t u, n;
    uint64_t limit;
    __device__ bool ready() const
    {
        if (u >= 1 && !loop_wait(sync, par_ctr(kSyncMerges, u - 1), par_target(u - 1, n), limit))
            return false;
        const uint32_t req = sync_load(&sync[kSyncFlushReq]) + 1;  // the turn alone raises it
        if ((threadIdx.x & 63) == 0) {
            __hip_atomic_store(&sync[kSyncFlushStep], u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            __hip_atomic_store(&sync[kSyncFlushReq], req, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        return loop_wait(sync, kSyncFlushDone, req * kLoopAppenders, limit);
    }
};

// Step t's kernel arguments: argument set and workspace t % 3, slots.
__device__ __forceinline__ FusedParams loop_step_params(const RL_CONST LoopParams &L, uint32_t t)
{
    const uint64_t k = L.first_step + t;
    const size_t si = k % L.input_slots, so = k % L.output_slots;
    FusedParams f = kcopy(L.f);
    if (const uint32_t x = t % 3u) {
        const LoopParams::Set z = kcopy(L.set[x - 1]);
        f.p.ctx = z.ctx;
        f.p.row_map = z.rmap;
        f.p.cum = z.cum;
        f.p.part = z.part;
        f.si_out = z.si_out;
        f.sp.seed = z.rseed;
        f.sp.steps = z.rstep;
        f.sp.draw_ids = z.rmap;
    }
    f.p.q = (const uint16_t *)((const uint8_t *)f.p.q + si * L.q_slot);
    f.p.out = (uint16_t *)((uint8_t *)f.p.out + so * L.out_slot);
    f.p.out_f32 = f.p.out_f32 ? f.p.out_f32 + so * L.out32_slot : nullptr;
    f.sp.logits = f.sp.logits + si * L.logits_slot;
    f.sp.token_out = f.sp.token_out + so * L.tok_slot;
    f.sp.logprob_out = f.sp.logprob_out + so * L.tok_slot;
    return f;
}

// Step u's split rows merged by the sampling waves of workgroup wg (one row
// per wave) - once every step workgroup has finished step u, which the
// caller may already know (wait false) - then counted.
template <int D, int G, int DT>
__device__ __forceinline__ bool loop_merge_step(uint32_t u, uint32_t wg, uint32_t n_wgs, bool wait, uint32_t *s_flag)
{
    if (wait) {
        const RL_CONST LoopParams &L = loop_args();
        if (!loop_wait_wg(L.sync, par_ctr(kSyncSteps, u), par_target(u, n_wgs), L.bar_ticks, s_flag))
            return false;
    }
    const RL_CONST LoopParams &L = loop_args();
    const FusedParams f = loop_step_params(L, u);
    AppendParams none = {};
    none.arena = nullptr;
    const uint32_t wave = (uint32_t)__builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    merge_rows_waves<D, G, DT, true>(f.p, none, f.si, wg * kFWaves + wave, f.si.sample_wgs * kFWaves,
                                     (int)(threadIdx.x & 63));
    loop_signal_wg(L.sync, par_ctr(kSyncMerges, u));
    return true;
}

// The sampling role of step t by sampling workgroup wg, compiled as a
// function of its own: with the sampling code in the same body as the
// attention, the compiler gives up the attention's tight per-tile loop.
// Arguments arrive in vector registers; they are wave-uniform, so they are
// read back from the first lane. args: the kernel-argument segment's address,
// which a called function cannot obtain itself.
template <int D, int G, int DT, int TPB>
__device__ __attribute__((noinline)) void loop_sample_fn(uint32_t args_lo, uint32_t args_hi, uint32_t t_in,
                                                         uint32_t wg_in, uint32_t lds_in)
{
    const auto first = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)v); };
    const uint64_t args = (uint64_t)first(args_lo) | ((uint64_t)first(args_hi) << 32);
    const uint32_t t = first(t_in);
    const uint32_t wg = first(wg_in);
    RL_LDS uint8_t *lds = (RL_LDS uint8_t *)(uintptr_t)first(lds_in);
    fused_sample_part<D, G, DT, TPB>(loop_step_params(loop_args_at(args), t), (uint8_t *)lds, wg);
}

template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void loop_steps(uint32_t wg, uint32_t n_wgs, uint8_t *lds, RL_LDS uint32_t *lctx,
                                           RL_LDS uint32_t *lrow, uint32_t *s_go, uint32_t *s_flag)
{
    const uint32_t n_samp = loop_args().f.si.sample_wgs;
    const bool sampler = wg < n_samp;
    for (uint32_t t = 0;; t++) {
        // (s_go is rewritten only after the barriers of a whole step; s_flag,
        // which the waits below write, may change while s_go is still read)
        if (threadIdx.x == 0) {
            const RL_CONST LoopParams &L = loop_args();
            *s_go = loop_go(L.sync, t, L.go_ticks) ? 1u : 0u;
        }
        __syncthreads();
        if (!*s_go) {
            // the loop ends before step t: the last step's merges
            if (sampler && t > 0)
                (void)loop_merge_step<D, G, DT>(t - 1, wg, n_wgs, true, s_flag);
            break;
        }
        if (sampler) {
            // ---- step t - 1's split rows (first when that step is already done
            // everywhere, else after the sampling), the sampling of step t's logits
            bool merged = t == 0;
            if (!merged) {
                if (threadIdx.x == 0) {
                    const RL_CONST LoopParams &L = loop_args();
                    *s_flag = sync_load(&L.sync[par_ctr(kSyncSteps, t - 1)]) >= par_target(t - 1, n_wgs) ? 1u : 0u;
                }
                __syncthreads();
                if (*s_flag) {
                    if (!loop_merge_step<D, G, DT>(t - 1, wg, n_wgs, true, s_flag))
                        break;
                    merged = true;
                }
            }
            {
                const uint64_t args = (uint64_t)__builtin_amdgcn_kernarg_segment_ptr();
                loop_sample_fn<D, G, DT, TPB>((uint32_t)args, (uint32_t)(args >> 32), t, wg,
                                              (uint32_t)(uintptr_t)(RL_LDS uint8_t *)lds);
            }
            if (!merged && !loop_merge_step<D, G, DT>(t - 1, wg, n_wgs, true, s_flag))
                break;
        }
        fused_attn_part<D, G, DT, TPB, true>(loop_step_params(loop_args(), t), lds, wg, lctx, lrow);
        loop_signal_wg(loop_args().sync, par_ctr(kSyncSteps, t));
    }
}

// Step u's split rows merged by append wave m (one row per wave of the
// kLoopAppenders), once every step workgroup has finished step u; counted in
// kSyncFlushDone. False when a wait ran out.
template <int D, int G, int DT>
__device__ __forceinline__ bool loop_flush_merge(uint32_t u, uint32_t m, int lane)
{
    const RL_CONST LoopParams &L = loop_args();
    if (!loop_wait(L.sync, par_ctr(kSyncSteps, u), par_target(u, L.f.si.wgs), L.bar_ticks))
        return false;
    const FusedParams f = loop_step_params(L, u);
    AppendParams none = {};
    none.arena = nullptr;
    merge_rows_waves<D, G, DT, true>(f.p, none, f.si, m, kLoopAppenders, lane);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
    rl_wait_vmcnt<0>();
    if (lane == 0)
        atomicAdd(&L.sync[kSyncFlushDone], 1u);
    return true;
}

// Append wave m (of kLoopAppenders): step t's K/V tokens, pairs m * 4 +
// lane / 16 + 4 * kLoopAppenders * i, sixteen lanes a pair; then counted.
// While it waits for a step it serves the turn's early-merge requests.
template <int D, int G, int DT>
__device__ __forceinline__ void loop_appends(uint32_t m, int lane)
{
    uint32_t served = 0;
    for (uint32_t t = 0;; t++) {
        bool go = false;
        {
            const RL_CONST LoopParams &L = loop_args();
            uint64_t t0 = __builtin_amdgcn_s_memrealtime();
            for (uint32_t polls = 0;; polls++) {
                const uint32_t v = sync_load(&L.sync[kSyncGo]);
                if ((v & 0x7FFFFFFFu) > t) {
                    go = true;
                    break;
                }
                if (v >> 31)
                    break;
                if (sync_load(&L.sync[kSyncFlushReq]) > served) {
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
                    const uint32_t u = sync_load(&L.sync[kSyncFlushStep]);
                    if (!loop_flush_merge<D, G, DT>(u, m, lane))
                        break;
                    served++;
                    t0 = __builtin_amdgcn_s_memrealtime();
                    polls = 0;
                    continue;
                }
                if (sync_load(&L.sync[kSyncError]) != 0 || __builtin_amdgcn_s_memrealtime() - t0 > L.go_ticks) {
                    __hip_atomic_store(&L.sync[kSyncError], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
                loop_backoff(polls);
            }
        }
        if (!go)
            break;
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        const RL_CONST LoopParams &L = loop_args();
        const uint64_t k = L.first_step + t;
        AppendParams ap = kcopy(L.ap);
        if (const uint32_t x = t % 3u) {
            ap.positions = L.set[x - 1].pos;
            ap.row_map = L.set[x - 1].rmap;
        }
        ap.k_new = ap.k_new + (k % L.input_slots) * L.kv_slot;
        ap.v_new = ap.v_new + (k % L.input_slots) * L.kv_slot;
        const uint32_t pairs = L.f.p.batch * ap.kv_heads;
        for (uint32_t pr = m * 4u + (uint32_t)lane / 16u; pr < pairs; pr += 4u * kLoopAppenders)
            append_row(ap, pr / ap.kv_heads, pr % ap.kv_heads, (uint32_t)lane % 16u, 16);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        rl_wait_vmcnt<0>();
        if (lane == 0)
            atomicAdd(&L.sync[kSyncAppends], 1u);
    }
}

// Completions written by turns but not yet visible, oldest first: the step
// they complete and the completion ring tail that publishes them.
struct PendingTails {
    uint32_t n;
    uint32_t step[3], tail[3];
};

// Stores the tail of every pending entry whose step's merges are done
// (waiting for them when block), in order; false when a wait ran out.
__device__ __forceinline__ bool loop_release(const RL_CONST LoopParams &L, PendingTails &q, bool block, int lane)
{
    uint32_t *sync = L.sync;
    const uint32_t n_samp = L.f.si.sample_wgs;
    uint32_t done = 0, tail = 0;
    for (; done < q.n; done++) {
        const uint32_t u = q.step[done];
        if (block) {
            if (!loop_wait(sync, par_ctr(kSyncMerges, u), par_target(u, n_samp), L.bar_ticks))
                return false;
        } else if (sync_load(&sync[par_ctr(kSyncMerges, u)]) < par_target(u, n_samp)) {
            break;
        } else {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        tail = q.tail[done];
    }
    if (done) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "");
        if (lane == 0)
            sys_store(&L.rp.dq->tail, tail);
        for (uint32_t i = done; i < q.n; i++) {
            q.step[i - done] = q.step[i];
            q.tail[i - done] = q.tail[i];
        }
        q.n -= done;
    }
    return true;
}

__device__ __forceinline__ void loop_turns(uint16_t *s_free, int lane)
{
    uint32_t t = 0;
    bool ok = true;
    PendingTails q;
    q.n = 0;
    for (;; t++) {
        const RL_CONST LoopParams &L = loop_args();
        uint32_t *sync = L.sync;
        const uint32_t n_samp = L.f.si.sample_wgs;
        const bool last = t >= L.max_steps;  // this turn only publishes
        // argument set and workspace t % 3 are free once step t - 3's merges are done
        if (t >= 3 &&
            !(ok = loop_wait(sync, par_ctr(kSyncMerges, t - 3), par_target(t - 3, n_samp), L.bar_ticks)))
            break;
        // completions whose steps are merged become visible; room for this turn's entry
        if (!(ok = loop_release(L, q, q.n == 3, lane)))
            break;
        RingParams rp = kcopy(L.rp);
        if (const uint32_t x = t % 3u) {
            const LoopParams::Set z = kcopy(L.set[x - 1]);
            rp.ctx = z.ctx;
            rp.pos = z.pos;
            rp.rmap = z.rmap;
            rp.rseed = z.rseed;
            rp.rstep = z.rstep;
        }
        const size_t so = (L.first_step + t) % L.output_slots;
        rp.row_rollout = L.row_rollout && !last ? L.row_rollout + so * rp.batch : nullptr;
        TurnOut to;
        const MergedBy rel{sync, t - 1, n_samp, L.bar_ticks};  // used only by turns that publish (t >= 1)
        const uint32_t held = ring_turn(rp, t > 0 ? 1u : 0u, last ? 0u : 1u, s_free, &to, rel);
        if (to.released)
            q.n = 0;  // the turn published every completion so far
        if (to.pending) {
            q.step[q.n] = t - 1;
            q.tail[q.n] = to.dtail;
            q.n++;
        }
        // admission over and every row free: later steps would decode nothing
        const bool end = last || (to.status != kRunning && held == 0);
        // step t reads the K/V tokens step t - 1 appended
        if (!end && t >= 1 && !(ok = loop_wait(sync, kSyncAppends, t * kLoopAppenders, L.bar_ticks)))
            break;
        if (lane == 0) {
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");  // the rows' step arguments before the word
            __hip_atomic_store(&sync[kSyncGo], end ? (t | 0x80000000u) : t + 1, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        }
        if (end) {
            // the last completions: visible once the sampling workgroups' final merges are done
            ok = loop_release(L, q, true, lane);
            break;
        }
    }
    if (lane == 0) {
        const RL_CONST LoopParams &L = loop_args();
        if (!ok)  // make sure every role stops
            __hip_atomic_store(&L.sync[kSyncGo], t | 0x80000000u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (L.steps_run)
            *L.steps_run = t;
        if (!ok || sync_load(&L.sync[kSyncError]) != 0)
            L.rp.stats[3] = kLoopSyncTimeout;
    }
}

template <int D, int G, int DT, int TPB>
__global__ __launch_bounds__(kFThreads) void ring_loop_kernel(LoopParams)
{
    using LY = FusedLayout<D, G, DT, TPB>;
    static_assert(LY::FITS, "fused step LDS");
    static_assert(2 * kMaxBatch <= LY::TOTAL, "the turn's free-row list fits the stage buffers");
    __shared__ __attribute__((aligned(1024))) uint8_t lds[LY::TOTAL];
    __shared__ uint32_t s_ctx[kFusedMaxBatch];  // the step's contexts and table rows (step workgroups)
    __shared__ uint32_t s_row[kFusedMaxBatch];
    __shared__ uint32_t s_go, s_flag;
    if (blockIdx.x >= kLoopService)
        loop_steps<D, G, DT, TPB>(blockIdx.x - kLoopService, gridDim.x - kLoopService, lds,
                                  (RL_LDS uint32_t *)s_ctx, (RL_LDS uint32_t *)s_row, &s_go, &s_flag);
    else if (blockIdx.x == 0 && threadIdx.x < 64)
        loop_turns(reinterpret_cast<uint16_t *>(lds), (int)threadIdx.x);
    else
        loop_appends<D, G, DT>(blockIdx.x * kFWaves + (threadIdx.x >> 6) - 1, (int)(threadIdx.x & 63));
}

struct FusedWs {
    size_t si_off, cum_off, part_off, total;
};

// Partials: at most one per wave-piece plus one per row (slot piece + row).
FusedWs fused_ws(const rl_attn_decode_args_t *a, const SplitIn &si)
{
    FusedWs w;
    const uint32_t G = a->q_heads / a->kv_heads;
    const size_t part = (size_t)G * a->layout.head_dim + 2 * G;
    const size_t rows = (size_t)a->batch * a->kv_heads;
    w.si_off = 0;
    w.cum_off = 256;
    w.part_off = w.cum_off + (((size_t)a->batch + 1) * 4 + 255) / 256 * 256;
    w.total = w.part_off + ((size_t)si.wgs * kFWaves + rows) * part * 4;
    return w;
}

template <int D, int G, int DT, int TPB>
bool fits()
{
    return FusedLayout<D, G, DT, TPB>::FITS;
}

enum : int { kRunFused = 1, kRunMerge = 2 };

template <int D, int G, int DT, int TPB>
int launch(int what, const FusedParams &f, const AppendParams &ap, hipStream_t stream)
{
    if constexpr (!FusedLayout<D, G, DT, TPB>::FITS) {
        rl_set_error("rl_hip_decode_sample_step: shape does not fit the fused step");
        return -1;
    } else {
        if (what & kRunFused) {
            hipLaunchKernelGGL((decode_fused_kernel<D, G, DT, TPB>), dim3(f.si.wgs), dim3(kFThreads), 0, stream, f);
            if (rl_check_launch("decode_fused_kernel launch"))
                return -1;
        }
        if (what & kRunMerge) {
            constexpr int HS = G >= 2 ? G / 2 : 1;
            // rows averaging more partials than the one-workgroup register path
            // holds (16 at two output elements per thread) take workgroups of
            // two heads, as attn_merge_kernel
            const uint64_t rows = (uint64_t)f.p.batch * f.p.kv_heads;
            if (HS > 1 && (uint64_t)f.si.wgs * kFWaves >= 16ull * rows)
                hipLaunchKernelGGL((merge_pieces_kernel<D, G, DT, HS>), dim3(f.p.kv_heads * HS, f.p.batch), dim3(256),
                                   0, stream, f.p, ap, (const SplitIn *)f.si_out);
            else
                hipLaunchKernelGGL((merge_pieces_kernel<D, G, DT, 1>), dim3(f.p.kv_heads, f.p.batch), dim3(256), 0,
                                   stream, f.p, ap, (const SplitIn *)f.si_out);
            if (rl_check_launch("merge_pieces_kernel launch"))
                return -1;
        }
        return 0;
    }
}

template <int D, int G>
bool fits_dt(uint32_t dt, uint32_t tpb)
{
    return dt == RL_DTYPE_BF16 ? (tpb == 16 ? fits<D, G, 0, 16>() : fits<D, G, 0, 32>())
                               : (tpb == 16 ? fits<D, G, 1, 16>() : fits<D, G, 1, 32>());
}

bool shape_fits(uint32_t D, uint32_t G, uint32_t dt, uint32_t tpb)
{
    if (D == 128) {
        switch (G) {
        case 1: return fits_dt<128, 1>(dt, tpb);
        case 2: return fits_dt<128, 2>(dt, tpb);
        case 4: return fits_dt<128, 4>(dt, tpb);
        default: return fits_dt<128, 8>(dt, tpb);
        }
    }
    switch (G) {
    case 1: return fits_dt<64, 1>(dt, tpb);
    case 2: return fits_dt<64, 2>(dt, tpb);
    case 4: return fits_dt<64, 4>(dt, tpb);
    default: return fits_dt<64, 8>(dt, tpb);
    }
}

template <int D, int G>
int launch_dt(int what, const FusedParams &f, const AppendParams &ap, hipStream_t st, uint32_t dt, uint32_t tpb)
{
    if (dt == RL_DTYPE_BF16)
        return tpb == 16 ? launch<D, G, 0, 16>(what, f, ap, st) : launch<D, G, 0, 32>(what, f, ap, st);
    return tpb == 16 ? launch<D, G, 1, 16>(what, f, ap, st) : launch<D, G, 1, 32>(what, f, ap, st);
}

template <int D>
int launch_g(int what, const FusedParams &f, const AppendParams &ap, hipStream_t st, uint32_t G, uint32_t dt,
             uint32_t tpb)
{
    switch (G) {
    case 1: return launch_dt<D, 1>(what, f, ap, st, dt, tpb);
    case 2: return launch_dt<D, 2>(what, f, ap, st, dt, tpb);
    case 4: return launch_dt<D, 4>(what, f, ap, st, dt, tpb);
    default: return launch_dt<D, 8>(what, f, ap, st, dt, tpb);
    }
}

int launch_shape(int what, const rl_attn_decode_args_t *attn, const FusedParams &f, const AppendParams &ap,
                 hipStream_t st)
{
    const uint32_t G = attn->q_heads / attn->kv_heads;
    if (attn->layout.head_dim == 128)
        return launch_g<128>(what, f, ap, st, G, attn->dtype, attn->layout.token_count);
    return launch_g<64>(what, f, ap, st, G, attn->dtype, attn->layout.token_count);
}

// Workgroups of the fused grid (one per compute unit, a multiple of 8) and
// of them the sampling ones: one per row up to 64, never more than half.
void grid_of(uint32_t rows, uint32_t &wgs, uint32_t &sample_wgs, uint32_t avail = 0)
{
    wgs = avail ? avail : rl_cu_count() / kXcds * kXcds;
    if (wgs < 2 * kXcds)
        wgs = 2 * kXcds;
    uint32_t s = (rows + kXcds - 1) / kXcds * kXcds;
    if (s > 64)
        s = 64;
    if (s > wgs / 2)
        s = wgs / 2 / kXcds * kXcds;
    sample_wgs = s;
}

// avail: workgroups the step may use (a multiple of 8; 0: one per compute
// unit).
SplitIn split_in_of(const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp, uint32_t avail = 0)
{
    SplitIn si;
    grid_of(samp->rows, si.wgs, si.sample_wgs, avail);
    si.tile_bytes = 2u * 16u * attn->layout.head_dim * 2u;
    const uint32_t rows_per_wg = (samp->rows + si.sample_wgs - 1) / si.sample_wgs;
    si.sample_bytes = (uint64_t)rows_per_wg * samp->vocab * 4u;
    si.sample_cost = kSampleCost;
    return si;
}

bool fused_eligible(const rl_attn_decode_args_t *a)
{
    const uint32_t G = a->q_heads / a->kv_heads;
    return a->batch <= kFusedMaxBatch && shape_fits(a->layout.head_dim, G, a->dtype, a->layout.token_count);
}

int fused_validate(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                   const rl_sample_args_t *samp, const char *who)
{
    if (rl_require_open(who) || rl_sample_check(samp))
        return -1;
    return append ? rl_decode_step_check(attn, append, who) : rl_attn_check(attn);
}

// The append of a step, or none (arena NULL: the kernels skip it).
AppendParams append_or_none(const rl_kv_append_args_t *append)
{
    if (append)
        return append_params(append);
    AppendParams ap = {};
    ap.arena = nullptr;
    return ap;
}

}  // namespace

extern "C" size_t rl_hip_decode_sample_step_workspace(const rl_attn_decode_args_t *attn,
                                                      const rl_sample_args_t *samp)
{
    if (rl_require_open("rl_hip_decode_sample_step_workspace") || rl_attn_check(attn) || rl_sample_check(samp))
        return 0;
    const size_t fused = fused_ws(attn, split_in_of(attn, samp)).total;
    // the shapes outside the fused kernel run the two steps one after the other
    const size_t a = rl_hip_attn_decode_workspace(attn);
    const size_t s = rl_hip_sample_workspace(samp);
    const size_t split = (a + 255) / 256 * 256 + s;
    return fused_eligible(attn) ? fused : split;
}

namespace {

// The kernel view of an attention call whose prefix and partials live in
// workspace ws (layout w).
AttnParams attn_params_of(const rl_attn_decode_args_t *attn, uint8_t *ws, const FusedWs &w)
{
    AttnParams p;
    p.arena = (const uint8_t *)attn->arena_base;
    p.block_bytes = attn->layout.block_bytes;
    p.arena_blocks = attn->arena_bytes / attn->layout.block_bytes;
    p.table = attn->block_table;
    p.table_stride = attn->table_stride;
    p.row_map = nullptr;
    p.ctx = attn->ctx_lens;
    p.max_ctx = attn->max_ctx;
    p.batch = attn->batch;
    p.q_heads = attn->q_heads;
    p.kv_heads = attn->kv_heads;
    p.q = (const uint16_t *)attn->q;
    p.out = (uint16_t *)attn->out;
    p.out_f32 = attn->out_f32;
    const float scale = attn->scale != 0.f ? attn->scale : 1.0f / sqrtf((float)attn->layout.head_dim);
    p.scale_log2 = scale * 1.4426950408889634f;
    p.nwaves = 0;  // the pieces replace the even split
    p.cum = (uint32_t *)(ws + w.cum_off);
    p.part = (float *)(ws + w.part_off);
    return p;
}

// The fused kernel's arguments for attention `attn` and sampling `samp` on
// workspace ws; the previous pipeline step, if any, filled in by the caller.
FusedParams fused_params_of(const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp, void *workspace,
                            uint32_t merge_rounds, uint32_t avail = 0)
{
    FusedParams f;
    f.si = split_in_of(attn, samp, avail);
    f.si.merge_rounds = merge_rounds;
    const FusedWs w = fused_ws(attn, f.si);
    uint8_t *ws = (uint8_t *)workspace;
    f.si_out = (SplitIn *)(ws + w.si_off);
    f.p = attn_params_of(attn, ws, w);
    f.sp = sample_params_of(samp);
    f.has_prev = 0;
    f.psi = nullptr;
    f.pp = f.p;
    f.pap.arena = nullptr;
    return f;
}

bool same_shape(const rl_attn_decode_args_t *a, const rl_attn_decode_args_t *b)
{
    return a->q_heads == b->q_heads && a->kv_heads == b->kv_heads && a->dtype == b->dtype &&
           a->layout.head_dim == b->layout.head_dim && a->layout.token_count == b->layout.token_count;
}

}  // namespace

namespace {

// rl_hip_decode_sample_step with batch row b reading the block-table row
// row_map[b] (row_map NULL: b itself), for the attention and the append.
int decode_sample_step_rows(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                            const rl_sample_args_t *samp, const uint32_t *row_map, void *workspace,
                            size_t workspace_bytes, const char *who)
{
    if (fused_validate(attn, append, samp, who))
        return -1;
    const size_t need = rl_hip_decode_sample_step_workspace(attn, samp);
    if (!workspace || workspace_bytes < need) {
        rl_set_error("%s: workspace %zu bytes < %zu required", who, workspace_bytes, need);
        return -1;
    }
    if (!fused_eligible(attn)) {
        // One decode step (or the attention alone), then the sampling, on
        // the library stream. A greedy batch that the sampler splits rides
        // in the attention's two launches instead: its slices as workgroups
        // after the attention's (they take compute units as the attention's
        // last waves retire), its row merges in the attention merge's grid.
        // (Running the sampler on a second stream beside the attention or
        // its merge made the step slower: the cross-stream event waits cost
        // more than the overlap saved.)
        const size_t a_bytes = (rl_hip_attn_decode_workspace(attn) + 255) / 256 * 256;
        rl_attn_decode_args_t a = *attn;
        a.workspace = workspace;
        a.workspace_bytes = a_bytes;
        if (!row_map) {
            rl_sample_args_t s = *samp;
            s.workspace = (uint8_t *)workspace + a_bytes;
            s.workspace_bytes = workspace_bytes - a_bytes;
            const int k = rl_decode_step_greedy_side(&a, append, &s);
            if (k <= 0)
                return k;
        }
        int rc;
        if (row_map)
            rc = append ? rl_decode_step_mapped(&a, append, row_map) : rl_attn_mapped(&a, row_map);
        else
            rc = append ? rl_hip_decode_step(&a, append) : rl_hip_attn_decode(&a);
        if (rc)
            return -1;
        rl_sample_args_t s = *samp;
        s.workspace = (uint8_t *)workspace + a_bytes;
        s.workspace_bytes = workspace_bytes - a_bytes;
        return rl_hip_sample(&s);
    }
    FusedParams f = fused_params_of(attn, samp, workspace, 0);
    f.p.row_map = row_map;
    AppendParams ap = append_or_none(append);
    ap.row_map = row_map;
    return launch_shape(kRunFused | kRunMerge, attn, f, ap, rl_stream());
}

}  // namespace

extern "C" int rl_hip_decode_sample_step(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                                         const rl_sample_args_t *samp, void *workspace, size_t workspace_bytes)
{
    return decode_sample_step_rows(attn, append, samp, nullptr, workspace, workspace_bytes,
                                   "rl_hip_decode_sample_step");
}

int rl_decode_sample_step_mapped(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                                 const rl_sample_args_t *samp, const uint32_t *row_map, void *workspace,
                                 size_t workspace_bytes, const char *who)
{
    if (!row_map) {
        rl_set_error("%s: NULL row map", who);
        return -1;
    }
    return decode_sample_step_rows(attn, append, samp, row_map, workspace, workspace_bytes, who);
}

namespace {

int pipeline_step_on(hipStream_t stream, const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp,
                     const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append, void *workspace,
                     void *prev_workspace, size_t workspace_bytes, const char *who)
{
    if (rl_require_open(who) || rl_attn_check(attn) || rl_sample_check(samp))
        return -1;
    if (!fused_eligible(attn)) {
        rl_set_error("%s: the shape does not fit the fused kernel (use rl_hip_decode_sample_step)", who);
        return -1;
    }
    const size_t need = rl_hip_decode_sample_step_workspace(attn, samp);
    if (!workspace || workspace_bytes < need) {
        rl_set_error("%s: workspace %zu bytes < %zu required", who, workspace_bytes, need);
        return -1;
    }
    uint32_t merge_rounds = 0;
    if (prev_attn) {
        if (rl_decode_step_check(prev_attn, prev_append, who))
            return -1;
        if (!same_shape(attn, prev_attn)) {
            rl_set_error("%s: the previous step's heads, dtype or layout differ from this step's", who);
            return -1;
        }
        if (!prev_workspace || prev_workspace == workspace ||
            workspace_bytes < fused_ws(prev_attn, split_in_of(prev_attn, samp)).total) {
            rl_set_error("%s: the previous step needs its own workspace of this size", who);
            return -1;
        }
        const uint32_t rows = prev_attn->batch * prev_attn->kv_heads;
        uint32_t wgs, sample_wgs;
        grid_of(samp->rows, wgs, sample_wgs);
        merge_rounds = (rows + sample_wgs * kFWaves - 1) / (sample_wgs * kFWaves);
    }
    FusedParams f = fused_params_of(attn, samp, workspace, merge_rounds);
    if (prev_attn) {
        const FusedWs pw = fused_ws(prev_attn, f.si);
        f.has_prev = 1;
        f.pp = attn_params_of(prev_attn, (uint8_t *)prev_workspace, pw);
        f.pap = append_params(prev_append);
        f.psi = (const SplitIn *)((uint8_t *)prev_workspace + pw.si_off);
    }
    return launch_shape(kRunFused, attn, f, f.pap, stream);
}

int pipeline_flush_on(hipStream_t stream, const rl_attn_decode_args_t *prev_attn,
                      const rl_kv_append_args_t *prev_append, void *prev_workspace, size_t workspace_bytes,
                      const char *who)
{
    if (rl_require_open(who) || rl_decode_step_check(prev_attn, prev_append, who))
        return -1;
    if (!fused_eligible(prev_attn)) {
        rl_set_error("%s: the shape does not fit the fused kernel", who);
        return -1;
    }
    // the workspace layout depends only on the attention and the grid
    rl_sample_args_t any = {};
    any.rows = 1;
    any.vocab = 1;
    const SplitIn si = split_in_of(prev_attn, &any);
    const FusedWs w = fused_ws(prev_attn, si);
    if (!prev_workspace || workspace_bytes < w.total) {
        rl_set_error("%s: workspace %zu bytes < %zu required", who, workspace_bytes, w.total);
        return -1;
    }
    FusedParams f;
    f.si = si;
    f.si_out = (SplitIn *)((uint8_t *)prev_workspace + w.si_off);  // recorded by the step that wrote the partials
    f.p = attn_params_of(prev_attn, (uint8_t *)prev_workspace, w);
    return launch_shape(kRunMerge, prev_attn, f, append_params(prev_append), stream);
}

}  // namespace

extern "C" int rl_hip_decode_pipeline_step(const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp,
                                           const rl_attn_decode_args_t *prev_attn,
                                           const rl_kv_append_args_t *prev_append, void *workspace,
                                           void *prev_workspace, size_t workspace_bytes)
{
    return pipeline_step_on(rl_stream(), attn, samp, prev_attn, prev_append, workspace, prev_workspace,
                            workspace_bytes, "rl_hip_decode_pipeline_step");
}



extern "C" int rl_hip_decode_lane_step(int lane, const rl_attn_decode_args_t *attn, const rl_sample_args_t *samp,
                                       const rl_attn_decode_args_t *prev_attn, const rl_kv_append_args_t *prev_append,
                                       void *workspace, void *prev_workspace, size_t workspace_bytes)
{
    const char *who = "rl_hip_decode_lane_step";
    hipStream_t st = rl_lane_stream(lane, who);
    if (!st)
        return -1;
    return pipeline_step_on(st, attn, samp, prev_attn, prev_append, workspace, prev_workspace, workspace_bytes, who);
}

extern "C" int rl_hip_decode_lane_flush(int lane, const rl_attn_decode_args_t *prev_attn,
                                        const rl_kv_append_args_t *prev_append, void *prev_workspace,
                                        size_t workspace_bytes)
{
    const char *who = "rl_hip_decode_lane_flush";
    hipStream_t st = rl_lane_stream(lane, who);
    if (!st)
        return -1;
    return pipeline_flush_on(st, prev_attn, prev_append, prev_workspace, workspace_bytes, who);
}

extern "C" int rl_hip_decode_pipeline_flush(const rl_attn_decode_args_t *prev_attn,
                                            const rl_kv_append_args_t *prev_append, void *prev_workspace,
                                            size_t workspace_bytes)
{
    return pipeline_flush_on(rl_stream(), prev_attn, prev_append, prev_workspace, workspace_bytes,
                             "rl_hip_decode_pipeline_flush");
}

// ---- the self-scheduled ring loop: host side ---------------------------------------

namespace {

template <int D, int G, int DT, int TPB>
int loop_launch(LoopParams &L, uint32_t grid)
{
    if constexpr (!FusedLayout<D, G, DT, TPB>::FITS) {
        rl_set_error("rl_hip_ring_loop_launch: shape does not fit the fused step");
        return -1;
    } else {
        void *args[] = {&L};
        return rl_check_hip(
            hipLaunchCooperativeKernel(reinterpret_cast<const void *>(&ring_loop_kernel<D, G, DT, TPB>), dim3(grid),
                                       dim3(kFThreads), args, 0, rl_stream()),
            "hipLaunchCooperativeKernel(ring_loop_kernel)");
    }
}

template <int D, int G>
int loop_dt(LoopParams &L, uint32_t grid, uint32_t dt, uint32_t tpb)
{
    if (dt == RL_DTYPE_BF16)
        return tpb == 16 ? loop_launch<D, G, 0, 16>(L, grid) : loop_launch<D, G, 0, 32>(L, grid);
    return tpb == 16 ? loop_launch<D, G, 1, 16>(L, grid) : loop_launch<D, G, 1, 32>(L, grid);
}

template <int D>
int loop_g(LoopParams &L, uint32_t grid, uint32_t G, uint32_t dt, uint32_t tpb)
{
    switch (G) {
    case 1: return loop_dt<D, 1>(L, grid, dt, tpb);
    case 2: return loop_dt<D, 2>(L, grid, dt, tpb);
    case 4: return loop_dt<D, 4>(L, grid, dt, tpb);
    default: return loop_dt<D, 8>(L, grid, dt, tpb);
    }
}

}  // namespace

extern "C" int rl_hip_ring_loop_launch(const rl_ring_step_args_t *a, uint32_t max_steps, uint64_t first_step,
                                       uint32_t *steps_run)
{
    const char *who = "rl_hip_ring_loop_launch";
    if (rl_require_open(who) || ring_validate(a, who))
        return -1;
    RingWs w;
    if (ring_layout(a, w))
        return -1;
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("%s: workspace %zu bytes < %zu required", who, a->workspace_bytes, w.total);
        return -1;
    }
    int coop = 0;
    if (rl_check_hip(hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, rl_device()),
                     "hipDeviceGetAttribute(CooperativeLaunch)"))
        return -1;
    if (!coop) {
        rl_set_error("%s: the device does not support cooperative launches", who);
        return -1;
    }
    uint8_t *ws = (uint8_t *)a->workspace;
    LoopParams L;
    L.rp = ring_params_of(a, ws, w);

    const size_t B = a->batch;
    const size_t qrow = (size_t)a->q_heads * a->layout.head_dim * 2;
    const size_t kvrow = (size_t)a->kv_heads * a->layout.head_dim * 2;
    rl_attn_decode_args_t t = attn_of(a, nullptr, 0);
    t.block_table = a->block_table;
    t.ctx_lens = L.rp.ctx;
    t.q = a->q;
    t.out = a->attn_out;
    t.out_f32 = a->attn_out_f32;
    if (!fused_eligible(&t)) {
        rl_set_error("%s: the shape does not fit the fused kernel (use rl_hip_ring_step_enqueue)", who);
        return -1;
    }
    if (a->output_slots < 3) {
        rl_set_error("%s: output_slots %u < 3 (a step's results are merged while the next two steps run)", who,
                     a->output_slots);
        return -1;
    }
    rl_sample_args_t s = samp_of(a);
    s.seed = L.rp.rseed;
    s.steps = L.rp.rstep;
    s.draw_ids = L.rp.rmap;  // the draw follows the rollout, not the row it was admitted into
    if (rl_attn_check(&t) || rl_sample_check(&s))
        return -1;
    const uint32_t grid = rl_cu_count() / kXcds * kXcds;
    if (grid < kLoopService + 2 * kXcds) {
        rl_set_error("%s: %u compute units are too few", who, rl_cu_count());
        return -1;
    }
    {
        // The sampling workgroups merge the previous step's rows, one per
        // wave. In the loop a merge runs while every other workgroup streams
        // (the pipelined step's estimate assumes a quieter device): it is
        // weighted at kLoopMergeWeight of those rounds in the split.
        uint32_t wgs, sample_wgs;
        grid_of(s.rows, wgs, sample_wgs, grid - kLoopService);
        const uint32_t rows = a->batch * a->kv_heads;
        const uint32_t rounds = (rows + sample_wgs * kFWaves - 1) / (sample_wgs * kFWaves);
        L.f = fused_params_of(&t, &s, ws + w.step, rounds * kLoopMergeWeight, grid - kLoopService);
    }
    L.f.p.row_map = L.rp.rmap;
    const FusedWs fw = fused_ws(&t, L.f.si);
    if (fw.total > w.step_bytes) {
        rl_set_error("%s: step workspace %zu bytes < %zu", who, w.step_bytes, fw.total);
        return -1;
    }
    // the counters (at most one per step workgroup and step) stay in 31 bits
    const uint64_t per_step = L.f.si.wgs;
    if (max_steps == 0 || (max_steps + 1ull) * per_step >= (1ull << 31)) {
        rl_set_error("%s: max_steps %u not in 1 .. %llu", who, max_steps,
                     (unsigned long long)((1ull << 31) / per_step - 2));
        return -1;
    }
    rl_kv_append_args_t apa = {};
    apa.arena_base = a->arena_base;
    apa.arena_bytes = a->arena_bytes;
    apa.layout = a->layout;
    apa.block_table = a->block_table;
    apa.table_stride = a->table_stride;
    apa.batch = a->batch;
    apa.kv_heads = a->kv_heads;
    apa.positions = L.rp.pos;
    apa.cow_src = nullptr;
    apa.k_new = a->k_new;
    apa.v_new = a->v_new;
    L.ap = append_params(&apa);
    L.ap.row_map = L.rp.rmap;
    for (int i = 0; i < 2; i++) {
        const RingWs::Set &x = w.set[i];
        L.set[i].ctx = (uint32_t *)(ws + x.ctx);
        L.set[i].pos = (uint32_t *)(ws + x.pos);
        L.set[i].rmap = (uint32_t *)(ws + x.rmap);
        L.set[i].rseed = (uint64_t *)(ws + x.rseed);
        L.set[i].rstep = (uint64_t *)(ws + x.rstep);
        L.set[i].cum = (uint32_t *)(ws + x.step + fw.cum_off);
        L.set[i].part = (float *)(ws + x.step + fw.part_off);
        L.set[i].si_out = (SplitIn *)(ws + x.step + fw.si_off);
    }
    L.q_slot = B * qrow;
    L.out_slot = B * qrow;
    L.out32_slot = B * qrow / 2;
    L.logits_slot = B * a->vocab;
    L.tok_slot = B;
    L.kv_slot = B * kvrow;
    L.row_rollout = a->row_rollout_out;
    L.steps_run = steps_run;
    L.input_slots = a->input_slots;
    L.output_slots = a->output_slots;
    L.first_step = first_step;
    L.max_steps = max_steps;
    L.sync = (uint32_t *)(ws + w.ctl + kLoopSyncOff);
    // A turn waits at most max_idle polls for room on the completion ring and
    // as many for a descriptor, each poll one PCIe round trip and a short
    // sleep (10 us is a generous bound), besides the merges of a step; a
    // step and its merges stream at most the device's memory once, far
    // below 2 s.
    L.bar_ticks = 200000000ull;
    L.go_ticks = 2000ull * L.rp.max_idle + 2 * L.bar_ticks;
    static_assert(kLoopSyncOff + kLoopSyncWords * 4 <= 256, "the sync words fit before the rows");
    if (rl_check_hip(hipMemsetAsync(L.sync, 0, kLoopSyncWords * sizeof(uint32_t), rl_stream()),
                     "hipMemsetAsync(loop sync)"))
        return -1;
    const uint32_t G = a->q_heads / a->kv_heads;
    if (a->layout.head_dim == 128)
        return loop_g<128>(L, grid, G, a->dtype, a->layout.token_count);
    return loop_g<64>(L, grid, G, a->dtype, a->layout.token_count);
}
