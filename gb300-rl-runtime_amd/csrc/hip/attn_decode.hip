// attn_decode.hip - single-query GQA decode attention over the block-paged KV
// arena, written for gfx950 (CDNA4, wave64).
//
// Replaces the reference microkernel attention_decode_step_fixed128
// (cu/attention_decode.cu:60-204: one warp, one head, <= 32 tokens, lane-0
// serial softmax) with a persistent, balanced split-KV kernel:
//
//  work   the KV of row (rollout b, kv head g) is ceil(ctx_b / 16) tiles of
//         16 tokens. All tiles of all rows, rows in (b, g) order, form one
//         sequence of U tiles; wave w of the NW = min(resident waves, U) waves
//         takes tiles [floor(w U / NW), floor((w + 1) U / NW)), so every wave
//         streams the same number of bytes whatever the context lengths, and
//         there is no tail of short workgroups. A wave that covers a whole row
//         writes the output; otherwise it writes an fp32 partial (max, sum,
//         unnormalised O) that attn_merge_kernel combines with a log-sum-exp
//         merge.
//  stage  each tile's K and V planes are copied HBM -> LDS with
//         global_load_lds_dwordx4 (16 B per lane, 1 KiB per instruction,
//         coalesced), double-buffered per wave and continuing across row
//         boundaries. Lanes fetch the 16-byte chunks of a row in XOR-permuted
//         order (chunk c of row t lands at position c ^ t in the K plane and
//         c ^ rotl4(t) in the V plane), which makes both MFMA operand reads
//         below free of LDS bank conflicts (the row-major K reads and the
//         transposed V reads need different permutations). The query of a
//         new row rides in the same copy stream into one of two q slots.
//  QK     v_mfma_f32_16x16x32_{bf16,f16}: A = the tile's 16 K rows, B = q^T
//         with the G heads of the group padded to 16 columns, so each K byte
//         is read from LDS once. The result S^T[token][head] has lane l
//         holding head l % 16 and tokens 4 (l / 16) .. + 3 - exactly the A
//         operand layout of the PV product.
//  softmax online, in the exp2 domain: per-head max over a lane's 4 tokens and
//         two cross-lane steps; per-lane partial sums reduced once per row;
//         the output is rescaled only when some head's max grows.
//  PV     v_mfma_f32_16x16x16_{bf16,f16}: A = P, B = V read with
//         ds_read_b64_tr_b16 (a 4x4 transpose inside each 16-lane group turns
//         row-major V into the k-major operand). P is split into a 16-bit
//         high part and the 16-bit remainder, two MFMAs per block, so the
//         products keep ~16 mantissa bits: fp32-grade accuracy.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "attn_core.h"
#include "kv_layout.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"
#include "kv_append_core.h"
#include "sample_core.h"

namespace {

// Greedy sampling that rides in the attention's launches (sp.splits == 0:
// none): workgroups attn_wgs and up of the attention kernel each run one
// slice of a row (split_slice), after every attention workgroup has been
// placed, so they take compute units as the attention's last waves retire;
// rows of the merge grid past the batch each merge greedy rows, one wave per
// row (greedy_merge_row). The kernel boundary between the two orders them.
struct SideSample {
    SampleParams sp;
    uint32_t attn_wgs;
};

// Stages of the per-wave tile ring. Two (one tile in flight while one is
// consumed) with two workgroups per CU measured faster than four stages with
// one workgroup per CU (120 vs 125 us on the 64-rollout ragged batch): the
// random-block stream saturates the same ~5.5 TB/s either way, and eight
// waves per CU overlap the consume phases better than four.
template <int D, int G, int DT, int TPB>
constexpr int stages_of()
{
    return 2;
}

// Workgroup b runs on XCD b % 8, each XCD behind its own L2. The logical
// index gives XCD x a contiguous eighth of the tile sequence, so rows that
// read the same KV blocks (the rollouts of a group over a shared prefix, which
// sit next to each other in the sequence) stream them through one L2.
__device__ __forceinline__ uint32_t xcd_contiguous_wg(uint32_t n)
{
    if (n % 8 != 0)
        return blockIdx.x;
    return (blockIdx.x % 8) * (n / 8) + blockIdx.x / 8;
}

template <int D, int G, int DT, int TPB>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnParams p, SideSample ss)
{
    using C = Cfg<D, G, DT, TPB>;
    constexpr int W = C::W;
    constexpr int NS = stages_of<D, G, DT, TPB>();
    static_assert(W * 64 == 256, "launch bounds");
    __shared__ __attribute__((aligned(1024))) uint8_t lds_st[NS][W * C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_q[W * NS * C::QSLOT];

    if (blockIdx.x >= ss.attn_wgs) {  // a slice of the greedy sampling riding in this launch
        const uint32_t e = blockIdx.x - ss.attn_wgs;
        split_slice(ss.sp, e % ss.sp.splits, e / ss.sp.splits, *reinterpret_cast<SplitLds *>(lds_q));
        return;
    }
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t wg = xcd_contiguous_wg(ss.attn_wgs);

    // ---- plan: tile prefix over rollouts, each wave's starting rollout -------
    // (q slot memory doubles as scratch until the copies start)
    RL_LDS uint32_t *wave_tot = (RL_LDS uint32_t *)lds_q;  // [W]
    RL_LDS uint32_t *start = wave_tot + W;                  // [W][2] rollout, tiles before it
    const uint32_t T = W * 64;
    const uint32_t per = (p.batch + T - 1) / T;
    const uint32_t b0 = min(threadIdx.x * per, p.batch);
    const uint32_t b1 = min(b0 + per, p.batch);
    uint32_t S = 0;
    for (uint32_t bb = b0; bb < b1; bb++)
        S += tiles_of(p, p.ctx[bb]) * p.kv_heads;
    // tiles of one rollout: its share of S when the thread has one, else reloaded
    auto tiles_at = [&](uint32_t bb) { return per == 1 ? S : tiles_of(p, p.ctx[bb]) * p.kv_heads; };
    const uint32_t inc = rl_wave_incl_scan_u32(S);
    if (lane == 63)
        wave_tot[wave] = inc;
    __syncthreads();
    uint32_t U = 0, before = 0;
#pragma unroll
    for (int v = 0; v < W; v++) {
        const uint32_t t = wave_tot[v];
        before += v < wave ? t : 0u;
        U += t;
    }
    const uint32_t P0 = before + inc - S;  // tiles before this thread's rollouts
    // Waves that share the tiles: never more than there are tiles, so every
    // wave of a row's range holds part of it.
    const uint32_t NW = min(p.nwaves, U);
#pragma unroll
    for (int v = 0; v < W; v++) {
        const uint32_t w = wg * W + v;
        if (w < NW && S > 0) {
            const uint32_t s = (uint32_t)(((uint64_t)w * U) / NW);
            if (s >= P0 && s < P0 + S) {
                uint32_t c = P0;
                for (uint32_t bb = b0; bb < b1; bb++) {
                    const uint32_t n = tiles_at(bb);
                    if (s < c + n) {
                        start[2 * v] = bb;
                        start[2 * v + 1] = c;
                        break;
                    }
                    c += n;
                }
            }
        }
    }
    if (blockIdx.x == 0) {
        uint32_t c = P0;
        for (uint32_t bb = b0; bb < b1; bb++) {
            p.cum[bb] = c;
            c += tiles_at(bb);
        }
        if (threadIdx.x == T - 1)
            p.cum[p.batch] = U;
    }
    __syncthreads();
    const uint32_t wave_id = wg * W + wave;
    const bool active = wave_id < NW;
    const uint32_t s_begin = active ? (uint32_t)(((uint64_t)wave_id * U) / NW) : 0u;
    const uint32_t s_end = active ? (uint32_t)(((uint64_t)(wave_id + 1) * U) / NW) : 0u;
    uint32_t rb = 0, rcum = 0;
    if (active) {
        rb = __builtin_amdgcn_readfirstlane(start[2 * wave]);
        rcum = __builtin_amdgcn_readfirstlane(start[2 * wave + 1]);
    }
    __syncthreads();  // scratch reads done before any copy lands in the q slots
    if (!active)
        return;

    RL_LDS uint8_t *st = (RL_LDS uint8_t *)lds_st[0] + wave * C::STAGE;
    RL_LDS uint8_t *qs = (RL_LDS uint8_t *)lds_q + wave * NS * C::QSLOT;
    attn_stream<D, G, DT, TPB, NS>(p, CtxFromArray{p.ctx}, wave_id, s_begin, s_end, rb, rcum, st, W * C::STAGE, qs,
                                   lane);
}

// Combines the partials of every row split across waves (merge_row) and
// writes rows without tiles (ctx 0: zeros; ctx beyond max_ctx: NaN). With
// HS > 1 each row's heads are shared by HS workgroups of G / HS heads
// (workgroup x of the grid: kv head x / HS, heads (x % HS) G / HS ... of its
// group), so the many partials of long rows are read through that many
// compute units. In a fused decode step (ap.arena set) the first workgroup
// of row (b, g) also appends that row's new K/V token: attn_decode_kernel has
// read every context already, and the merge reads only the partials.
template <int G>
constexpr int merge_heads_of()
{
    return G >= 2 ? G / 2 : 1;
}

template <int D, int G, int DT, int HS>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p, AppendParams ap, SideSample ss)
{
    constexpr int GH = G / HS;
    if (blockIdx.y >= p.batch) {  // greedy rows of the sampling riding in this launch, one wave each
        const uint32_t r = ((blockIdx.y - p.batch) * gridDim.x + blockIdx.x) * 4 + (threadIdx.x >> 6);
        if (r < ss.sp.rows)
            greedy_merge_row(ss.sp, r, (int)(threadIdx.x & 63), true);
        return;
    }
    __shared__ float s_f[kMergeLds * G];
    __shared__ float s_L[G];
    const uint32_t g = blockIdx.x / HS;
    const uint32_t h0 = (blockIdx.x % HS) * GH;
    const uint32_t b = blockIdx.y;
    // the three values the row's partials are located by, loaded together
    // (cum has batch + 1 entries whatever the context)
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
    const uint32_t NW = min(p.nwaves, U);  // U > 0: this row has tiles
    const uint32_t R0 = cum_b + g * nu;
    merge_row<D, G, DT, 256, GH>(p, b, g, h0, R0, nu, U, NW, bad, threadIdx.x, s_f, s_L);
}
}  // namespace

// ---- launcher ------------------------------------------------------------------

namespace {

uint32_t part_floats(const rl_attn_decode_args_t *a)
{
    const uint32_t G = a->q_heads / a->kv_heads;
    return G * a->layout.head_dim + 2 * G;
}

uint32_t waves_of(const rl_attn_decode_args_t *a)
{
    if (a->grid_waves)
        return a->grid_waves;
    const uint32_t G = a->q_heads / a->kv_heads;
    const uint32_t D = a->layout.head_dim;
    // LDS per wave: NS stages of one tile's K and V and NS q slots, NS as in
    // stages_of()
    const uint32_t per_stage = 2 * 16 * 2 * D + ((G * D * 2 + 1023) / 1024) * 1024;
    const uint32_t ns = 2;
    uint32_t wg = (160u * 1024u) / (4 * ns * per_stage);
    wg = wg > 4 ? 4 : wg;
    return rl_cu_count() * wg * 4;
}

struct WsLayout {
    size_t cum_off, part_off, total;
};

WsLayout ws_layout(const rl_attn_decode_args_t *a)
{
    WsLayout w;
    const size_t rows = (size_t)a->batch * a->kv_heads;
    w.cum_off = 0;
    w.part_off = (((size_t)a->batch + 1) * 4 + 255) / 256 * 256;
    w.total = w.part_off + ((size_t)waves_of(a) + rows) * part_floats(a) * 4;
    return w;
}

template <int D, int G, int DT, int TPB>
int launch(const AttnParams &p, const AppendParams &ap, SideSample ss)
{
    using C = Cfg<D, G, DT, TPB>;
    const uint32_t wgs = (p.nwaves + C::W - 1) / C::W;
    ss.attn_wgs = wgs;
    const uint32_t slices = ss.sp.splits * ss.sp.rows;  // 0 without a side sampling
    hipLaunchKernelGGL((attn_decode_kernel<D, G, DT, TPB>), dim3(wgs + slices), dim3(C::W * 64), 0, rl_stream(), p,
                       ss);
    if (rl_check_launch("attn_decode_kernel launch"))
        return -1;
    // Rows averaging 8 or more partials (waves per row) take workgroups of
    // two heads; shorter rows one workgroup per row, whose partials arrive
    // in one batch of loads. Greedy rows of a side sampling: four per
    // workgroup in extra grid rows.
    constexpr int HS = merge_heads_of<G>();
    const bool hs = HS > 1 && (uint64_t)p.nwaves >= 8ull * p.batch * p.kv_heads;
    const uint32_t gx = hs ? p.kv_heads * HS : p.kv_heads;
    const uint32_t gy = p.batch + (slices ? (ss.sp.rows + 4 * gx - 1) / (4 * gx) : 0u);
    if (hs)
        hipLaunchKernelGGL((attn_merge_kernel<D, G, DT, HS>), dim3(gx, gy), dim3(256), 0, rl_stream(), p, ap, ss);
    else
        hipLaunchKernelGGL((attn_merge_kernel<D, G, DT, 1>), dim3(gx, gy), dim3(256), 0, rl_stream(), p, ap, ss);
    return rl_check_launch("attn_merge_kernel launch");
}

template <int D, int G, int DT>
int dispatch_tpb(const AttnParams &p, const AppendParams &ap, const SideSample &ss, uint32_t tpb)
{
    return tpb == 16 ? launch<D, G, DT, 16>(p, ap, ss) : launch<D, G, DT, 32>(p, ap, ss);
}

template <int D, int G>
int dispatch_dt(const AttnParams &p, const AppendParams &ap, const SideSample &ss, uint32_t dt, uint32_t tpb)
{
    return dt == RL_DTYPE_BF16 ? dispatch_tpb<D, G, 0>(p, ap, ss, tpb) : dispatch_tpb<D, G, 1>(p, ap, ss, tpb);
}

template <int D>
int dispatch_g(const AttnParams &p, const AppendParams &ap, const SideSample &ss, uint32_t G, uint32_t dt,
               uint32_t tpb)
{
    switch (G) {
    case 1: return dispatch_dt<D, 1>(p, ap, ss, dt, tpb);
    case 2: return dispatch_dt<D, 2>(p, ap, ss, dt, tpb);
    case 4: return dispatch_dt<D, 4>(p, ap, ss, dt, tpb);
    default: return dispatch_dt<D, 8>(p, ap, ss, dt, tpb);
    }
}

int validate(const rl_attn_decode_args_t *a)
{
    if (!a) {
        rl_set_error("rl_hip_attn_decode: NULL args");
        return -1;
    }
    if (kv_layout_check_paged(&a->layout) != 0) {
        rl_set_error("rl_hip_attn_decode: unsupported KV layout (token_count %u, head_dim %u, scalar %u)",
                     a->layout.token_count, a->layout.head_dim, a->layout.scalar_bytes);
        return -1;
    }
    if (a->kv_heads == 0 || a->q_heads % a->kv_heads != 0) {
        rl_set_error("rl_hip_attn_decode: q_heads %u not a multiple of kv_heads %u", a->q_heads, a->kv_heads);
        return -1;
    }
    const uint32_t G = a->q_heads / a->kv_heads;
    if (G != 1 && G != 2 && G != 4 && G != 8) {
        rl_set_error("rl_hip_attn_decode: GQA group %u not in {1,2,4,8}", G);
        return -1;
    }
    if (a->dtype != RL_DTYPE_BF16 && a->dtype != RL_DTYPE_FP16) {
        rl_set_error("rl_hip_attn_decode: dtype %u", a->dtype);
        return -1;
    }
    if (!a->arena_base || !a->block_table || !a->ctx_lens || !a->q || !a->out) {
        rl_set_error("rl_hip_attn_decode: NULL device pointer");
        return -1;
    }
    if (a->arena_bytes < a->layout.block_bytes) {
        rl_set_error("rl_hip_attn_decode: arena of %llu bytes holds no block", (unsigned long long)a->arena_bytes);
        return -1;
    }
    if (a->batch == 0 || a->batch > 65535 || a->kv_heads > 65535) {
        rl_set_error("rl_hip_attn_decode: batch %u / kv_heads %u out of range", a->batch, a->kv_heads);
        return -1;
    }
    const uint64_t max_tiles = (a->max_ctx + 15ull) / 16ull;
    if ((uint64_t)a->batch * a->kv_heads * max_tiles >= (1ull << 32)) {
        rl_set_error("rl_hip_attn_decode: batch %u x kv_heads %u x %llu tiles of max_ctx %u exceeds 2^32 tiles",
                     a->batch, a->kv_heads, (unsigned long long)max_tiles, a->max_ctx);
        return -1;
    }
    if (a->grid_waves > (1u << 20)) {
        rl_set_error("rl_hip_attn_decode: grid_waves %u above 2^20", a->grid_waves);
        return -1;
    }
    const uint32_t table_need = (a->max_ctx + a->layout.token_count - 1) / a->layout.token_count;
    if (a->table_stride < table_need) {
        rl_set_error("rl_hip_attn_decode: table_stride %u < %u blocks needed for max_ctx %u", a->table_stride,
                     table_need, a->max_ctx);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" size_t rl_hip_attn_decode_workspace(const rl_attn_decode_args_t *a)
{
    if (rl_require_open("rl_hip_attn_decode_workspace") || validate(a))
        return 0;
    return ws_layout(a).total;
}

namespace {

SideSample no_side()
{
    SideSample ss;
    ss.sp = SampleParams{};
    ss.sp.splits = 0;
    ss.sp.rows = 0;
    ss.attn_wgs = 0;
    return ss;
}

int attn_run(const rl_attn_decode_args_t *a, const AppendParams &ap, const uint32_t *row_map = nullptr,
             const SideSample &ss = no_side())
{
    const WsLayout w = ws_layout(a);
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_attn_decode: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    AttnParams p;
    p.arena = (const uint8_t *)a->arena_base;
    p.block_bytes = a->layout.block_bytes;
    p.arena_blocks = a->arena_bytes / a->layout.block_bytes;
    p.table = a->block_table;
    p.table_stride = a->table_stride;
    p.row_map = row_map;
    p.ctx = a->ctx_lens;
    p.max_ctx = a->max_ctx;
    p.batch = a->batch;
    p.q_heads = a->q_heads;
    p.kv_heads = a->kv_heads;
    p.q = (const uint16_t *)a->q;
    p.out = (uint16_t *)a->out;
    p.out_f32 = a->out_f32;
    const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)a->layout.head_dim);
    p.scale_log2 = scale * 1.4426950408889634f;
    p.nwaves = waves_of(a);
    uint8_t *ws = (uint8_t *)a->workspace;
    p.cum = (uint32_t *)(ws + w.cum_off);
    p.part = (float *)(ws + w.part_off);

    const uint32_t G = a->q_heads / a->kv_heads;
    if (a->layout.head_dim == 128)
        return dispatch_g<128>(p, ap, ss, G, a->dtype, a->layout.token_count);
    return dispatch_g<64>(p, ap, ss, G, a->dtype, a->layout.token_count);
}

}  // namespace

extern "C" int rl_hip_attn_decode(const rl_attn_decode_args_t *a)
{
    if (rl_require_open("rl_hip_attn_decode") || validate(a))
        return -1;
    AppendParams none = {};
    none.arena = nullptr;
    return attn_run(a, none);
}

namespace {

int step_validate(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append, const char *who)
{
    if (rl_require_open(who) || validate(attn) || append_validate(append, who))
        return -1;
    if (append->batch != attn->batch || append->kv_heads != attn->kv_heads) {
        rl_set_error("%s: append batch %u / kv_heads %u differ from attention %u / %u", who, append->batch,
                     append->kv_heads, attn->batch, attn->kv_heads);
        return -1;
    }
    return 0;
}

}  // namespace

extern "C" int rl_hip_decode_step(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append)
{
    if (step_validate(attn, append, "rl_hip_decode_step"))
        return -1;
    return attn_run(attn, append_params(append));
}

int rl_attn_check(const rl_attn_decode_args_t *a)
{
    return validate(a);
}

int rl_decode_step_check(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append, const char *who)
{
    return step_validate(attn, append, who);
}

int rl_decode_step_mapped(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                          const uint32_t *row_map)
{
    if (step_validate(attn, append, "rl_hip_decode_step") || !row_map) {
        if (!row_map)
            rl_set_error("rl_hip_decode_step: NULL row map");
        return -1;
    }
    AppendParams ap = append_params(append);
    ap.row_map = row_map;
    return attn_run(attn, ap, row_map);
}

int rl_decode_step_greedy_side(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append,
                               const rl_sample_args_t *samp)
{
    const char *who = "rl_hip_decode_sample_step";
    if (append ? step_validate(attn, append, who) : (rl_require_open(who) || validate(attn)))
        return -1;
    uint32_t splits = 0;
    size_t cand_off = 0;
    const int k = rl_sample_greedy_split(samp, &splits, &cand_off);
    if (k <= 0)
        return k < 0 ? -1 : 1;
    SideSample ss = no_side();
    ss.sp = sample_params_of(samp);
    ss.sp.splits = splits;
    ss.sp.stats = (SplitStat *)samp->workspace;  // the slice records start the sampler's workspace
    ss.sp.cand = (uint2 *)((uint8_t *)samp->workspace + cand_off);
    AppendParams ap = {};
    ap.arena = nullptr;
    if (append)
        ap = append_params(append);
    return attn_run(attn, ap, nullptr, ss);
}

int rl_attn_mapped(const rl_attn_decode_args_t *attn, const uint32_t *row_map)
{
    if (rl_require_open("rl_hip_attn_decode") || validate(attn))
        return -1;
    if (!row_map) {
        rl_set_error("rl_hip_attn_decode: NULL row map");
        return -1;
    }
    AppendParams none = {};
    none.arena = nullptr;
    return attn_run(attn, none, row_map);
}

// ---- the decode step without allocation ---------------------------------------
// The workspace of rl_hip_decode_step_noalloc (cum[batch + 1], then the fp32
// partials) lives in this file-scope array; every device the library runs on
// holds its own copy until the process ends. On the host, `scratch` names a
// host-side stand-in, not device memory: kernels get the device address that
// hipGetSymbolAddress returned for the device at rl_hip_open, kept in
// g_scratch_dev. Nothing in the workspace has to start at zero: cum is written
// by attn_decode_kernel's first workgroup and every partial the merge reads is
// written earlier in the same call.
static __device__ __align__(256) uint8_t scratch[RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kScratchDevices = 64;
void *g_scratch_dev[kScratchDevices];

}  // namespace

int rl_attn_scratch_setup(int device)
{
    if (device < 0 || device >= kScratchDevices) {
        rl_set_error("rl_hip_open: device %d beyond the %d devices the decode-step scratch covers", device,
                     kScratchDevices);
        return -1;
    }
    if (g_scratch_dev[device])
        return 0;
    void *p = nullptr;
    if (rl_check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)"))
        return -1;
    if (!p) {
        rl_set_error("hipGetSymbolAddress(scratch) returned NULL on device %d", device);
        return -1;
    }
    g_scratch_dev[device] = p;
    return 0;
}

extern "C" int rl_hip_decode_step_noalloc(const rl_attn_decode_args_t *attn, const rl_kv_append_args_t *append)
{
    if (step_validate(attn, append, "rl_hip_decode_step_noalloc"))
        return -1;
    const int dev = rl_device();
    void *ws = dev >= 0 && dev < kScratchDevices ? g_scratch_dev[dev] : nullptr;
    if (!ws) {
        rl_set_error("rl_hip_decode_step_noalloc: no scratch address for device %d", dev);
        return -1;
    }
    const size_t need = ws_layout(attn).total;
    if (need > RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES) {
        rl_set_error("rl_hip_decode_step_noalloc: the step needs %zu bytes of workspace, above the %u-byte "
                     "scratch (use rl_hip_decode_step with a caller workspace)",
                     need, (unsigned)RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES);
        return -1;
    }
    rl_attn_decode_args_t a = *attn;
    a.workspace = ws;
    a.workspace_bytes = RL_DECODE_STEP_NOALLOC_SCRATCH_BYTES;
    return attn_run(&a, append_params(append));
}
