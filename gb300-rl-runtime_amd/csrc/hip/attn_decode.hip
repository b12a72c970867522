// attn_decode.hip - single-query GQA decode attention over the block-paged KV
// arena, written for gfx950 (CDNA4, wave64).
//
// Replaces the reference microkernel attention_decode_step_fixed128
// (cu/attention_decode.cu:60-204: one warp, one head, <= 32 tokens, lane-0
// serial softmax) with a split-KV kernel for batched GQA decode:
//
//  grid   (chunk, kv_head, rollout); one workgroup of W wave64s per chunk of
//         `chunk_tiles` 16-token tiles of one (rollout, kv head).
//  stage  every tile's K and V planes are copied HBM -> LDS with
//         global_load_lds_dwordx4 (16 B per lane, 1 KiB per instruction,
//         fully coalesced), double-buffered per wave so the next tile's
//         loads are in flight while the current one is consumed.
//  QK     lane (row r, lane t) of a 16-lane DPP row owns token t and q head
//         r (GQA group <= 4; two heads per lane for groups of 8): a full
//         head_dim dot product with v_dot2_f32_bf16 against q held in VGPRs.
//         K rows are read from LDS with an XOR swizzle (chunk j ^ t) so the
//         16 lanes of a row hit 16 different bank groups.
//  softmax online, in the exp2 domain (scale folded with log2 e); row max
//         and row sum with four DPP steps (quad_perm x2, row_half_mirror,
//         row_mirror); p and the rescale factor go through LDS.
//  PV     lane owns one dword (2 dims) of V for every head of the group, so
//         each V element is converted to fp32 once; p is a broadcast LDS read.
//  merge  waves of a workgroup merge through LDS; the chunks of a long
//         context write fp32 partials (max, sum, unnormalised output) that a
//         second small kernel combines with an fp32 log-sum-exp merge. (A
//         last-workgroup merge inside the same launch needs agent-scope
//         release/acquire fences, which on gfx950 write back and invalidate
//         the whole L2 of the XCD for every workgroup: measured 12x slower.)
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_layout.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr int kTileTokens = 16;

struct AttnParams {
    const uint8_t *arena;
    uint64_t block_bytes;
    uint64_t arena_blocks;  // blocks at or past this index are never read
    uint32_t max_ctx;
    const uint32_t *table;
    uint32_t table_stride;
    const uint32_t *ctx;
    const uint16_t *q;
    uint16_t *out;
    float *out_f32;
    float scale_log2;      // softmax scale * log2(e)
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t chunk_tiles;  // tiles per workgroup (multiple of 4)
    uint32_t max_chunks;
    float *ws_o;           // [rollout][kv_head][chunk][G][D]
    float *ws_ml;          // [rollout][kv_head][chunk][G][2]
};

template <int D, int G, int DT, int TPB, int W>
struct Cfg {
    static constexpr int RB = 2 * D;                 // bytes per K/V row
    static constexpr int NC = D / 8;                 // 16-byte chunks per row
    static constexpr int PLANE = kTileTokens * RB;   // bytes of one tile's K (or V)
    static constexpr int GH = G < 4 ? G : 4;         // heads per DPP row set
    static constexpr int HPL = G / GH;               // heads per lane in QK
    static constexpr int NT = 4 / GH;                // tiles per iteration ("unit")
    static constexpr int UNIT_TOK = NT * kTileTokens;
    static constexpr int STAGE = NT * 2 * PLANE;     // LDS bytes of one unit
    static constexpr int DW = D / 2;                 // dwords per row
    static constexpr int TG = 64 / DW;               // PV token groups
    static constexpr int SUB = TPB / kTileTokens;    // tiles per arena block
    static constexpr int PBUF = UNIT_TOK * G + G;    // p[token][head] + alpha[head]
    static constexpr int MERGE_FLOATS = W * (TG * G * D + 2 * G);
    static_assert(D == 64 || D == 128, "head_dim");
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group");
    static_assert(PLANE % 1024 == 0, "plane must be whole 1 KiB DMA rows");
    // Stage 0 doubles as the merge area once the unit loop is done.
    static constexpr int STAGE0_BYTES = MERGE_FLOATS * 4 > W * STAGE ? MERGE_FLOATS * 4 : W * STAGE;
};

// Per-wave decode state: q in VGPRs, running max/sum, PV accumulators.
template <int D, int G, int DT, int TPB, int W>
struct WaveState {
    using C = Cfg<D, G, DT, TPB, W>;
    uint32_t qreg[C::HPL][C::NC][4];  // register j holds q chunk j ^ tsw
    float m_run[C::HPL];
    float l_run[C::HPL];
    float acc[G][2];
};

// Issues the HBM -> LDS copies of one unit (NT tiles, K and V planes).
// The chunk's block-table entries, loaded once into VGPRs (entry j of the
// chunk in lane j % 64 of word j / 64) so that no table load latency sits
// between consuming a unit and issuing the next unit's copies.
struct ChunkTable {
    uint32_t w0, w1;
    uint32_t first;  // first logical block of the chunk

    __device__ __forceinline__ uint32_t block(uint32_t logical) const
    {
        const uint32_t j = logical - first;  // wave-uniform, < 128
        const uint32_t v = j < 64 ? w0 : w1;
        return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)(j & 63));
    }
};

// Returns false if the block table names a block outside the arena (that
// block is not read).
template <int D, int G, int DT, int TPB, int W>
__device__ __forceinline__ bool stage_unit(const AttnParams &p, const ChunkTable &tbl, uint32_t tile0,
                                           uint32_t tile_end, uint32_t lane_off, RL_LDS uint8_t *dst)
{
    using C = Cfg<D, G, DT, TPB, W>;
    bool ok = true;
#pragma unroll
    for (int n = 0; n < C::NT; n++) {
        const uint32_t tile = tile0 + n;
        if (tile < tile_end) {
            const uint32_t blk = tbl.block(tile / C::SUB);
            if (blk >= p.arena_blocks) {
                ok = false;
                continue;
            }
            const uint8_t *kp = p.arena + (uint64_t)blk * p.block_bytes + (tile % C::SUB) * C::PLANE;
            const uint8_t *vp = kp + TPB * C::RB;
#pragma unroll
            for (int i = 0; i < C::PLANE / 1024; i++) {
                rl_g2lds_16(kp + lane_off + i * 1024, dst + n * 2 * C::PLANE + i * 1024);
                rl_g2lds_16(vp + lane_off + i * 1024, dst + n * 2 * C::PLANE + C::PLANE + i * 1024);
            }
        }
    }
    return ok;
}

// Consumes one staged unit: QK, online softmax update, PV. FULL units lie
// entirely below ctx and skip the masking of tokens past the end.
template <int D, int G, int DT, int TPB, int W, bool FULL>
__device__ __forceinline__ void consume_unit(const AttnParams &p, WaveState<D, G, DT, TPB, W> &ws,
                                             RL_LDS const uint8_t *st, RL_LDS float *pbuf, uint32_t unit_tok0,
                                             uint32_t ctx, int lane)
{
    using C = Cfg<D, G, DT, TPB, W>;
    const int r = lane >> 4;
    const int t = lane & 15;
    const int n_qk = r / C::GH;
    const int hb = r % C::GH;
    const int dw = lane % C::DW;
    const int tg = lane / C::DW;
    const int tsw = t & (C::NC - 1);

    // ---- QK: lane (row r, t) computes the full dot product of token t ------
    float s2[C::HPL];
    {
        RL_LDS const uint8_t *krow = st + n_qk * 2 * C::PLANE + t * C::RB;
        float dot[C::HPL];
#pragma unroll
        for (int i = 0; i < C::HPL; i++)
            dot[i] = 0.f;
#pragma unroll
        for (int j = 0; j < C::NC; j++) {
            const rl_u32x4 kv = *(RL_LDS const rl_u32x4 *)(krow + ((j ^ tsw) << 4));
#pragma unroll
            for (int i = 0; i < C::HPL; i++) {
                dot[i] = rl_dot2<DT>(kv.x, ws.qreg[i][j][0], dot[i]);
                dot[i] = rl_dot2<DT>(kv.y, ws.qreg[i][j][1], dot[i]);
                dot[i] = rl_dot2<DT>(kv.z, ws.qreg[i][j][2], dot[i]);
                dot[i] = rl_dot2<DT>(kv.w, ws.qreg[i][j][3], dot[i]);
            }
        }
        const bool valid = FULL || (unit_tok0 + n_qk * kTileTokens + t < ctx);
#pragma unroll
        for (int i = 0; i < C::HPL; i++)
            s2[i] = valid ? dot[i] * p.scale_log2 : -INFINITY;
    }

    // ---- online softmax over the unit ---------------------------------------
#pragma unroll
    for (int i = 0; i < C::HPL; i++) {
        float mx = rl_row_max(s2[i]);
        if constexpr (C::NT > 1) {
#pragma unroll
            for (int off = 16 * C::GH; off < 64; off <<= 1)
                mx = fmaxf(mx, __shfl_xor(mx, off));
        }
        const float m_new = fmaxf(ws.m_run[i], mx);
        const float m_use = (m_new == -INFINITY) ? 0.f : m_new;
        const float pv = exp2f(s2[i] - m_use);
        float sum = rl_row_sum(pv);
        if constexpr (C::NT > 1) {
#pragma unroll
            for (int off = 16 * C::GH; off < 64; off <<= 1)
                sum += __shfl_xor(sum, off);
        }
        const float alpha = exp2f(ws.m_run[i] - m_use);
        ws.l_run[i] = ws.l_run[i] * alpha + sum;
        ws.m_run[i] = m_new;
        const int head = hb + 4 * i;
        pbuf[(n_qk * kTileTokens + t) * G + head] = pv;
        if (t == 0 && n_qk == 0)
            pbuf[C::UNIT_TOK * G + head] = alpha;
    }
    rl_wave_lds_fence();

    // ---- PV: lane owns dword dw (2 dims) of V for all G heads ------------------
    {
#pragma unroll
        for (int h = 0; h < G; h++) {
            const float alpha = pbuf[C::UNIT_TOK * G + h];
            ws.acc[h][0] *= alpha;
            ws.acc[h][1] *= alpha;
        }
#pragma unroll
        for (int k = 0; k < C::UNIT_TOK / C::TG; k++) {
            const int tok = k * C::TG + tg;
            const int n = tok / kTileTokens;
            const int tt = tok % kTileTokens;
            uint32_t vw = *(RL_LDS const uint32_t *)(st + n * 2 * C::PLANE + C::PLANE + tt * C::RB + dw * 4);
            if (!FULL && unit_tok0 + tok >= ctx)
                vw = 0u;  // stale or uninitialised slot: contributes exactly 0
            float v0, v1;
            rl_unpack2<DT>(vw, v0, v1);
#pragma unroll
            for (int h = 0; h < G; h++) {
                const float pw = pbuf[tok * G + h];
                ws.acc[h][0] = fmaf(pw, v0, ws.acc[h][0]);
                ws.acc[h][1] = fmaf(pw, v1, ws.acc[h][1]);
            }
        }
    }
    rl_wave_lds_fence();
}

template <int D, int G, int DT, int TPB, int W>
__device__ __forceinline__ void consume_any(const AttnParams &p, WaveState<D, G, DT, TPB, W> &ws,
                                            RL_LDS const uint8_t *st, RL_LDS float *pbuf, uint32_t unit_tok0,
                                            uint32_t ctx, int lane)
{
    using C = Cfg<D, G, DT, TPB, W>;
    if (unit_tok0 + C::UNIT_TOK <= ctx)
        consume_unit<D, G, DT, TPB, W, true>(p, ws, st, pbuf, unit_tok0, ctx, lane);
    else
        consume_unit<D, G, DT, TPB, W, false>(p, ws, st, pbuf, unit_tok0, ctx, lane);
}

template <int D, int G, int DT, int TPB, int W>
__global__ __launch_bounds__(W * 64) void attn_decode_kernel(AttnParams p)
{
    using C = Cfg<D, G, DT, TPB, W>;
    // Two static stage buffers (not one indexed array) so the waitcnt pass can
    // tell the DMA into stage 1 apart from reads of stage 0 and leave the next
    // unit's loads in flight while the current unit is consumed.
    __shared__ __attribute__((aligned(1024))) uint8_t lds_stage0[C::STAGE0_BYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_stage1[W * C::STAGE];
    __shared__ float lds_p[W * C::PBUF];
    __shared__ uint32_t s_bad;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t chunk = blockIdx.x;
    const uint32_t g = blockIdx.y;
    const uint32_t b = blockIdx.z;

    const uint32_t ctx_in = rl_sload(p.ctx + b);
    // A context past max_ctx cannot be covered by the grid: clamp it, and
    // poison the output below.
    bool bad = ctx_in > p.max_ctx;
    const uint32_t ctx = bad ? p.max_ctx : ctx_in;
    const uint32_t ntiles = (ctx + kTileTokens - 1) / kTileTokens;
    const uint32_t nchunks = (ntiles + p.chunk_tiles - 1) / p.chunk_tiles;
    const uint32_t row_id = b * p.kv_heads + g;

    if (ctx == 0) {
        if (chunk == 0) {
            for (int e = threadIdx.x; e < G * D; e += W * 64) {
                const size_t o = ((size_t)b * p.q_heads + g * G) * D + e;
                const float v = bad ? __builtin_nanf("") : 0.f;
                p.out[o] = rl_from_f32<DT>(v);
                if (p.out_f32)
                    p.out_f32[o] = v;
            }
        }
        return;
    }
    if (chunk >= nchunks)
        return;

    const uint32_t tile_begin = chunk * p.chunk_tiles;
    const uint32_t tile_end = min(tile_begin + p.chunk_tiles, ntiles);
    const uint32_t units = (tile_end - tile_begin + C::NT - 1) / C::NT;
    const uint32_t lane_off = (uint32_t)lane * 16u;
    ChunkTable tbl;
    {
        const uint32_t *table_row = p.table + (size_t)row_id * p.table_stride;
        tbl.first = tile_begin / C::SUB;
        const uint32_t last = (tile_end + C::SUB - 1) / C::SUB;  // one past the chunk's last block
        tbl.w0 = (tbl.first + lane < last) ? table_row[tbl.first + lane] : 0u;
        tbl.w1 = (tbl.first + 64 + lane < last) ? table_row[tbl.first + 64 + lane] : 0u;
    }

    RL_LDS uint8_t *st0 = (RL_LDS uint8_t *)lds_stage0 + wave * C::STAGE;
    RL_LDS uint8_t *st1 = (RL_LDS uint8_t *)lds_stage1 + wave * C::STAGE;
    RL_LDS float *pbuf = (RL_LDS float *)lds_p + wave * C::PBUF;

    WaveState<D, G, DT, TPB, W> ws;
    {
        const int r = lane >> 4;
        const int hb = r % C::GH;
        const int tsw = (lane & 15) & (C::NC - 1);
#pragma unroll
        for (int i = 0; i < C::HPL; i++) {
            const uint16_t *qrow = p.q + ((size_t)b * p.q_heads + g * G + hb + 4 * i) * D;
#pragma unroll
            for (int j = 0; j < C::NC; j++) {
                const rl_u32x4 v = *(const rl_u32x4 *)(qrow + (j ^ tsw) * 8);
                ws.qreg[i][j][0] = v.x;
                ws.qreg[i][j][1] = v.y;
                ws.qreg[i][j][2] = v.z;
                ws.qreg[i][j][3] = v.w;
            }
            ws.m_run[i] = -INFINITY;
            ws.l_run[i] = 0.f;
        }
#pragma unroll
        for (int h = 0; h < G; h++)
            ws.acc[h][0] = ws.acc[h][1] = 0.f;
    }

    // Copies per staged unit. Vector-memory operations retire in issue order,
    // so "at most UNIT_OPS outstanding" means every copy older than the most
    // recently staged unit (and the q loads above) has landed in LDS. Units
    // of several tiles can be partial at the end of a chunk, so those waves
    // drain fully instead.
    constexpr int UNIT_OPS = C::NT == 1 ? 2 * (C::PLANE / 1024) : 0;

    if ((uint32_t)wave < units)
        bad |= !stage_unit<D, G, DT, TPB, W>(p, tbl, tile_begin + wave * C::NT, tile_end, lane_off, st0);
    if ((uint32_t)wave + W < units)
        bad |= !stage_unit<D, G, DT, TPB, W>(p, tbl, tile_begin + (wave + W) * C::NT, tile_end, lane_off, st1);

    for (uint32_t u = wave; u < units; u += 2 * W) {
        // stage 0 holds unit u; stage 1 may hold unit u + W (in flight)
        if (u + W < units)
            rl_wait_vmcnt<UNIT_OPS>();
        else
            rl_wait_vmcnt<0>();
        consume_any<D, G, DT, TPB, W>(p, ws, st0, pbuf, (tile_begin + u * C::NT) * kTileTokens, ctx, lane);
        if (u + 2 * W < units) {
            rl_wait_lgkmcnt0();
            bad |= !stage_unit<D, G, DT, TPB, W>(p, tbl, tile_begin + (u + 2 * W) * C::NT, tile_end, lane_off,
                                                 st0);
        }
        if (u + W >= units)
            break;
        // stage 1 holds unit u + W; stage 0 may hold unit u + 2W (in flight)
        if (u + 2 * W < units)
            rl_wait_vmcnt<UNIT_OPS>();
        else
            rl_wait_vmcnt<0>();
        consume_any<D, G, DT, TPB, W>(p, ws, st1, pbuf, (tile_begin + (u + W) * C::NT) * kTileTokens, ctx,
                                       lane);
        if (u + 3 * W < units) {
            rl_wait_lgkmcnt0();
            bad |= !stage_unit<D, G, DT, TPB, W>(p, tbl, tile_begin + (u + 3 * W) * C::NT, tile_end, lane_off,
                                                 st1);
        }
    }

    // ---- merge the waves of the workgroup (merge area aliases stage 0) -------
    if (threadIdx.x == 0)
        s_bad = 0;
    __syncthreads();
    if (bad && lane == 0)
        s_bad = 1;
    RL_LDS float *mo = (RL_LDS float *)lds_stage0;      // [W][TG][G][D]
    RL_LDS float *mml = mo + W * C::TG * G * D;         // [W][G][2]
    {
        const int r = lane >> 4;
        const int t = lane & 15;
        const int dw = lane % C::DW;
        const int tg = lane / C::DW;
#pragma unroll
        for (int h = 0; h < G; h++) {
            mo[((wave * C::TG + tg) * G + h) * D + dw * 2 + 0] = ws.acc[h][0];
            mo[((wave * C::TG + tg) * G + h) * D + dw * 2 + 1] = ws.acc[h][1];
        }
        if (t == 0 && r / C::GH == 0) {
#pragma unroll
            for (int i = 0; i < C::HPL; i++) {
                mml[(wave * G + r % C::GH + 4 * i) * 2 + 0] = ws.m_run[i];
                mml[(wave * G + r % C::GH + 4 * i) * 2 + 1] = ws.l_run[i];
            }
        }
    }
    __syncthreads();

    const bool poison = s_bad != 0;
    const bool split = nchunks > 1;
    float *ws_o = p.ws_o + ((size_t)row_id * p.max_chunks + chunk) * G * D;
    float *ws_ml = p.ws_ml + ((size_t)row_id * p.max_chunks + chunk) * G * 2;

    for (int e = threadIdx.x; e < G * D; e += W * 64) {
        const int h = e / D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; w++)
            M = fmaxf(M, mml[(w * G + h) * 2]);
        float L = 0.f, O = 0.f;
#pragma unroll
        for (int w = 0; w < W; w++) {
            const float mw = mml[(w * G + h) * 2];
            const float f = (mw == -INFINITY) ? 0.f : exp2f(mw - M);
            L = fmaf(mml[(w * G + h) * 2 + 1], f, L);
            float ow = 0.f;
#pragma unroll
            for (int q = 0; q < C::TG; q++)
                ow += mo[((w * C::TG + q) * G + h) * D + (e % D)];
            O = fmaf(ow, f, O);
        }
        if (poison) {
            O = __builtin_nanf("");
            L = __builtin_nanf("");
        }
        if (!split) {
            const float v = L > 0.f ? O / L : (poison ? L : 0.f);
            const size_t o = ((size_t)b * p.q_heads + g * G) * D + e;
            p.out[o] = rl_from_f32<DT>(v);
            if (p.out_f32)
                p.out_f32[o] = v;
        } else {
            ws_o[e] = O;
            if (e % D == 0) {
                ws_ml[h * 2 + 0] = M;
                ws_ml[h * 2 + 1] = L;
            }
        }
    }
}

// Combines the chunk partials of every split (rollout, kv head):
// M = max_c m_c, L = sum_c l_c 2^(m_c - M), O = sum_c o_c 2^(m_c - M), out = O / L.
// The per-chunk scale factors go through LDS so every partial-output load
// is independent of the others and they can all be in flight together.
constexpr int kMergeMaxChunks = 128;

template <int D, int G, int DT>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p)
{
    __shared__ float s_f[kMergeMaxChunks * G];
    __shared__ float s_l[G];
    const uint32_t g = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const uint32_t ctx_in = rl_sload(p.ctx + b);
    const uint32_t ctx = ctx_in > p.max_ctx ? p.max_ctx : ctx_in;
    const uint32_t ntiles = (ctx + kTileTokens - 1) / kTileTokens;
    const uint32_t nchunks = (ntiles + p.chunk_tiles - 1) / p.chunk_tiles;
    if (nchunks <= 1)
        return;  // written directly by the decode kernel
    const uint32_t row_id = b * p.kv_heads + g;
    const float *row_o = p.ws_o + (size_t)row_id * p.max_chunks * G * D;
    const float *row_ml = p.ws_ml + (size_t)row_id * p.max_chunks * G * 2;
    if (threadIdx.x < G) {
        const int h = threadIdx.x;
        float M = -INFINITY;
        for (uint32_t c = 0; c < nchunks; c++)
            M = fmaxf(M, row_ml[(c * G + h) * 2]);
        float L = 0.f;
        for (uint32_t c = 0; c < nchunks; c++) {
            const float mc = row_ml[(c * G + h) * 2];
            const float f = (mc == -INFINITY) ? 0.f : exp2f(mc - M);
            s_f[c * G + h] = f;
            L = fmaf(row_ml[(c * G + h) * 2 + 1], f, L);
        }
        s_l[h] = L;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < G * D; e += 256) {
        const int h = e / D;
        float O = 0.f;
#pragma unroll 8
        for (uint32_t c = 0; c < nchunks; c++)
            O = fmaf(row_o[c * G * D + e], s_f[c * G + h], O);
        const float L = s_l[h];
        const float v = (L > 0.f || L != L) ? O / L : 0.f;
        const size_t o = ((size_t)b * p.q_heads + g * G) * D + e;
        p.out[o] = rl_from_f32<DT>(v);
        if (p.out_f32)
            p.out_f32[o] = v;
    }
}

}  // namespace

// ---- launcher ------------------------------------------------------------------

namespace {

// Waves per workgroup: up to 4, with both stage buffers within 64 KiB so two
// workgroups share a CU's 160 KiB of LDS.
template <int D, int G>
constexpr int waves_for()
{
    constexpr int nt = 4 / (G < 4 ? G : 4);
    constexpr int stage = nt * 2 * kTileTokens * 2 * D;
    constexpr int w = 65536 / (2 * stage);
    return w < 1 ? 1 : (w > 4 ? 4 : w);
}
constexpr uint32_t kDefaultChunkTokens = 512;

struct WsLayout {
    size_t ml_off, o_off, total;
};

WsLayout ws_layout(const rl_attn_decode_args_t *a, uint32_t chunk_tiles)
{
    const uint32_t G = a->q_heads / a->kv_heads;
    const uint32_t D = a->layout.head_dim;
    const uint32_t max_tiles = (a->max_ctx + kTileTokens - 1) / kTileTokens;
    const uint32_t max_chunks = max_tiles == 0 ? 1 : (max_tiles + chunk_tiles - 1) / chunk_tiles;
    const size_t rows = (size_t)a->batch * a->kv_heads;
    WsLayout w;
    w.ml_off = 0;
    w.o_off = w.ml_off + ((rows * max_chunks * G * 2 * 4 + 255) / 256) * 256;
    w.total = w.o_off + rows * max_chunks * G * D * 4;
    return w;
}

uint32_t chunk_tiles_of(const rl_attn_decode_args_t *a)
{
    const uint32_t tok = a->chunk_tokens ? a->chunk_tokens : kDefaultChunkTokens;
    return tok / kTileTokens;
}

template <int D, int G, int DT, int TPB>
int launch(const AttnParams &p, dim3 grid)
{
    constexpr int W = waves_for<D, G>();
    auto kern = attn_decode_kernel<D, G, DT, TPB, W>;
    hipLaunchKernelGGL(kern, grid, dim3(W * 64), 0, rl_stream(), p);
    if (rl_check_launch("attn_decode_kernel launch"))
        return -1;
    if (grid.x > 1) {
        hipLaunchKernelGGL((attn_merge_kernel<D, G, DT>), dim3(grid.y, grid.z), dim3(256), 0, rl_stream(), p);
        return rl_check_launch("attn_merge_kernel launch");
    }
    return 0;
}

template <int D, int G, int DT>
int dispatch_tpb(const AttnParams &p, dim3 grid, uint32_t tpb)
{
    return tpb == 16 ? launch<D, G, DT, 16>(p, grid) : launch<D, G, DT, 32>(p, grid);
}

template <int D, int G>
int dispatch_dt(const AttnParams &p, dim3 grid, uint32_t dt, uint32_t tpb)
{
    return dt == RL_DTYPE_BF16 ? dispatch_tpb<D, G, 0>(p, grid, tpb) : dispatch_tpb<D, G, 1>(p, grid, tpb);
}

template <int D>
int dispatch_g(const AttnParams &p, dim3 grid, uint32_t G, uint32_t dt, uint32_t tpb)
{
    switch (G) {
    case 1: return dispatch_dt<D, 1>(p, grid, dt, tpb);
    case 2: return dispatch_dt<D, 2>(p, grid, dt, tpb);
    case 4: return dispatch_dt<D, 4>(p, grid, dt, tpb);
    default: return dispatch_dt<D, 8>(p, grid, dt, tpb);
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
    const uint32_t tok = a->chunk_tokens ? a->chunk_tokens : kDefaultChunkTokens;
    if (tok % 64 != 0 || tok == 0 || tok > 2048) {
        rl_set_error("rl_hip_attn_decode: chunk_tokens %u must be a multiple of 64 in [64, 2048]", tok);
        return -1;
    }
    if (!a->arena_base || !a->block_table || !a->ctx_lens || !a->q || !a->out) {
        rl_set_error("rl_hip_attn_decode: NULL device pointer");
        return -1;
    }
    if (a->batch == 0 || a->batch > 65535 || a->kv_heads > 65535) {
        rl_set_error("rl_hip_attn_decode: batch %u / kv_heads %u out of range", a->batch, a->kv_heads);
        return -1;
    }
    const uint32_t max_tiles = (a->max_ctx + kTileTokens - 1) / kTileTokens;
    if ((max_tiles + tok / kTileTokens - 1) / (tok / kTileTokens) > (uint32_t)kMergeMaxChunks) {
        rl_set_error("rl_hip_attn_decode: max_ctx %u needs more than %d chunks of %u tokens", a->max_ctx,
                     kMergeMaxChunks, tok);
        return -1;
    }
    const uint32_t table_need = (max_tiles + a->layout.token_count / kTileTokens - 1) /
                                (a->layout.token_count / kTileTokens);
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
    if (validate(a))
        return 0;
    return ws_layout(a, chunk_tiles_of(a)).total;
}

extern "C" int rl_hip_attn_decode(const rl_attn_decode_args_t *a)
{
    if (rl_require_open("rl_hip_attn_decode") || validate(a))
        return -1;
    const uint32_t chunk_tiles = chunk_tiles_of(a);
    const WsLayout w = ws_layout(a, chunk_tiles);
    if (!a->workspace || a->workspace_bytes < w.total) {
        rl_set_error("rl_hip_attn_decode: workspace %zu bytes < %zu required", a->workspace_bytes, w.total);
        return -1;
    }
    const uint32_t max_tiles = (a->max_ctx + kTileTokens - 1) / kTileTokens;
    const uint32_t max_chunks = max_tiles == 0 ? 1 : (max_tiles + chunk_tiles - 1) / chunk_tiles;

    AttnParams p;
    p.arena = (const uint8_t *)a->arena_base;
    p.block_bytes = a->layout.block_bytes;
    p.arena_blocks = a->arena_bytes / a->layout.block_bytes;
    p.max_ctx = a->max_ctx;
    p.table = a->block_table;
    p.table_stride = a->table_stride;
    p.ctx = a->ctx_lens;
    p.q = (const uint16_t *)a->q;
    p.out = (uint16_t *)a->out;
    p.out_f32 = a->out_f32;
    const float scale = a->scale != 0.f ? a->scale : 1.0f / sqrtf((float)a->layout.head_dim);
    p.scale_log2 = scale * 1.4426950408889634f;
    p.q_heads = a->q_heads;
    p.kv_heads = a->kv_heads;
    p.chunk_tiles = chunk_tiles;
    p.max_chunks = max_chunks;
    uint8_t *ws = (uint8_t *)a->workspace;
    p.ws_ml = (float *)(ws + w.ml_off);
    p.ws_o = (float *)(ws + w.o_off);

    const dim3 grid(max_chunks, a->kv_heads, a->batch);
    const uint32_t G = a->q_heads / a->kv_heads;
    if (a->layout.head_dim == 128)
        return dispatch_g<128>(p, grid, G, a->dtype, a->layout.token_count);
    return dispatch_g<64>(p, grid, G, a->dtype, a->layout.token_count);
}
