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
//         order (chunk c of row t lands at position c ^ t), which makes both
//         MFMA operand reads below free of LDS bank conflicts. The query of a
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

#include "kv_layout.h"
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr int kTile = 16;  // tokens per tile (the MFMA M/K block)

typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

struct AttnParams {
    const uint8_t *arena;
    uint64_t block_bytes;
    uint64_t arena_blocks;  // blocks at or past this index are never read
    const uint32_t *table;
    uint32_t table_stride;
    const uint32_t *ctx;
    uint32_t max_ctx;
    uint32_t batch;
    uint32_t q_heads;
    uint32_t kv_heads;
    const uint16_t *q;
    uint16_t *out;
    float *out_f32;
    float scale_log2;  // softmax scale * log2(e)
    uint32_t nwaves;   // waves sharing the tile sequence
    float *part;       // [nwaves + rows][G * D + 2 * G] partials of split rows
    uint32_t *cum;     // [batch + 1] tiles of all rows before rollout b
};

template <int D, int G, int DT, int TPB>
struct Cfg {
    static constexpr int W = 4;                   // waves per workgroup
    static constexpr int RB = 2 * D;              // bytes per K or V row
    static constexpr int NC = D / 8;              // 16-byte chunks per row
    static constexpr int PLANE = kTile * RB;      // one tile of K (or V)
    static constexpr int POPS = PLANE / 1024;     // copies per plane
    static constexpr int UNIT_OPS = 2 * POPS;     // copies per staged tile
    static constexpr int STAGE = 2 * PLANE;
    static constexpr int QBYTES = G * D * 2;
    static constexpr int QOPS = (QBYTES + 1023) / 1024;
    static constexpr int QSLOT = QOPS * 1024;
    static constexpr int WAVE_LDS = 2 * STAGE + 2 * QSLOT;
    static constexpr int KS = D / 32;             // QK MFMA k-steps
    static constexpr int NB = D / 16;             // PV MFMA column blocks
    static constexpr int SUB = TPB / kTile;       // tiles per arena block
    static constexpr int PART = G * D + 2 * G;    // floats per partial
    static constexpr int LDS_CU = 160 * 1024;
    static constexpr int WG_PER_CU_LDS = LDS_CU / (W * WAVE_LDS);
    static constexpr int WG_PER_CU = WG_PER_CU_LDS > 4 ? 4 : WG_PER_CU_LDS;
    static_assert(D == 64 || D == 128, "head_dim");
    static_assert(G == 1 || G == 2 || G == 4 || G == 8, "group");
    static_assert(PLANE % 1024 == 0, "plane must be whole 1 KiB copies");
    static_assert(WG_PER_CU >= 1, "LDS budget");
    static_assert(2 * QSLOT >= 16 * 4, "q slots double as prologue scratch");
};

// ---- 16-bit element helpers -----------------------------------------------

template <int DT>
__device__ __forceinline__ uint16_t to16(float f)
{
    if constexpr (DT == 0)
        return __builtin_bit_cast(uint16_t, (__bf16)f);
    else
        return __builtin_bit_cast(uint16_t, (_Float16)f);
}

template <int DT>
__device__ __forceinline__ float from16(uint16_t h)
{
    if constexpr (DT == 0)
        return __uint_as_float((uint32_t)h << 16);
    else
        return (float)__builtin_bit_cast(_Float16, h);
}

template <int DT>
__device__ __forceinline__ rl_f32x4 mfma_qk(s16x8 a, s16x8 b, rl_f32x4 c)
{
    if constexpr (DT == 0)
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
}

template <int DT>
__device__ __forceinline__ rl_f32x4 mfma_pv(s16x4 a, s16x4 b, rl_f32x4 c)
{
    if constexpr (DT == 0)
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
    else
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c,
                                                     0, 0, 0);
}

__device__ __forceinline__ uint32_t tiles_of(const AttnParams &p, uint32_t ctx_in)
{
    const uint32_t c = ctx_in > p.max_ctx ? p.max_ctx : ctx_in;
    return (c + kTile - 1) / kTile;
}

// What the copy stream put into one stage, read back when it is consumed.
struct StageMeta {
    uint32_t b, g, u, nu, ctx;  // row, tile index within the row, tiles of the row, clamped ctx
    uint32_t qslot;
    bool first;                 // first tile of its row in this wave (q arrives with it)
    bool last;                  // last tile of its row in this wave
    bool bad;                   // ctx beyond max_ctx or a block outside the arena
};

// Issue side of a wave: walks the wave's tile range and starts the copies.
template <int D, int G, int DT, int TPB>
struct Issuer {
    using C = Cfg<D, G, DT, TPB>;
    uint32_t b, g, u, nu, ctx;
    bool ctx_bad;
    bool first;
    uint32_t left;     // tiles still to issue
    uint32_t qcount;   // rows entered so far (q slot parity)
    uint32_t win0, win1, wrow, wfirst;  // block-table window: entries wfirst .. wfirst + 127 of row wrow
    uint32_t soff[C::POPS];             // per-lane source offset of each copy within a plane

    __device__ __forceinline__ void init_offsets(int lane)
    {
#pragma unroll
        for (int i = 0; i < C::POPS; i++) {
            const uint32_t byte = (uint32_t)i * 1024u + (uint32_t)lane * 16u;
            const uint32_t t = byte / C::RB;
            const uint32_t pos = (byte % C::RB) / 16u;
            soff[i] = t * C::RB + ((pos ^ (t & (C::NC - 1))) * 16u);
        }
    }

    __device__ __forceinline__ void set_rollout(const AttnParams &p, uint32_t nb)
    {
        b = nb;
        const uint32_t cin = rl_sload(p.ctx + nb);
        ctx_bad = cin > p.max_ctx;
        ctx = ctx_bad ? p.max_ctx : cin;
        nu = (ctx + kTile - 1) / kTile;
    }

    __device__ __forceinline__ void issue(const AttnParams &p, RL_LDS uint8_t *st, RL_LDS uint8_t *qslots,
                                          StageMeta &m, int lane)
    {
        const uint32_t row = b * p.kv_heads + g;
        const uint32_t lb = u / C::SUB;
        if (row != wrow || lb < wfirst || lb >= wfirst + 128u) {
            // New row or past the window: reload 128 table entries. The wait
            // drains the copies in flight, once per row change.
            const uint32_t nblk = (ctx + TPB - 1) / TPB;
            const uint32_t *trow = p.table + (size_t)row * p.table_stride;
            win0 = (lb + (uint32_t)lane < nblk) ? trow[lb + lane] : 0u;
            win1 = (lb + 64u + (uint32_t)lane < nblk) ? trow[lb + 64u + lane] : 0u;
            rl_wait_vmcnt<0>();
            wrow = row;
            wfirst = lb;
        }
        const uint32_t j = lb - wfirst;
        uint32_t blk = (uint32_t)__builtin_amdgcn_readlane((int)(j < 64u ? win0 : win1), (int)(j & 63u));
        m.bad = ctx_bad;
        if (blk >= p.arena_blocks) {
            // Never read outside the arena; copy block 0 instead so the number
            // of copies per tile stays fixed, and poison the row.
            m.bad = true;
            blk = 0;
        }
        m.b = b;
        m.g = g;
        m.u = u;
        m.nu = nu;
        m.ctx = ctx;
        m.first = first;
        if (first) {
            m.qslot = qcount & 1u;
            qcount++;
            const uint8_t *qsrc = (const uint8_t *)(p.q + ((size_t)b * p.q_heads + (size_t)g * G) * D);
#pragma unroll
            for (int i = 0; i < C::QOPS; i++) {
                uint32_t off = (uint32_t)i * 1024u + (uint32_t)lane * 16u;
                off = off < (uint32_t)C::QBYTES ? off : (uint32_t)C::QBYTES - 16u;
                rl_g2lds_16_off(qsrc, off, qslots + m.qslot * C::QSLOT + i * 1024);
            }
        }
        const uint8_t *kp = p.arena + (uint64_t)blk * p.block_bytes + (u % C::SUB) * C::PLANE;
        const uint8_t *vp = kp + TPB * C::RB;
#pragma unroll
        for (int i = 0; i < C::POPS; i++) {
            rl_g2lds_16_off(kp, soff[i], st + i * 1024);
            rl_g2lds_16_off(vp, soff[i], st + C::PLANE + i * 1024);
        }
        // advance
        left--;
        u++;
        first = false;
        m.last = (u == nu) || (left == 0);
        if (u == nu && left != 0) {
            u = 0;
            first = true;
            if (++g == p.kv_heads) {
                g = 0;
                // tiles remain, so a later rollout has some (bounded anyway)
                uint32_t nb = b;
                do {
                    set_rollout(p, ++nb);
                } while (nu == 0 && nb + 1 < p.batch);
            }
        }
    }
};

// Consume side: running softmax state of the current row and its output.
template <int D, int G, int DT, int TPB>
struct RowState {
    using C = Cfg<D, G, DT, TPB>;
    s16x8 qf[C::KS];          // B operand of QK: q[head lane%16][32 s + 8 (lane/16) .. + 7]
    rl_f32x4 acc[C::NB];      // O[head 4 (lane/16) + r][16 n + lane % 16]
    float m_run;              // running max (log2 domain) of head lane % 16
    float l_run;              // this lane's share of the running sum
    bool from0;               // the row started at tile 0 in this wave
    bool bad;
};

template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void row_begin(RowState<D, G, DT, TPB> &rs, RL_LDS const uint8_t *qslot,
                                          const StageMeta &m, int lane)
{
    using C = Cfg<D, G, DT, TPB>;
    const int h = lane & 15;
    const int hs = h < G ? h : G - 1;
#pragma unroll
    for (int s = 0; s < C::KS; s++) {
        s16x8 v = *(RL_LDS const s16x8 *)(qslot + hs * C::RB + (32 * s + 8 * (lane >> 4)) * 2);
        if (h >= G)
            v = s16x8{0, 0, 0, 0, 0, 0, 0, 0};
        rs.qf[s] = v;
    }
#pragma unroll
    for (int n = 0; n < C::NB; n++)
        rs.acc[n] = rl_f32x4{0.f, 0.f, 0.f, 0.f};
    rs.m_run = -INFINITY;
    rs.l_run = 0.f;
    rs.from0 = m.u == 0;
    rs.bad = false;
}

// One staged tile: QK (MFMA), online softmax, PV (MFMA).
template <int D, int G, int DT, int TPB, bool FULL>
__device__ __forceinline__ void consume_tile(const AttnParams &p, RowState<D, G, DT, TPB> &rs,
                                             RL_LDS const uint8_t *st, const StageMeta &m, int lane)
{
    using C = Cfg<D, G, DT, TPB>;
    const int h = lane & 15;   // head (QK output column / PV A row)
    const int tg = lane >> 4;  // token group: tokens 4 tg .. 4 tg + 3

    // ---- S^T = K q^T ---------------------------------------------------------
    rl_f32x4 sc = {0.f, 0.f, 0.f, 0.f};
    {
        const int t = lane & 15;
#pragma unroll
        for (int s = 0; s < C::KS; s++) {
            const int c = 4 * s + tg;
            const s16x8 kf = *(RL_LDS const s16x8 *)(st + t * C::RB + ((c ^ (t & (C::NC - 1))) << 4));
            sc = mfma_qk<DT>(kf, rs.qf[s], sc);
        }
    }

    // ---- online softmax ------------------------------------------------------
    const uint32_t tok0 = m.u * kTile + 4 * tg;
    float sv[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const bool ok = (h < G) && (FULL || tok0 + r < m.ctx);
        sv[r] = ok ? sc[r] * p.scale_log2 : -INFINITY;
    }
    float mx = fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3]));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(rs.m_run, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const bool grow = (m_new > rs.m_run) && (rs.m_run != -INFINITY);
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float alpha = grow ? exp2f(rs.m_run - m_use) : 1.f;
        rs.l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float a = __shfl(alpha, 4 * tg + r);
#pragma unroll
            for (int n = 0; n < C::NB; n++)
                rs.acc[n][r] *= a;
        }
    }
    rs.m_run = m_new;
    float pr[4];
#pragma unroll
    for (int r = 0; r < 4; r++)
        pr[r] = exp2f(sv[r] - m_use);
    rs.l_run += (pr[0] + pr[1]) + (pr[2] + pr[3]);

    // ---- P split into high and low 16-bit parts --------------------------------
    s16x4 phi, plo;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const uint16_t hi = to16<DT>(pr[r]);
        const uint16_t lo = to16<DT>(pr[r] - from16<DT>(hi));
        phi[r] = (short)hi;
        plo[r] = (short)lo;
    }

    // ---- O += P V --------------------------------------------------------------
    uint32_t vm0 = 0xFFFFFFFFu, vm1 = 0xFFFFFFFFu;
    if constexpr (!FULL) {
        // element r of the transposed operand is token 4 tg + r
        vm0 = (tok0 + 0 < m.ctx ? 0x0000FFFFu : 0u) | (tok0 + 1 < m.ctx ? 0xFFFF0000u : 0u);
        vm1 = (tok0 + 2 < m.ctx ? 0x0000FFFFu : 0u) | (tok0 + 3 < m.ctx ? 0xFFFF0000u : 0u);
    }
    {
        const int L = lane & 15;
        const int t = 4 * tg + (L >> 2);
        const int sw = t & (C::NC - 1);
        RL_LDS const uint8_t *vrow = st + C::PLANE + t * C::RB + 8 * (L & 1);
#pragma unroll
        for (int n = 0; n < C::NB; n++) {
            const int c = 2 * n + ((L & 3) >> 1);
            s16x4 vb = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (RL_LDS s16x4 *)(vrow + ((c ^ sw) << 4)));
            if constexpr (!FULL) {
                // stale slots past ctx may hold anything, NaN included: zero them
                uint32_t w0 = __builtin_bit_cast(uint32_t, __builtin_shufflevector(vb, vb, 0, 1)) & vm0;
                uint32_t w1 = __builtin_bit_cast(uint32_t, __builtin_shufflevector(vb, vb, 2, 3)) & vm1;
                typedef short s16x2 __attribute__((ext_vector_type(2)));
                const s16x2 a = __builtin_bit_cast(s16x2, w0);
                const s16x2 b2 = __builtin_bit_cast(s16x2, w1);
                vb = s16x4{a[0], a[1], b2[0], b2[1]};
            }
            rs.acc[n] = mfma_pv<DT>(phi, vb, rs.acc[n]);
            rs.acc[n] = mfma_pv<DT>(plo, vb, rs.acc[n]);
        }
    }
}

// Row done in this wave: direct output, or an fp32 partial for the merge.
template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void row_end(const AttnParams &p, RowState<D, G, DT, TPB> &rs, const StageMeta &m,
                                        uint32_t wave_id, int lane)
{
    using C = Cfg<D, G, DT, TPB>;
    const int h = lane & 15;
    const int tg = lane >> 4;
    float lt = rs.l_run + __shfl_xor(rs.l_run, 16);
    lt += __shfl_xor(lt, 32);
    const bool poison = rs.bad || m.bad;
    const uint32_t row = m.b * p.kv_heads + m.g;
    if (rs.from0 && m.u + 1 == m.nu) {
        const size_t obase = ((size_t)m.b * p.q_heads + (size_t)m.g * G) * D;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float L = __shfl(lt, 4 * tg + r);
            const int hh = 4 * tg + r;
            if (hh < G) {
#pragma unroll
                for (int n = 0; n < C::NB; n++) {
                    float v = L > 0.f ? rs.acc[n][r] / L : 0.f;
                    if (poison)
                        v = __builtin_nanf("");
                    const size_t o = obase + (size_t)hh * D + 16 * n + h;
                    p.out[o] = rl_from_f32<DT>(v);
                    if (p.out_f32)
                        p.out_f32[o] = v;
                }
            }
        }
    } else {
        float *part = p.part + (size_t)(wave_id + row) * C::PART;
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int hh = 4 * tg + r;
            if (hh < G) {
#pragma unroll
                for (int n = 0; n < C::NB; n++)
                    part[hh * D + 16 * n + h] = rs.acc[n][r];
            }
        }
        if (lane < G) {
            part[G * D + 2 * lane + 0] = rs.m_run;
            part[G * D + 2 * lane + 1] = poison ? __builtin_nanf("") : lt;
        }
    }
}

template <int D, int G, int DT, int TPB>
__device__ __forceinline__ void consume(const AttnParams &p, RowState<D, G, DT, TPB> &rs, RL_LDS const uint8_t *st,
                                        RL_LDS const uint8_t *qslots, const StageMeta &m, uint32_t wave_id, int lane)
{
    using C = Cfg<D, G, DT, TPB>;
    if (m.first)
        row_begin<D, G, DT, TPB>(rs, qslots + m.qslot * C::QSLOT, m, lane);
    rs.bad |= m.bad;
    if (m.u * kTile + kTile <= m.ctx)
        consume_tile<D, G, DT, TPB, true>(p, rs, st, m, lane);
    else
        consume_tile<D, G, DT, TPB, false>(p, rs, st, m, lane);
    if (m.last)
        row_end<D, G, DT, TPB>(p, rs, m, wave_id, lane);
}

template <int D, int G, int DT, int TPB>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnParams p)
{
    using C = Cfg<D, G, DT, TPB>;
    constexpr int W = C::W;
    static_assert(W * 64 == 256, "launch bounds");
    // Separate arrays per stage so the compiler's wait insertion can tell a
    // copy into one stage from reads of the other.
    __shared__ __attribute__((aligned(1024))) uint8_t lds_st0[W * C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_st1[W * C::STAGE];
    __shared__ __attribute__((aligned(1024))) uint8_t lds_q[W * 2 * C::QSLOT];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

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
    uint32_t inc = S;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const uint32_t v = __shfl_up(inc, off);
        if (lane >= off)
            inc += v;
    }
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
        const uint32_t w = blockIdx.x * W + v;
        if (w < NW && S > 0) {
            const uint32_t s = (uint32_t)(((uint64_t)w * U) / NW);
            if (s >= P0 && s < P0 + S) {
                uint32_t c = P0;
                for (uint32_t bb = b0; bb < b1; bb++) {
                    const uint32_t n = tiles_of(p, p.ctx[bb]) * p.kv_heads;
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
            c += tiles_of(p, p.ctx[bb]) * p.kv_heads;
        }
        if (threadIdx.x == T - 1)
            p.cum[p.batch] = U;
    }
    __syncthreads();
    const uint32_t wave_id = blockIdx.x * W + wave;
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

    RL_LDS uint8_t *st0 = (RL_LDS uint8_t *)lds_st0 + wave * C::STAGE;
    RL_LDS uint8_t *st1 = (RL_LDS uint8_t *)lds_st1 + wave * C::STAGE;
    RL_LDS uint8_t *qs = (RL_LDS uint8_t *)lds_q + wave * 2 * C::QSLOT;

    Issuer<D, G, DT, TPB> is;
    is.init_offsets(lane);
    is.set_rollout(p, rb);
    {
        const uint32_t rem = s_begin - rcum;
        is.g = rem / is.nu;
        is.u = rem % is.nu;
    }
    is.left = s_end - s_begin;
    is.first = true;
    is.qcount = 0;
    is.wrow = 0xFFFFFFFFu;
    is.wfirst = 0;
    is.win0 = is.win1 = 0;

    RowState<D, G, DT, TPB> rs;
    StageMeta mc, mn;  // tile to consume next, tile in flight behind it
    RL_LDS uint8_t *stc = st0;
    RL_LDS uint8_t *stn = st1;
    bool has_next = false;
    is.issue(p, stc, qs, mc, lane);
    if (is.left) {
        is.issue(p, stn, qs, mn, lane);
        has_next = true;
    }
    for (;;) {
        // Copies complete in issue order: once at most one tile's worth is
        // outstanding, everything older - this tile and its q - has landed.
        // (A tile that brings a q slot issues one more copy: the wait is then
        // slightly stronger than needed, never weaker.)
        if (has_next)
            rl_wait_vmcnt<C::UNIT_OPS>();
        else
            rl_wait_vmcnt<0>();
        consume<D, G, DT, TPB>(p, rs, stc, qs, mc, wave_id, lane);
        if (!has_next)
            break;
        // the stage just consumed takes the tile after next
        StageMeta mi;
        bool has_after = false;
        if (is.left) {
            rl_wait_lgkmcnt0();
            is.issue(p, stc, qs, mi, lane);
            has_after = true;
        }
        RL_LDS uint8_t *t = stc;
        stc = stn;
        stn = t;
        mc = mn;
        mn = mi;
        has_next = has_after;
    }
}

// Combines the partials of every row split across waves:
// M = max_w m_w, L = sum_w l_w 2^(m_w - M), O = sum_w o_w 2^(m_w - M), out = O / L.
// Also writes rows without tiles (ctx 0: zeros; ctx beyond max_ctx: NaN).
// The (max, sum) pairs of up to kMergeLds partials are loaded in parallel into
// LDS, the per-head scale factors computed once, and every output element then
// sums its partials with independent loads.
constexpr int kMergeLds = 256;

template <int D, int G, int DT>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnParams p)
{
    constexpr int PART = G * D + 2 * G;
    __shared__ float s_f[kMergeLds * G];  // m, then the scale 2^(m - M)
    __shared__ float s_l[kMergeLds * G];
    __shared__ float s_L[G];
    const uint32_t g = blockIdx.x;
    const uint32_t b = blockIdx.y;
    const uint32_t row = b * p.kv_heads + g;
    const uint32_t cin = rl_sload(p.ctx + b);
    const bool bad = cin > p.max_ctx;
    const uint32_t nu = tiles_of(p, cin);
    const size_t obase = ((size_t)b * p.q_heads + (size_t)g * G) * D;
    if (nu == 0) {
        for (int e = threadIdx.x; e < G * D; e += 256) {
            const float v = bad ? __builtin_nanf("") : 0.f;
            p.out[obase + e] = rl_from_f32<DT>(v);
            if (p.out_f32)
                p.out_f32[obase + e] = v;
        }
        return;
    }
    const uint32_t U = rl_sload(p.cum + p.batch);  // > 0: this row has tiles
    const uint32_t NW = min(p.nwaves, U);
    const uint32_t R0 = rl_sload(p.cum + b) + g * nu;
    const uint32_t R1 = R0 + nu;
    // wave holding tile R0 / tile R1 - 1: the largest w with floor(w U / NW) <= tile
    const uint32_t wf = (uint32_t)((((uint64_t)R0 + 1) * NW - 1) / U);
    const uint32_t wl = (uint32_t)(((uint64_t)R1 * NW - 1) / U);
    if (wf == wl)
        return;  // one wave covered the row and wrote it
    const float *part = p.part + (size_t)(wf + row) * PART;
    const uint32_t np = wl - wf + 1;
    constexpr int EPT = (G * D + 255) / 256;  // output elements per thread
    constexpr int NPR = 8;                    // partials merged from registers
    if (np <= (uint32_t)NPR) {
        // few partials: every load is issued before the first use
        float o[NPR][EPT], mm[NPR][EPT], ll[NPR][EPT];
#pragma unroll
        for (int i = 0; i < NPR; i++)
#pragma unroll
            for (int k = 0; k < EPT; k++) {
                const int e = threadIdx.x + 256 * k;
                const bool ok = (uint32_t)i < np && e < G * D;
                const float *pp = part + (size_t)(ok ? i : 0) * PART;
                const int h = (e < G * D ? e : 0) / D;
                o[i][k] = ok ? pp[e] : 0.f;
                mm[i][k] = ok ? pp[G * D + 2 * h] : -INFINITY;
                ll[i][k] = ok ? pp[G * D + 2 * h + 1] : 0.f;
            }
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const int e = threadIdx.x + 256 * k;
            if (e >= G * D)
                break;
            float M = -INFINITY;
#pragma unroll
            for (int i = 0; i < NPR; i++)
                M = fmaxf(M, mm[i][k]);
            float L = 0.f, O = 0.f;
#pragma unroll
            for (int i = 0; i < NPR; i++) {
                const float f = mm[i][k] == -INFINITY ? 0.f : exp2f(mm[i][k] - M);
                L = fmaf(ll[i][k], f, L);
                O = fmaf(o[i][k], f, O);
            }
            float v = (L > 0.f || L != L) ? O / L : 0.f;
            if (bad)
                v = __builtin_nanf("");
            p.out[obase + e] = rl_from_f32<DT>(v);
            if (p.out_f32)
                p.out_f32[obase + e] = v;
        }
        return;
    }
    if (np <= (uint32_t)kMergeLds) {
        for (uint32_t t = threadIdx.x; t < np * G; t += 256) {
            const uint32_t i = t / G, h = t % G;
            s_f[t] = part[(size_t)i * PART + G * D + 2 * h];
            s_l[t] = part[(size_t)i * PART + G * D + 2 * h + 1];
        }
        __syncthreads();
        if (threadIdx.x < G) {
            const int h = threadIdx.x;
            float M = -INFINITY;
            for (uint32_t i = 0; i < np; i++)
                M = fmaxf(M, s_f[i * G + h]);
            float L = 0.f;
            for (uint32_t i = 0; i < np; i++) {
                const float mi = s_f[i * G + h];
                const float f = mi == -INFINITY ? 0.f : exp2f(mi - M);
                s_f[i * G + h] = f;
                L = fmaf(s_l[i * G + h], f, L);
            }
            s_L[h] = L;
        }
        __syncthreads();
        for (int e = threadIdx.x; e < G * D; e += 256) {
            const int h = e / D;
            float O = 0.f;
#pragma unroll 8
            for (uint32_t i = 0; i < np; i++)
                O = fmaf(part[(size_t)i * PART + e], s_f[i * G + h], O);
            const float L = s_L[h];
            float v = (L > 0.f || L != L) ? O / L : 0.f;
            if (bad)
                v = __builtin_nanf("");
            p.out[obase + e] = rl_from_f32<DT>(v);
            if (p.out_f32)
                p.out_f32[obase + e] = v;
        }
        return;
    }
    // very long rows: stream the partials per element
    for (int e = threadIdx.x; e < G * D; e += 256) {
        const int h = e / D;
        float M = -INFINITY;
        for (uint32_t i = 0; i < np; i++)
            M = fmaxf(M, part[(size_t)i * PART + G * D + 2 * h]);
        float L = 0.f, O = 0.f;
        for (uint32_t i = 0; i < np; i++) {
            const float *pp = part + (size_t)i * PART;
            const float mi = pp[G * D + 2 * h];
            const float f = mi == -INFINITY ? 0.f : exp2f(mi - M);
            L = fmaf(pp[G * D + 2 * h + 1], f, L);
            O = fmaf(pp[e], f, O);
        }
        float v = (L > 0.f || L != L) ? O / L : 0.f;
        if (bad)
            v = __builtin_nanf("");
        p.out[obase + e] = rl_from_f32<DT>(v);
        if (p.out_f32)
            p.out_f32[obase + e] = v;
    }
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
    // LDS per wave: two stages of one tile's K and V, two q slots
    const uint32_t wave_lds = 2 * (2 * 16 * 2 * D) + 2 * ((G * D * 2 + 1023) / 1024) * 1024;
    uint32_t wg = (160u * 1024u) / (4 * wave_lds);
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
int launch(const AttnParams &p)
{
    using C = Cfg<D, G, DT, TPB>;
    const uint32_t wgs = (p.nwaves + C::W - 1) / C::W;
    hipLaunchKernelGGL((attn_decode_kernel<D, G, DT, TPB>), dim3(wgs), dim3(C::W * 64), 0, rl_stream(), p);
    if (rl_check_launch("attn_decode_kernel launch"))
        return -1;
    hipLaunchKernelGGL((attn_merge_kernel<D, G, DT>), dim3(p.kv_heads, p.batch), dim3(256), 0, rl_stream(), p);
    return rl_check_launch("attn_merge_kernel launch");
}

template <int D, int G, int DT>
int dispatch_tpb(const AttnParams &p, uint32_t tpb)
{
    return tpb == 16 ? launch<D, G, DT, 16>(p) : launch<D, G, DT, 32>(p);
}

template <int D, int G>
int dispatch_dt(const AttnParams &p, uint32_t dt, uint32_t tpb)
{
    return dt == RL_DTYPE_BF16 ? dispatch_tpb<D, G, 0>(p, tpb) : dispatch_tpb<D, G, 1>(p, tpb);
}

template <int D>
int dispatch_g(const AttnParams &p, uint32_t G, uint32_t dt, uint32_t tpb)
{
    switch (G) {
    case 1: return dispatch_dt<D, 1>(p, dt, tpb);
    case 2: return dispatch_dt<D, 2>(p, dt, tpb);
    case 4: return dispatch_dt<D, 4>(p, dt, tpb);
    default: return dispatch_dt<D, 8>(p, dt, tpb);
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

extern "C" int rl_hip_attn_decode(const rl_attn_decode_args_t *a)
{
    if (rl_require_open("rl_hip_attn_decode") || validate(a))
        return -1;
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
        return dispatch_g<128>(p, G, a->dtype, a->layout.token_count);
    return dispatch_g<64>(p, G, a->dtype, a->layout.token_count);
}
