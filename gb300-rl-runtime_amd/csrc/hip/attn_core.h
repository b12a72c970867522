// attn_core.h - device building blocks of the paged GQA decode attention
// (gfx950): tile staging, MFMA QK/PV with online softmax, per-wave tile
// streams and the log-sum-exp merge of split rows. Used by the batched
// attention kernel and by the persistent ring worker.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "kv_layout.h"
#include "rl_dev_common.h"

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
    const uint32_t *row_map;  // [batch]: the table row (rollout) of batch row b, or NULL: b itself
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

    // LDS position of 16-byte chunk c of tile row t is c ^ swizzle(t). K rows
    // are read 16 rows x one chunk per 16 lanes (ds_read_b128): t itself
    // spreads them over the 16 bank groups. V is read transposed, 8 rows x two
    // adjacent chunks per 32 lanes (ds_read_tr16_b64): with t the pairs of
    // rows 2i, 2i + 1 land on the same 8 groups (2-way conflicts), so V rows
    // use t rotated left by one bit, which gives each of the 8 rows its own
    // pair of groups. (Measured on gfx950: 0 conflict cycles per read for
    // both, against 2 per V read with t.) D = 64 keeps t for both planes.
    static __device__ __forceinline__ uint32_t kswz(uint32_t t) { return t & (NC - 1); }
    static __device__ __forceinline__ uint32_t vswz(uint32_t t)
    {
        return NC == 16 ? (((t << 1) | (t >> 3)) & 15u) : (t & (NC - 1));
    }
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

// Context length of rollout b and the block-table row it reads: from the
// ctx array and p.row_map (scalar loads), or one context fixed by the
// caller, or from copies in LDS (a persistent kernel's per-step arguments,
// which the launch itself rewrites between steps).
__device__ __forceinline__ uint32_t table_row_of(const AttnParams &p, uint32_t b)
{
    return p.row_map ? rl_sload(p.row_map + b) : b;
}
struct CtxFromArray {
    const uint32_t *ctx;
    __device__ __forceinline__ uint32_t operator()(uint32_t b) const { return rl_sload(ctx + b); }
    __device__ __forceinline__ uint32_t table_row(const AttnParams &p, uint32_t b) const { return table_row_of(p, b); }
};
struct CtxFixed {
    uint32_t value;
    __device__ __forceinline__ uint32_t operator()(uint32_t) const { return value; }
    __device__ __forceinline__ uint32_t table_row(const AttnParams &p, uint32_t b) const { return table_row_of(p, b); }
};
struct CtxLds {
    RL_LDS const uint32_t *ctx;  // [batch]
    RL_LDS const uint32_t *row;  // [batch]: the table row of each rollout
    __device__ __forceinline__ uint32_t operator()(uint32_t b) const { return ctx[b]; }
    __device__ __forceinline__ uint32_t table_row(const AttnParams &, uint32_t b) const { return row[b]; }
};

// Issue side of a wave: walks the wave's tile range and starts the copies.
// NS stages (tiles in the pipeline) need NS q slots: every row whose first
// tile is staged but not yet consumed holds one.
template <int D, int G, int DT, int TPB, int NS, class CtxFn>
struct Issuer {
    using C = Cfg<D, G, DT, TPB>;
    CtxFn cf;
    uint32_t b, g, u, nu, ctx;
    uint32_t tb;       // table row of rollout b
    bool ctx_bad;
    bool first;
    uint32_t left;     // tiles still to issue
    uint32_t qcount;   // rows entered so far (q slot parity)
    uint32_t win0, win1, wrow, wfirst;  // block-table window: entries wfirst .. wfirst + 127 of row wrow
    uint32_t soff[C::POPS], svoff[C::POPS];  // per-lane source offset of each copy within the K / V plane

    __device__ __forceinline__ void init_offsets(int lane)
    {
#pragma unroll
        for (int i = 0; i < C::POPS; i++) {
            const uint32_t byte = (uint32_t)i * 1024u + (uint32_t)lane * 16u;
            const uint32_t t = byte / C::RB;
            const uint32_t pos = (byte % C::RB) / 16u;
            soff[i] = t * C::RB + ((pos ^ C::kswz(t)) * 16u);
            svoff[i] = t * C::RB + ((pos ^ C::vswz(t)) * 16u);
        }
    }

    __device__ __forceinline__ void set_rollout(const AttnParams &p, uint32_t nb)
    {
        b = nb;
        tb = cf.table_row(p, nb);
        const uint32_t cin = cf(nb);
        ctx_bad = cin > p.max_ctx;
        ctx = ctx_bad ? p.max_ctx : cin;
        nu = (ctx + kTile - 1) / kTile;
    }

    __device__ __forceinline__ void issue(const AttnParams &p, RL_LDS uint8_t *st, RL_LDS uint8_t *qslots,
                                          StageMeta &m, int lane)
    {
        const uint32_t row = tb * p.kv_heads + g;
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
            m.qslot = qcount % (uint32_t)NS;
            qcount++;
            const uint8_t *qsrc = (const uint8_t *)(p.q + ((size_t)b * p.q_heads + (size_t)g * G) * D);
            // head h's chunk c lands at c ^ h: the heads' rows (RB apart,
            // read at one column by row_begin) then sit in distinct banks
#pragma unroll
            for (int i = 0; i < C::QOPS; i++) {
                const uint32_t byte = (uint32_t)i * 1024u + (uint32_t)lane * 16u;
                const uint32_t h = byte / C::RB, pos = (byte % C::RB) / 16u;
                const uint32_t off = byte < (uint32_t)C::QBYTES ? h * C::RB + ((pos ^ C::kswz(h)) * 16u)
                                                                : (uint32_t)C::QBYTES - 16u;
                rl_g2lds_16_off(qsrc, off, qslots + m.qslot * C::QSLOT + i * 1024);
            }
        }
        const uint8_t *kp = p.arena + (uint64_t)blk * p.block_bytes + (u % C::SUB) * C::PLANE;
        const uint8_t *vp = kp + TPB * C::RB;
#pragma unroll
        for (int i = 0; i < C::POPS; i++) {
            rl_g2lds_16_off(kp, soff[i], st + i * 1024);
            rl_g2lds_16_off(vp, svoff[i], st + C::PLANE + i * 1024);
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
        const uint32_t c = 4u * s + (uint32_t)(lane >> 4);  // chunk of dims 32 s + 8 (lane / 16) ..
        s16x8 v = *(RL_LDS const s16x8 *)(qslot + hs * C::RB + ((c ^ C::kswz((uint32_t)hs)) << 4));
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
            const s16x8 kf = *(RL_LDS const s16x8 *)(st + t * C::RB + ((c ^ C::kswz(t)) << 4));
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
        const int sw = (int)C::vswz((uint32_t)t);
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
                    if (p.out)
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


// Waits until at most n staged tiles' copies of this wave are outstanding
// (copies complete in issue order; n * UNIT stays below the 6-bit vmcnt).
template <int UNIT, int NMAX>
__device__ __forceinline__ void wait_tiles(uint32_t n)
{
    static_assert(NMAX * UNIT < 64, "vmcnt range");
    if constexpr (NMAX >= 7) { if (n >= 7) { rl_wait_vmcnt<7 * UNIT>(); return; } }
    if constexpr (NMAX >= 6) { if (n == 6) { rl_wait_vmcnt<6 * UNIT>(); return; } }
    if constexpr (NMAX >= 5) { if (n == 5) { rl_wait_vmcnt<5 * UNIT>(); return; } }
    if constexpr (NMAX >= 4) { if (n == 4) { rl_wait_vmcnt<4 * UNIT>(); return; } }
    if constexpr (NMAX >= 3) { if (n == 3) { rl_wait_vmcnt<3 * UNIT>(); return; } }
    if constexpr (NMAX >= 2) { if (n == 2) { rl_wait_vmcnt<2 * UNIT>(); return; } }
    if (n >= 1)
        rl_wait_vmcnt<UNIT>();
    else
        rl_wait_vmcnt<0>();
}

// The main loop of one wave: stream tiles [s_begin, s_end) of the row
// sequence, starting in rollout start_b whose first tile is start_cum.
// NS stages form a ring (stage k at st + k * st_stride; q slots at qs): while
// one tile is consumed the next NS - 1 are in flight, and the consumed stage
// takes the tile NS ahead. Rows finished in this wave are written directly or
// as partials.
template <int D, int G, int DT, int TPB, int NS, class CtxFn>
__device__ __forceinline__ void attn_stream(const AttnParams &p, const CtxFn &cf, uint32_t wave_id, uint32_t s_begin,
                                            uint32_t s_end, uint32_t start_b, uint32_t start_cum,
                                            RL_LDS uint8_t *st, uint32_t st_stride, RL_LDS uint8_t *qs, int lane)
{
    using C = Cfg<D, G, DT, TPB>;
    static_assert(NS >= 2 && NS <= 8, "stages");
    Issuer<D, G, DT, TPB, NS, CtxFn> is;
    is.cf = cf;
    is.init_offsets(lane);
    is.set_rollout(p, start_b);
    {
        const uint32_t rem = s_begin - start_cum;
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
    StageMeta m[NS];  // indexed with compile-time slots only (the ring loop is unrolled)
    uint32_t n_in = 0;  // tiles staged and not yet consumed
#pragma unroll
    for (int k = 0; k < NS; k++)
        if (is.left) {
            is.issue(p, st + k * st_stride, qs, m[k], lane);
            n_in++;
        }
    for (;;) {
#pragma unroll
        for (int k = 0; k < NS; k++) {
            // Once at most n_in - 1 tiles' copies are outstanding, this tile
            // and its q have landed. (A younger tile that brings a q slot
            // issues more copies: the wait is then stronger, never weaker.)
            wait_tiles<C::UNIT_OPS, NS - 1>(n_in - 1);
            consume<D, G, DT, TPB>(p, rs, st + k * st_stride, qs, m[k], wave_id, lane);
            n_in--;
            if (is.left) {
                // the consumed stage takes the tile NS ahead
                rl_wait_lgkmcnt0();
                is.issue(p, st + k * st_stride, qs, m[k], lane);
                n_in++;
            } else if (n_in == 0) {
                return;
            }
        }
    }
}

// Log-sum-exp merge of one split row (rollout b, kv head g) whose tiles are
// [R0, R0 + nu) of a sequence of U tiles shared by NW waves, the partials of
// waves wf..wl at p.part[(w + row)]: M = max_w m_w, L = sum_w l_w 2^(m_w - M),
// O = sum_w o_w 2^(m_w - M), out = O / L. Threads tid, tid + NTHR, ... of the
// caller take the output elements (NTHR a multiple of 64); s_f holds
// kMergeLds * G floats and s_L G floats of LDS. Returns without writing when one wave covered the row.
constexpr int kMergeLds = 256;

// Wave-wide max / sum of a float (butterfly: every lane ends with the same
// value).
__device__ __forceinline__ float wave_max_f32(float x)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        x = fmaxf(x, __shfl_xor(x, o));
    return x;
}

__device__ __forceinline__ float wave_sum_f32(float x)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1)
        x += __shfl_xor(x, o);
    return x;
}

// The merge of row (b, g) from the partials of streams wf .. wl at
// p.part[(w + row)] (a stream being a wave of an even split or a piece of
// the fused step); nothing to do when one stream covered the row.
template <int D, int G, int DT, int NTHR, int GH>
__device__ __forceinline__ void merge_span(const AttnParams &p, uint32_t b, uint32_t g, uint32_t h0, uint32_t wf,
                                           uint32_t wl, bool bad, uint32_t tid, float *s_f, float *s_L)
{
    static_assert(G % GH == 0, "head subset");
    constexpr int PART = G * D + 2 * G;
    constexpr int NE = GH * D;  // output elements of the head subset: global element h0 * D + e
    constexpr uint32_t nthr = NTHR;
    const uint32_t row = b * p.kv_heads + g;
    const size_t obase = ((size_t)b * p.q_heads + (size_t)g * G) * D;
    if (wf == wl)
        return;
    const float *part = p.part + (size_t)(wf + row) * PART;
    const uint32_t np = wl - wf + 1;
    auto store = [&](uint32_t e, float O, float L) {
        float v = (L > 0.f || L != L) ? O / L : 0.f;
        if (bad)
            v = __builtin_nanf("");
        if (p.out)
            p.out[obase + e] = rl_from_f32<DT>(v);
        if (p.out_f32)
            p.out_f32[obase + e] = v;
    };
    constexpr int EPT = (NE + NTHR - 1) / NTHR;         // output elements per thread
    // partials merged from registers, all loaded in one round: up to 40 when
    // a thread has one output element (long rows over a head subset), 16 with
    // two, 8 else
    constexpr int NPR = EPT == 1 ? 40 : EPT == 2 ? 16 : 8;
    if (np <= (uint32_t)NPR) {
        // few partials: every load is issued before the first use
        float o[NPR][EPT], mm[NPR][EPT], ll[NPR][EPT];
#pragma unroll
        for (int i = 0; i < NPR; i++)
#pragma unroll
            for (int k = 0; k < EPT; k++) {
                const uint32_t e = tid + nthr * k;
                const bool ok = (uint32_t)i < np && e < (uint32_t)NE;
                const float *pp = part + (size_t)(ok ? i : 0) * PART;
                const uint32_t eg = h0 * D + (ok ? e : 0);
                const int h = eg / D;
                o[i][k] = ok ? pp[eg] : 0.f;
                mm[i][k] = ok ? pp[G * D + 2 * h] : -INFINITY;
                ll[i][k] = ok ? pp[G * D + 2 * h + 1] : 0.f;
            }
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const uint32_t e = tid + nthr * k;
            if (e >= (uint32_t)NE)
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
            store(h0 * D + e, O, L);
        }
        return;
    }
    if (np <= (uint32_t)kMergeLds) {
        // the weights 2^(m_w - M) of each head's partials: wave v takes heads
        // h0 + v, h0 + v + NTHR / 64, ..., lane j partials j, j + 64, ... (all
        // loaded at once), with M and L reduced across the wave
        constexpr uint32_t nwav = nthr / 64;
        constexpr int PL = kMergeLds / 64;  // partials per lane at most
        const uint32_t wv = tid / 64, ln = tid % 64;
        for (uint32_t h = h0 + wv; h < h0 + (uint32_t)GH; h += nwav) {
            float mv[PL], lv[PL];
#pragma unroll
            for (int j = 0; j < PL; j++) {
                const uint32_t i = ln + 64u * (uint32_t)j;
                const bool ok = i < np;
                const float *pp = part + (size_t)(ok ? i : 0) * PART + G * D + 2 * h;
                mv[j] = ok ? pp[0] : -INFINITY;
                lv[j] = ok ? pp[1] : 0.f;
            }
            float M = -INFINITY;
#pragma unroll
            for (int j = 0; j < PL; j++)
                M = fmaxf(M, mv[j]);
            M = wave_max_f32(M);
            float L = 0.f;
#pragma unroll
            for (int j = 0; j < PL; j++) {
                const uint32_t i = ln + 64u * (uint32_t)j;
                const float f = mv[j] == -INFINITY ? 0.f : exp2f(mv[j] - M);
                if (i < np)
                    s_f[i * G + h] = f;
                L = fmaf(lv[j], f, L);
            }
            L = wave_sum_f32(L);
            if (ln == 0)
                s_L[h] = L;
        }
        __syncthreads();
        // the outputs, kC partials at a time: the loads of all of a thread's
        // elements for the chunk (16 in all) are issued before the first use
        constexpr int kC = EPT >= 8 ? 2 : 16 / EPT;
        float O[EPT];
#pragma unroll
        for (int k = 0; k < EPT; k++)
            O[k] = 0.f;
        for (uint32_t i0 = 0; i0 < np; i0 += kC) {
            float v[kC][EPT];
#pragma unroll
            for (int c = 0; c < kC; c++)
#pragma unroll
                for (int k = 0; k < EPT; k++) {
                    const uint32_t i = i0 + (uint32_t)c, e = tid + nthr * (uint32_t)k;
                    const bool ok = i < np && e < (uint32_t)NE;
                    v[c][k] = ok ? part[(size_t)i * PART + h0 * D + e] : 0.f;
                }
#pragma unroll
            for (int c = 0; c < kC; c++)
#pragma unroll
                for (int k = 0; k < EPT; k++) {
                    const uint32_t i = i0 + (uint32_t)c, e = tid + nthr * (uint32_t)k;
                    if (i < np && e < (uint32_t)NE)
                        O[k] = fmaf(v[c][k], s_f[i * G + h0 + e / D], O[k]);
                }
        }
#pragma unroll
        for (int k = 0; k < EPT; k++) {
            const uint32_t e = tid + nthr * (uint32_t)k;
            if (e < (uint32_t)NE)
                store(h0 * D + e, O[k], s_L[h0 + e / D]);
        }
        __syncthreads();
        return;
    }
    // very long rows: stream the partials per element
    for (uint32_t e = tid; e < (uint32_t)NE; e += nthr) {
        const uint32_t eg = h0 * D + e;
        const int h = eg / D;
        float M = -INFINITY;
        for (uint32_t i = 0; i < np; i++)
            M = fmaxf(M, part[(size_t)i * PART + G * D + 2 * h]);
        float L = 0.f, O = 0.f;
        for (uint32_t i = 0; i < np; i++) {
            const float *pp = part + (size_t)i * PART;
            const float mi = pp[G * D + 2 * h];
            const float f = mi == -INFINITY ? 0.f : exp2f(mi - M);
            L = fmaf(pp[G * D + 2 * h + 1], f, L);
            O = fmaf(pp[eg], f, O);
        }
        store(eg, O, L);
    }
}

// merge_span of one whole row (all G heads) by one wave, with the arithmetic
// of merge_span's register path in the same order: M = max_w m_w per head,
// then L = sum l_w f_w and O = sum o_w f_w over w ascending (fmaf), f_w =
// 2^(m_w - M), out = O / L. The partials go 64 at a time: lane j of a round
// loads partial (round start + j)'s (m, l) of every head, which gives M by a
// wave reduction and each f_w by readlane (a row of at most 64 partials, the
// usual case, loads them once); lane l owns output elements l + 64 k. The O
// loads of up to 8 partials are in flight together with the (m, l) loads.
template <int D, int G, int DT>
__device__ __forceinline__ void merge_row_wave(const AttnParams &p, uint32_t b, uint32_t g, uint32_t wf, uint32_t wl,
                                               bool bad, int lane)
{
    constexpr int PART = G * D + 2 * G;
    constexpr int EPL = G * D / 64;  // output elements per lane
    constexpr int CH = 8;            // partials per round of O loads
    static_assert(G * D % 64 == 0, "lane mapping");
    if (wf == wl)
        return;
    const uint32_t row = b * p.kv_heads + g;
    const uint32_t np = wl - wf + 1;
    const float *part = p.part + (size_t)(wf + row) * PART;
    // lane j: partial c0 + j's (m, l) per head (clamped addresses, masked)
    float mj[G], lj[G];
    auto load_ml = [&](uint32_t c0) {
        const float *pj = part + (size_t)min(c0 + (uint32_t)lane, np - 1) * PART + G * D;
#pragma unroll
        for (int h = 0; h < G; h++) {
            mj[h] = pj[2 * h];
            lj[h] = pj[2 * h + 1];
        }
    };
    load_ml(0);
    float ov[CH][EPL];
    auto load_o = [&](uint32_t i0) {
#pragma unroll
        for (int c = 0; c < CH; c++) {
            const float *pc = part + (size_t)min(i0 + (uint32_t)c, np - 1) * PART;
#pragma unroll
            for (int k = 0; k < EPL; k++)
                ov[c][k] = pc[lane + 64 * k];
        }
    };
    load_o(0);
    float M[G];
#pragma unroll
    for (int h = 0; h < G; h++)
        M[h] = wave_max_f32((uint32_t)lane < np ? mj[h] : -INFINITY);
    for (uint32_t c0 = 64; c0 < np; c0 += 64) {  // rows of more than 64 partials
        const float *pj = part + (size_t)min(c0 + (uint32_t)lane, np - 1) * PART + G * D;
#pragma unroll
        for (int h = 0; h < G; h++)
            M[h] = fmaxf(M[h], wave_max_f32(c0 + (uint32_t)lane < np ? pj[2 * h] : -INFINITY));
    }
    float L[G], O[EPL];
#pragma unroll
    for (int h = 0; h < G; h++)
        L[h] = 0.f;
#pragma unroll
    for (int k = 0; k < EPL; k++)
        O[k] = 0.f;
    for (uint32_t c0 = 0; c0 < np; c0 += 64) {
        if (c0 > 0)
            load_ml(c0);
        const uint32_t n = min(np - c0, 64u);
        for (uint32_t i0 = 0; i0 < n; i0 += CH) {
            if (c0 + i0 > 0)
                load_o(c0 + i0);
#pragma unroll
            for (int c = 0; c < CH; c++) {
                const uint32_t i = i0 + (uint32_t)c;
                if (i >= n)
                    break;
                float f[G];
#pragma unroll
                for (int h = 0; h < G; h++) {
                    const float m = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mj[h]), (int)i));
                    const float l = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lj[h]), (int)i));
                    f[h] = m == -INFINITY ? 0.f : exp2f(m - M[h]);
                    L[h] = fmaf(l, f[h], L[h]);
                }
#pragma unroll
                for (int k = 0; k < EPL; k++)
                    O[k] = fmaf(ov[c][k], f[(lane + 64 * k) / D], O[k]);
            }
        }
    }
    const size_t obase = ((size_t)b * p.q_heads + (size_t)g * G) * D;
#pragma unroll
    for (int k = 0; k < EPL; k++) {
        const uint32_t e = (uint32_t)lane + 64u * k;
        const float Lh = L[e / D];
        float v = (Lh > 0.f || Lh != Lh) ? O[k] / Lh : 0.f;
        if (bad)
            v = __builtin_nanf("");
        if (p.out)
            p.out[obase + e] = rl_from_f32<DT>(v);
        if (p.out_f32)
            p.out_f32[obase + e] = v;
    }
}

template <int D, int G, int DT, int NTHR, int GH>
__device__ __forceinline__ void merge_row(const AttnParams &p, uint32_t b, uint32_t g, uint32_t h0, uint32_t R0,
                                          uint32_t nu, uint32_t U, uint32_t NW, bool bad, uint32_t tid, float *s_f,
                                          float *s_L)
{
    // wave holding tile R0 / tile R0 + nu - 1: the largest w with floor(w U / NW) <= tile
    const uint32_t wf = (uint32_t)((((uint64_t)R0 + 1) * NW - 1) / U);
    const uint32_t wl = (uint32_t)((((uint64_t)R0 + nu) * NW - 1) / U);
    merge_span<D, G, DT, NTHR, GH>(p, b, g, h0, wf, wl, bad, tid, s_f, s_L);
}

// Writes heads h0 .. h0 + GH - 1 of a row without tiles: zeros (ctx 0) or
// NaN (ctx beyond max_ctx).
template <int D, int G, int DT, int GH>
__device__ __forceinline__ void empty_row(const AttnParams &p, uint32_t b, uint32_t g, uint32_t h0, bool bad,
                                          uint32_t tid, uint32_t nthr)
{
    const size_t obase = ((size_t)b * p.q_heads + (size_t)g * G + h0) * D;
    for (uint32_t e = tid; e < (uint32_t)(GH * D); e += nthr) {
        const float v = bad ? __builtin_nanf("") : 0.f;
        if (p.out)
            p.out[obase + e] = rl_from_f32<DT>(v);
        if (p.out_f32)
            p.out_f32[obase + e] = v;
    }
}
}  // namespace
