// logits_proj.hip - the dense hidden-to-vocab logits projection on gfx950:
// logits[M][N] (fp32) = X[M][K] (bf16) . W[N][K]^T (bf16), fp32 accumulate.
//
// No reference kernel exists; the nearest analog is the
// fp16 GEMV query_prepare_kernel (cu/query_producer.cu:5-26). W is stored
// like an lm_head weight, one row of K per vocabulary entry, so both
// operands are K-contiguous.
//
//  tiles   one 512-thread workgroup (8 waves, 4 along M x 2 along N) per
//          output tile, K in steps of 64:
//          - up to 256 rows: 256 x 128 tiles, waves of 64 x 64 (4 x 4 MFMA
//            blocks of 16 x 16), a 3-stage LDS ring (144 KiB). Every W tile
//            is read by exactly one workgroup, and the grid (one workgroup
//            per 128 vocabulary rows) fits the device in one round.
//          - above 256 rows: 256 x 256 tiles, waves of 64 x 128, a 2-stage
//            ring (128 KiB). The larger wave tile reads fewer LDS bytes per
//            MFMA, and at 512 rows the grid is again one round.
//          X (at most 2 MiB per M tile) is read from L2.
//  staging the X and W tiles of a K step are copied HBM -> LDS with
//          global_load_lds_dwordx4, NS - 1 steps ahead of the MFMAs, with one
//          barrier per step; 16-byte chunk c of row r lands at chunk position
//          c ^ (r & 7) (lanes fetch permuted sources), so the MFMA operand
//          reads are free of bank conflicts.
//  MFMA    v_mfma_f32_16x16x32_bf16: lane l reads 16 B of row l % 16 at
//          k-chunk 4 s + l / 16 for both operands.
//  When several M tiles share a W tile, they run side by side on one XCD.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BM = 256, BK = 64;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kWavesM = 4, kWavesN = 2;
constexpr int TM = BM / kWavesM / 16;        // 16-row MFMA blocks per wave along M: 4

// Tile shape by TN, the 16-column MFMA blocks per wave along N.
template <int TN>
struct Tile {
    static constexpr int BN = kWavesN * TN * 16;          // 128 or 256
    static constexpr int NSTAGE = TN == 4 ? 3 : 2;        // 144 or 128 KiB of LDS
    static constexpr int XBYTES = BM * BK * 2;            // 32 KiB of X per step
    static constexpr int WBYTES = BN * BK * 2;            // 16 or 32 KiB of W per step
    static constexpr int XOPS = XBYTES / 1024 / kWaves;   // 1 KiB copies per wave and step: 4 of X
    static constexpr int WOPS = WBYTES / 1024 / kWaves;   // ... and 2 or 4 of W
    static constexpr int STEP_OPS = XOPS + WOPS;
    static constexpr int STAGE = XBYTES + WBYTES;
};

struct ProjParams {
    const uint16_t *x;  // [M][ldx]
    const uint16_t *w;  // [N][ldw]
    float *out;         // [M][ldo]
    uint32_t M, N, K, ldx, ldw, ldo;
    uint32_t m_tiles, n_tiles;
};

// Workgroups are dispatched to the 8 XCDs round-robin (workgroup b on XCD
// b % 8), each XCD with its own L2. The M tiles of one N tile (which share
// the N tile's W rows) are given consecutive workgroups of one XCD, so they
// run side by side behind one L2 and W leaves HBM about once.
constexpr uint32_t kXcds = 8;

// Per-lane source offsets of the `nops` 1 KiB pieces op0 .. op0 + nops - 1
// (8 rows x 64 k each) of a tile of a K-contiguous operand, relative to the
// tile's first row at the step's k: piece op, lane l fetches chunk
// (l % 8) ^ (r & 7) of row r = 8 op + l / 8, so chunk c of row r lands at
// c ^ (r & 7). Rows past `rows` re-read the last row (in bounds; their
// results are never stored). The same for every K step: computed once.
template <int NOPS>
__device__ __forceinline__ void piece_offsets(uint32_t ld, uint32_t rows, uint32_t row0, int op0, int lane,
                                              uint32_t (&off)[NOPS])
{
    const uint32_t first = min(row0, rows - 1);
#pragma unroll
    for (int j = 0; j < NOPS; j++) {
        const uint32_t r = (uint32_t)(op0 + j) * 8 + (uint32_t)lane / 8;
        const uint32_t c = ((uint32_t)lane % 8) ^ (r & 7);
        off[j] = (min(row0 + r, rows - 1) - first) * ld * 2u + c * 16u;
    }
}

// Copies the pieces of one K step: base is the tile's first row at the
// step's k (wave-uniform).
template <int NOPS>
__device__ __forceinline__ void stage_rows(const uint16_t *base, const uint32_t (&off)[NOPS], RL_LDS uint8_t *dst,
                                           int op0)
{
#pragma unroll
    for (int j = 0; j < NOPS; j++)
        rl_g2lds_16_off(base, off[j], dst + (op0 + j) * 1024);
}

template <int TN>
__global__ __launch_bounds__(kThreads) void logits_proj_kernel(ProjParams p)
{
    using T = Tile<TN>;
    __shared__ __attribute__((aligned(1024))) uint8_t smem[T::NSTAGE * T::STAGE];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
    const uint32_t mt = local % p.m_tiles;
    const uint32_t nt = xcd + kXcds * (local / p.m_tiles);
    if (nt >= p.n_tiles)
        return;
    const uint32_t m0 = mt * BM, n0 = nt * T::BN;
    const int wm = wave % kWavesM, wn = wave / kWavesM;

    rl_f32x4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int j = 0; j < TN; j++)
            acc[i][j] = rl_f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t ksteps = p.K / BK;
    // fragment addressing inside a tile: row (l % 16) of block i, chunk 4 s + l / 16
    const int fr = lane & 15;
    const int fc = lane >> 4;
    uint32_t xoff[T::XOPS], woff[T::WOPS];
    piece_offsets<T::XOPS>(p.ldx, p.M, m0, wave * T::XOPS, lane, xoff);
    piece_offsets<T::WOPS>(p.ldw, p.N, n0, wave * T::WOPS, lane, woff);
    const uint16_t *xbase = p.x + (size_t)min(m0, p.M - 1) * p.ldx;
    const uint16_t *wbase = p.w + (size_t)min(n0, p.N - 1) * p.ldw;
    auto sx = [&](int b) { return (RL_LDS uint8_t *)(smem + b * T::STAGE); };
    auto sw = [&](int b) { return (RL_LDS uint8_t *)(smem + b * T::STAGE + T::XBYTES); };
    auto stage = [&](uint32_t kt) {
        const int b = (int)(kt % T::NSTAGE);
        stage_rows<T::XOPS>(xbase + kt * BK, xoff, sx(b), wave * T::XOPS);
        stage_rows<T::WOPS>(wbase + kt * BK, woff, sw(b), wave * T::WOPS);
    };

#pragma unroll
    for (int s = 0; s < T::NSTAGE - 1; s++)
        if ((uint32_t)s < ksteps)
            stage(s);
    for (uint32_t kt = 0; kt < ksteps; kt++) {
        // this wave's copies of step kt have landed once at most the ones
        // issued after them (steps kt + 1 .. kt + NSTAGE - 2) are outstanding:
        // copies complete in issue order
        if (T::NSTAGE == 3 && kt + 1 < ksteps)
            rl_wait_vmcnt<(T::NSTAGE == 3 ? T::STEP_OPS : 0)>();
        else
            rl_wait_vmcnt<0>();
        // every wave's copies of step kt have landed, and every wave is done
        // with step kt - 1, whose buffer step kt + NSTAGE - 1 takes
        __syncthreads();
        if (kt + T::NSTAGE - 1 < ksteps)
            stage(kt + T::NSTAGE - 1);
        const int buf = (int)(kt % T::NSTAGE);
        RL_LDS const uint8_t *xs = sx(buf);
        RL_LDS const uint8_t *ws = sw(buf);
#pragma unroll
        for (int s = 0; s < BK / 32; s++) {
            s16x8 af[TM], bf[TN];
            const int c = 4 * s + fc;
#pragma unroll
            for (int i = 0; i < TM; i++) {
                const int ra = wm * TM * 16 + i * 16 + fr;
                af[i] = *(RL_LDS const s16x8 *)(xs + ra * (BK * 2) + ((c ^ (ra & 7)) << 4));
            }
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const int rb = wn * TN * 16 + j * 16 + fr;
                bf[j] = *(RL_LDS const s16x8 *)(ws + rb * (BK * 2) + ((c ^ (rb & 7)) << 4));
            }
#pragma unroll
            for (int i = 0; i < TM; i++)
#pragma unroll
                for (int j = 0; j < TN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                                        __builtin_bit_cast(bf16x8, bf[j]),
                                                                        acc[i][j], 0, 0, 0);
        }
    }

    // C block (i, j): lane holds rows 4 (l / 16) + r, column l % 16
#pragma unroll
    for (int i = 0; i < TM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m0 + wm * TM * 16 + i * 16 + 4 * fc + r;
            if (m >= p.M)
                continue;
            float *orow = p.out + (size_t)m * p.ldo;
#pragma unroll
            for (int j = 0; j < TN; j++) {
                const uint32_t n = n0 + wn * TN * 16 + j * 16 + fr;
                if (n < p.N)
                    orow[n] = acc[i][j][r];
            }
        }
}

template <int TN>
int launch_proj(ProjParams p)
{
    p.m_tiles = (p.M + BM - 1) / BM;
    p.n_tiles = (p.N + Tile<TN>::BN - 1) / Tile<TN>::BN;
    const uint64_t grid = (uint64_t)(p.n_tiles + kXcds - 1) / kXcds * kXcds * p.m_tiles;
    if (grid > 0x7FFFFFFFull) {
        rl_set_error("rl_hip_logits_proj: %llu workgroups", (unsigned long long)grid);
        return -1;
    }
    hipLaunchKernelGGL(logits_proj_kernel<TN>, dim3((uint32_t)grid), dim3(kThreads), 0, rl_stream(), p);
    return rl_check_launch("logits_proj_kernel launch");
}

}  // namespace

extern "C" int rl_hip_logits_proj(const rl_logits_proj_args_t *a)
{
    if (rl_require_open("rl_hip_logits_proj"))
        return -1;
    if (!a || !a->x || !a->w || !a->logits) {
        rl_set_error("rl_hip_logits_proj: NULL argument");
        return -1;
    }
    if (a->rows == 0 || a->vocab == 0 || a->hidden == 0 || a->hidden % BK != 0) {
        rl_set_error("rl_hip_logits_proj: rows %u vocab %u hidden %u (hidden must be a positive multiple of %d)",
                     a->rows, a->vocab, a->hidden, BK);
        return -1;
    }
    if (a->x_stride < a->hidden || a->w_stride < a->hidden || a->logits_stride < a->vocab ||
        a->x_stride % 8 != 0 || a->w_stride % 8 != 0) {
        rl_set_error("rl_hip_logits_proj: strides x %u w %u logits %u invalid (x, w multiples of 8 elements)",
                     a->x_stride, a->w_stride, a->logits_stride);
        return -1;
    }
    ProjParams p;
    p.x = (const uint16_t *)a->x;
    p.w = (const uint16_t *)a->w;
    p.out = a->logits;
    p.M = a->rows;
    p.N = a->vocab;
    p.K = a->hidden;
    p.ldx = a->x_stride;
    p.ldw = a->w_stride;
    p.ldo = a->logits_stride;
    // above 256 rows the 256 x 256 tile (more MFMA work per LDS byte); up to
    // 256 rows the 256 x 128 tile, whose grid still fills the device
    return a->rows > (uint32_t)BM ? launch_proj<8>(p) : launch_proj<4>(p);
}
