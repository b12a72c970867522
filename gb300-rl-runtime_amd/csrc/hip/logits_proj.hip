// logits_proj.hip - the dense hidden-to-vocab logits projection on gfx950:
// logits[M][N] (fp32) = X[M][K] (bf16) . W[N][K]^T (bf16), fp32 accumulate.
//
// No reference kernel exists; the nearest analog is the
// fp16 GEMV query_prepare_kernel (cu/query_producer.cu:5-26). W is stored
// like an lm_head weight, one row of K per vocabulary entry, so both
// operands are K-contiguous.
//
//  tiles   256 x 128 output tile per 512-thread workgroup (8 waves of
//          64 x 64: 4 x 4 MFMA blocks of 16 x 16), K in steps of 64. At 256
//          rows every W tile is read by exactly one workgroup and the grid
//          (one workgroup per 128 vocabulary rows) fits the device in one
//          round; X (at most 2 MiB per M tile) is read from L2.
//  staging the X and W tiles of a K step (32 + 16 KiB) are copied HBM -> LDS
//          with global_load_lds_dwordx4 into a 3-stage ring (144 KiB, one
//          workgroup per CU), two steps ahead of the MFMAs, with one barrier
//          per step; 16-byte chunk c of row r lands at chunk position
//          c ^ (r & 7) (lanes fetch permuted sources), so the MFMA operand
//          reads are free of bank conflicts.
//  MFMA    v_mfma_f32_16x16x32_bf16: lane l reads 16 B of row l % 16 at
//          k-chunk 4 s + l / 16 for both operands; 32 MFMAs per wave and K step.
//  When several M tiles share a W tile, they run side by side on one XCD.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BM = 256, BN = 128, BK = 64;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int NSTAGE = 3;
constexpr int XBYTES = BM * BK * 2;          // 32 KiB of X per step
constexpr int WBYTES = BN * BK * 2;          // 16 KiB of W per step
constexpr int XOPS = XBYTES / 1024 / kWaves; // 1 KiB copies per wave and step: 4 of X
constexpr int WOPS = WBYTES / 1024 / kWaves; // ... and 2 of W
constexpr int STEP_OPS = XOPS + WOPS;

struct ProjParams {
    const uint16_t *x;  // [M][ldx]
    const uint16_t *w;  // [N][ldw]
    float *out;         // [M][ldo]
    uint32_t M, N, K, ldx, ldw, ldo;
    uint32_t m_tiles, n_tiles;
};

// Workgroups are dispatched to the 8 XCDs round-robin (workgroup b on XCD
// b % 8), each XCD with its own L2. The M tiles of one N tile (which share
// the 128-row W tile) are given consecutive workgroups of one XCD, so they
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

__global__ __launch_bounds__(kThreads) void logits_proj_kernel(ProjParams p)
{
    __shared__ __attribute__((aligned(1024))) uint8_t sX[NSTAGE][XBYTES];
    __shared__ __attribute__((aligned(1024))) uint8_t sW[NSTAGE][WBYTES];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t xcd = blockIdx.x % kXcds, local = blockIdx.x / kXcds;
    const uint32_t mt = local % p.m_tiles;
    const uint32_t nt = xcd + kXcds * (local / p.m_tiles);
    if (nt >= p.n_tiles)
        return;
    const uint32_t m0 = mt * BM, n0 = nt * BN;
    const int wm = wave & 3, wn = wave >> 2;

    rl_f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++)
            acc[i][j] = rl_f32x4{0.f, 0.f, 0.f, 0.f};

    const uint32_t ksteps = p.K / BK;
    // fragment addressing inside a tile: row (l % 16) of block i, chunk 4 s + l / 16
    const int fr = lane & 15;
    const int fc = lane >> 4;
    uint32_t xoff[XOPS], woff[WOPS];
    piece_offsets<XOPS>(p.ldx, p.M, m0, wave * XOPS, lane, xoff);
    piece_offsets<WOPS>(p.ldw, p.N, n0, wave * WOPS, lane, woff);
    const uint16_t *xbase = p.x + (size_t)min(m0, p.M - 1) * p.ldx;
    const uint16_t *wbase = p.w + (size_t)min(n0, p.N - 1) * p.ldw;
    auto stage = [&](uint32_t kt) {
        const int buf = (int)(kt % NSTAGE);
        stage_rows<XOPS>(xbase + kt * BK, xoff, (RL_LDS uint8_t *)sX[buf], wave * XOPS);
        stage_rows<WOPS>(wbase + kt * BK, woff, (RL_LDS uint8_t *)sW[buf], wave * WOPS);
    };

    stage(0);
    if (ksteps > 1)
        stage(1);
    for (uint32_t kt = 0; kt < ksteps; kt++) {
        // this wave's copies of step kt have landed once at most the next
        // step's are outstanding (copies complete in issue order)
        if (kt + 1 < ksteps)
            rl_wait_vmcnt<STEP_OPS>();
        else
            rl_wait_vmcnt<0>();
        // every wave's copies of step kt have landed, and every wave is done
        // with step kt - 1, whose buffer step kt + 2 takes
        __syncthreads();
        if (kt + 2 < ksteps)
            stage(kt + 2);
        const int buf = (int)(kt % NSTAGE);
        RL_LDS const uint8_t *xs = (RL_LDS const uint8_t *)sX[buf];
        RL_LDS const uint8_t *ws = (RL_LDS const uint8_t *)sW[buf];
#pragma unroll
        for (int s = 0; s < BK / 32; s++) {
            s16x8 af[4], bf[4];
            const int c = 4 * s + fc;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int ra = wm * 64 + i * 16 + fr;
                const int rb = wn * 64 + i * 16 + fr;
                af[i] = *(RL_LDS const s16x8 *)(xs + ra * (BK * 2) + ((c ^ (ra & 7)) << 4));
                bf[i] = *(RL_LDS const s16x8 *)(ws + rb * (BK * 2) + ((c ^ (rb & 7)) << 4));
            }
#pragma unroll
            for (int i = 0; i < 4; i++)
#pragma unroll
                for (int j = 0; j < 4; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, af[i]),
                                                                        __builtin_bit_cast(bf16x8, bf[j]),
                                                                        acc[i][j], 0, 0, 0);
        }
    }

    // C block (i, j): lane holds rows 4 (l / 16) + r, column l % 16
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const uint32_t m = m0 + wm * 64 + i * 16 + 4 * fc + r;
            if (m >= p.M)
                continue;
            float *orow = p.out + (size_t)m * p.ldo;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t n = n0 + wn * 64 + j * 16 + fr;
                if (n < p.N)
                    orow[n] = acc[i][j][r];
            }
        }
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
    p.m_tiles = (a->rows + BM - 1) / BM;
    p.n_tiles = (a->vocab + BN - 1) / BN;
    const uint64_t grid = (uint64_t)(p.n_tiles + kXcds - 1) / kXcds * kXcds * p.m_tiles;
    if (grid > 0x7FFFFFFFull) {
        rl_set_error("rl_hip_logits_proj: %llu workgroups", (unsigned long long)grid);
        return -1;
    }
    hipLaunchKernelGGL(logits_proj_kernel, dim3((uint32_t)grid), dim3(kThreads), 0, rl_stream(), p);
    return rl_check_launch("logits_proj_kernel launch");
}
