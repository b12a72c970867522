// rl_dev_common.h - gfx950 device helpers shared by the kernels: bf16/fp16
// conversion, DPP row reductions, LDS-direct (global_load_lds) staging.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

typedef __bf16 rl_bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 rl_f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t rl_u32x4 __attribute__((ext_vector_type(4)));
typedef float rl_f32x4 __attribute__((ext_vector_type(4)));

#define RL_LDS __attribute__((address_space(3)))
#define RL_GLOBAL __attribute__((address_space(1)))
#define RL_CONST __attribute__((address_space(4)))

// Load through the constant address space: memory the kernel never writes,
// read at a wave-uniform address, becomes a scalar (s_load) access.
template <typename T>
__device__ __forceinline__ T rl_sload(const T *p)
{
    return *(const RL_CONST T *)p;
}

// Wave-uniform load of a word that the same launch rewrites between reads (a
// persistent kernel's per-step arguments): a relaxed device-scope atomic
// load, which is never a scalar-cache access and never moved out of a loop,
// broadcast from the first lane. Ordering comes from the caller's fences.
__device__ __forceinline__ uint32_t rl_live_u32(const uint32_t *p)
{
    return __builtin_amdgcn_readfirstlane(
        __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// ---- scalar conversions ---------------------------------------------------

__device__ __forceinline__ float rl_bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float rl_bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

__device__ __forceinline__ float rl_f16_lo(uint32_t w)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xFFFFu));
}
__device__ __forceinline__ float rl_f16_hi(uint32_t w)
{
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// float -> bf16 bits, round to nearest even (finite inputs).
__device__ __forceinline__ uint16_t rl_f32_to_bf16(float f)
{
    const uint32_t u = __float_as_uint(f);
    return (uint16_t)((u + 0x7FFFu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint16_t rl_f32_to_f16(float f)
{
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element pair of a packed dword -> two fp32 values.
template <int DT>
__device__ __forceinline__ void rl_unpack2(uint32_t w, float &lo, float &hi)
{
    if constexpr (DT == 0) {
        lo = rl_bf16_lo(w);
        hi = rl_bf16_hi(w);
    } else {
        lo = rl_f16_lo(w);
        hi = rl_f16_hi(w);
    }
}

// acc + a.x*b.x + a.y*b.y with 2-byte operands and an fp32 accumulator.
template <int DT>
__device__ __forceinline__ float rl_dot2(uint32_t a, uint32_t b, float acc)
{
    if constexpr (DT == 0)
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(rl_bf16x2, a),
                                               __builtin_bit_cast(rl_bf16x2, b), acc, false);
    else
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(rl_f16x2, a), __builtin_bit_cast(rl_f16x2, b),
                                      acc, false);
}

template <int DT>
__device__ __forceinline__ uint16_t rl_from_f32(float f)
{
    if constexpr (DT == 0)
        return rl_f32_to_bf16(f);
    else
        return rl_f32_to_f16(f);
}

// ---- DPP reductions inside a row of 16 lanes ------------------------------
// quad_perm(1,0,3,2) = 0xB1, quad_perm(2,3,0,1) = 0x4E, row_half_mirror =
// 0x141, row_mirror = 0x140. After the four steps every lane of the row holds
// the reduction over its 16 lanes.

template <int CTRL>
__device__ __forceinline__ float rl_dpp(float x)
{
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

__device__ __forceinline__ float rl_row_max(float x)
{
    x = fmaxf(x, rl_dpp<0xB1>(x));
    x = fmaxf(x, rl_dpp<0x4E>(x));
    x = fmaxf(x, rl_dpp<0x141>(x));
    x = fmaxf(x, rl_dpp<0x140>(x));
    return x;
}

__device__ __forceinline__ float rl_row_sum(float x)
{
    x += rl_dpp<0xB1>(x);
    x += rl_dpp<0x4E>(x);
    x += rl_dpp<0x141>(x);
    x += rl_dpp<0x140>(x);
    return x;
}

// ---- whole-wave scans and reductions on u32 (DPP, no LDS crossbar) ---------
// row_shr:1/2/4/8 (0x111, 0x112, 0x114, 0x118; lanes without a source read 0)
// give an inclusive scan inside each row of 16 lanes; row_bcast:15 (0x142) on
// rows 1 and 3 and row_bcast:31 (0x143) on rows 2 and 3 carry the row totals.

template <int CTRL, int ROW_MASK, bool BOUND_ZERO>
__device__ __forceinline__ uint32_t rl_dpp_u32(uint32_t x)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROW_MASK, 0xF, BOUND_ZERO);
}

__device__ __forceinline__ uint32_t rl_wave_incl_scan_u32(uint32_t x)
{
    x += rl_dpp_u32<0x111, 0xF, true>(x);
    x += rl_dpp_u32<0x112, 0xF, true>(x);
    x += rl_dpp_u32<0x114, 0xF, true>(x);
    x += rl_dpp_u32<0x118, 0xF, true>(x);
    x += rl_dpp_u32<0x142, 0xA, false>(x);
    x += rl_dpp_u32<0x143, 0xC, false>(x);
    return x;
}

__device__ __forceinline__ uint32_t rl_readlane(uint32_t x, int lane)
{
    return (uint32_t)__builtin_amdgcn_readlane((int)x, lane);
}

// Wave broadcast: every lane gets lane `src`'s value (src wave-uniform), in
// a scalar register. The ring workers use it for the values one lane reads
// from a ring (the reference's warp_broadcast_u32 / _u64,
// include/warp_broadcast.cuh).
__device__ __forceinline__ uint32_t rl_wave_bcast_u32(uint32_t x, int src) { return rl_readlane(x, src); }

__device__ __forceinline__ uint64_t rl_wave_bcast_u64(uint64_t x, int src)
{
    return ((uint64_t)rl_readlane((uint32_t)(x >> 32), src) << 32) | rl_readlane((uint32_t)x, src);
}

// One 64-byte ring record between registers and fine-grained host memory as
// eight relaxed system-scope 8-byte accesses. They are issued back to back
// with one wait for the loads, where a volatile access would wait for the
// previous one to complete: four PCIe round trips for a record in 16-byte
// volatile pieces, one here.
__device__ __forceinline__ void rl_sys_load_64B(const void *src, uint64_t (&w)[8])
{
    const uint64_t *s = (const uint64_t *)src;
#pragma unroll
    for (int j = 0; j < 8; j++)
        w[j] = __hip_atomic_load((uint64_t *)(s + j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

__device__ __forceinline__ void rl_sys_store_64B(void *dst, const uint64_t (&w)[8])
{
    uint64_t *d = (uint64_t *)dst;
#pragma unroll
    for (int j = 0; j < 8; j++)
        __hip_atomic_store(d + j, w[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}

// Wave-uniform min / max / sum of a u32 held by every lane.
__device__ __forceinline__ uint32_t rl_wave_min_u32(uint32_t x)
{
    x = min(x, rl_dpp_u32<0xB1, 0xF, false>(x));
    x = min(x, rl_dpp_u32<0x4E, 0xF, false>(x));
    x = min(x, rl_dpp_u32<0x141, 0xF, false>(x));
    x = min(x, rl_dpp_u32<0x140, 0xF, false>(x));
    return min(min(rl_readlane(x, 0), rl_readlane(x, 16)), min(rl_readlane(x, 32), rl_readlane(x, 48)));
}

__device__ __forceinline__ uint32_t rl_wave_max_u32(uint32_t x)
{
    x = max(x, rl_dpp_u32<0xB1, 0xF, false>(x));
    x = max(x, rl_dpp_u32<0x4E, 0xF, false>(x));
    x = max(x, rl_dpp_u32<0x141, 0xF, false>(x));
    x = max(x, rl_dpp_u32<0x140, 0xF, false>(x));
    return max(max(rl_readlane(x, 0), rl_readlane(x, 16)), max(rl_readlane(x, 32), rl_readlane(x, 48)));
}

__device__ __forceinline__ uint32_t rl_wave_sum_u32(uint32_t x)
{
    return rl_readlane(rl_wave_incl_scan_u32(x), 63);
}

// ---- LDS-direct staging ---------------------------------------------------
// global_load_lds_dwordx4: each lane fetches 16 bytes from its own global
// address; they land at lds_base + lane * 16 (lds_base wave-uniform).
__device__ __forceinline__ void rl_g2lds_16(const void *gsrc, RL_LDS void *lds_base)
{
    __builtin_amdgcn_global_load_lds(gsrc, lds_base, 16, 0, 0);
}

// The same copy with a wave-uniform global base and a per-lane 32-bit offset,
// issued as inline assembly: the compiler's wait insertion does not see it,
// so it adds no conservative vmcnt(0) before LDS reads it cannot prove
// disjoint. The caller orders every use with rl_wait_vmcnt. (Writing M0 needs
// one wait state before an LDS-direct load reads it. M0 is reserved to the
// compiler, which does not keep values in it across inline assembly; the
// kernels using this helper make no other use of M0.)
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void rl_g2lds_16_off(const void *gbase, uint32_t voff, RL_LDS void *lds_base)
{
    // base and LDS address are wave-uniform; readfirstlane puts them in SGPRs
    const uint64_t a = (uint64_t)(uintptr_t)gbase;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)a);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(a >> 32));
    const uint64_t base = ((uint64_t)hi << 32) | lo;
    const uint32_t lds = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)lds_base);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                 :
                 : "v"(voff), "s"(base), "s"(lds)
                 : "memory", "m0");
}
#pragma clang diagnostic pop

// Waits until at most N vector-memory operations of this wave are
// outstanding (loads retire in issue order), e.g. the LDS-direct copies of
// one staged unit while the next unit's copies stay in flight. The memory
// clobber keeps the compiler from hoisting LDS reads above the wait.
template <int N>
__device__ __forceinline__ void rl_wait_vmcnt()
{
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits for all of this wave's LDS reads to return (before an LDS-direct
// copy may overwrite what they read).
__device__ __forceinline__ void rl_wait_lgkmcnt0()
{
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Orders this wave's LDS writes before its later LDS reads (the LDS unit
// serves one wave in issue order; this keeps the compiler from reordering).
__device__ __forceinline__ void rl_wave_lds_fence()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}
