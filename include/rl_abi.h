/*
 * rl_abi.h - portability macros shared by every ABI header.
 *
 * The ABI headers are consumed by three compilers: gcc (C11 host library and
 * oracle), g++/clang++ (C++ host code) and hipcc (gfx950 device code that
 * reads the same ring and descriptor structs out of coherent host memory).
 * These macros keep one struct definition valid in all three.
 */
#pragma once

#ifdef __cplusplus
#define RL_ALIGNAS(n) alignas(n)
#define RL_STATIC_ASSERT(cond, msg) static_assert(cond, msg)
#define RL_EXTERN_C_BEGIN extern "C" {
#define RL_EXTERN_C_END }
#else
#define RL_ALIGNAS(n) _Alignas(n)
#define RL_STATIC_ASSERT(cond, msg) _Static_assert(cond, msg)
#define RL_EXTERN_C_BEGIN
#define RL_EXTERN_C_END
#endif

#define RL_OFFSETOF(type, field) __builtin_offsetof(type, field)

/* Host-side acquire/release helpers (GCC/clang builtins, valid in C and C++). */
#define RL_LOAD_ACQ_U32(p) __atomic_load_n((p), __ATOMIC_ACQUIRE)
#define RL_LOAD_RLX_U32(p) __atomic_load_n((p), __ATOMIC_RELAXED)
#define RL_STORE_REL_U32(p, v) __atomic_store_n((p), (v), __ATOMIC_RELEASE)
