/*
 * mmio.h - doorbell write/read with store/load ordering.
 *
 * Semantics of the reference helpers (include/mmio.h:5-34): a store fence
 * precedes the doorbell store so every descriptor byte is globally visible
 * before the device can observe the new tail; an aarch64 read is followed by
 * a load barrier. On an MI355X host (x86-64) the fence is sfence.
 */
#pragma once

#include <stdint.h>

static inline void
mmio_wmb(void)
{
#if defined(__x86_64__)
    __asm__ volatile("sfence" ::: "memory");
#elif defined(__aarch64__)
    __asm__ volatile("dsb st" ::: "memory");
#else
    __atomic_thread_fence(__ATOMIC_SEQ_CST);
#endif
}

static inline void
mmio_write32(volatile uint32_t *addr, uint32_t value)
{
    mmio_wmb();
    *addr = value;
}

static inline uint32_t
mmio_read32(volatile uint32_t *addr)
{
    const uint32_t v = *addr;
#if defined(__aarch64__)
    __asm__ volatile("dmb oshld" ::: "memory");
#else
    __asm__ volatile("" ::: "memory");
#endif
    return v;
}
