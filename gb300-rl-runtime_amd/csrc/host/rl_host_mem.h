/*
 * rl_host_mem.h - where the host C runtime puts ring memory.
 *
 * Coherent hipHostMalloc memory when a device is open (the device polls it),
 * otherwise zeroed 64-byte aligned pageable memory. rl_ring_mem_free tells
 * the two apart, so a ring created before rl_hip_open() is still freed
 * correctly.
 */
#pragma once

#include <stddef.h>

__attribute__((visibility("hidden"))) void *rl_ring_mem_alloc(size_t bytes);
__attribute__((visibility("hidden"))) void rl_ring_mem_free(void *p);
