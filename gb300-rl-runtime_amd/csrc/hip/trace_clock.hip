// trace_clock.hip - samples of the GPU's constant 100 MHz clock
// (s_memrealtime) against the host's CLOCK_MONOTONIC, for mapping
// device-stamped trace records onto the host timeline.
//
// A one-wave kernel and the host play ping-pong through a flag in coherent
// host memory: for sample i the host reads its clock (t0) and raises the flag
// to 2i + 1; the kernel, polling the flag at system scope, reads the GPU
// clock, writes it to ticks[i] and releases the flag to 2i + 2; the host
// reads its clock again when it sees that (t1). The GPU reading lies in
// [t0, t1], so the sample is (ticks[i], (t0 + t1) / 2) with an error of at
// most half the round trip; the sample with the shortest round trip wins.
// The kernel's wait for each sample is bounded (it exits after kSpinLimit
// polls), and the host stops waiting after 50 ms per sample.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <time.h>

#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

constexpr uint64_t kSpinLimit = 1ull << 22;
constexpr uint32_t kMaxSamples = 1024;

__global__ void clock_pingpong_kernel(uint32_t *flag, uint64_t *ticks, uint32_t n)
{
    if (threadIdx.x != 0)
        return;
    for (uint32_t i = 0; i < n; i++) {
        uint64_t spins = 0;
        while (__hip_atomic_load(flag, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_SYSTEM) != 2u * i + 1u) {
            if (++spins > kSpinLimit)
                return;
            __builtin_amdgcn_s_sleep(1);
        }
        ticks[i] = __builtin_amdgcn_s_memrealtime();
        __hip_atomic_store(flag, 2u * i + 2u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

uint64_t host_ns()
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

}  // namespace

extern "C" int rl_hip_trace_clock_sample(uint32_t samples, uint64_t *ticks_out, double *host_ns_out,
                                         uint64_t *rtt_ns_out)
{
    if (rl_require_open("rl_hip_trace_clock_sample"))
        return -1;
    if (!ticks_out || !host_ns_out || samples == 0 || samples > kMaxSamples) {
        rl_set_error("rl_hip_trace_clock_sample: NULL output or %u samples (1..%u)", samples, kMaxSamples);
        return -1;
    }
    uint8_t *mem = nullptr;
    if (rl_check_hip(hipHostMalloc((void **)&mem, 64 + (size_t)samples * 8, hipHostMallocMapped | hipHostMallocCoherent),
                     "hipHostMalloc"))
        return -1;
    memset(mem, 0, 64 + (size_t)samples * 8);
    uint32_t *flag = (uint32_t *)mem;
    uint64_t *ticks = (uint64_t *)(mem + 64);
    hipStream_t s = nullptr;
    if (rl_check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags")) {
        (void)hipHostFree(mem);
        return -1;
    }
    hipLaunchKernelGGL(clock_pingpong_kernel, dim3(1), dim3(64), 0, s, flag, ticks, samples);
    int rc = rl_check_launch("clock_pingpong_kernel launch");
    uint64_t best_rtt = UINT64_MAX;
    uint32_t got = 0;
    for (uint32_t i = 0; rc == 0 && i < samples; i++) {
        const uint64_t t0 = host_ns();
        __atomic_store_n(flag, 2u * i + 1u, __ATOMIC_RELEASE);
        uint64_t t1 = t0;
        while (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != 2u * i + 2u) {
            t1 = host_ns();
            if (t1 - t0 > 50000000ull)
                break;
        }
        if (__atomic_load_n(flag, __ATOMIC_ACQUIRE) != 2u * i + 2u)
            break;              // the kernel is gone (it gives up on its own)
        t1 = host_ns();
        got++;
        if (t1 - t0 < best_rtt) {
            best_rtt = t1 - t0;
            *ticks_out = ticks[i];
            *host_ns_out = 0.5 * ((double)t0 + (double)t1);
        }
    }
    // a kernel still waiting for a sample that will not come exits by itself
    if (rl_check_hip(hipStreamSynchronize(s), "hipStreamSynchronize"))
        rc = -1;
    (void)hipStreamDestroy(s);
    (void)hipHostFree(mem);
    if (rc == 0 && got == 0) {
        rl_set_error("rl_hip_trace_clock_sample: no sample came back");
        rc = -1;
    }
    if (rc == 0 && rtt_ns_out)
        *rtt_ns_out = best_rtt;
    return rc;
}
