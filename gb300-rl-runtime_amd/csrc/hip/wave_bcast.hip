// wave_bcast.hip - self-test of the wave broadcast the ring workers use
// (rl_wave_bcast_u32 / _u64), in the shape of the reference's warp broadcast
// test (test/test_bench.cu:47-59 and 623-656) on a 64-lane wave.
#include "rl_dev_common.h"
#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

// Wave w: lane src_w = (w ? 37 : 0) holds the values, every other lane zeros;
// each lane writes what the broadcast gives it.
__global__ __launch_bounds__(128) void wave_bcast_kernel(uint64_t *seq_out, uint32_t *off_out, uint64_t *cookie_out)
{
    const uint32_t tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int src = wave ? 37 : 0;
    const bool holder = lane == src;
    const uint64_t seq = holder ? 0x123456789ABCDEF0ull + (uint64_t)wave : 0ull;
    const uint32_t off = holder ? 77u + (uint32_t)wave : 0u;
    const uint64_t cookie = holder ? 0x0FEDCBA987654321ull ^ (uint64_t)wave : 0ull;
    seq_out[tid] = rl_wave_bcast_u64(seq, src);
    off_out[tid] = rl_wave_bcast_u32(off, src);
    cookie_out[tid] = rl_wave_bcast_u64(cookie, src);
}

}  // namespace

extern "C" int rl_hip_wave_broadcast_selftest(uint64_t *seq_out, uint32_t *offset_out, uint64_t *cookie_out)
{
    if (rl_require_open("rl_hip_wave_broadcast_selftest"))
        return -1;
    if (!seq_out || !offset_out || !cookie_out) {
        rl_set_error("rl_hip_wave_broadcast_selftest: NULL device pointer");
        return -1;
    }
    hipLaunchKernelGGL(wave_bcast_kernel, dim3(1), dim3(128), 0, rl_stream(), seq_out, offset_out, cookie_out);
    if (rl_check_launch("wave_bcast_kernel launch"))
        return -1;
    return rl_check_hip(hipStreamSynchronize(rl_stream()), "hipStreamSynchronize");
}
