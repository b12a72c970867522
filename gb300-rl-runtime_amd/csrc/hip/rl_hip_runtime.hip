// rl_hip_runtime.hip - session, memory and timing half of the thin C ABI
// (rl_hip.h). One device, one non-blocking library stream plus two lane
// streams for overlapped decode steps, one host thread.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>

#include "rl_hip.h"
#include "rl_hip_internal.h"

namespace {

struct CoherentBlock {
    void *ptr;
    size_t bytes;
};

constexpr int kMaxCoherent = 4096;

struct Session {
    int open = 0;
    int device = -1;
    uint32_t cu_count = 0;
    hipStream_t stream = nullptr;
    hipStream_t lanes[RL_HIP_LANES] = {};
    hipEvent_t ev_begin = nullptr;
    hipEvent_t ev_end = nullptr;
    hipEvent_t ev_fork = nullptr;
    hipEvent_t ev_lane[RL_HIP_LANES] = {};
    std::mutex mu;
    CoherentBlock coherent[kMaxCoherent];
    int n_coherent = 0;
};

Session g_session;
thread_local char g_err[512] = "";

}  // namespace

void rl_set_error(const char *fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int rl_check_hip(hipError_t e, const char *what)
{
    if (e == hipSuccess)
        return 0;
    rl_set_error("%s: %s", what, hipGetErrorString(e));
    return -1;
}

hipStream_t rl_stream(void) { return g_session.stream; }

hipStream_t rl_lane_stream(int lane, const char *what)
{
    if (rl_require_open(what))
        return nullptr;
    if (lane < 0 || lane >= RL_HIP_LANES) {
        rl_set_error("%s: lane %d out of range [0, %d)", what, lane, RL_HIP_LANES);
        return nullptr;
    }
    return g_session.lanes[lane];
}

uint32_t rl_cu_count(void) { return g_session.cu_count; }

int rl_device(void) { return g_session.open ? g_session.device : -1; }

int rl_require_open(const char *what)
{
    if (g_session.open)
        return 0;
    rl_set_error("%s: no device open (call rl_hip_open first)", what);
    return -1;
}

extern "C" {

const char *rl_hip_last_error(void) { return g_err; }

int rl_hip_is_open(void) { return g_session.open; }

int rl_hip_open(int device)
{
    if (g_session.open)
        return g_session.device == device ? 0 : (rl_set_error("rl_hip_open: device %d already open", g_session.device), -1);
    int count = 0;
    if (rl_check_hip(hipGetDeviceCount(&count), "hipGetDeviceCount"))
        return -1;
    if (device < 0 || device >= count) {
        rl_set_error("rl_hip_open: device %d out of range (%d devices)", device, count);
        return -1;
    }
    if (rl_check_hip(hipSetDevice(device), "hipSetDevice"))
        return -1;
    if (rl_attn_scratch_setup(device))
        return -1;
    if (rl_check_hip(hipStreamCreateWithFlags(&g_session.stream, hipStreamNonBlocking), "hipStreamCreateWithFlags"))
        return -1;
    if (rl_check_hip(hipEventCreate(&g_session.ev_begin), "hipEventCreate") ||
        rl_check_hip(hipEventCreate(&g_session.ev_end), "hipEventCreate"))
        return -1;
    // lanes keep the default priority, like the library stream; their events
    // only order work, so they record no timestamps
    if (rl_check_hip(hipEventCreateWithFlags(&g_session.ev_fork, hipEventDisableTiming), "hipEventCreateWithFlags"))
        return -1;
    for (int l = 0; l < RL_HIP_LANES; l++)
        if (rl_check_hip(hipStreamCreateWithFlags(&g_session.lanes[l], hipStreamNonBlocking),
                         "hipStreamCreateWithFlags") ||
            rl_check_hip(hipEventCreateWithFlags(&g_session.ev_lane[l], hipEventDisableTiming),
                         "hipEventCreateWithFlags"))
            return -1;
    int cus = 0;
    if (rl_check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                     "hipDeviceGetAttribute(MultiprocessorCount)"))
        return -1;
    g_session.cu_count = cus > 0 ? (uint32_t)cus : 1u;
    g_session.device = device;
    g_session.open = 1;
    return 0;
}

int rl_hip_close(void)
{
    if (!g_session.open)
        return 0;
    int rc = rl_check_hip(hipStreamSynchronize(g_session.stream), "hipStreamSynchronize");
    for (int l = 0; l < RL_HIP_LANES; l++) {
        if (rl_check_hip(hipStreamSynchronize(g_session.lanes[l]), "hipStreamSynchronize"))
            rc = -1;
        (void)hipEventDestroy(g_session.ev_lane[l]);
        (void)hipStreamDestroy(g_session.lanes[l]);
        g_session.lanes[l] = nullptr;
        g_session.ev_lane[l] = nullptr;
    }
    (void)hipEventDestroy(g_session.ev_fork);
    (void)hipEventDestroy(g_session.ev_begin);
    (void)hipEventDestroy(g_session.ev_end);
    (void)hipStreamDestroy(g_session.stream);
    g_session.stream = nullptr;
    g_session.open = 0;
    return rc;
}

int rl_hip_device_info(rl_hip_device_info_t *out)
{
    if (!out)
        return -1;
    if (rl_require_open("rl_hip_device_info"))
        return -1;
    std::memset(out, 0, sizeof(*out));
    hipDeviceProp_t prop;
    if (rl_check_hip(hipGetDeviceProperties(&prop, g_session.device), "hipGetDeviceProperties"))
        return -1;
    int v = 0;
    out->device = g_session.device;
    (void)hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, g_session.device);
    out->cu_count = (uint32_t)v;
    out->wave_size = (uint32_t)prop.warpSize;
    out->lds_bytes_per_block = (uint32_t)prop.sharedMemPerBlock;
    (void)hipDeviceGetAttribute(&v, hipDeviceAttributeClockRate, g_session.device);
    out->clock_khz = (uint32_t)v;
    (void)hipDeviceGetAttribute(&v, hipDeviceAttributeMemoryClockRate, g_session.device);
    out->mem_clock_khz = (uint32_t)v;
    (void)hipDeviceGetAttribute(&v, hipDeviceAttributeMemoryBusWidth, g_session.device);
    out->mem_bus_width_bits = (uint32_t)v;
    (void)hipDeviceGetAttribute(&v, hipDeviceAttributeL2CacheSize, g_session.device);
    out->l2_bytes = (uint32_t)v;
    out->hbm_bytes = (uint64_t)prop.totalGlobalMem;
    std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
    return 0;
}

void *rl_hip_host_alloc_coherent(size_t bytes)
{
    if (rl_require_open("rl_hip_host_alloc_coherent"))
        return nullptr;
    void *p = nullptr;
    if (rl_check_hip(hipHostMalloc(&p, bytes, hipHostMallocMapped | hipHostMallocCoherent), "hipHostMalloc"))
        return nullptr;
    void *dp = nullptr;
    if (rl_check_hip(hipHostGetDevicePointer(&dp, p, 0), "hipHostGetDevicePointer") || dp != p) {
        if (dp != p)
            rl_set_error("rl_hip_host_alloc_coherent: device alias %p differs from host pointer %p", dp, p);
        (void)hipHostFree(p);
        return nullptr;
    }
    std::memset(p, 0, bytes);
    std::lock_guard<std::mutex> lk(g_session.mu);
    if (g_session.n_coherent >= kMaxCoherent) {
        (void)hipHostFree(p);
        rl_set_error("rl_hip_host_alloc_coherent: more than %d live allocations", kMaxCoherent);
        return nullptr;
    }
    g_session.coherent[g_session.n_coherent++] = {p, bytes};
    return p;
}

int rl_hip_is_coherent_host(const void *p)
{
    std::lock_guard<std::mutex> lk(g_session.mu);
    const char *c = static_cast<const char *>(p);
    for (int i = 0; i < g_session.n_coherent; i++) {
        const char *b = static_cast<const char *>(g_session.coherent[i].ptr);
        if (c >= b && c < b + g_session.coherent[i].bytes)
            return 1;
    }
    return 0;
}

int rl_hip_host_free(void *p)
{
    std::lock_guard<std::mutex> lk(g_session.mu);
    for (int i = 0; i < g_session.n_coherent; i++) {
        if (g_session.coherent[i].ptr == p) {
            g_session.coherent[i] = g_session.coherent[--g_session.n_coherent];
            return rl_check_hip(hipHostFree(p), "hipHostFree");
        }
    }
    rl_set_error("rl_hip_host_free: %p is not a coherent host allocation", p);
    return -1;
}

void *rl_hip_dev_alloc(size_t bytes)
{
    if (rl_require_open("rl_hip_dev_alloc"))
        return nullptr;
    void *p = nullptr;
    if (rl_check_hip(hipMalloc(&p, bytes == 0 ? 1 : bytes), "hipMalloc"))
        return nullptr;
    return p;
}

int rl_hip_is_device_ptr(const void *p)
{
    if (!g_session.open || !p)
        return 0;
    hipPointerAttribute_t attr;
    if (hipPointerGetAttributes(&attr, p) != hipSuccess) {
        (void)hipGetLastError();
        return 0;
    }
    return attr.type == hipMemoryTypeDevice ? 1 : 0;
}

int rl_hip_dev_free(void *p)
{
    if (!p)
        return 0;
    return rl_check_hip(hipFree(p), "hipFree");
}

int rl_hip_memcpy_h2d(void *dst, const void *src, size_t bytes)
{
    if (rl_require_open("rl_hip_memcpy_h2d"))
        return -1;
    if (rl_check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_session.stream), "hipMemcpyAsync(H2D)"))
        return -1;
    return rl_check_hip(hipStreamSynchronize(g_session.stream), "hipStreamSynchronize");
}

int rl_hip_memcpy_d2h(void *dst, const void *src, size_t bytes)
{
    if (rl_require_open("rl_hip_memcpy_d2h"))
        return -1;
    if (rl_check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_session.stream), "hipMemcpyAsync(D2H)"))
        return -1;
    return rl_check_hip(hipStreamSynchronize(g_session.stream), "hipStreamSynchronize");
}

int rl_hip_memcpy_d2d(void *dst, const void *src, size_t bytes)
{
    if (rl_require_open("rl_hip_memcpy_d2d"))
        return -1;
    return rl_check_hip(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, g_session.stream), "hipMemcpyAsync(D2D)");
}

int rl_hip_memset_d(void *dst, int value, size_t bytes)
{
    if (rl_require_open("rl_hip_memset_d"))
        return -1;
    return rl_check_hip(hipMemsetAsync(dst, value, bytes, g_session.stream), "hipMemsetAsync");
}

int rl_hip_sync(void)
{
    if (rl_require_open("rl_hip_sync"))
        return -1;
    for (int l = 0; l < RL_HIP_LANES; l++)
        if (rl_check_hip(hipStreamSynchronize(g_session.lanes[l]), "hipStreamSynchronize"))
            return -1;
    return rl_check_hip(hipStreamSynchronize(g_session.stream), "hipStreamSynchronize");
}

int rl_hip_lanes_fork(void)
{
    if (rl_require_open("rl_hip_lanes_fork"))
        return -1;
    if (rl_check_hip(hipEventRecord(g_session.ev_fork, g_session.stream), "hipEventRecord"))
        return -1;
    for (int l = 0; l < RL_HIP_LANES; l++)
        if (rl_check_hip(hipStreamWaitEvent(g_session.lanes[l], g_session.ev_fork, 0), "hipStreamWaitEvent"))
            return -1;
    return 0;
}

int rl_hip_lanes_join(void)
{
    if (rl_require_open("rl_hip_lanes_join"))
        return -1;
    for (int l = 0; l < RL_HIP_LANES; l++)
        if (rl_check_hip(hipEventRecord(g_session.ev_lane[l], g_session.lanes[l]), "hipEventRecord") ||
            rl_check_hip(hipStreamWaitEvent(g_session.stream, g_session.ev_lane[l], 0), "hipStreamWaitEvent"))
            return -1;
    return 0;
}

int rl_hip_timer_begin(void)
{
    if (rl_require_open("rl_hip_timer_begin"))
        return -1;
    return rl_check_hip(hipEventRecord(g_session.ev_begin, g_session.stream), "hipEventRecord");
}

int rl_hip_timer_end(float *elapsed_ms)
{
    if (rl_require_open("rl_hip_timer_end"))
        return -1;
    if (rl_check_hip(hipEventRecord(g_session.ev_end, g_session.stream), "hipEventRecord") ||
        rl_check_hip(hipEventSynchronize(g_session.ev_end), "hipEventSynchronize"))
        return -1;
    float ms = 0.f;
    if (rl_check_hip(hipEventElapsedTime(&ms, g_session.ev_begin, g_session.ev_end), "hipEventElapsedTime"))
        return -1;
    if (elapsed_ms)
        *elapsed_ms = ms;
    return 0;
}

int rl_hip_capture_begin(void)
{
    if (rl_require_open("rl_hip_capture_begin"))
        return -1;
    return rl_check_hip(hipStreamBeginCapture(g_session.stream, hipStreamCaptureModeThreadLocal),
                        "hipStreamBeginCapture");
}

int rl_hip_capture_end(void **graph)
{
    if (rl_require_open("rl_hip_capture_end"))
        return -1;
    if (!graph) {
        rl_set_error("rl_hip_capture_end: NULL output");
        return -1;
    }
    *graph = nullptr;
    hipGraph_t g = nullptr;
    if (rl_check_hip(hipStreamEndCapture(g_session.stream, &g), "hipStreamEndCapture"))
        return -1;
    hipGraphExec_t exec = nullptr;
    const int rc = rl_check_hip(hipGraphInstantiate(&exec, g, nullptr, nullptr, 0), "hipGraphInstantiate");
    (void)hipGraphDestroy(g);
    if (rc)
        return -1;
    *graph = exec;
    return 0;
}

int rl_hip_graph_launch(void *graph)
{
    if (rl_require_open("rl_hip_graph_launch"))
        return -1;
    if (!graph) {
        rl_set_error("rl_hip_graph_launch: NULL graph");
        return -1;
    }
    return rl_check_hip(hipGraphLaunch((hipGraphExec_t)graph, g_session.stream), "hipGraphLaunch");
}

int rl_hip_graph_destroy(void *graph)
{
    if (!graph)
        return 0;
    return rl_check_hip(hipGraphExecDestroy((hipGraphExec_t)graph), "hipGraphExecDestroy");
}

}  // extern "C"
