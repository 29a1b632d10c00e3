// Implementation of the thin HIP C ABI (see hip_backend.h).
#include "backends/hip_backend.h"

#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstring>

namespace {
hipStream_t as_stream(dlh_stream s) { return reinterpret_cast<hipStream_t>(s); }
hipEvent_t as_event(dlh_event e) { return reinterpret_cast<hipEvent_t>(e); }
hipGraphExec_t as_graph(dlh_graph g) { return reinterpret_cast<hipGraphExec_t>(g); }
int code(hipError_t e) { return static_cast<int>(e); }
} // namespace

extern "C" {

const char* dlh_error_string(int c) { return hipGetErrorString(static_cast<hipError_t>(c)); }

int dlh_device_count(int* count) {
    *count = 0;
    const hipError_t e = hipGetDeviceCount(count);
    if (e == hipErrorNoDevice) { *count = 0; (void)hipGetLastError(); return 0; }
    return code(e);
}

int dlh_set_device(int device) { return code(hipSetDevice(device)); }
int dlh_get_device(int* device) { return code(hipGetDevice(device)); }

int dlh_device_properties_get(int device, dlh_device_properties* out) {
    hipDeviceProp_t p;
    const hipError_t e = hipGetDeviceProperties(&p, device);
    if (e != hipSuccess) return code(e);
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%.*s", static_cast<int>(sizeof(out->name) - 1), p.name);
    std::snprintf(out->arch, sizeof(out->arch), "%.*s", static_cast<int>(sizeof(out->arch) - 1), p.gcnArchName);
    out->compute_units = p.multiProcessorCount;
    out->wavefront_size = p.warpSize;
    out->clock_khz = p.clockRate;
    out->memory_clock_khz = p.memoryClockRate;
    out->memory_bus_width = p.memoryBusWidth;
    out->global_memory_bytes = p.totalGlobalMem;
    out->shared_memory_per_block = p.sharedMemPerBlock;
    out->l2_cache_bytes = static_cast<uint64_t>(p.l2CacheSize);
    return 0;
}

int dlh_stream_create(dlh_stream* stream) {
    hipStream_t s = nullptr;
    const hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    *stream = reinterpret_cast<dlh_stream>(s);
    return code(e);
}
int dlh_stream_destroy(dlh_stream stream) { return code(hipStreamDestroy(as_stream(stream))); }
int dlh_stream_synchronize(dlh_stream stream) { return code(hipStreamSynchronize(as_stream(stream))); }

int dlh_pool_configure(int device) {
    hipMemPool_t pool;
    hipError_t e = hipDeviceGetDefaultMemPool(&pool, device);
    if (e != hipSuccess) return code(e);
    uint64_t threshold = UINT64_MAX; // keep freed blocks for reuse instead of returning them at every sync
    return code(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &threshold));
}

int dlh_malloc_async(void** pointer, size_t bytes, dlh_stream stream) {
    return code(hipMallocAsync(pointer, bytes, as_stream(stream)));
}
int dlh_free_async(void* pointer, dlh_stream stream) { return code(hipFreeAsync(pointer, as_stream(stream))); }

int dlh_pool_stats(int device, uint64_t* used, uint64_t* reserved, uint64_t* peak_used, uint64_t* peak_reserved,
                   uint64_t* threshold) {
    hipMemPool_t pool;
    hipError_t e = hipDeviceGetDefaultMemPool(&pool, device);
    if (e != hipSuccess) return code(e);
    e = hipMemPoolGetAttribute(pool, hipMemPoolAttrUsedMemCurrent, used);
    if (e == hipSuccess) e = hipMemPoolGetAttribute(pool, hipMemPoolAttrReservedMemCurrent, reserved);
    if (e == hipSuccess) e = hipMemPoolGetAttribute(pool, hipMemPoolAttrUsedMemHigh, peak_used);
    if (e == hipSuccess) e = hipMemPoolGetAttribute(pool, hipMemPoolAttrReservedMemHigh, peak_reserved);
    if (e == hipSuccess) e = hipMemPoolGetAttribute(pool, hipMemPoolAttrReleaseThreshold, threshold);
    return code(e);
}

int dlh_pool_trim(int device) {
    hipMemPool_t pool;
    hipError_t e = hipDeviceGetDefaultMemPool(&pool, device);
    if (e != hipSuccess) return code(e);
    return code(hipMemPoolTrimTo(pool, 0));
}

int dlh_pool_set_threshold(int device, uint64_t bytes) {
    hipMemPool_t pool;
    hipError_t e = hipDeviceGetDefaultMemPool(&pool, device);
    if (e != hipSuccess) return code(e);
    return code(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &bytes));
}

int dlh_pool_reset_peaks(int device) {
    hipMemPool_t pool;
    hipError_t e = hipDeviceGetDefaultMemPool(&pool, device);
    if (e != hipSuccess) return code(e);
    uint64_t zero = 0; // the high-water attributes accept only zero
    e = hipMemPoolSetAttribute(pool, hipMemPoolAttrUsedMemHigh, &zero);
    if (e == hipSuccess) e = hipMemPoolSetAttribute(pool, hipMemPoolAttrReservedMemHigh, &zero);
    return code(e);
}

int dlh_memcpy_async(void* destination, const void* source, size_t bytes, int kind, dlh_stream stream) {
    hipMemcpyKind k = kind == DLH_HOST_TO_DEVICE   ? hipMemcpyHostToDevice
                      : kind == DLH_DEVICE_TO_HOST ? hipMemcpyDeviceToHost
                                                   : hipMemcpyDeviceToDevice;
    return code(hipMemcpyAsync(destination, source, bytes, k, as_stream(stream)));
}

int dlh_event_create(dlh_event* event) {
    hipEvent_t e = nullptr;
    const hipError_t r = hipEventCreate(&e);
    *event = reinterpret_cast<dlh_event>(e);
    return code(r);
}
int dlh_event_destroy(dlh_event event) { return code(hipEventDestroy(as_event(event))); }
int dlh_event_record(dlh_event event, dlh_stream stream) {
    return code(hipEventRecord(as_event(event), as_stream(stream)));
}
int dlh_event_synchronize(dlh_event event) { return code(hipEventSynchronize(as_event(event))); }
int dlh_event_elapsed(dlh_event start, dlh_event stop, float* milliseconds) {
    return code(hipEventElapsedTime(milliseconds, as_event(start), as_event(stop)));
}

int dlh_capture_begin(dlh_stream stream) {
    return code(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal));
}
int dlh_stream_capturing(dlh_stream stream, int* capturing) {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    const hipError_t e = hipStreamIsCapturing(as_stream(stream), &status);
    *capturing = status == hipStreamCaptureStatusActive ? 1 : 0;
    return code(e);
}
int dlh_capture_end(dlh_stream stream, dlh_graph* executable) {
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(as_stream(stream), &graph);
    if (e != hipSuccess) return code(e);
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    *executable = reinterpret_cast<dlh_graph>(exec);
    return code(e);
}
int dlh_graph_launch(dlh_graph executable, dlh_stream stream) {
    return code(hipGraphLaunch(as_graph(executable), as_stream(stream)));
}
int dlh_graph_destroy(dlh_graph executable) { return code(hipGraphExecDestroy(as_graph(executable))); }

int dlh_last_launch_error(void) { return code(hipGetLastError()); }

} // extern "C"
