// Thin C ABI over the HIP runtime.  The C++20 host layers (core, nn, api) reach the GPU only through these
// functions and the kernel launch entries of kernels/kernels.h; neither header exposes HIP types.
//
// Replaces the reference's device plugin layer for the GPU: the CUDA Context with its stream-ordered pool,
// compute/copy streams and transfers (src/backends/cuda_context.h:17-107, cuda_context.cpp:18-210) and the
// Backend function table (src/backends/backend.h:21-108).  Every entry returns 0 on success or a HIP error
// code, which the C++ side turns into std::runtime_error("HIP: ...").
#pragma once

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dlh_stream_opaque* dlh_stream;
typedef struct dlh_event_opaque* dlh_event;
typedef struct dlh_graph_opaque* dlh_graph;

typedef struct dlh_device_properties {
    char name[256];
    char arch[64];
    int compute_units;
    int wavefront_size;
    int clock_khz;
    int memory_clock_khz;
    int memory_bus_width;
    uint64_t global_memory_bytes;
    uint64_t shared_memory_per_block;
    uint64_t l2_cache_bytes;
} dlh_device_properties;

enum { DLH_HOST_TO_DEVICE = 1, DLH_DEVICE_TO_HOST = 2, DLH_DEVICE_TO_DEVICE = 3 };

const char* dlh_error_string(int code);
int dlh_device_count(int* count);
int dlh_set_device(int device);
int dlh_get_device(int* device);
int dlh_device_properties_get(int device, dlh_device_properties* out);

int dlh_stream_create(dlh_stream* stream);
int dlh_stream_destroy(dlh_stream stream);
int dlh_stream_synchronize(dlh_stream stream);

/* Stream-ordered allocation from the device's default memory pool, which keeps freed memory for reuse. */
int dlh_pool_configure(int device);
int dlh_malloc_async(void** pointer, size_t bytes, dlh_stream stream);
int dlh_free_async(void* pointer, dlh_stream stream);
int dlh_pool_stats(int device, uint64_t* used, uint64_t* reserved, uint64_t* peak_used, uint64_t* peak_reserved,
                   uint64_t* threshold);
int dlh_pool_trim(int device);
int dlh_pool_set_threshold(int device, uint64_t bytes);
int dlh_pool_reset_peaks(int device);

int dlh_memcpy_async(void* destination, const void* source, size_t bytes, int kind, dlh_stream stream);

int dlh_event_create(dlh_event* event);
int dlh_event_destroy(dlh_event event);
int dlh_event_record(dlh_event event, dlh_stream stream);
int dlh_event_synchronize(dlh_event event);
int dlh_event_elapsed(dlh_event start, dlh_event stop, float* milliseconds);

/* Stream capture into an executable graph (thread-local capture mode). */
int dlh_capture_begin(dlh_stream stream);
/* *capturing = 1 while the stream records into a graph. */
int dlh_stream_capturing(dlh_stream stream, int* capturing);
int dlh_capture_end(dlh_stream stream, dlh_graph* executable);
int dlh_graph_launch(dlh_graph executable, dlh_stream stream);
int dlh_graph_destroy(dlh_graph executable);

/* Error left by the most recent kernel launch on this thread (hipGetLastError). */
int dlh_last_launch_error(void);

#ifdef __cplusplus
}
#endif
