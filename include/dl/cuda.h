#pragma once
// The reference's device-pool statistics under their own names (include/dl/cuda.h:5-28, namespace dl::cuda),
// so that its callers compile unchanged.  In this library they read and control the HIP device's stream-ordered
// pool: the same calls as dl::gpu (dl/gpu.h).

#include "dl/gpu.h"

namespace dl::cuda {

using MemoryStats = gpu::MemoryStats;

inline MemoryStats memory_stats(int device = 0) { return gpu::memory_stats(device); }
inline void set_memory_release_threshold(std::uint64_t bytes, int device = 0) {
    gpu::set_memory_release_threshold(bytes, device);
}
inline void reset_peak_memory_stats(int device = 0) { gpu::reset_peak_memory_stats(device); }
inline void release_unused_memory(int device = 0) { gpu::release_unused_memory(device); }

} // namespace dl::cuda
