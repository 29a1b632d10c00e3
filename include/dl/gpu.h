#pragma once
// Statistics and control of this library's device memory pool.  Mirrors include/dl/cuda.h:10-26 of the reference
// (namespace dl::cuda there): the same four calls over the GPU's default stream-ordered pool
// (reference src/core/cuda_memory.cpp:27-63).

#include "dl/types.h"

#include <cstdint>

namespace dl::gpu {

/// Bytes of the device's pool as the HIP runtime reports them.  `used` counts live allocations, `reserved` adds
/// the free blocks the pool keeps for reuse; pinned host memory and the HIP runtime's own allocations are not
/// counted.
struct MemoryStats {
    std::uint64_t used_bytes, reserved_bytes;
    std::uint64_t peak_used_bytes, peak_reserved_bytes;
    std::uint64_t release_threshold;
};

/// Reads the pool's attributes without waiting for the stream (synchronize first for figures at a phase
/// boundary).  The first call creates the device's context.
DL_API MemoryStats memory_stats(int device = 0);
/// Free bytes above this threshold go back to the device at synchronisation points.  The library's default keeps
/// every freed block for reuse; zero returns all of them.  It is not a capacity limit.
DL_API void set_memory_release_threshold(std::uint64_t bytes, int device = 0);
/// Restarts both peak figures (HIP sets them to zero; the next allocation raises them again).
DL_API void reset_peak_memory_stats(int device = 0);
/// Waits for the device's stream and then returns every free block of the pool to the device; live tensors and
/// the release threshold are kept.
DL_API void release_unused_memory(int device = 0);

} // namespace dl::gpu
