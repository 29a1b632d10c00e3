// Per-GPU context (compute stream + stream-ordered pool) and the storage owner shared by all tensors.
// Mirrors the reference's lazily created, mutex-guarded per-device Context (src/backends/cuda_context.cpp:121-133)
// and its Allocation {address, release} owner (src/core/tensor_data.h:11-15), over the HIP C ABI only.
#pragma once

#include "dl/types.h"
#include "backends/hip_backend.h"
#include "kernels/kernels.h"

#include <cstddef>
#include <memory>
#include <string>

namespace dl::detail {

/// Throws std::runtime_error("HIP: <what>: <error>") for a nonzero HIP status.
void hip_check(int status, const char* what);

struct GpuContext {
    int index = 0;
    dlh_stream stream = nullptr;
    dlh_device_properties properties{};
    int32_t* error_flag = nullptr; // device flag set by kernels that detect invalid input (e.g. token ids)
};

/// Returns the context of GPU `index`, creating it on first use, and makes the device current on this thread.
GpuContext& gpu_context(int index);
/// Throws when the library runs without a usable GPU (the product has no CPU compute path).
void require_gpu(Device device, const char* operation);

struct Storage {
    void* data = nullptr;
    std::size_t bytes = 0;
    Device device{};
    Storage() = default;
    Storage(const Storage&) = delete;
    Storage& operator=(const Storage&) = delete;
    ~Storage();
};

std::shared_ptr<Storage> allocate_storage(std::size_t bytes, Device device);

/// Checks and clears the device error flag of `device` (blocking read); throws with `what` if it was set.
void check_device_errors(Device device, const char* what);

} // namespace dl::detail
