#include "core/device.h"

#include "dl/gpu.h"

#include <cstdlib>
#include <cstring>
#include <mutex>
#include <stdexcept>
#include <vector>

namespace dl::detail {

void hip_check(int status, const char* what) {
    if (status != 0) throw std::runtime_error(std::string("HIP: ") + what + ": " + dlh_error_string(status));
}

namespace {
std::mutex context_mutex;
std::vector<std::unique_ptr<GpuContext>>& contexts() {
    // intentionally leaked: tensors released during interpreter or static teardown still find their stream
    static auto* value = new std::vector<std::unique_ptr<GpuContext>>();
    return *value;
}
thread_local int current_device = -1;
} // namespace

GpuContext& gpu_context(int index) {
    GpuContext* context = nullptr;
    {
        std::lock_guard<std::mutex> lock(context_mutex);
        auto& all = contexts();
        if (all.empty()) {
            int count = 0;
            hip_check(dlh_device_count(&count), "device count");
            all.resize(static_cast<std::size_t>(count));
        }
        if (index < 0 || static_cast<std::size_t>(index) >= all.size())
            throw std::runtime_error("HIP: GPU " + std::to_string(index) + " is not available (" +
                                     std::to_string(all.size()) + " visible)");
        auto& slot = all[static_cast<std::size_t>(index)];
        if (!slot) {
            auto created = std::make_unique<GpuContext>();
            created->index = index;
            hip_check(dlh_set_device(index), "set device");
            hip_check(dlh_device_properties_get(index, &created->properties), "device properties");
            hip_check(dlh_pool_configure(index), "memory pool");
            hip_check(dlh_stream_create(&created->stream), "stream create");
            void* flag = nullptr;
            hip_check(dlh_malloc_async(&flag, 256, created->stream), "error flag");
            hip_check(dlk_fill(flag, DLK_F32, 1, 0.0, created->stream), "error flag reset");
            created->error_flag = static_cast<int32_t*>(flag);
            slot = std::move(created);
        }
        context = slot.get();
    }
    if (current_device != index) {
        hip_check(dlh_set_device(index), "set device");
        current_device = index;
    }
    return *context;
}

void require_gpu(Device device, const char* operation) {
    if (device.type != DeviceType::gpu)
        throw std::invalid_argument(std::string(operation) +
                                    ": this build computes on the GPU only; move the tensors/modules with to(gpu)");
}

Storage::~Storage() {
    if (!data) return;
    if (device.type == DeviceType::cpu) {
        std::free(data);
    } else {
        // stream-ordered release: later work on the compute stream may reuse the block immediately
        GpuContext& context = gpu_context(device.index);
        (void)dlh_free_async(data, context.stream);
    }
}

std::shared_ptr<Storage> allocate_storage(std::size_t bytes, Device device) {
    auto storage = std::make_shared<Storage>();
    storage->bytes = bytes;
    storage->device = device;
    const std::size_t rounded = bytes == 0 ? 64 : (bytes + 63) / 64 * 64;
    if (device.type == DeviceType::cpu) {
        storage->data = std::aligned_alloc(64, rounded);
        if (!storage->data) throw std::bad_alloc();
        std::memset(storage->data, 0, rounded);
    } else {
        GpuContext& context = gpu_context(device.index);
        hip_check(dlh_malloc_async(&storage->data, rounded, context.stream), "allocate");
    }
    return storage;
}

void check_device_errors(Device device, const char* what) {
    if (device.type != DeviceType::gpu) return;
    GpuContext& context = gpu_context(device.index);
    int32_t flag = 0;
    hip_check(dlh_memcpy_async(&flag, context.error_flag, sizeof(flag), DLH_DEVICE_TO_HOST, context.stream), what);
    hip_check(dlh_stream_synchronize(context.stream), what);
    if (flag != 0) {
        hip_check(dlk_fill(context.error_flag, DLK_F32, 1, 0.0, context.stream), what);
        throw std::out_of_range(std::string(what) + ": index out of range");
    }
}

} // namespace dl::detail

namespace dl {
void synchronize(Device device) {
    if (device.type != DeviceType::gpu) return;
    auto& context = detail::gpu_context(device.index);
    detail::hip_check(dlh_stream_synchronize(context.stream), "synchronize");
}
} // namespace dl

namespace dl::gpu {
MemoryStats memory_stats(int device) {
    detail::gpu_context(device);
    MemoryStats out{};
    detail::hip_check(dlh_pool_stats(device, &out.used_bytes, &out.reserved_bytes, &out.peak_used_bytes,
                                     &out.peak_reserved_bytes, &out.release_threshold),
                      "pool statistics");
    return out;
}

void set_memory_release_threshold(std::uint64_t bytes, int device) {
    detail::gpu_context(device);
    detail::hip_check(dlh_pool_set_threshold(device, bytes), "pool release threshold");
}

void reset_peak_memory_stats(int device) {
    detail::gpu_context(device);
    detail::hip_check(dlh_pool_reset_peaks(device), "pool peak reset");
}

void release_unused_memory(int device) {
    auto& context = detail::gpu_context(device);
    detail::hip_check(dlh_stream_synchronize(context.stream), "synchronize");
    detail::hip_check(dlh_pool_trim(device), "pool trim");
}
} // namespace dl::gpu
