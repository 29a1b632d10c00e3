// Entries of <dl/generate_c_api.h>: the on-device token loop, per-kernel profiling, device timers, keyed
// normal weights and the streaming-copy bandwidth probe.
#include "api/common.h"
#include "core/tensor_impl.h"

#include <cstring>
#include <stdexcept>

using namespace dl::capi;

namespace {
template <class T> std::shared_ptr<T> cast_module(const dl_module* module, const char* what) {
    auto value = std::dynamic_pointer_cast<T>(require(module, what).value);
    if (!value) throw std::invalid_argument(std::string(what) + " has the wrong module type");
    return value;
}
} // namespace

extern "C" {

dl_status dl_decoder_lm_create(const dl_module* embedding, const dl_module* decoder, const dl_module* head,
                               dl_decoder_lm** output) {
    if (!output) return DL_ERROR;
    *output = nullptr;
    return invoke([&] {
        auto e = cast_module<dl::nn::Embedding>(embedding, "embedding");
        auto d = cast_module<dl::nn::TransformerDecoder>(decoder, "decoder");
        auto h = cast_module<dl::nn::Linear>(head, "head");
        auto lm = std::make_unique<dl_decoder_lm>();
        lm->embedding = e;
        lm->decoder = d;
        lm->head = h;
        lm->value = std::make_unique<dl::detail::DecoderLM>(e, d, h);
        *output = lm.release();
    });
}

void dl_decoder_lm_release(dl_decoder_lm* lm) { delete lm; }

dl_status dl_decoder_lm_logits(dl_decoder_lm* lm, const dl_tensor* ids, dl_decoder_cache* cache, dl_tensor** logits) {
    return make_handle(logits, [&] {
        return require(lm, "lm").value->logits(require(ids, "ids").value, require(cache, "cache").value);
    });
}

dl_status dl_decoder_lm_generate(dl_decoder_lm* lm, const dl_tensor* prompt, dl_decoder_cache* cache, int64_t steps,
                                 double temperature, dl_random_key key, int32_t use_graph, dl_tensor** tokens,
                                 dl_tensor** last_logits) {
    if (tokens) *tokens = nullptr;
    if (last_logits) *last_logits = nullptr;
    return invoke([&] {
        auto [t, l] = require(lm, "lm").value->generate(require(prompt, "prompt").value, require(cache, "cache").value,
                                                         steps, temperature, convert(key), use_graph != 0);
        auto th = tokens ? std::make_unique<dl_tensor>(dl_tensor{t}) : nullptr;
        auto lh = last_logits ? std::make_unique<dl_tensor>(dl_tensor{l}) : nullptr;
        if (tokens) *tokens = th.release();
        if (last_logits) *last_logits = lh.release();
    });
}

dl_status dl_decoder_lm_benchmark(dl_decoder_lm* lm, const dl_tensor* prompt, dl_decoder_cache* cache, int64_t warmup,
                                  int64_t timed, double temperature, dl_random_key key, int32_t use_graph,
                                  double* milliseconds, dl_tensor** tokens) {
    if (tokens) *tokens = nullptr;
    return invoke([&] {
        dl::Tensor t;
        const double ms = require(lm, "lm").value->benchmark(require(prompt, "prompt").value,
                                                             require(cache, "cache").value, warmup, timed, temperature,
                                                             convert(key), use_graph != 0, tokens ? &t : nullptr);
        if (milliseconds) *milliseconds = ms;
        if (tokens) *tokens = new dl_tensor{t};
    });
}

dl_status dl_decoder_lm_profile(dl_decoder_lm* lm, const dl_tensor* ids, dl_decoder_cache* cache, int64_t rounds,
                                dl_kernel_timing* timings, size_t capacity, size_t* count) {
    return invoke([&] {
        auto result = require(lm, "lm").value->profile(require(ids, "ids").value, require(cache, "cache").value, rounds);
        const size_t n = std::min(capacity, result.size());
        for (size_t i = 0; i < n; ++i) {
            std::memset(timings[i].name, 0, sizeof(timings[i].name));
            std::strncpy(timings[i].name, result[i].name.c_str(), sizeof(timings[i].name) - 1);
            timings[i].launches = result[i].launches;
            timings[i].total_ms = result[i].total_ms;
            timings[i].bytes = result[i].bytes;
        }
        if (count) *count = n;
    });
}

dl_status dl_decoder_lm_set_weight_repack(dl_decoder_lm* lm, int32_t enabled) {
    return invoke([&] { require(lm, "lm").value->set_weight_repack(enabled != 0); });
}

dl_status dl_sample(const dl_tensor* logits, double temperature, dl_random_key key, dl_tensor** output) {
    return make_handle(output, [&] { return dl::sample(require(logits, "logits").value, temperature, convert(key)); });
}

dl_status dl_normal_with_key(dl_random_key key, dl_shape shape, double scale, dl_tensor_options options,
                             dl_tensor** output) {
    return make_handle(output, [&] { return dl::normal(convert(key), convert(shape), scale, convert(options)); });
}

dl_status dl_timer_create(dl_device device, dl_timer** output) {
    if (!output) return DL_ERROR;
    *output = nullptr;
    return invoke([&] {
        dl::detail::require_gpu(convert(device), "timer");
        dl::detail::gpu_context(device.index);
        auto timer = std::make_unique<dl_timer>();
        timer->device = device.index;
        dl::detail::hip_check(dlh_event_create(&timer->start), "event");
        dl::detail::hip_check(dlh_event_create(&timer->stop), "event");
        *output = timer.release();
    });
}

void dl_timer_release(dl_timer* timer) {
    if (!timer) return;
    (void)dlh_event_destroy(timer->start);
    (void)dlh_event_destroy(timer->stop);
    delete timer;
}

dl_status dl_timer_start(dl_timer* timer) {
    return invoke([&] {
        auto& t = require(timer, "timer");
        auto& context = dl::detail::gpu_context(t.device);
        dl::detail::hip_check(dlh_event_record(t.start, context.stream), "event record");
    });
}

dl_status dl_timer_stop(dl_timer* timer, double* milliseconds) {
    return invoke([&] {
        auto& t = require(timer, "timer");
        auto& context = dl::detail::gpu_context(t.device);
        dl::detail::hip_check(dlh_event_record(t.stop, context.stream), "event record");
        dl::detail::hip_check(dlh_event_synchronize(t.stop), "event wait");
        float ms = 0.0f;
        dl::detail::hip_check(dlh_event_elapsed(t.start, t.stop, &ms), "event elapsed");
        *milliseconds = ms;
    });
}

dl_status dl_gpu_copy_bandwidth(int32_t device, uint64_t bytes, int32_t iterations, double* gigabytes_per_second) {
    return invoke([&] {
        if (bytes % 16 != 0 || iterations <= 0) throw std::invalid_argument("bytes must be a multiple of 16");
        const dl::Device gpu = dl::Device::gpu(device);
        auto& context = dl::detail::gpu_context(device);
        dl::Tensor src = dl::zeros({static_cast<dl::Index>(bytes / 4)}, {.dtype = dl::DType::f32, .device = gpu});
        dl::Tensor dst = dl::empty({static_cast<dl::Index>(bytes / 4)}, {.dtype = dl::DType::f32, .device = gpu});
        dl::detail::hip_check(dlk_stream_copy(src.data<void>(), dl::detail::mutable_data(dst), bytes, context.stream), "copy");
        dlh_event start = nullptr, stop = nullptr;
        dl::detail::hip_check(dlh_event_create(&start), "event");
        dl::detail::hip_check(dlh_event_create(&stop), "event");
        dl::detail::hip_check(dlh_event_record(start, context.stream), "event record");
        for (int i = 0; i < iterations; ++i)
            dl::detail::hip_check(dlk_stream_copy(src.data<void>(), dl::detail::mutable_data(dst), bytes, context.stream),
                                  "copy");
        dl::detail::hip_check(dlh_event_record(stop, context.stream), "event record");
        dl::detail::hip_check(dlh_event_synchronize(stop), "event wait");
        float ms = 0.0f;
        dl::detail::hip_check(dlh_event_elapsed(start, stop, &ms), "event elapsed");
        (void)dlh_event_destroy(start);
        (void)dlh_event_destroy(stop);
        *gigabytes_per_second = 2.0 * static_cast<double>(bytes) * iterations / (ms * 1e-3) / 1e9;
    });
}

} // extern "C"
