// On-device token loop (see language_model.h).  A step is: embedding gather of the current ids, the fused
// decoder layers, the LM head for the last position with the final RMSNorm fused into its prologue and the
// sampling candidates in its epilogue, and one finalize launch that writes the token, feeds it back as the
// next ids and advances the device step counter.  Nothing in a single-token step depends on host values, so
// steps 3.. replay a HIP graph captured from step 3.
#include "nn/language_model.h"

#include <algorithm>
#include <cstring>
#include <stdexcept>

namespace dl::detail {

DecoderLM::DecoderLM(std::shared_ptr<nn::Embedding> embedding, std::shared_ptr<nn::TransformerDecoder> decoder,
                     std::shared_ptr<nn::Linear> head)
    : embedding_(std::move(embedding)), decoder_(std::move(decoder)), head_(std::move(head)) {
    const Device device = decoder_->layer(0).attention().query().weight().device();
    require_gpu(device, "decoder language model");
    if (!(embedding_->weight().device() == device) || !(head_->weight().device() == device))
        throw std::invalid_argument("embedding, decoder and head must live on one GPU");
    const Index d = decoder_->layer(0).attention().dimensions();
    if (embedding_->weight().size(1) != d || head_->weight().size(1) != d)
        throw std::invalid_argument("embedding / head width differs from the decoder width");
    if (head_->bias()) throw std::invalid_argument("the fused LM head takes a bias-free Linear");
    context_ = &gpu_context(device.index);
    // the token loop runs many steps over the same weights: the batched decode reads them repacked in its
    // matrix-core kernel's tile order, a second copy of the bf16 projection and head weights in HBM (1B: 1.6 GB,
    // 8B: 14 GB) for a faster step (MI355X, 1B at batch 32: 1.44 -> 1.33 ms; 8B at batch 8: 10.2 -> 9.6 ms)
    ws_.pack_weights = true;
}

DecoderLM::~DecoderLM() { release_graph(); }

void DecoderLM::set_weight_repack(bool enabled) {
    ws_.pack_weights = enabled;
    if (!enabled) {
        // launches already queued may still read the packed copies: they finish before the memory is returned
        hip_check(dlh_stream_synchronize(context_->stream), "weight repack off");
        ws_.release_packs();
    }
}

void DecoderLM::release_graph() {
    if (graph_) {
        (void)dlh_stream_synchronize(context_->stream);
        (void)dlh_graph_destroy(graph_);
        graph_ = nullptr;
    }
}

void DecoderLM::check_caches(std::span<nn::KVCache> cache, Index batch, Index length) const {
    if (cache.size() != static_cast<std::size_t>(decoder_->layer_count()))
        throw std::invalid_argument("decoder requires one cache per layer");
    const Index prefix = cache.front().length();
    for (std::size_t i = 0; i < cache.size(); ++i) {
        if (cache[i].length() != prefix) throw std::invalid_argument("decoder cache positions differ");
        if (length > cache[i].capacity() - prefix)
            throw std::invalid_argument("KV cache append exceeds capacity or has unequal key/value lengths");
        if (prefix + length > decoder_->layer(static_cast<Index>(i)).attention().rotary().cosine().size(0))
            throw std::out_of_range("RoPE positions exceed the table capacity");
        const auto& layer = decoder_->layer(static_cast<Index>(i));
        cache[i].check_layout(batch, layer.attention().kv_heads(), layer.attention().head_dim(), cache_dtype(layer),
                              embedding_->weight().device());
    }
}

void DecoderLM::forward_chunk(const Index* ids, Index batch, Index length, std::span<nn::KVCache> cache,
                              int sample_mode, double temperature, RandomKey key, bool capacity_splits,
                              LaunchObserver* observer) {
    const Index d = embedding_->weight().size(1), V = head_->weight().size(0);
    const Index rows = batch * length;
    const Device device = embedding_->weight().device();
    if (!x_.defined() || x_rows_ < rows) {
        x_ = empty_tensor({rows, d}, DType::f32, device);
        x_rows_ = rows;
    }
    if (!logits_.defined() || logits_.size(0) != batch) logits_ = empty_tensor({batch, V}, DType::f32, device);
    float* x = static_cast<float*>(mutable_data(x_));
    GpuContext* context = context_;

    if (ids) {
        const void* table = embedding_->weight().data<void>();
        const int table_dtype = dlk_dtype(embedding_->weight().dtype());
        const Index vocabulary = embedding_->weight().size(0);
        issue(observer, "embedding",
              static_cast<double>(rows * d) * static_cast<double>(element_size(embedding_->weight().dtype())),
              [=](bool) {
                  hip_check(dlk_embedding(ids, rows, table, table_dtype, vocabulary, d, x, DLK_F32, context->error_flag,
                                          context->stream),
                            "embedding");
              });
    }

    const auto& first = decoder_->layer(0).attention();
    int splits = 1, chunk = 64;
    const Index source = capacity_splits ? cache.front().capacity() : cache.front().length() + length;
    attention_split(batch, first.heads(), first.kv_heads(), first.head_dim(),
                    cache_dtype(decoder_->layer(0)) == DType::bf16, length, source, splits, chunk);
    for (Index i = 0; i < decoder_->layer_count(); ++i) {
        auto& layer = decoder_->layer(i);
        cache[static_cast<std::size_t>(i)].reserve(batch, layer.attention().kv_heads(), layer.attention().head_dim(),
                                                   cache_dtype(layer), device);
        decode_layer(layer, x, x, batch, length, cache[static_cast<std::size_t>(i)], ws_, splits, chunk, *context_,
                     observer);
    }

    // LM head on the last position of every sequence, final RMSNorm fused in, sampling candidates out
    int hb = 0, nb = 0;
    const auto& norm = decoder_->normalization();
    dlk_gemv_params p = gemv_params(x + (length - 1) * d, batch, d, DLK_EPI_LOGITS);
    p.ldx = length * d;
    p.apply_norm = 1;
    p.norm_weight = norm.weight() ? norm.weight()->data<void>() : nullptr;
    nb = norm.weight() && norm.weight()->dtype() == DType::bf16;
    p.norm_bf16 = nb;
    p.epsilon = static_cast<float>(norm.epsilon());
    p.nseg = 1;
    p.w[0] = weight_data(head_->weight(), hb, "LM head");
    p.seg_rows[0] = static_cast<int>(V);
    p.w_bf16 = hb;
    p.y = static_cast<float*>(mutable_data(logits_));
    p.ldy = V;
    p.sample_mode = sample_mode;
    p.temperature = temperature;
    p.key_seed = key.seed;
    p.key_stream = key.stream;
    if (sample_mode > 0) {
        p.key_label = static_cast<const Index*>(step_.data<void>());
        const int blocks = dlk_gemv_blocks(&p);
        if (blocks <= 0) throw std::invalid_argument("LM head: no projection kernel fits this shape");
        if (!partial_.defined() || blocks_ != blocks || partial_.numel() < batch * blocks * 2) {
            partial_ = empty_tensor({batch * blocks * 2}, DType::i64, device);
            blocks_ = blocks;
        }
        p.partial = static_cast<dlk_sample_partial*>(mutable_data(partial_));
        p.partial_blocks = blocks;
    }
    if (dlk_gemv_uses_rows(&p)) p.w_tiles[0] = ws_.tiles_of(head_->weight(), nullptr, context->stream);
    issue(observer, "lm_head", static_cast<double>(V * d) * (hb ? 2 : 4),
          [p, context](bool) { hip_check(dlk_gemv(&p, context->stream), "LM head"); });
    if (sample_mode > 0) {
        // the sampled ids are fed back: their embedding rows become the next step's input x[0:B]
        const auto* partial = static_cast<const dlk_sample_partial*>(partial_.data<void>());
        Index* next = static_cast<Index*>(mutable_data(next_ids_));
        Index* tokens = tokens_.defined() ? static_cast<Index*>(mutable_data(tokens_)) : nullptr;
        Index* step = static_cast<Index*>(mutable_data(step_));
        const void* table = embedding_->weight().data<void>();
        const int table_dtype = dlk_dtype(embedding_->weight().dtype());
        const int blocks = blocks_;
        const Index columns = token_columns_;
        issue(observer, "sample_finalize", 0.0, [=](bool) {
            hip_check(dlk_sample_finalize(partial, batch, blocks, nullptr, next, tokens, columns, step, table,
                                          table_dtype, d, x, context->stream),
                      "sample");
        });
    }
}

Tensor DecoderLM::logits(const Tensor& ids, std::span<nn::KVCache> cache) {
    if (ids.ndim() != 2 || ids.dtype() != DType::i64) throw std::invalid_argument("ids must be i64 [B, L]");
    const Index B = ids.size(0), L = ids.size(1);
    if (L <= 0 || B <= 0) throw std::invalid_argument("ids must be non-empty");
    check_caches(cache, B, L);
    const Device device = embedding_->weight().device();
    Tensor dev_ids = ids.to(device).contiguous();
    const Index prefix = cache.front().length();
    try {
        forward_chunk(dev_ids.data<Index>(), B, L, cache, 0, 0.0, {0, 0}, false, nullptr);
    } catch (...) {
        for (auto& c : cache) c.truncate(std::min(prefix, c.length()));
        throw;
    }
    check_device_errors(device, "embedding");
    return logits_.clone();
}

DecoderLM::RunResult DecoderLM::run(const Tensor& prompt, std::span<nn::KVCache> cache, Index steps,
                                    double temperature, RandomKey key, bool use_graph, Index timed) {
    if (prompt.ndim() != 2 || prompt.dtype() != DType::i64) throw std::invalid_argument("prompt must be i64 [B, P]");
    if (steps <= 0) throw std::invalid_argument("steps must be positive");
    if (timed < 0 || timed > steps - 1) throw std::invalid_argument("timed steps must follow the prompt step");
    const Index B = prompt.size(0), P = prompt.size(1);
    if (P <= 0 || B <= 0) throw std::invalid_argument("prompt must be non-empty");
    // the whole request must fit: prompt plus steps-1 fed-back tokens
    check_caches(cache, B, P + steps - 1);
    const Device device = embedding_->weight().device();
    Tensor dev_prompt = prompt.to(device).contiguous();
    step_ = zeros({1}, {.dtype = DType::i64, .device = device});
    next_ids_ = empty_tensor({B}, DType::i64, device);
    tokens_ = empty_tensor({B, steps}, DType::i64, device);
    token_columns_ = steps;
    const int mode = temperature > 0.0 ? 2 : 1;
    const Index prefix = cache.front().length();
    const Index first_timed = steps - timed;
    dlh_event start = nullptr, stop = nullptr;
    RunResult result;
    auto mark_start = [&](Index s) {
        if (timed > 0 && s == first_timed) {
            hip_check(dlh_stream_synchronize(context_->stream), "benchmark synchronize");
            hip_check(dlh_event_record(start, context_->stream), "event record");
        }
    };
    try {
        if (timed > 0) {
            hip_check(dlh_event_create(&start), "event");
            hip_check(dlh_event_create(&stop), "event");
        }
        forward_chunk(dev_prompt.data<Index>(), B, P, cache, mode, temperature, key, false, nullptr);
        // eager steps size every buffer; with graphs the step after them is captured and replayed
        const Index eager_steps = use_graph ? std::min<Index>(steps, 2) : steps;
        for (Index s = 1; s < eager_steps; ++s) {
            mark_start(s);
            forward_chunk(nullptr, B, 1, cache, mode, temperature, key, use_graph, nullptr);
        }
        if (use_graph && steps > 2) {
            // capture one single-token step; host lengths are restored because capture does not execute
            std::vector<Index> lengths;
            for (auto& c : cache) lengths.push_back(c.length());
            release_graph();
            hip_check(dlh_capture_begin(context_->stream), "graph capture");
            try {
                forward_chunk(nullptr, B, 1, cache, mode, temperature, key, true, nullptr);
            } catch (...) {
                dlh_graph discard = nullptr;
                (void)dlh_capture_end(context_->stream, &discard);
                if (discard) (void)dlh_graph_destroy(discard);
                throw;
            }
            hip_check(dlh_capture_end(context_->stream, &graph_), "graph instantiate");
            // truncate re-writes the (unchanged) device length of every layer
            for (std::size_t i = 0; i < cache.size(); ++i) cache[i].truncate(lengths[i]);
            for (Index s = 2; s < steps; ++s) {
                mark_start(s);
                hip_check(dlh_graph_launch(graph_, context_->stream), "graph launch");
                for (auto& c : cache) c.advance(1);
            }
        }
        if (timed > 0) {
            hip_check(dlh_event_record(stop, context_->stream), "event record");
            hip_check(dlh_event_synchronize(stop), "event wait");
            float ms = 0.0f;
            hip_check(dlh_event_elapsed(start, stop, &ms), "event elapsed");
            result.timed_ms = ms;
        }
        release_graph();
    } catch (...) {
        release_graph();
        if (start) (void)dlh_event_destroy(start);
        if (stop) (void)dlh_event_destroy(stop);
        for (auto& c : cache) c.truncate(std::min(prefix, c.length()));
        throw;
    }
    if (start) (void)dlh_event_destroy(start);
    if (stop) (void)dlh_event_destroy(stop);
    check_device_errors(device, "embedding");
    result.tokens = tokens_;
    result.logits = logits_.clone();
    tokens_ = Tensor();
    return result;
}

std::pair<Tensor, Tensor> DecoderLM::generate(const Tensor& prompt, std::span<nn::KVCache> cache, Index steps,
                                              double temperature, RandomKey key, bool use_graph) {
    RunResult r = run(prompt, cache, steps, temperature, key, use_graph, 0);
    return {r.tokens, r.logits};
}

double DecoderLM::benchmark(const Tensor& prompt, std::span<nn::KVCache> cache, Index warmup, Index timed,
                            double temperature, RandomKey key, bool use_graph, Tensor* tokens) {
    if (warmup < 0 || timed <= 0) throw std::invalid_argument("benchmark needs warmup >= 0 and timed > 0");
    // token 0 comes from the prompt step; steps 1 and 2 size buffers / are captured; then warmup, then timed
    const Index steps = 1 + 2 + warmup + timed;
    RunResult r = run(prompt, cache, steps, temperature, key, use_graph, timed);
    if (tokens) *tokens = r.tokens;
    return r.timed_ms;
}

namespace {
// Records every launch of a step (and issues it); the profile then repeats each kernel class on its own.
struct ReplayObserver final : LaunchObserver {
    struct Entry {
        std::string name;
        double bytes;
        std::function<void(bool)> fn;
    };
    std::vector<Entry> entries;
    void launch(const char* name, double bytes, std::function<void(bool)> fn) override {
        fn(false);
        entries.push_back({name, bytes, std::move(fn)});
    }
};
} // namespace

std::vector<KernelTiming> DecoderLM::profile(const Tensor& ids, std::span<nn::KVCache> cache, Index rounds) {
    if (ids.ndim() != 2 || ids.dtype() != DType::i64 || ids.size(1) != 1)
        throw std::invalid_argument("profile ids must be i64 [B, 1]");
    if (rounds <= 0) throw std::invalid_argument("profile needs rounds > 0");
    const Index B = ids.size(0);
    check_caches(cache, B, 2); // the step's own token plus the slot its QKV repeats write
    const Device device = embedding_->weight().device();
    Tensor dev_ids = ids.to(device).contiguous();
    step_ = zeros({1}, {.dtype = DType::i64, .device = device});
    tokens_ = Tensor();
    // One unobserved step first: every workspace of the step reaches its size for this batch, so the buffers the
    // recorded launches point at are the ones that stay (a later launch of the same step may otherwise grow and
    // reallocate a workspace an earlier recorded launch uses).  The caches go back to their lengths afterwards.
    const Index prefix = cache.front().length();
    next_ids_ = dev_ids.clone();
    forward_chunk(next_ids_.data<Index>(), B, 1, cache, 1, 0.0, {0, 0}, false, nullptr);
    for (auto& c : cache) c.truncate(prefix);
    next_ids_ = dev_ids.clone();
    ReplayObserver observer;
    forward_chunk(next_ids_.data<Index>(), B, 1, cache, 1, 0.0, {0, 0}, false, &observer);
    hip_check(dlh_stream_synchronize(context_->stream), "profile");

    // each class: all of its launches of the step (one per layer), `rounds` times back to back between two events
    std::vector<KernelTiming> out;
    dlh_event start = nullptr, stop = nullptr;
    hip_check(dlh_event_create(&start), "event");
    hip_check(dlh_event_create(&stop), "event");
    try {
        for (const auto& first : observer.entries) {
            if (std::any_of(out.begin(), out.end(), [&](const KernelTiming& k) { return k.name == first.name; }))
                continue;
            KernelTiming timing{first.name, 0, 0.0, 0.0};
            for (const auto& e : observer.entries)
                if (e.name == first.name) e.fn(true); // warm-up round
            hip_check(dlh_event_record(start, context_->stream), "event record");
            for (Index r = 0; r < rounds; ++r)
                for (const auto& e : observer.entries)
                    if (e.name == first.name) {
                        e.fn(true);
                        timing.launches += 1;
                        timing.bytes += e.bytes;
                    }
            hip_check(dlh_event_record(stop, context_->stream), "event record");
            hip_check(dlh_stream_synchronize(context_->stream), "profile");
            float ms = 0.0f;
            hip_check(dlh_event_elapsed(start, stop, &ms), "event elapsed");
            timing.total_ms = ms;
            out.push_back(timing);
        }
    } catch (...) {
        (void)dlh_event_destroy(start);
        (void)dlh_event_destroy(stop);
        throw;
    }
    (void)dlh_event_destroy(start);
    (void)dlh_event_destroy(stop);
    for (auto& c : cache) c.truncate(c.length()); // repeats never moved the lengths; rewrite them on the device
    check_device_errors(device, "embedding");
    return out;
}

} // namespace dl::detail
