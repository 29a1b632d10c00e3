// On-device token loop over Embedding -> TransformerDecoder -> Linear head (the reference's application-level
// composition, examples/decoder_model.h:10-39 and examples/decoder_generate.cpp:20-31).
#pragma once

#include "nn/decode_step.h"

#include <map>
#include <string>

namespace dl::detail {

struct KernelTiming {
    std::string name;
    Index launches = 0;
    double total_ms = 0.0;
    double bytes = 0.0;
};

class DecoderLM {
public:
    DecoderLM(std::shared_ptr<nn::Embedding> embedding, std::shared_ptr<nn::TransformerDecoder> decoder,
              std::shared_ptr<nn::Linear> head);
    ~DecoderLM();

    /// Logits [B, V] of the last position after feeding ids [B, L].
    Tensor logits(const Tensor& ids, std::span<nn::KVCache> cache);
    /// Prompt then `steps` sampled tokens; returns tokens [B, steps] and the last logits [B, V].
    std::pair<Tensor, Tensor> generate(const Tensor& prompt, std::span<nn::KVCache> cache, Index steps,
                                       double temperature, RandomKey key, bool use_graph);
    std::vector<KernelTiming> profile(const Tensor& ids, std::span<nn::KVCache> cache, Index rounds);
    /// Whether batched decode (3 to 64 rows) reads a second, repacked copy of every bf16 weight (on by default:
    /// faster, at the cost of that copy's memory).  Turning it off drops the copies now held.
    void set_weight_repack(bool enabled);
    /// Prompt, then warmup + timed single-token steps; the last `timed` steps are bracketed by HIP events on
    /// the compute stream (after a synchronize) and their device time is returned in milliseconds.
    double benchmark(const Tensor& prompt, std::span<nn::KVCache> cache, Index warmup, Index timed,
                     double temperature, RandomKey key, bool use_graph, Tensor* tokens);

private:
    struct StepBuffers;
    void check_caches(std::span<nn::KVCache> cache, Index batch, Index length) const;
    /// Feeds B*L ids already on the device (ids == nullptr: the input rows were already gathered into x_ by
    /// the previous step's sampler); writes logits of the last position and, when sample_mode > 0, samples
    /// into the token / next-id buffers (key label = device step counter) and gathers the next input rows.
    void forward_chunk(const Index* ids, Index batch, Index length, std::span<nn::KVCache> cache, int sample_mode,
                       double temperature, RandomKey key, bool capacity_splits, LaunchObserver* observer);
    void release_graph();
    struct RunResult {
        Tensor tokens, logits;
        double timed_ms = 0.0;
    };
    RunResult run(const Tensor& prompt, std::span<nn::KVCache> cache, Index steps, double temperature, RandomKey key,
                  bool use_graph, Index timed);

    std::shared_ptr<nn::Embedding> embedding_;
    std::shared_ptr<nn::TransformerDecoder> decoder_;
    std::shared_ptr<nn::Linear> head_;
    GpuContext* context_;
    DecodeWorkspace ws_;
    Tensor x_, logits_, partial_, step_, next_ids_, tokens_;
    Index x_rows_ = 0, batch_ = 0, token_columns_ = 0;
    int blocks_ = 0;
    dlh_graph graph_ = nullptr;
    Index graph_batch_ = 0;
    const void* graph_cache_key_ = nullptr;
    std::uint64_t graph_signature_ = 0;
};

} // namespace dl::detail
