#pragma once
// Decoder stack and KV cache.  Mirrors include/dl/decoder.h:7-107 of the reference (SwiGLU, LoRALinear,
// RotaryEmbedding, KVCache, GroupedQueryAttention, TransformerDecoderLayer, TransformerDecoder) with the same
// constructor arguments, state names and decode semantics.  Additive extensions, each documented where it
// is declared: a RoPE base for the attention/decoder (the reference hard-codes 10000), unmerged LoRA
// adapters attached to the query/value projections, and an opt-in bf16 KV storage dtype (the default, as in the
// reference, stores K/V in the f32 dtype the projections produce).

#include "dl/nn.h"

#include <span>

namespace dl::nn {

class DL_API SwiGLU : public UnaryModule {
public:
    SwiGLU(Index dimensions, Index hidden, bool bias = false, TensorOptions options = {});
    Tensor forward(const Tensor& input) override;
    const Linear& gate() const { return *gate_; }
    const Linear& up() const { return *up_; }
    const Linear& down() const { return *down_; }

private:
    std::shared_ptr<Linear> gate_, up_, down_;
};

/// Frozen copy of a base Linear plus alpha/rank * up(down(x)); up starts at zero.  merged() returns an
/// independent Linear with W + (alpha/rank) * up.weight @ down.weight rounded to W's dtype.
class DL_API LoRALinear : public UnaryModule {
public:
    LoRALinear(const Linear& base, Index rank, double alpha = 1.0);
    Tensor forward(const Tensor& input) override;
    std::shared_ptr<Linear> merged() const;
    const Linear& down() const { return *down_; }
    const Linear& up() const { return *up_; }
    double scale() const { return scale_; }

private:
    Tensor weight_;
    std::optional<Tensor> bias_;
    double scale_;
    std::shared_ptr<Linear> down_, up_;
};

/// Unmerged low-rank adapter on a projection owned elsewhere (extension: the reference cannot attach
/// LoRALinear to GroupedQueryAttention, whose projections are plain Linear members).  Adds
/// scale * up(down(x)) with scale = alpha / rank; `up` starts at zero.
class DL_API LoRAAdapter : public Module {
public:
    LoRAAdapter(Index input_features, Index output_features, Index rank, double alpha, TensorOptions options = {});
    const Linear& down() const { return *down_; }
    const Linear& up() const { return *up_; }
    Index rank() const { return rank_; }
    double scale() const { return scale_; }

private:
    Index rank_;
    double scale_;
    std::shared_ptr<Linear> down_, up_;
};

/// Frequencies base^(-2i/dimensions); rotates adjacent feature pairs; the f32 angle tables are buffers.
class DL_API RotaryEmbedding : public UnaryModule {
public:
    RotaryEmbedding(Index dimensions, Index capacity, double base = 10000.0, TensorOptions options = {});
    Tensor forward(const Tensor& input) override { return forward(input, 0); }
    Tensor forward(const Tensor& input, Index offset);
    const Tensor& cosine() const { return cosine_; }
    const Tensor& sine() const { return sine_; }

private:
    Tensor cosine_, sine_;
};

/// Per-request K/V store appended along the second-to-last axis.  Storage [B, KV, capacity, D] is allocated
/// once by the first append (which also fixes the other dimensions, dtype and device: a later append of another
/// shape, dtype or device throws); clear/truncate reuse it and key()/value() are views of it.  On the GPU the
/// cache also keeps its length in device memory so that a captured token step reads the current position
/// without host arguments.
class DL_API KVCache {
public:
    explicit KVCache(Index capacity);
    KVCache(const KVCache&) = delete;
    KVCache& operator=(const KVCache&) = delete;
    KVCache(KVCache&&) = default;
    KVCache& operator=(KVCache&&) = default;
    void append(const Tensor& key, const Tensor& value);
    Tensor key() const;
    Tensor value() const;
    Index length() const { return length_; }
    Index capacity() const { return capacity_; }
    void clear();
    void truncate(Index length);

    /// Allocates [batch, heads, capacity, head_dim] storage of `dtype` on `device` if absent (a no-op when
    /// the same layout already exists; throws if it differs).  Used by the fused decode path.
    void reserve(Index batch, Index heads, Index head_dim, DType dtype, Device device);
    /// Throws std::invalid_argument unless reserve() with these arguments would succeed: no storage yet, or
    /// key and value storage both of exactly this layout.  Allocates nothing; the fused paths call it for every
    /// layer before their first launch.
    void check_layout(Index batch, Index heads, Index head_dim, DType dtype, Device device) const;
    bool reserved() const { return key_.has_value(); }
    /// Device pointers for kernels (valid after reserve on a GPU).
    void* key_data() const;
    void* value_data() const;
    std::int64_t* position_data() const;
    /// Host bookkeeping after a device kernel appended `count` positions and advanced the device length.
    void advance(Index count) { length_ += count; }

private:
    void sync_position() const;
    Index capacity_, length_ = 0;
    std::optional<Tensor> key_, value_;
    std::optional<Tensor> position_; // i64[1] on the cache's GPU
};

/// Causal self-attention with grouped K/V heads, bias-free projections and RoPE.
class DL_API GroupedQueryAttention : public UnaryModule {
public:
    GroupedQueryAttention(Index dimensions, Index heads, Index kv_heads, Index context, TensorOptions options = {},
                          double rope_base = 10000.0);
    Tensor forward(const Tensor& input) override;
    /// Computes only the new tokens; the offset is cache.length(); no gradients are recorded.
    Tensor decode(const Tensor& input, KVCache& cache);

    /// Extension: attaches unmerged rank-`rank` adapters to the query and/or value projection.
    void attach_lora(Index rank, double alpha, bool query = true, bool value = true);
    /// Extension: the dtype of the K/V storage this module's decode reserves.  The default is f32, the dtype of
    /// the projections' output, which the reference's cache takes from its first append
    /// (src/nn/kv_cache.cpp:16-21); bf16 halves the cache bytes of long-context decode at the cost of rounding
    /// every stored key and value.  Set it before the first decode into a cache.
    void set_cache_dtype(DType dtype);
    DType cache_dtype() const { return cache_dtype_; }

    Index dimensions() const { return dimensions_; }
    Index heads() const { return heads_; }
    Index kv_heads() const { return kv_heads_; }
    Index head_dim() const { return dimensions_ / heads_; }
    const Linear& query() const { return *query_; }
    const Linear& key() const { return *key_; }
    const Linear& value() const { return *value_; }
    const Linear& output() const { return *output_; }
    const RotaryEmbedding& rotary() const { return *rotary_; }
    const LoRAAdapter* query_adapter() const { return query_adapter_.get(); }
    const LoRAAdapter* value_adapter() const { return value_adapter_.get(); }

private:
    Tensor run(const Tensor& input, KVCache* cache);
    Index dimensions_, heads_, kv_heads_;
    DType cache_dtype_ = DType::f32;
    std::shared_ptr<Linear> query_, key_, value_, output_;
    std::shared_ptr<RotaryEmbedding> rotary_;
    std::shared_ptr<LoRAAdapter> query_adapter_, value_adapter_;
    friend class TransformerDecoderLayer;
};

/// Pre-norm layer: RMSNorm, causal GQA, SwiGLU, two residual additions.
class DL_API TransformerDecoderLayer : public UnaryModule {
public:
    static constexpr double norm_epsilon = 1e-5;
    TransformerDecoderLayer(Index dimensions, Index heads, Index kv_heads, Index hidden, Index context,
                            TensorOptions options = {}, double rope_base = 10000.0);
    Tensor forward(const Tensor& input) override;
    Tensor decode(const Tensor& input, KVCache& cache);

    GroupedQueryAttention& attention() { return *attention_; }
    const GroupedQueryAttention& attention() const { return *attention_; }
    const SwiGLU& feedforward() const { return *feedforward_; }
    const RMSNorm& attention_norm() const { return *attention_norm_; }
    const RMSNorm& feedforward_norm() const { return *feedforward_norm_; }

private:
    std::shared_ptr<GroupedQueryAttention> attention_;
    std::shared_ptr<SwiGLU> feedforward_;
    std::shared_ptr<RMSNorm> attention_norm_, feedforward_norm_;
};

/// Input and output [batch, length, dimensions]; a final RMSNorm normalises the stack.  Each request makes
/// its caches with make_cache; all layers advance by the same token chunk, and a failed chunk leaves every
/// cache at the prefix it started from.
class DL_API TransformerDecoder : public UnaryModule {
public:
    TransformerDecoder(Index layers, Index dimensions, Index heads, Index kv_heads, Index hidden, Index context,
                       TensorOptions options = {}, double rope_base = 10000.0);
    Tensor forward(const Tensor& input) override;
    std::vector<KVCache> make_cache() const;
    Index layer_count() const { return static_cast<Index>(layers_.size()); }
    Tensor decode(const Tensor& input, std::span<KVCache> cache);

    /// Extension: attaches unmerged adapters to every layer's query/value projections.
    void attach_lora(Index rank, double alpha, bool query = true, bool value = true);
    /// Extension: every layer's K/V storage dtype (GroupedQueryAttention::set_cache_dtype): f32 by default,
    /// bf16 as an opt-in for long-context decode.
    void set_cache_dtype(DType dtype);
    DType cache_dtype() const;

    Index context() const { return context_; }
    TransformerDecoderLayer& layer(Index i) { return *layers_.at(static_cast<std::size_t>(i)); }
    const TransformerDecoderLayer& layer(Index i) const { return *layers_.at(static_cast<std::size_t>(i)); }
    const RMSNorm& normalization() const { return *normalization_; }

private:
    Index context_;
    std::vector<std::shared_ptr<TransformerDecoderLayer>> layers_;
    std::shared_ptr<RMSNorm> normalization_;
};

} // namespace dl::nn
