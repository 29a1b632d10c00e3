// The fused per-layer decode step shared by TransformerDecoderLayer::decode, TransformerDecoder::decode and the
// on-device token loop.  One layer is five launches: QKV projection (RMSNorm prologue, RoPE + KV-append
// epilogue), attention (+ a combine launch when the keys are split), output projection (+ residual, advances the device length),
// gate/up projection (RMSNorm prologue, SiLU*up epilogue), down projection (+ residual).
#pragma once

#include "nn/ops_internal.h"

#include <cstdint>
#include <functional>
#include <map>
#include <tuple>
#include <utility>

namespace dl::detail {

/// Scratch of one decode chunk of `rows` = B * L activation rows.
struct DecodeWorkspace {
    Index rows = 0, splits_capacity = 0;
    Tensor q, attention, hidden, activation, partial_o, partial_ml;
    Tensor lora; ///< LoRA hidden rows [rows, rank_q + rank_v]: the query adapter's, then the value adapter's
    Tensor split; ///< key-split partials of the matrix-core projections (shared: launches are stream-ordered)
    Tensor stage_ffn; ///< prefill: the SwiGLU rows already split for the down projection's tiled path
    Tensor stage_attn; ///< prefill: the attention rows already split for the output projection's tiled path
    Tensor stage; ///< prefill projections: activation rows split into bf16 hi + lo, per-row norm factors
    Tensor kv_split; ///< prefill attention over an f32 cache: the K/V tiles split into bf16 hi + lo planes
    /// Points `p` at the staging workspace when its shape takes the tiled prefill path and at the split
    /// workspace when its launch would split the keys (both grown as needed).
    void attach_workspace(dlk_gemv_params& p, Device device);
    void ensure(const nn::TransformerDecoderLayer& layer, Index rows, Index heads_total, Index hidden_features,
                int splits, Device device);

    /// Batched decode: bf16 projection weights repacked in the matrix-core kernel's tile order (dlk_pack_tiles),
    /// so that each of its weight loads reads 1 KB contiguous.  Off unless set (it costs a second copy of every
    /// packed weight in HBM); a weight is packed on the first eager launch that takes that kernel, and the packs
    /// are dropped when the parameter epoch moves (weights loaded or moved).
    bool pack_weights = false;
    /// The packed tiles of `w0` [rows, K] (with `w1`: gate and up, interleaved for the SwiGLU launch), or null
    /// (packing off, not bf16, a shape the pack does not cover, or no current pack while `stream` captures).
    const void* tiles_of(const Tensor& w0, const Tensor* w1, dlh_stream stream);
    /// Drops every packed copy (their memory returns to the pool once no launch uses it).
    void release_packs() { packed_.clear(); }

private:
    struct Packed {
        Tensor source, second, tiles; // the sources keep the weights' storage (the key) alive while the pack exists
    };
    // a pack is found by everything that shapes it: w0's address, rows and K, and w1's address (gate/up), so a
    // view at the same address with another shape, or w0 paired with another w1, makes a pack of its own
    using PackKey = std::tuple<const void*, Index, Index, const void*>;
    std::map<PackKey, Packed> packed_;
    uint64_t packed_epoch_ = 0;
};

/// Launch hook for profiling (null in normal operation).  Every launch of a step is handed over as a closure
/// with its kernel-class name and algorithmic HBM bytes: `fn(false)` issues the step's own launch, `fn(true)`
/// issues the identical launch again without side effects on cache lengths (a timing repeat).
struct LaunchObserver {
    virtual ~LaunchObserver() = default;
    virtual void launch(const char* name, double bytes, std::function<void(bool repeat)> fn) = 0;
};

/// Issues one launch: directly, or through the observer.
template <typename F>
void issue(LaunchObserver* observer, const char* name, double bytes, F&& fn) {
    if (observer) observer->launch(name, bytes, std::function<void(bool)>(std::forward<F>(fn)));
    else fn(false);
}

/// Runs one layer on x_in [B*L, d] f32 (device) and writes x_out (may alias x_in).  The cache must be
/// reserved; its device length is advanced by L on the device, and on the host by the caller.
/// `splits`/`chunk` choose the attention key split (attention_split for eager calls).
void decode_layer(const nn::TransformerDecoderLayer& layer, const float* x_in, float* x_out, Index batch, Index length,
                  nn::KVCache& cache, DecodeWorkspace& ws, int splits, int chunk, GpuContext& context,
                  LaunchObserver* observer = nullptr);

/// The KV storage dtype the fused path reserves for a layer (its attention's cache dtype: f32 unless bf16 was
/// chosen).
DType cache_dtype(const nn::TransformerDecoderLayer& layer);

} // namespace dl::detail
