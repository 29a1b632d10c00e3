// The fused per-layer decode step shared by TransformerDecoderLayer::decode, TransformerDecoder::decode and the
// on-device token loop.  One layer is five launches: QKV projection (RMSNorm prologue, RoPE + KV-append
// epilogue), split-K attention (+ combine), output projection (+ residual, advances the device length),
// gate/up projection (RMSNorm prologue, SiLU*up epilogue), down projection (+ residual).
#pragma once

#include "nn/ops_internal.h"

namespace dl::detail {

/// Scratch of one decode chunk of `rows` = B * L activation rows.
struct DecodeWorkspace {
    Index rows = 0, splits_capacity = 0;
    Tensor q, attention, hidden, activation, partial_o, partial_ml, lora_query, lora_value, counters;
    /// Zeroed i32 split-merge counters for the attention kernel (at least `count`).
    int* merge_counters(Index count, Device device, GpuContext& context);
    void ensure(const nn::TransformerDecoderLayer& layer, Index rows, Index heads_total, Index hidden_features,
                int splits, Device device);
};

/// Per-launch timing hook (profiling); called with a kernel-class name and the algorithmic bytes before and
/// after each launch.  Null in normal operation.
struct LaunchObserver {
    virtual ~LaunchObserver() = default;
    virtual void before(const char* name, double bytes) = 0;
    virtual void after() = 0;
};

/// Runs one layer on x_in [B*L, d] f32 (device) and writes x_out (may alias x_in).  The cache must be
/// reserved; its device length is advanced by L on the device, and on the host by the caller.
/// `splits`/`chunk` choose the attention key split (attention_split for eager calls).
void decode_layer(const nn::TransformerDecoderLayer& layer, const float* x_in, float* x_out, Index batch, Index length,
                  nn::KVCache& cache, DecodeWorkspace& ws, int splits, int chunk, GpuContext& context,
                  LaunchObserver* observer = nullptr);

/// The KV storage dtype the fused path uses for a layer: bf16 when the projections are bf16, else f32.
DType cache_dtype(const nn::TransformerDecoderLayer& layer);

} // namespace dl::detail
