#pragma once
// Free functions on the decode path.  Mirrors include/dl/ops.h:100-101,149-158,191,341 of the reference
// (argmax, rotary_embedding, grouped_query_attention, linear, embedding, rms_norm); `sample` has no
// reference counterpart (the reference samples on the host, examples/text_generate.cpp:29-41).
// All arithmetic runs on the GPU; bf16 storage computes and returns f32.

#include "dl/random.h"

namespace dl {

/// Index of the first maximum along `axis` (a NaN wins, first NaN first).  Result is i64.
DL_API Tensor argmax(const Tensor& input, Index axis, KeepDim keep = KeepDim::no);
/// Rotates interleaved pairs (2i, 2i+1) of the last axis by cosine/sine [L, D/2] (broadcast over leading
/// axes, L = input.size(-2)).
DL_API Tensor rotary_embedding(const Tensor& input, const Tensor& cosine, const Tensor& sine);
/// Q [B,H,L,D], K [B,KV,S,D], V [B,KV,S,D]; query head h reads KV head h / (H/KV).  With no mask every query
/// row sees all S keys, as in the reference (src/ops/attention.cpp:161-164: no causal window); the decoder's
/// causal rule is applied by its own layers.  An explicit keep mask (reference include/dl/ops.h:149-153,
/// src/ops/attention.cpp:48-50,156-183) is a bool tensor broadcast to [B,H,L,S] by the trailing-axis rule: a
/// false entry drops that key from that row's softmax (its score becomes -inf), and a row that keeps no key
/// comes out NaN, as the reference's softmax of an all -inf row does.  Masked calls take the general kernels.
DL_API Tensor grouped_query_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                                      std::optional<Tensor> keep_mask = std::nullopt);
/// input [..., in] times weight [out, in]^T (+ bias [out]).
DL_API Tensor linear(const Tensor& input, const Tensor& weight, std::optional<Tensor> bias = std::nullopt);
/// Row gather of weight [V, D] by i64 indices of any shape; the weight dtype is preserved.
DL_API Tensor embedding(const Tensor& indices, const Tensor& weight);
/// x / sqrt(mean(x*x) + epsilon) * weight over the trailing `normalized_shape`.
DL_API Tensor rms_norm(const Tensor& input, const Shape& normalized_shape,
                       std::optional<Tensor> weight = std::nullopt, std::optional<double> epsilon = std::nullopt);
/// Draws one index per row of logits [B, V]: temperature <= 0 is argmax; otherwise Gumbel-max,
/// argmax_i(logit_i / T + g_i) with g = -log(-log u), u from Philox(key, b*V + i) on (0, 1).
DL_API Tensor sample(const Tensor& logits, double temperature, RandomKey key);

} // namespace dl
