// Helpers shared by the operator, module and token-loop layers: tensor checks and kernel parameter filling.
#pragma once

#include "core/tensor_impl.h"
#include "dl/decoder.h"

#include <string>

namespace dl::detail {

/// The GPU context of a tensor that must live on a GPU (throws for CPU tensors).
GpuContext& gpu_of(const Tensor& t, const char* operation);
/// A contiguous f32 copy (or the tensor itself when it already is one) on the same device.
Tensor contiguous_f32(const Tensor& t);
/// Weight pointer and dtype flag for the projection kernels; weight must be contiguous bf16 or f32.
const void* weight_data(const Tensor& w, int& is_bf16, const char* operation);
/// Fills the fields common to every projection launch.
dlk_gemv_params gemv_params(const float* x, Index rows, Index k, int epilogue);
/// y[rows, out] = x W^T (+ bias) on the GPU, f32 output rows with leading dimension ldy.
void linear_into(const float* x, Index rows, Index k, const Tensor& weight, const std::optional<Tensor>& bias,
                 float* y, Index ldy, GpuContext& context);

/// Number of key splits and keys per split for attention of `length` new positions over `source` keys.
void attention_split(Index batch, Index heads, Index kv_heads, Index head_dim, bool kv_bf16, Index length,
                     Index source, int& splits, int& chunk);

} // namespace dl::detail
