// Decode-path operators on GPU tensors (reference include/dl/ops.h:100-101,149-158,191,341 and their
// numeric layer, src/ops/numeric.cpp:178-226,252-254).  Low-precision inputs compute and return f32.
#include "nn/ops_internal.h"

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <stdexcept>

namespace dl::detail {

GpuContext& gpu_of(const Tensor& t, const char* operation) {
    require_gpu(t.device(), operation);
    return gpu_context(t.device().index);
}

Tensor contiguous_f32(const Tensor& t) {
    if (t.dtype() == DType::f32 && t.is_contiguous()) return t;
    Tensor out = empty_tensor(t.shape(), DType::f32, t.device());
    copy_into(out, t);
    return out;
}

const void* weight_data(const Tensor& w, int& is_bf16, const char* operation) {
    if (w.dtype() != DType::bf16 && w.dtype() != DType::f32)
        throw std::invalid_argument(std::string(operation) + ": weights must be bf16 or f32");
    if (!w.is_contiguous()) throw std::invalid_argument(std::string(operation) + ": weights must be contiguous");
    is_bf16 = w.dtype() == DType::bf16;
    return w.data<void>();
}

dlk_gemv_params gemv_params(const float* x, Index rows, Index k, int epilogue) {
    dlk_gemv_params p{};
    p.x = x;
    p.ldx = k;
    p.M = static_cast<int>(rows);
    p.K = static_cast<int>(k);
    p.epilogue = epilogue;
    p.epsilon = 1e-5f;
    p.acc_scale = 1.0f;
    p.length = 1;
    return p;
}

void linear_into(const float* x, Index rows, Index k, const Tensor& weight, const std::optional<Tensor>& bias,
                 float* y, Index ldy, GpuContext& context) {
    if (weight.ndim() != 2 || weight.size(1) != k)
        throw std::invalid_argument("linear: weight must be [out, " + std::to_string(k) + "], got " +
                                    shape_string(weight.shape()));
    int wb = 0;
    const void* w = weight_data(weight, wb, "linear");
    const Index n = weight.size(0);
    if (bias && (bias->ndim() != 1 || bias->size(0) != n)) throw std::invalid_argument("linear: bias must be [out]");
    const int chunk = wb ? 8 : 4;
    if (rows == 0 || n == 0) return;
    const bool aligned = reinterpret_cast<std::uintptr_t>(x) % 16 == 0 && reinterpret_cast<std::uintptr_t>(w) % 16 == 0;
    if (k % chunk != 0 || ldy != n || !aligned) {
        hip_check(dlk_linear_generic(x, rows, k, w, wb ? DLK_BF16 : DLK_F32, n, bias ? bias->data<void>() : nullptr,
                                     bias ? dlk_dtype(bias->dtype()) : DLK_F32, y, context.stream),
                  "linear");
        return;
    }
    dlk_gemv_params p = gemv_params(x, rows, k, DLK_EPI_STORE);
    p.nseg = 1;
    p.w[0] = w;
    p.seg_rows[0] = static_cast<int>(n);
    p.w_bf16 = wb;
    p.y = y;
    p.ldy = ldy;
    if (bias) {
        const Tensor b = bias->is_contiguous() ? *bias : bias->contiguous();
        if (b.dtype() != DType::f32 && b.dtype() != DType::bf16) throw std::invalid_argument("linear: bias dtype");
        p.bias = b.data<void>();
        p.bias_bf16 = b.dtype() == DType::bf16;
        hip_check(dlk_gemv(&p, context.stream), "linear");
        return;
    }
    hip_check(dlk_gemv(&p, context.stream), "linear");
}

void attention_split(Index batch, Index heads, Index kv_heads, Index head_dim, bool kv_bf16, Index length,
                     Index source, int& splits, int& chunk) {
    constexpr Index tile = 64;
    const bool matrix = dlk_attention_matrix_heads(static_cast<int>(heads), static_cast<int>(kv_heads),
                                                   static_cast<int>(head_dim)) != 0;
    if (length == 1 && matrix && (batch * kv_heads * source >= DLK_STREAM_DECODE_KEYS || !kv_bf16)) {
        // many keys in all, or an f32 cache: each wave of the matrix-core kernel streams its run of keys (four
        // waves per work-group when the keys split).  With 256 or more (sequence, KV head) pairs there is a
        // work-group per pair already, so each takes all of its keys (no partials, no combine launch: C3); an
        // f32 cache of at most 512 keys stays in one work-group per pair (C2: eight waves); otherwise runs of
        // 64..256 keys per wave, about total / 1024 keys (measured on MI355X at b=4 over 4100 keys: bf16 14.6 us
        // per layer at 192 keys per wave against 15.8 at 64 and 256; f32 19.8 us at 192 against 22.9 at 256 and
        // 25.8 at 128; C4 keeps 256)
        const Index total = batch * kv_heads * source;
        if (batch * kv_heads >= 256) {
            chunk = static_cast<int>(4 * (((source + 3) / 4 + 63) / 64 * 64));
        } else if (!kv_bf16 && source <= DLK_DECODE_CHUNK_MAX) {
            chunk = DLK_DECODE_CHUNK_MAX;
        } else {
            const Index per_run = 1024;
            chunk = static_cast<int>(4 * std::clamp<Index>(((total + per_run - 1) / per_run + 63) / 64 * 64, 64, 256));
        }
        splits = static_cast<int>((source + chunk - 1) / chunk);
        return;
    }
    if (length == 1) {
        // one new position over few keys: one work-group of 256 or 512 keys (the matrix-core kernel; the general
        // kernel for other head layouts takes up to 1024), split only beyond it (the split partials take a
        // second, combine launch)
        const Index widest = matrix ? DLK_DECODE_CHUNK_MAX : 16 * tile;
        Index per = 4 * tile;
        while (per < source && per < widest) per *= 2;
        chunk = static_cast<int>(per);
        splits = static_cast<int>(std::max<Index>(1, (source + per - 1) / per));
        return;
    }
    const Index groups = batch * kv_heads;
    const Index tiles = std::max<Index>(1, (source + tile - 1) / tile);
    Index wanted = 1;
    // decode: enough key splits for ~2 work-groups per CU slot of a 256-CU chip; prefill rows already spread
    if (length <= 4) wanted = std::max<Index>(1, (1024 + groups - 1) / groups);
    wanted = std::min(wanted, tiles);
    const Index per = (tiles + wanted - 1) / wanted;
    splits = static_cast<int>((tiles + per - 1) / per);
    chunk = static_cast<int>(per * tile);
}

} // namespace dl::detail

namespace dl {

using namespace detail;

Tensor linear(const Tensor& input, const Tensor& weight, std::optional<Tensor> bias) {
    GpuContext& context = gpu_of(input, "linear");
    if (!(weight.device() == input.device())) throw std::invalid_argument("linear: weight on another device");
    const Index k = input.size(-1);
    const Index n = weight.size(0);
    Tensor x = contiguous_f32(input);
    const Index rows = k == 0 ? 0 : x.numel() / k;
    Shape out_shape = input.shape();
    out_shape.back() = n;
    Tensor y = empty_tensor(out_shape, DType::f32, input.device());
    linear_into(x.data<float>(), rows, k, weight, bias, static_cast<float*>(mutable_data(y)), n, context);
    return y;
}

Tensor embedding(const Tensor& indices, const Tensor& weight) {
    GpuContext& context = gpu_of(weight, "embedding");
    if (weight.ndim() != 2) throw std::invalid_argument("embedding: weight must be [V, D]");
    if (indices.dtype() != DType::i64) throw std::invalid_argument("embedding: indices must be i64");
    Tensor ids = indices.to(weight.device()).contiguous();
    Tensor w = weight.contiguous();
    Shape out_shape = indices.shape();
    out_shape.push_back(weight.size(1));
    Tensor out = empty_tensor(out_shape, weight.dtype(), weight.device());
    hip_check(dlk_embedding(ids.data<Index>(), ids.numel(), w.data<void>(), dlk_dtype(w.dtype()), w.size(0), w.size(1),
                            mutable_data(out), dlk_dtype(out.dtype()), context.error_flag, context.stream),
              "embedding");
    return out;
}

Tensor rms_norm(const Tensor& input, const Shape& normalized_shape, std::optional<Tensor> weight,
                std::optional<double> epsilon) {
    GpuContext& context = gpu_of(input, "rms_norm");
    Index width = 1;
    for (Index s : normalized_shape) width *= s;
    if (input.ndim() < static_cast<Index>(normalized_shape.size())) throw std::invalid_argument("rms_norm: rank");
    for (std::size_t i = 0; i < normalized_shape.size(); ++i)
        if (input.shape()[input.shape().size() - normalized_shape.size() + i] != normalized_shape[i])
            throw std::invalid_argument("rms_norm: trailing shape differs from normalized_shape");
    Tensor x = contiguous_f32(input);
    Tensor y = empty_tensor(input.shape(), DType::f32, input.device());
    const void* w = nullptr;
    int wb = 0;
    Tensor wc;
    if (weight) {
        wc = weight->contiguous();
        if (wc.numel() != width) throw std::invalid_argument("rms_norm: weight size");
        if (wc.dtype() != DType::f32 && wc.dtype() != DType::bf16) wc = wc.astype(DType::f32);
        w = wc.data<void>();
        wb = wc.dtype() == DType::bf16;
    }
    // the default epsilon is the f32 machine epsilon of the accumulation dtype (reference ops.h:338-341)
    const double eps = epsilon ? *epsilon : static_cast<double>(std::numeric_limits<float>::epsilon());
    const Index rows = width == 0 ? 0 : x.numel() / width;
    hip_check(dlk_rms_norm(x.data<float>(), rows, width, w, wb, static_cast<float>(eps),
                           static_cast<float*>(mutable_data(y)), context.stream),
              "rms_norm");
    return y;
}

Tensor rotary_embedding(const Tensor& input, const Tensor& cosine, const Tensor& sine) {
    GpuContext& context = gpu_of(input, "rotary_embedding");
    if (input.ndim() < 2) throw std::invalid_argument("rotary_embedding: input needs [..., L, D]");
    const Index length = input.size(-2), dim = input.size(-1);
    if (dim % 2 != 0) throw std::invalid_argument("rotary_embedding: D must be even");
    if (cosine.numel() != length * (dim / 2) || sine.numel() != length * (dim / 2))
        throw std::invalid_argument("rotary_embedding: tables must be [L, D/2]");
    Tensor x = contiguous_f32(input);
    Tensor c = contiguous_f32(cosine.to(input.device())), s = contiguous_f32(sine.to(input.device()));
    Tensor y = empty_tensor(input.shape(), DType::f32, input.device());
    const Index outer = length * dim == 0 ? 0 : x.numel() / (length * dim);
    hip_check(dlk_rope(x.data<float>(), outer, length, dim, c.data<float>(), s.data<float>(),
                       static_cast<float*>(mutable_data(y)), context.stream),
              "rotary_embedding");
    return y;
}

Tensor grouped_query_attention(const Tensor& query, const Tensor& key, const Tensor& value,
                               std::optional<Tensor> keep_mask) {
    GpuContext& context = gpu_of(query, "grouped_query_attention");
    if (query.ndim() != 4 || key.ndim() != 4 || value.ndim() != 4)
        throw std::invalid_argument("grouped_query_attention: expects [B,H,L,D] and [B,KV,S,D]");
    const Index B = query.size(0), H = query.size(1), L = query.size(2), D = query.size(3);
    const Index KV = key.size(1), S = key.size(2);
    if (key.shape() != value.shape() || key.size(0) != B || key.size(3) != D || KV <= 0 || H % KV != 0)
        throw std::invalid_argument("grouped_query_attention: shapes differ or H is not a multiple of KV");
    if (D != 2 && D != 4 && D != 8 && D != 16 && D != 32 && D != 64 && D != 128)
        throw std::invalid_argument("grouped_query_attention: head size 2, 4, 8, 16, 32, 64 or 128");
    Tensor q = contiguous_f32(query.transpose(1, 2)); // [B, L, H, D] = rows (b, l)
    const DType kv_dtype = key.dtype() == DType::bf16 && value.dtype() == DType::bf16 ? DType::bf16 : DType::f32;
    Tensor k = key.dtype() == kv_dtype && key.is_contiguous() ? key : key.astype(kv_dtype).contiguous();
    Tensor v = value.dtype() == kv_dtype && value.is_contiguous() ? value : value.astype(kv_dtype).contiguous();
    Tensor out = empty_tensor({B, L, H, D}, DType::f32, query.device());
    dlk_attention_params p{};
    p.q = q.data<float>();
    p.ldq = H * D;
    p.k = k.data<void>();
    p.v = v.data<void>();
    p.kv_bf16 = kv_dtype == DType::bf16;
    p.capacity = S;
    p.first_host = S - L; // unused: no causal window without a mask
    p.early_keys = S;
    p.B = static_cast<int>(B); p.L = static_cast<int>(L); p.H = static_cast<int>(H); p.KV = static_cast<int>(KV);
    p.hd = static_cast<int>(D);
    p.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
    p.causal = 0;
    p.out = static_cast<float*>(mutable_data(out));
    p.ldo = H * D;
    if (S < L) throw std::invalid_argument("grouped_query_attention: needs S >= L");
    // The keep mask, as the reference applies it (src/ops/attention.cpp:48-50,80,156-183): a bool tensor that
    // broadcasts to [B, H, L, S] by the trailing-axis rule; the kernels read it in place through its strides
    // (0 on the broadcast axes), on the query's device
    Tensor mask;
    if (keep_mask) {
        if (keep_mask->dtype() != DType::boolean)
            throw std::invalid_argument("grouped_query_attention: keep mask must be bool");
        mask = keep_mask->device() == query.device() ? *keep_mask : keep_mask->to(query.device());
        const Shape want{B, H, L, S};
        const Index rank = mask.ndim();
        for (Index axis = 0; axis + 4 < rank; ++axis)
            if (mask.size(axis) != 1)
                throw std::invalid_argument("grouped_query_attention: keep mask " + shape_string(mask.shape()) +
                                            " does not broadcast to " + shape_string(want));
        for (int axis = 0; axis < 4; ++axis) {
            const Index from = rank - 4 + axis; // the mask axis aligned with output axis `axis`, if any
            const Index size = from >= 0 ? mask.size(from) : 1;
            if (size != 1 && size != want[axis])
                throw std::invalid_argument("grouped_query_attention: keep mask " + shape_string(mask.shape()) +
                                            " does not broadcast to " + shape_string(want));
            p.mask_stride[axis] = size == 1 ? 0 : mask.strides()[static_cast<std::size_t>(from)];
        }
        p.keep_mask = static_cast<const unsigned char*>(mask.data<void>());
    }
    attention_split(B, H, KV, D, kv_dtype == DType::bf16, L, S, p.splits, p.chunk);
    Tensor po, pml;
    if (p.splits > 1) {
        po = empty_tensor({B * H * L, p.splits, D}, DType::f32, query.device());
        pml = empty_tensor({B * H * L, p.splits, 2}, DType::f32, query.device());
        p.partial_o = static_cast<float*>(mutable_data(po));
        p.partial_ml = static_cast<float*>(mutable_data(pml));
    }
    hip_check(dlk_attention(&p, context.stream), "grouped_query_attention");
    return out.transpose(1, 2);
}

Tensor argmax(const Tensor& input, Index axis, KeepDim keep) {
    GpuContext& context = gpu_of(input, "argmax");
    const Index rank = input.ndim();
    const Index a = axis < 0 ? axis + rank : axis;
    if (a < 0 || a >= rank) throw std::out_of_range("argmax axis out of range");
    if (input.size(a) == 0) throw std::invalid_argument("argmax over an empty axis");
    Tensor moved = a == rank - 1 ? input : input.transpose(a, rank - 1);
    Tensor x = contiguous_f32(moved);
    const Index n = x.size(-1), rows = x.numel() / n;
    Shape out_shape = moved.shape();
    out_shape.pop_back();
    Tensor out = empty_tensor(out_shape, DType::i64, input.device());
    hip_check(dlk_argmax(x.data<float>(), rows, n, static_cast<Index*>(mutable_data(out)), context.stream), "argmax");
    if (a != rank - 1 && rank > 1) {
        // undo the axis move: the reduced axis was last; the moved-in axis sits at position a
        Tensor fixed = out;
        if (a < rank - 1) {
            // out axes: [.. a-1, (rank-1 moved to a), a+1 .. rank-2]; move axis a back to the end
            for (Index i = a; i < rank - 2; ++i) fixed = fixed.transpose(i, i + 1);
        }
        out = fixed.contiguous();
    }
    if (keep == KeepDim::yes) out = out.unsqueeze(a);
    return out;
}

Tensor sample(const Tensor& logits, double temperature, RandomKey key) {
    GpuContext& context = gpu_of(logits, "sample");
    if (logits.ndim() != 2) throw std::invalid_argument("sample: logits must be [B, V]");
    Tensor x = contiguous_f32(logits);
    const Index rows = x.size(0), n = x.size(1);
    if (n == 0) throw std::invalid_argument("sample: empty vocabulary");
    const int blocks = dlk_sample_blocks(n);
    Tensor partial = empty_tensor({rows * blocks * 2}, DType::i64, logits.device());
    Tensor out = empty_tensor({rows}, DType::i64, logits.device());
    const int mode = temperature > 0.0 ? 2 : 1;
    auto* parts = static_cast<dlk_sample_partial*>(mutable_data(partial));
    hip_check(dlk_sample_partials(x.data<float>(), rows, n, mode, temperature, key.seed, key.stream, nullptr, parts,
                                  blocks, context.stream),
              "sample");
    hip_check(dlk_sample_finalize(parts, rows, blocks, static_cast<Index*>(mutable_data(out)), nullptr, nullptr, 0,
                                  nullptr, nullptr, 0, 0, nullptr, context.stream),
              "sample");
    return out;
}

} // namespace dl
