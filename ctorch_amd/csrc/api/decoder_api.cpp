// Entries of <dl/decoder_c_api.h> (reference src/api/decoder.cpp:4-70).
#include "api/common.h"
#include "core/tensor_impl.h"
#include "nn/decode_step.h"

#include <cmath>

#include <numeric>
#include <stdexcept>

using namespace dl::capi;

namespace {
template <class T> T& as(dl_module* module, const char* what) {
    auto* value = dynamic_cast<T*>(require(module, "module").value.get());
    if (!value) throw std::invalid_argument(std::string("module is not a ") + what);
    return *value;
}
template <class T> const T& as(const dl_module* module, const char* what) {
    auto* value = dynamic_cast<const T*>(require(module, "module").value.get());
    if (!value) throw std::invalid_argument(std::string("module is not a ") + what);
    return *value;
}
std::shared_ptr<dl::nn::UnaryModule> unary(std::shared_ptr<dl::nn::UnaryModule> m) { return m; }

// general contraction over the listed axes: permute both operands so the contracted axes meet, then one
// projection launch computes [rows(a), contracted] x [cols(b), contracted]^T
dl::Tensor tensordot(const dl::Tensor& a, const dl::Tensor& b, const dl::Shape& axes_a, const dl::Shape& axes_b) {
    if (axes_a.size() != axes_b.size()) throw std::invalid_argument("tensordot axis lists differ in length");
    auto norm = [](dl::Index axis, dl::Index rank) { return axis < 0 ? axis + rank : axis; };
    std::vector<bool> used_a(static_cast<std::size_t>(a.ndim()), false), used_b(static_cast<std::size_t>(b.ndim()), false);
    dl::Index k = 1;
    for (std::size_t i = 0; i < axes_a.size(); ++i) {
        const dl::Index ia = norm(axes_a[i], a.ndim()), ib = norm(axes_b[i], b.ndim());
        if (ia < 0 || ia >= a.ndim() || ib < 0 || ib >= b.ndim() || used_a[static_cast<std::size_t>(ia)] ||
            used_b[static_cast<std::size_t>(ib)] || a.size(ia) != b.size(ib))
            throw std::invalid_argument("tensordot axes are invalid or sizes differ");
        used_a[static_cast<std::size_t>(ia)] = used_b[static_cast<std::size_t>(ib)] = true;
        k *= a.size(ia);
    }
    dl::Shape out_shape;
    dl::Index rows = 1, cols = 1;
    // move free axes first (a) / first (b), contracted axes last in the listed order, via copies
    auto arrange = [&](const dl::Tensor& t, const dl::Shape& axes, std::vector<bool>& used, dl::Index& free_count) {
        std::vector<dl::Index> order;
        for (dl::Index i = 0; i < t.ndim(); ++i)
            if (!used[static_cast<std::size_t>(i)]) { order.push_back(i); out_shape.push_back(t.size(i)); free_count *= t.size(i); }
        for (dl::Index axis : axes) order.push_back(norm(axis, t.ndim()));
        // permutation as a strided view, then a contiguous copy
        auto impl = std::make_shared<dl::detail::TensorImpl>(*dl::detail::TensorAccess::impl(t));
        dl::Shape shape, strides;
        for (dl::Index i : order) {
            shape.push_back(t.shape()[static_cast<std::size_t>(i)]);
            strides.push_back(t.strides()[static_cast<std::size_t>(i)]);
        }
        impl->shape = shape;
        impl->strides = strides;
        return dl::detail::contiguous_f32(dl::detail::TensorAccess::make(impl));
    };
    dl::Tensor left = arrange(a, axes_a, used_a, rows);
    dl::Tensor right = arrange(b, axes_b, used_b, cols);
    dl::Tensor y = dl::linear(left.reshape({rows, k}), right.reshape({cols, k}));
    return y.reshape(out_shape);
}
} // namespace

extern "C" {

dl_status dl_tensordot(const dl_tensor* a, const dl_tensor* b, dl_shape axes_a, dl_shape axes_b, dl_tensor** output) {
    return make_handle(output, [&] {
        return tensordot(require(a, "a").value, require(b, "b").value, convert(axes_a), convert(axes_b));
    });
}

dl_status dl_rotary_embedding(const dl_tensor* input, const dl_tensor* cosine, const dl_tensor* sine, dl_tensor** output) {
    return make_handle(output, [&] {
        return dl::rotary_embedding(require(input, "input").value, require(cosine, "cosine").value,
                                    require(sine, "sine").value);
    });
}

dl_status dl_grouped_query_attention(const dl_tensor* query, const dl_tensor* key, const dl_tensor* value,
                                     const dl_tensor* keep_mask, dl_tensor** output) {
    return make_handle(output, [&] {
        return dl::grouped_query_attention(require(query, "query").value, require(key, "key").value,
                                           require(value, "value").value,
                                           keep_mask ? std::optional<dl::Tensor>{keep_mask->value} : std::nullopt);
    });
}

dl_status dl_grouped_query_attention_noalloc(const float* query, const void* key, const void* value, dl_dtype kv_dtype,
                                             int64_t batch, int64_t heads, int64_t kv_heads, int64_t length,
                                             int64_t source, int64_t head_dim, float* output, int32_t device) {
    return invoke([&] {
        if (!query || !key || !value || !output) throw std::invalid_argument("attention pointers must not be NULL");
        if (kv_dtype != DL_F32 && kv_dtype != DL_BF16) throw std::invalid_argument("attention K/V dtype must be f32 or bf16");
        if (batch <= 0 || heads <= 0 || kv_heads <= 0 || length <= 0 || heads % kv_heads != 0)
            throw std::invalid_argument("attention dimensions must be positive and heads a multiple of kv_heads");
        if (source < length) throw std::invalid_argument("attention needs source >= length");
        const int64_t D = head_dim;
        if (D != 2 && D != 4 && D != 8 && D != 16 && D != 32 && D != 64 && D != 128)
            throw std::invalid_argument("attention head size 2, 4, 8, 16, 32, 64 or 128");
        dlk_attention_params p{};
        p.kv_bf16 = kv_dtype == DL_BF16;
        dl::detail::attention_split(batch, heads, kv_heads, D, p.kv_bf16 != 0, length, source, p.splits, p.chunk);
        const int64_t rows = batch * heads * length;
        const int64_t need = p.splits > 1 ? rows * p.splits * (D + 2) : 0;
        if (need > DLK_ATTENTION_SCRATCH_FLOATS)
            throw std::invalid_argument("attention partials need " + std::to_string(need) +
                                        " floats, more than the allocation-free entry's " +
                                        std::to_string(DLK_ATTENTION_SCRATCH_FLOATS) + "-float scratch");
        auto& context = dl::detail::gpu_context(device);
        float* scratch = nullptr;
        dl::detail::hip_check(dlk_attention_scratch(device, &scratch), "attention scratch");
        p.q = query;
        p.ldq = heads * D;
        p.k = key;
        p.v = value;
        p.capacity = source;
        p.first_host = source - length;
        p.early_keys = source;
        p.B = static_cast<int>(batch); p.L = static_cast<int>(length); p.H = static_cast<int>(heads);
        p.KV = static_cast<int>(kv_heads); p.hd = static_cast<int>(D);
        p.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(D)));
        p.causal = 0;
        p.out = output;
        p.ldo = heads * D;
        if (p.splits > 1) {
            // every split writes its (max, sum) pair and, when it holds keys, its partial output row; the merge
            // skips splits without keys, so nothing has to start at zero
            p.partial_o = scratch;
            p.partial_ml = scratch + rows * p.splits * D;
        }
        dl::detail::hip_check(dlk_attention(&p, context.stream), "grouped_query_attention_noalloc");
    });
}

dl_status dl_swiglu_create(int64_t dimensions, int64_t hidden, int32_t bias, dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::SwiGLU>(dimensions, hidden, bias != 0, convert(options)));
    });
}

dl_status dl_lora_linear_create(const dl_module* base, int64_t rank, double alpha, dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::LoRALinear>(as<dl::nn::Linear>(base, "Linear"), rank, alpha));
    });
}

dl_status dl_lora_linear_merge(const dl_module* adapter, dl_module** output) {
    return make_handle(output, [&] { return unary(as<dl::nn::LoRALinear>(adapter, "LoRALinear").merged()); });
}

dl_status dl_rotary_embedding_create(int64_t dimensions, int64_t capacity, double base, dl_tensor_options options,
                                     dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::RotaryEmbedding>(dimensions, capacity, base, convert(options)));
    });
}

dl_status dl_rotary_embedding_forward(dl_module* rotary, const dl_tensor* input, int64_t offset, dl_tensor** output) {
    return make_handle(output, [&] {
        return as<dl::nn::RotaryEmbedding>(rotary, "RotaryEmbedding").forward(require(input, "input").value, offset);
    });
}

dl_status dl_grouped_query_attention_create(int64_t dimensions, int64_t heads, int64_t kv_heads, int64_t context,
                                            dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::GroupedQueryAttention>(dimensions, heads, kv_heads, context, convert(options)));
    });
}

dl_status dl_transformer_decoder_create(int64_t layers, int64_t dimensions, int64_t heads, int64_t kv_heads,
                                        int64_t hidden, int64_t context, dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::TransformerDecoder>(layers, dimensions, heads, kv_heads, hidden, context,
                                                                  convert(options)));
    });
}

dl_status dl_transformer_decoder_create_with_base(int64_t layers, int64_t dimensions, int64_t heads, int64_t kv_heads,
                                                  int64_t hidden, int64_t context, double rope_base,
                                                  dl_tensor_options options, dl_module** output) {
    return make_handle(output, [&] {
        return unary(std::make_shared<dl::nn::TransformerDecoder>(layers, dimensions, heads, kv_heads, hidden, context,
                                                                  convert(options), rope_base));
    });
}

dl_status dl_transformer_decoder_attach_lora(dl_module* decoder, int64_t rank, double alpha, int32_t query,
                                             int32_t value) {
    return invoke([&] {
        as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder").attach_lora(rank, alpha, query != 0, value != 0);
    });
}

dl_status dl_transformer_decoder_set_cache_dtype(dl_module* decoder, dl_dtype dtype) {
    return invoke([&] {
        as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder").set_cache_dtype(static_cast<dl::DType>(dtype));
    });
}

dl_status dl_transformer_decoder_cache_dtype(const dl_module* decoder, dl_dtype* dtype) {
    return invoke([&] {
        *dtype = static_cast<dl_dtype>(as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder").cache_dtype());
    });
}

dl_status dl_decoder_cache_create(const dl_module* decoder, dl_decoder_cache** output) {
    return make_handle(output, [&] { return as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder").make_cache(); });
}

void dl_decoder_cache_release(dl_decoder_cache* cache) { delete cache; }

dl_status dl_decoder_cache_clear(dl_decoder_cache* cache) {
    return invoke([&] { for (auto& layer : require(cache, "cache").value) layer.clear(); });
}

dl_status dl_decoder_cache_truncate(dl_decoder_cache* cache, int64_t length) {
    return invoke([&] {
        auto& layers = require(cache, "cache").value;
        for (auto& layer : layers)
            if (length < 0 || length > layer.length())
                throw std::out_of_range("KV cache truncation must keep an existing prefix");
        for (auto& layer : layers) layer.truncate(length);
    });
}

dl_status dl_decoder_cache_length(const dl_decoder_cache* cache, int64_t* length) {
    return invoke([&] {
        const auto& layers = require(cache, "cache").value;
        *length = layers.empty() ? 0 : layers.front().length();
    });
}

dl_status dl_decoder_cache_append(dl_decoder_cache* cache, int64_t layer, const dl_tensor* key, const dl_tensor* value) {
    return invoke([&] {
        auto& layers = require(cache, "cache").value;
        if (layer < 0 || layer >= static_cast<int64_t>(layers.size())) throw std::out_of_range("cache layer out of range");
        layers[static_cast<std::size_t>(layer)].append(require(key, "key").value, require(value, "value").value);
    });
}

dl_status dl_decoder_cache_state(const dl_decoder_cache* cache, dl_state** output) {
    return make_handle(output, [&] {
        const auto& layers = require(cache, "cache").value;
        dl::StateDict state;
        for (std::size_t i = 0; i < layers.size(); ++i) {
            if (!layers[i].reserved())
                throw std::logic_error("cache layer " + std::to_string(i) + " holds no keys yet (its batch is unknown)");
            // a snapshot: an f32 cache's contiguous prefix would otherwise come back as a view of live storage
            auto snapshot = [](const dl::Tensor& t) {
                return t.dtype() == dl::DType::f32 ? t.clone() : t.astype(dl::DType::f32);
            };
            state.emplace_back("past_key_" + std::to_string(i), snapshot(layers[i].key()));
            state.emplace_back("past_value_" + std::to_string(i), snapshot(layers[i].value()));
        }
        return state;
    });
}

dl_status dl_decoder_cache_load_state(const dl_module* decoder, dl_decoder_cache* cache, const dl_state* state) {
    return invoke([&] {
        const auto& dec = as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder");
        auto& layers = require(cache, "cache").value;
        const auto& entries = require(state, "state").value;
        if (layers.size() != static_cast<std::size_t>(dec.layer_count()))
            throw std::invalid_argument("cache and decoder have different layer counts");
        auto find = [&](const std::string& kind, std::size_t layer) -> const dl::Tensor& {
            const dl::Tensor* found = nullptr;
            for (const char* prefix : {"past_", "present_"}) {
                const std::string name = prefix + kind + "_" + std::to_string(layer);
                for (const auto& [n, t] : entries) {
                    if (n != name) continue;
                    if (found) throw std::invalid_argument("cache state names layer " + std::to_string(layer) + " " +
                                                           kind + " twice");
                    found = &t;
                }
            }
            if (!found) throw std::invalid_argument("cache state has no past_" + kind + "_" + std::to_string(layer));
            return *found;
        };
        // validate every layer before touching the cache
        std::vector<std::pair<const dl::Tensor*, const dl::Tensor*>> kv;
        dl::Index batch = -1, length = -1;
        for (std::size_t i = 0; i < layers.size(); ++i) {
            const auto& attention = dec.layer(static_cast<dl::Index>(i)).attention();
            const dl::Tensor& k = find("key", i);
            const dl::Tensor& v = find("value", i);
            for (const dl::Tensor* t : {&k, &v})
                if (t->ndim() != 4 || t->size(1) != attention.kv_heads() || t->size(3) != attention.head_dim())
                    throw std::invalid_argument("cache state layer " + std::to_string(i) +
                                                " must be [batch, kv_heads, length, head_dim]");
            if (k.shape() != v.shape()) throw std::invalid_argument("cache state key and value shapes differ");
            if (batch < 0) { batch = k.size(0); length = k.size(2); }
            if (k.size(0) != batch || k.size(2) != length)
                throw std::invalid_argument("cache state layers must share batch and length");
            if (length > layers[i].capacity()) throw std::invalid_argument("cache state exceeds the cache capacity");
            kv.emplace_back(&k, &v);
        }
        for (std::size_t i = 0; i < layers.size(); ++i) {
            const auto& layer = dec.layer(static_cast<dl::Index>(i));
            const auto& attention = layer.attention();
            const dl::Device device = attention.query().weight().device();
            const dl::DType dtype = dl::detail::cache_dtype(layer);
            layers[i] = dl::nn::KVCache(layers[i].capacity());
            layers[i].reserve(batch, attention.kv_heads(), attention.head_dim(), dtype, device);
            layers[i].append(kv[i].first->to(device).astype(dtype), kv[i].second->to(device).astype(dtype));
        }
    });
}

dl_status dl_transformer_decoder_decode(dl_module* decoder, const dl_tensor* input, dl_decoder_cache* cache,
                                        dl_tensor** output) {
    return make_handle(output, [&] {
        return as<dl::nn::TransformerDecoder>(decoder, "TransformerDecoder")
            .decode(require(input, "input").value, require(cache, "cache").value);
    });
}

} // extern "C"
