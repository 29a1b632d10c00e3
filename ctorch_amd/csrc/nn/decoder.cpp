// Decoder stack (reference src/nn/decoder.cpp:11-142) over the fused GPU decode step.
//
// Semantics kept from the reference: state names (layer{i}.attention.{query,key,value,output}.weight,
// layer{i}.attention.rotary.{cosine,sine}, layer{i}.feedforward.{gate,up,down}.weight,
// layer{i}.{attention,feedforward}_norm.weight, normalization.weight), f32 RoPE tables from
// exp(i * (-2 ln base / D)) with interleaved pairs, GQA head mapping h -> h / (H/KV), the causal rule
// k <= offset + row, decode of only the new positions with the offset taken from the cache, and chunk
// atomicity: a chunk that cannot be appended leaves every cache at the prefix it started from.
#include "nn/decode_step.h"

#include <cmath>
#include <stdexcept>

namespace dl::nn {

using namespace dl::detail;

// ------------------------------------------------------------------------------------------------ SwiGLU
SwiGLU::SwiGLU(Index dimensions, Index hidden, bool bias, TensorOptions options) {
    gate_ = add_module<Linear>("gate", dimensions, hidden, bias, options);
    up_ = add_module<Linear>("up", dimensions, hidden, bias, options);
    down_ = add_module<Linear>("down", hidden, dimensions, bias, options);
}

Tensor SwiGLU::forward(const Tensor& input) {
    GpuContext& context = gpu_of(input, "SwiGLU");
    const Index d = input.size(-1), F = gate_->weight().size(0);
    Tensor x = contiguous_f32(input);
    const Index rows = x.numel() / d;
    Shape hidden_shape = input.shape();
    hidden_shape.back() = F;
    Tensor act = empty_tensor(hidden_shape, DType::f32, input.device());
    int gb = 0, ub = 0;
    const void* g = weight_data(gate_->weight(), gb, "SwiGLU");
    const void* u = weight_data(up_->weight(), ub, "SwiGLU");
    if (gate_->bias() || gb != ub || d % (gb ? 8 : 4) != 0)
        throw std::invalid_argument("SwiGLU on the GPU needs bias-free gate/up of one dtype and a width multiple of 8");
    dlk_gemv_params p = gemv_params(x.data<float>(), rows, d, DLK_EPI_SWIGLU);
    p.nseg = 2;
    p.w[0] = g;
    p.w[1] = u;
    p.seg_rows[0] = p.seg_rows[1] = static_cast<int>(F);
    p.w_bf16 = gb;
    p.y = static_cast<float*>(mutable_data(act));
    p.ldy = F;
    hip_check(dlk_gemv(&p, context.stream), "SwiGLU gate/up");
    return linear(act, down_->weight(), down_->bias());
}

// ------------------------------------------------------------------------------------------------ LoRA
LoRALinear::LoRALinear(const Linear& base, Index rank, double alpha)
    : weight_(register_parameter("weight", base.weight().clone())), scale_(alpha / static_cast<double>(rank)) {
    if (rank <= 0) throw std::invalid_argument("LoRA rank must be positive");
    if (base.bias()) bias_ = register_parameter("bias", base.bias()->clone());
    const TensorOptions options{.dtype = weight_.dtype(), .device = weight_.device(), .requires_grad = true};
    down_ = add_module<Linear>("down", weight_.size(1), rank, false, options);
    up_ = add_module<Linear>("up", zeros({weight_.size(0), rank}, options));
}

namespace {
// y = base + scale * (x A^T) B^T with A = down [r, in], B = up [out, r]: two projections, the second with a
// residual epilogue scaled by `scale`.
Tensor lora_forward(const Tensor& input, const Tensor& weight, const std::optional<Tensor>& bias, const Linear& down,
                    const Linear& up, double scale) {
    GpuContext& context = gpu_of(input, "LoRALinear");
    Tensor base = linear(input, weight, bias);
    Tensor hidden = linear(input, down.weight(), std::nullopt);
    const Index r = up.weight().size(1), n = up.weight().size(0);
    const Index rows = hidden.numel() / r;
    int ub = 0;
    const void* uw = weight_data(up.weight(), ub, "LoRALinear");
    dlk_gemv_params p = gemv_params(hidden.data<float>(), rows, r, DLK_EPI_RESIDUAL);
    p.nseg = 1;
    p.w[0] = uw;
    p.seg_rows[0] = static_cast<int>(n);
    p.w_bf16 = ub;
    p.acc_scale = static_cast<float>(scale);
    p.y = static_cast<float*>(mutable_data(base));
    p.ldy = n;
    p.residual = base.data<float>();
    p.ldres = n;
    if (r % (ub ? 8 : 4) != 0) throw std::invalid_argument("LoRA rank must be a multiple of 8 (bf16) or 4 (f32)");
    hip_check(dlk_gemv(&p, context.stream), "LoRA up");
    return base;
}
} // namespace

Tensor LoRALinear::forward(const Tensor& input) { return lora_forward(input, weight_, bias_, *down_, *up_, scale_); }

std::shared_ptr<Linear> LoRALinear::merged() const {
    // W + scale * up @ down, accumulated in f32 on the GPU and rounded once to W's dtype
    GpuContext& context = gpu_of(weight_, "LoRALinear::merged");
    const Index out = weight_.size(0), in = weight_.size(1), r = down_->weight().size(0);
    Tensor up32 = contiguous_f32(up_->weight());                          // [out, r] as activation rows
    Tensor downT = down_->weight().transpose(0, 1).contiguous();          // [in, r] as weight rows
    Tensor merged = contiguous_f32(weight_).clone();
    int db = 0;
    const void* dw = weight_data(downT, db, "LoRALinear::merged");
    if (r % (db ? 8 : 4) != 0) throw std::invalid_argument("LoRA rank must be a multiple of 8 (bf16) or 4 (f32)");
    dlk_gemv_params p = gemv_params(up32.data<float>(), out, r, DLK_EPI_RESIDUAL);
    p.nseg = 1;
    p.w[0] = dw;
    p.seg_rows[0] = static_cast<int>(in);
    p.w_bf16 = db;
    p.acc_scale = static_cast<float>(scale_);
    p.y = static_cast<float*>(mutable_data(merged));
    p.ldy = in;
    p.residual = merged.data<float>();
    p.ldres = in;
    hip_check(dlk_gemv(&p, context.stream), "LoRA merge");
    Tensor weight = merged.astype(weight_.dtype());
    return std::make_shared<Linear>(weight, bias_ ? std::optional<Tensor>{bias_->clone()} : std::nullopt);
}

LoRAAdapter::LoRAAdapter(Index input_features, Index output_features, Index rank, double alpha, TensorOptions options)
    : rank_(rank), scale_(alpha / static_cast<double>(rank)) {
    if (rank <= 0) throw std::invalid_argument("LoRA rank must be positive");
    down_ = add_module<Linear>("down", input_features, rank, false, options);
    up_ = add_module<Linear>("up", zeros({output_features, rank}, options));
}

// ------------------------------------------------------------------------------------------------ RoPE
namespace {
// Angle tables as the reference builds them (src/nn/decoder.cpp:38-46): frequencies in f32 from
// exp(arange(D/2) * f32(-2 ln base / D)), angles = f32(p) * frequency, then f32 cos/sin.
std::pair<Tensor, Tensor> rotary_tables(Index dimensions, Index capacity, double base, Device device) {
    if (dimensions <= 0 || dimensions % 2 != 0 || capacity <= 0 || base <= 0)
        throw std::invalid_argument("RoPE needs an even positive dimension, positive capacity and base");
    const Index half = dimensions / 2;
    Tensor c = empty_tensor({capacity, half}, DType::f32, Device::cpu());
    Tensor s = empty_tensor({capacity, half}, DType::f32, Device::cpu());
    float* cd = static_cast<float*>(mutable_data(c));
    float* sd = static_cast<float*>(mutable_data(s));
    const float factor = static_cast<float>(-2.0 * std::log(base) / static_cast<double>(dimensions));
    std::vector<float> frequencies(static_cast<std::size_t>(half));
    for (Index i = 0; i < half; ++i) frequencies[static_cast<std::size_t>(i)] = std::exp(static_cast<float>(i) * factor);
    for (Index p = 0; p < capacity; ++p) {
        for (Index i = 0; i < half; ++i) {
            const float angle = static_cast<float>(p) * frequencies[static_cast<std::size_t>(i)];
            cd[p * half + i] = std::cos(angle);
            sd[p * half + i] = std::sin(angle);
        }
    }
    if (device.type == DeviceType::cpu) return {c, s};
    return {c.to(device), s.to(device)};
}
} // namespace

RotaryEmbedding::RotaryEmbedding(Index dimensions, Index capacity, double base, TensorOptions options) {
    auto [c, s] = rotary_tables(dimensions, capacity, base, options.device);
    cosine_ = register_buffer("cosine", c);
    sine_ = register_buffer("sine", s);
}

Tensor RotaryEmbedding::forward(const Tensor& input, Index offset) {
    if (offset < 0 || input.size(-2) > cosine_.size(0) - offset)
        throw std::out_of_range("RoPE positions exceed the table capacity");
    return rotary_embedding(input, cosine_.narrow(0, offset, input.size(-2)), sine_.narrow(0, offset, input.size(-2)));
}

// ------------------------------------------------------------------------------------------------ GQA
GroupedQueryAttention::GroupedQueryAttention(Index dimensions, Index heads, Index kv_heads, Index context,
                                             TensorOptions options, double rope_base)
    : dimensions_(dimensions), heads_(heads), kv_heads_(kv_heads) {
    if (heads <= 0 || kv_heads <= 0 || dimensions <= 0 || dimensions % heads || heads % kv_heads)
        throw std::invalid_argument("attention dimensions and query/key head counts must divide evenly");
    query_ = add_module<Linear>("query", dimensions, dimensions, false, options);
    key_ = add_module<Linear>("key", dimensions, kv_heads * (dimensions / heads), false, options);
    value_ = add_module<Linear>("value", dimensions, kv_heads * (dimensions / heads), false, options);
    output_ = add_module<Linear>("output", dimensions, dimensions, false, options);
    rotary_ = add_module<RotaryEmbedding>("rotary", dimensions / heads, context, rope_base, options);
}

void GroupedQueryAttention::attach_lora(Index rank, double alpha, bool query, bool value) {
    const TensorOptions options{.dtype = query_->weight().dtype(), .device = query_->weight().device()};
    if (query && !query_adapter_)
        query_adapter_ = add_module<LoRAAdapter>("query_adapter", dimensions_, dimensions_, rank, alpha, options);
    if (value && !value_adapter_)
        value_adapter_ = add_module<LoRAAdapter>("value_adapter", dimensions_, kv_heads_ * head_dim(), rank, alpha, options);
}

void GroupedQueryAttention::set_cache_dtype(DType dtype) {
    if (dtype != DType::f32 && dtype != DType::bf16) throw std::invalid_argument("KV cache dtype must be f32 or bf16");
    cache_dtype_ = dtype;
}

Tensor GroupedQueryAttention::forward(const Tensor& input) { return run(input, nullptr); }

Tensor GroupedQueryAttention::decode(const Tensor& input, KVCache& cache) { return run(input, &cache); }

Tensor GroupedQueryAttention::run(const Tensor& input, KVCache* cache) {
    if (input.ndim() != 3 || input.size(2) != dimensions_)
        throw std::invalid_argument("attention input must be [batch, length, dimensions]");
    KVCache local(std::max<Index>(1, input.size(1)));
    KVCache& target = cache ? *cache : local;
    target.check_layout(input.size(0), kv_heads_, head_dim(), cache_dtype_, input.device());
    GpuContext& context = gpu_of(input, "GroupedQueryAttention");
    const Index B = input.size(0), L = input.size(1), d = dimensions_;
    const Index offset = target.length();
    if (L > target.capacity() - offset)
        throw std::invalid_argument("KV cache append exceeds capacity or has unequal key/value lengths");
    if (offset + L > rotary_->cosine().size(0)) throw std::out_of_range("RoPE positions exceed the table capacity");
    // a standalone attention block sees its input unnormalised: the layer step's kernels without the norm
    // prologue and without the residual
    Tensor x = contiguous_f32(input);
    Tensor out = empty_tensor({B, L, d}, DType::f32, input.device());
    const Index hd = head_dim();
    const DType kv_dtype = cache_dtype_;
    target.reserve(B, kv_heads_, hd, kv_dtype, input.device());
    const Index rows = B * L;
    Tensor q = empty_tensor({rows, heads_ * hd}, DType::f32, input.device());
    Tensor attended = empty_tensor({rows, d}, DType::f32, input.device());
    int qb = 0, kb = 0, vb = 0, ob = 0;
    dlk_gemv_params p = gemv_params(x.data<float>(), rows, d, DLK_EPI_QKV);
    p.nseg = 3;
    p.w[0] = weight_data(query_->weight(), qb, "attention");
    p.w[1] = weight_data(key_->weight(), kb, "attention");
    p.w[2] = weight_data(value_->weight(), vb, "attention");
    if (qb != kb || qb != vb) throw std::invalid_argument("attention projections must share one dtype");
    p.seg_rows[0] = static_cast<int>(heads_ * hd);
    p.seg_rows[1] = p.seg_rows[2] = static_cast<int>(kv_heads_ * hd);
    p.w_bf16 = qb;
    p.y = static_cast<float*>(mutable_data(q));
    p.ldy = heads_ * hd;
    p.head_dim = static_cast<int>(hd);
    p.kv_heads = static_cast<int>(kv_heads_);
    p.length = static_cast<int>(L);
    p.cosine = rotary_->cosine().data<float>();
    p.sine = rotary_->sine().data<float>();
    p.position = target.position_data();
    p.k_cache = target.key_data();
    p.v_cache = target.value_data();
    p.cache_bf16 = kv_dtype == DType::bf16;
    p.cache_capacity = target.capacity();
    Tensor lq, lv;
    auto adapter_hidden = [&](const LoRAAdapter* adapter, Tensor& hidden, int segment) {
        if (!adapter) return;
        hidden = empty_tensor({rows, adapter->rank()}, DType::f32, input.device());
        linear_into(x.data<float>(), rows, d, adapter->down().weight(), std::nullopt,
                    static_cast<float*>(mutable_data(hidden)), adapter->rank(), context);
        int ab = 0;
        p.lora_hidden[segment] = hidden.data<float>();
        p.lora_up[segment] = weight_data(adapter->up().weight(), ab, "LoRA");
        if (ab != qb) throw std::invalid_argument("LoRA adapters must share the projection dtype");
        p.lora_rank = static_cast<int>(adapter->rank());
        p.lora_scale = static_cast<float>(adapter->scale());
    };
    adapter_hidden(query_adapter_.get(), lq, 0);
    adapter_hidden(value_adapter_.get(), lv, 2);
    if (d % (qb ? 8 : 4) != 0) throw std::invalid_argument("attention width must be a multiple of 8");
    hip_check(dlk_gemv(&p, context.stream), "attention QKV");

    dlk_attention_params a{};
    a.q = q.data<float>();
    a.ldq = heads_ * hd;
    a.k = target.key_data();
    a.v = target.value_data();
    a.kv_bf16 = p.cache_bf16;
    a.capacity = target.capacity();
    a.position = target.position_data();
    a.early_keys = offset + L; // the host length plus this chunk
    a.B = static_cast<int>(B); a.L = static_cast<int>(L); a.H = static_cast<int>(heads_); a.KV = static_cast<int>(kv_heads_);
    a.hd = static_cast<int>(hd);
    a.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(hd)));
    a.causal = 1;
    a.out = static_cast<float*>(mutable_data(attended));
    a.ldo = d;
    attention_split(B, heads_, kv_heads_, hd, a.kv_bf16 != 0, L, offset + L, a.splits, a.chunk);
    Tensor po, pml;
    if (a.splits > 1) {
        po = empty_tensor({B * heads_ * L, a.splits, hd}, DType::f32, input.device());
        pml = empty_tensor({B * heads_ * L, a.splits, 2}, DType::f32, input.device());
        a.partial_o = static_cast<float*>(mutable_data(po));
        a.partial_ml = static_cast<float*>(mutable_data(pml));
    }
    hip_check(dlk_attention(&a, context.stream), "attention");

    dlk_gemv_params o = gemv_params(attended.data<float>(), rows, d, DLK_EPI_STORE);
    o.nseg = 1;
    o.w[0] = weight_data(output_->weight(), ob, "attention");
    o.seg_rows[0] = static_cast<int>(d);
    o.w_bf16 = ob;
    o.y = static_cast<float*>(mutable_data(out));
    o.ldy = d;
    o.bump_position = target.position_data();
    o.bump_count = L;
    hip_check(dlk_gemv(&o, context.stream), "attention output");
    target.advance(L);
    return out;
}

// ------------------------------------------------------------------------------------------------ layer
TransformerDecoderLayer::TransformerDecoderLayer(Index dimensions, Index heads, Index kv_heads, Index hidden,
                                                 Index context, TensorOptions options, double rope_base) {
    attention_ = add_module<GroupedQueryAttention>("attention", dimensions, heads, kv_heads, context, options, rope_base);
    feedforward_ = add_module<SwiGLU>("feedforward", dimensions, hidden, false, options);
    attention_norm_ = add_module<RMSNorm>("attention_norm", Shape{dimensions}, norm_epsilon, true, options);
    feedforward_norm_ = add_module<RMSNorm>("feedforward_norm", Shape{dimensions}, norm_epsilon, true, options);
}

Tensor TransformerDecoderLayer::forward(const Tensor& input) {
    KVCache cache(std::max<Index>(1, input.size(1)));
    return decode(input, cache);
}

Tensor TransformerDecoderLayer::decode(const Tensor& input, KVCache& cache) {
    if (input.ndim() != 3 || input.size(2) != attention_->dimensions())
        throw std::invalid_argument("decoder layer input must be [batch, length, dimensions]");
    cache.check_layout(input.size(0), attention_->kv_heads(), attention_->head_dim(), cache_dtype(*this),
                       input.device());
    GpuContext& context = gpu_of(input, "TransformerDecoderLayer");
    const Index B = input.size(0), L = input.size(1), d = attention_->dimensions();
    if (L > cache.capacity() - cache.length())
        throw std::invalid_argument("KV cache append exceeds capacity or has unequal key/value lengths");
    if (cache.length() + L > attention_->rotary().cosine().size(0))
        throw std::out_of_range("RoPE positions exceed the table capacity");
    cache.reserve(B, attention_->kv_heads(), attention_->head_dim(), cache_dtype(*this), input.device());
    Tensor x = contiguous_f32(input);
    Tensor out = empty_tensor({B, L, d}, DType::f32, input.device());
    DecodeWorkspace ws;
    int splits = 1, chunk = 64;
    attention_split(B, attention_->heads(), attention_->kv_heads(), attention_->head_dim(),
                    cache_dtype(*this) == DType::bf16, L, cache.length() + L, splits, chunk);
    decode_layer(*this, x.data<float>(), static_cast<float*>(mutable_data(out)), B, L, cache, ws, splits, chunk, context);
    return out;
}

// ------------------------------------------------------------------------------------------------ decoder
TransformerDecoder::TransformerDecoder(Index layers, Index dimensions, Index heads, Index kv_heads, Index hidden,
                                       Index context, TensorOptions options, double rope_base)
    : context_(context) {
    if (layers <= 0) throw std::invalid_argument("decoder requires at least one layer");
    for (Index i = 0; i < layers; ++i)
        layers_.push_back(add_module<TransformerDecoderLayer>("layer" + std::to_string(i), dimensions, heads, kv_heads,
                                                              hidden, context, options, rope_base));
    normalization_ = add_module<RMSNorm>("normalization", Shape{dimensions}, TransformerDecoderLayer::norm_epsilon,
                                         true, options);
}

void TransformerDecoder::attach_lora(Index rank, double alpha, bool query, bool value) {
    for (auto& layer : layers_) layer->attention().attach_lora(rank, alpha, query, value);
}

void TransformerDecoder::set_cache_dtype(DType dtype) {
    for (auto& layer : layers_) layer->attention().set_cache_dtype(dtype);
}

DType TransformerDecoder::cache_dtype() const { return layers_.front()->attention().cache_dtype(); }

Tensor TransformerDecoder::forward(const Tensor& input) {
    std::vector<KVCache> cache;
    for (std::size_t i = 0; i < layers_.size(); ++i) cache.emplace_back(std::max<Index>(1, input.size(1)));
    return decode(input, cache);
}

std::vector<KVCache> TransformerDecoder::make_cache() const {
    std::vector<KVCache> result;
    result.reserve(layers_.size());
    for (std::size_t i = 0; i < layers_.size(); ++i) result.emplace_back(context_);
    return result;
}

Tensor TransformerDecoder::decode(const Tensor& input, std::span<KVCache> cache) {
    if (cache.size() != layers_.size()) throw std::invalid_argument("decoder requires one cache per layer");
    const auto prefix = cache.front().length();
    for (const auto& layer : cache)
        if (layer.length() != prefix) throw std::invalid_argument("decoder cache positions differ");
    if (input.ndim() != 3 || input.size(2) != layers_.front()->attention().dimensions())
        throw std::invalid_argument("decoder input must be [batch, length, dimensions]");
    for (std::size_t i = 0; i < layers_.size(); ++i)
        cache[i].check_layout(input.size(0), layers_[i]->attention().kv_heads(), layers_[i]->attention().head_dim(),
                              detail::cache_dtype(*layers_[i]), input.device());
    GpuContext& context = gpu_of(input, "TransformerDecoder");
    const Index B = input.size(0), L = input.size(1), d = input.size(2);
    // every layer's append is checked before anything is launched: a chunk that does not fit leaves all
    // caches at the prefix, as the reference's truncate-and-rethrow does (src/nn/decoder.cpp:133-141)
    for (std::size_t i = 0; i < cache.size(); ++i) {
        if (L > cache[i].capacity() - prefix)
            throw std::invalid_argument("KV cache append exceeds capacity or has unequal key/value lengths");
        if (prefix + L > layers_[i]->attention().rotary().cosine().size(0))
            throw std::out_of_range("RoPE positions exceed the table capacity");
    }
    try {
        Tensor x = input.dtype() == DType::f32 && input.is_contiguous() ? input.clone() : contiguous_f32(input);
        float* xd = static_cast<float*>(mutable_data(x));
        DecodeWorkspace ws;
        int splits = 1, chunk = 64;
        const auto& front = layers_.front()->attention();
        attention_split(B, front.heads(), front.kv_heads(), front.head_dim(),
                        detail::cache_dtype(*layers_.front()) == DType::bf16, L, prefix + L, splits, chunk);
        for (std::size_t i = 0; i < layers_.size(); ++i) {
            cache[i].reserve(B, layers_[i]->attention().kv_heads(), layers_[i]->attention().head_dim(),
                             detail::cache_dtype(*layers_[i]), input.device());
            decode_layer(*layers_[i], xd, xd, B, L, cache[i], ws, splits, chunk, context);
        }
        Tensor out = empty_tensor({B, L, d}, DType::f32, input.device());
        const auto& w = normalization_->weight();
        hip_check(dlk_rms_norm(xd, B * L, d, w ? w->data<void>() : nullptr, w && w->dtype() == DType::bf16,
                               static_cast<float>(normalization_->epsilon()), static_cast<float*>(mutable_data(out)),
                               context.stream),
                  "final norm");
        return out;
    } catch (...) {
        for (auto& layer : cache) layer.truncate(std::min(prefix, layer.length()));
        throw;
    }
}

} // namespace dl::nn
