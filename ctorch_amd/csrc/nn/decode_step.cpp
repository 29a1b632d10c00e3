// Fused per-layer decode step (see decode_step.h).
#include "nn/decode_step.h"

#include <cmath>
#include <stdexcept>

namespace dl::detail {

using nn::KVCache;
using nn::TransformerDecoderLayer;

DType cache_dtype(const TransformerDecoderLayer& layer) { return layer.attention().cache_dtype(); }

void DecodeWorkspace::ensure(const TransformerDecoderLayer& layer, Index n, Index heads_total, Index hidden_features,
                             int splits, Device device) {
    const Index d = layer.attention().dimensions();
    const Index hd = layer.attention().head_dim();
    if (!q.defined() || rows < n || q.size(1) != heads_total || activation.size(1) != hidden_features ||
        !(q.device() == device)) {
        rows = n;
        q = empty_tensor({n, heads_total}, DType::f32, device);
        attention = empty_tensor({n, d}, DType::f32, device);
        hidden = empty_tensor({n, d}, DType::f32, device);
        activation = empty_tensor({n, hidden_features}, DType::f32, device);
        splits_capacity = 0;
        lora = Tensor();
    }
    const Index heads = layer.attention().heads();
    const Index partial_rows = n * heads; // one partial row per (b, h, l)
    if (splits > 1 && (splits_capacity < splits || partial_o.size(0) < partial_rows)) {
        splits_capacity = splits;
        partial_o = empty_tensor({partial_rows, splits, hd}, DType::f32, device);
        partial_ml = empty_tensor({partial_rows, splits, 2}, DType::f32, device);
    }
    const auto* qa = layer.attention().query_adapter();
    const auto* va = layer.attention().value_adapter();
    const Index ranks = (qa ? qa->rank() : 0) + (va ? va->rank() : 0);
    if (ranks > 0 && (!lora.defined() || lora.size(0) < n || lora.size(1) != ranks))
        lora = empty_tensor({n, ranks}, DType::f32, device);
}

void DecodeWorkspace::attach_workspace(dlk_gemv_params& p, Device device) {
    const int64_t stage_need = dlk_gemv_stage_bytes(&p);
    if (stage_need > 0) {
        if (!stage.defined() || stage.numel() * 4 < stage_need || !(stage.device() == device))
            stage = empty_tensor({(stage_need + 3) / 4}, DType::f32, device);
        p.stage = mutable_data(stage);
        p.stage_bytes = stage.numel() * 4;
    }
    const int64_t need = dlk_gemv_split_floats(&p);
    if (need <= 0) return;
    if (!split.defined() || split.numel() < need || !(split.device() == device))
        split = empty_tensor({need}, DType::f32, device);
    p.split_partial = static_cast<float*>(mutable_data(split));
    p.split_capacity = split.numel();
}

const void* DecodeWorkspace::tiles_of(const Tensor& w0, const Tensor* w1, dlh_stream stream) {
    if (!pack_weights || w0.dtype() != DType::bf16 || w0.ndim() != 2 || !w0.is_contiguous()) return nullptr;
    const Index rows = w0.size(0), K = w0.size(1);
    if (w1 && (w1->dtype() != DType::bf16 || w1->shape() != w0.shape() || !w1->is_contiguous())) return nullptr;
    if (K % 32 != 0 || rows % (w1 ? 8 : 16) != 0) return nullptr;
    int capturing = 0;
    hip_check(dlh_stream_capturing(stream, &capturing), "stream capture status");
    const uint64_t epoch = parameter_epoch();
    if (epoch != packed_epoch_) {
        if (capturing) return nullptr;
        packed_.clear();
        packed_epoch_ = epoch;
    }
    const PackKey key{w0.data<void>(), rows, K, w1 ? w1->data<void>() : nullptr};
    const auto it = packed_.find(key);
    if (it != packed_.end()) return it->second.tiles.data<void>();
    if (capturing) return nullptr;
    Tensor tiles = empty_tensor({(w1 ? 2 : 1) * rows * K}, DType::bf16, w0.device());
    hip_check(dlk_pack_tiles(w0.data<void>(), w1 ? w1->data<void>() : nullptr, w1 ? 1 : 0, rows, K,
                             mutable_data(tiles), stream),
              "weight repack");
    packed_[key] = Packed{w0, w1 ? *w1 : Tensor(), tiles};
    return tiles.data<void>();
}

namespace {
const void* norm_data(const nn::RMSNorm& norm, int& bf16) {
    const auto& w = norm.weight();
    if (!w) { bf16 = 0; return nullptr; }
    if (w->dtype() != DType::f32 && w->dtype() != DType::bf16) throw std::invalid_argument("RMSNorm weight dtype");
    bf16 = w->dtype() == DType::bf16;
    return w->data<void>();
}

} // namespace

void decode_layer(const TransformerDecoderLayer& layer, const float* x_in, float* x_out, Index batch, Index length,
                  KVCache& cache, DecodeWorkspace& ws, int splits, int chunk, GpuContext& context,
                  LaunchObserver* observer) {
    const auto& attention = layer.attention();
    const auto& ff = layer.feedforward();
    const Index d = attention.dimensions(), H = attention.heads(), KV = attention.kv_heads(), hd = attention.head_dim();
    const Index F = ff.gate().weight().size(0);
    const Index rows = batch * length;
    const Device device = attention.query().weight().device();
    ws.ensure(layer, rows, H * hd, F, splits, device);
    if (!cache.reserved()) throw std::logic_error("decode_layer needs a reserved cache");
    const bool kv_bf16 = cache.key().dtype() == DType::bf16;
    const double kv_bytes_per = static_cast<double>(batch) * KV * hd * (kv_bf16 ? 2 : 4);

    // The LoRA down projections and the QKV projection read the same normalised rows: when consecutive launches
    // take the tiled path with the same staging workspace, the rows are split once.
    const void* staged = nullptr;
    auto share_stage = [&](dlk_gemv_params& p) {
        const bool tiled = p.stage != nullptr && dlk_gemv_stage_bytes(&p) > 0;
        p.stage_ready = tiled && staged == p.stage ? 1 : 0;
        staged = tiled ? p.stage : nullptr;
    };

    // 2. QKV projection: fused RMSNorm prologue, (LoRA,) RoPE and KV append epilogue; issued with the attention.
    //    Its parameters come first: over few rows the launch may apply the LoRA down rows itself, and then 1 is
    //    not issued.
    const nn::LoRAAdapter* adapters[2] = {attention.query_adapter(), attention.value_adapter()};
    const Index lora_width = ws.lora.defined() ? ws.lora.size(1) : 0;
    bool lora_folded = false;
    dlk_gemv_params qkv{};
    double qkv_bytes = 0.0;
    {
        int qb = 0, kb = 0, vb = 0, nb = 0;
        dlk_gemv_params p = gemv_params(x_in, rows, d, DLK_EPI_QKV);
        p.apply_norm = 1;
        p.norm_weight = norm_data(layer.attention_norm(), nb);
        p.norm_bf16 = nb;
        p.epsilon = static_cast<float>(layer.attention_norm().epsilon());
        p.nseg = 3;
        p.w[0] = weight_data(attention.query().weight(), qb, "QKV");
        p.w[1] = weight_data(attention.key().weight(), kb, "QKV");
        p.w[2] = weight_data(attention.value().weight(), vb, "QKV");
        if (qb != kb || qb != vb) throw std::invalid_argument("attention projections must share one dtype");
        p.seg_rows[0] = static_cast<int>(H * hd);
        p.seg_rows[1] = p.seg_rows[2] = static_cast<int>(KV * hd);
        p.w_bf16 = qb;
        p.y = static_cast<float*>(mutable_data(ws.q));
        p.ldy = H * hd;
        p.head_dim = static_cast<int>(hd);
        p.kv_heads = static_cast<int>(KV);
        p.length = static_cast<int>(length);
        p.cosine = attention.rotary().cosine().data<float>();
        p.sine = attention.rotary().sine().data<float>();
        p.position = cache.position_data();
        p.k_cache = cache.key_data();
        p.v_cache = cache.value_data();
        p.cache_bf16 = kv_bf16;
        p.cache_capacity = cache.capacity();
        bool down_bf16 = true;
        for (int i = 0; i < 2; ++i) {
            const nn::LoRAAdapter* a = adapters[i];
            if (!a) continue;
            const int seg = 2 * i; // q or v
            int ub = 0, db = 0;
            p.lora_hidden[seg] = ws.lora.data<float>() + (i == 1 && adapters[0] ? adapters[0]->rank() : 0);
            p.lora_up[seg] = weight_data(a->up().weight(), ub, "LoRA up");
            if (ub != qb) throw std::invalid_argument("LoRA up weights must share the projection dtype");
            p.lora_down[seg] = weight_data(a->down().weight(), db, "LoRA down");
            down_bf16 = down_bf16 && db;
            p.lora_rank = static_cast<int>(a->rank());
            p.lora_scale = static_cast<float>(a->scale());
        }
        p.lora_ld = lora_width;
        if (adapters[0] && adapters[1] &&
            (adapters[0]->rank() != adapters[1]->rank() || adapters[0]->scale() != adapters[1]->scale()))
            throw std::invalid_argument("query and value adapters must share rank and alpha");
        qkv_bytes = static_cast<double>((H + 2 * KV) * hd * d) * (qb ? 2 : 4) + 2.0 * kv_bytes_per * length;
        ws.attach_workspace(p, device);
        // the fold reads the down rows in place of the hidden rows of 1
        if (adapters[0] || adapters[1]) {
            const float* hidden[2] = {p.lora_hidden[0], p.lora_hidden[2]};
            p.lora_hidden[0] = p.lora_hidden[2] = nullptr;
            lora_folded = down_bf16 && dlk_gemv_folds_lora(&p) != 0;
            if (!lora_folded) {
                p.lora_hidden[0] = hidden[0];
                p.lora_hidden[2] = hidden[1];
                p.lora_down[0] = p.lora_down[2] = nullptr;
            }
        }
        qkv = p;
    }

    // 1. LoRA hidden states (down projections of the normalised input), when adapters are attached and the QKV
    //    launch does not fold them into its key loop: one launch for both adapters, their down matrices as two
    //    weight segments whose outputs sit side by side in a row of ws.lora (query adapter first)
    if ((adapters[0] || adapters[1]) && !lora_folded) {
        int nb = 0, wb = -1;
        dlk_gemv_params p = gemv_params(x_in, rows, d, DLK_EPI_STORE);
        p.apply_norm = 1;
        p.norm_weight = norm_data(layer.attention_norm(), nb);
        p.norm_bf16 = nb;
        p.epsilon = static_cast<float>(layer.attention_norm().epsilon());
        double bytes = 0.0;
        for (const auto* adapter : adapters) {
            if (!adapter) continue;
            int ab = 0;
            p.w[p.nseg] = weight_data(adapter->down().weight(), ab, "LoRA down");
            if (wb >= 0 && ab != wb) throw std::invalid_argument("LoRA adapters must share one dtype");
            wb = ab;
            p.seg_rows[p.nseg++] = static_cast<int>(adapter->rank());
            bytes += static_cast<double>(adapter->down().weight().numel()) * (ab ? 2 : 4);
        }
        p.w_bf16 = wb;
        p.y = static_cast<float*>(mutable_data(ws.lora));
        p.ldy = lora_width;
        ws.attach_workspace(p, device);
        share_stage(p);
        issue(observer, "lora_down", bytes,
              [p, &context](bool) { hip_check(dlk_gemv(&p, context.stream), "LoRA down projection"); });
    }

    // 4's parameters first: when the output projection takes the tiled (prefill) path and the attention the
    // prefill kernel, the attention writes its rows already split for the projection, which skips its split pass
    dlk_gemv_params out{};
    {
        int ob = 0;
        dlk_gemv_params p = gemv_params(ws.attention.data<float>(), rows, d, DLK_EPI_RESIDUAL);
        p.nseg = 1;
        p.w[0] = weight_data(attention.output().weight(), ob, "output projection");
        p.seg_rows[0] = static_cast<int>(d);
        p.w_bf16 = ob;
        p.y = static_cast<float*>(mutable_data(ws.hidden));
        p.ldy = d;
        p.residual = x_in;
        p.ldres = d;
        p.bump_position = cache.position_data();
        p.bump_count = length;
        ws.attach_workspace(p, device);
        out = p;
    }
    // the output projection's attach may have grown the split buffer: the QKV launch takes the current one (the
    // attention may read its partials), which already fits both launches
    ws.attach_workspace(qkv, device);
    share_stage(qkv);
    if (dlk_gemv_uses_rows(&qkv)) {
        qkv.w_tiles[0] = ws.tiles_of(attention.query().weight(), nullptr, context.stream);
        qkv.w_tiles[1] = ws.tiles_of(attention.key().weight(), nullptr, context.stream);
        qkv.w_tiles[2] = ws.tiles_of(attention.value().weight(), nullptr, context.stream);
    }
    if (dlk_gemv_uses_rows(&out)) out.w_tiles[0] = ws.tiles_of(attention.output().weight(), nullptr, context.stream);

    // 3. split-K attention over the cache (reads the device length, sees the keys just appended)
    {
        dlk_attention_params a{};
        a.q = ws.q.data<float>();
        a.ldq = H * hd;
        a.k = cache.key_data();
        a.v = cache.value_data();
        a.kv_bf16 = kv_bf16;
        a.capacity = cache.capacity();
        a.position = cache.position_data();
        // the host length plus this chunk: at graph capture, the fewest keys any replay sees
        a.early_keys = cache.length() + length;
        a.B = static_cast<int>(batch); a.L = static_cast<int>(length); a.H = static_cast<int>(H);
        a.KV = static_cast<int>(KV); a.hd = static_cast<int>(hd);
        a.scale = static_cast<float>(1.0 / std::sqrt(static_cast<double>(hd)));
        a.causal = 1;
        a.out = static_cast<float*>(mutable_data(ws.attention));
        a.ldo = d;
        a.splits = splits;
        a.chunk = chunk;
        if (splits > 1) {
            a.partial_o = static_cast<float*>(mutable_data(ws.partial_o));
            a.partial_ml = static_cast<float*>(mutable_data(ws.partial_ml));
        }
        const int64_t out_stage = dlk_gemv_stage_bytes(&out);
        if (out.stage && out_stage > 0 && dlk_attention_prefill_eligible(&a) && (H * hd) % 32 == 0) {
            if (!ws.stage_attn.defined() || ws.stage_attn.numel() * 4 < out_stage || !(ws.stage_attn.device() == device))
                ws.stage_attn = empty_tensor({(out_stage + 3) / 4}, DType::f32, device);
            a.stage_out = mutable_data(ws.stage_attn);
            out.stage = a.stage_out;
            out.stage_bytes = ws.stage_attn.numel() * 4;
            out.stage_ready = 1;
        }
        // One new position without adapters, when the projection splits its keys and the attention's work-groups
        // fit one per CU: the attention finishes the projection from its partials (sums them, normalises,
        // rotates, appends K/V), which drops the reduce launch.  Every work-group pays the partials' round trip
        // before its first tile, so a grid of several work-groups per CU (MI355X, 8B at b=8 over 32768 keys:
        // 10.2 -> 10.8 ms a step; measured again with the first tile requested before the length, 9.31 -> 9.84 ms)
        // keeps the reduce launch; at one per CU (1B at b=32: 1.49 -> 1.45 ms) it pays.
        const bool one_per_cu = static_cast<int64_t>(a.splits) * batch * KV <= 256;
        const int qkv_splits = length == 1 && !adapters[0] && !adapters[1] && !a.stage_out && one_per_cu
                                   ? dlk_gemv_split_count(&qkv)
                                   : 1;
        if (qkv_splits > 1) {
            dlk_attention_params f = a;
            f.qkv_partial = qkv.split_partial;
            f.qkv_splits = qkv_splits;
            f.qkv_width = static_cast<int>((H + 2 * KV) * hd);
            f.qkv_K = static_cast<int>(d);
            f.qkv_norm = qkv.apply_norm;
            f.qkv_scale = qkv.acc_scale;
            f.qkv_epsilon = qkv.epsilon;
            f.rope_cos = qkv.cosine;
            f.rope_sin = qkv.sine;
            if (dlk_attention_matrix_eligible(&f)) {
                a = f;
                qkv.defer_reduce = 1;
            }
        }
        // the label names what the launch leaves: finished rows, or the partials the attention finishes
        issue(observer, qkv.defer_reduce ? "qkv_split" : "qkv_rope_append", qkv_bytes,
              [p = qkv, &context](bool) { hip_check(dlk_gemv(&p, context.stream), "QKV projection"); });
        // Prefill over an f32 cache: the K/V tiles are split into bf16 planes once for the launch (a workspace
        // covering the capacity; kept within 1 GiB, past which the kernel splits each tile it reads itself)
        const int64_t split_bytes = length > 1 ? dlk_attention_split_bytes(&a) : 0;
        if (split_bytes > 0 && split_bytes <= (int64_t(1) << 30)) {
            if (!ws.kv_split.defined() || ws.kv_split.numel() * 4 < split_bytes || !(ws.kv_split.device() == device))
                ws.kv_split = empty_tensor({(split_bytes + 3) / 4}, DType::f32, device);
            a.kv_split = mutable_data(ws.kv_split);
            a.kv_split_tiles = static_cast<int>((cache.capacity() + 63) / 64);
        }
        const double bytes = 2.0 * kv_bytes_per * static_cast<double>(cache.length() + length);
        issue(observer, "attention", bytes,
              [a, &context](bool) { hip_check(dlk_attention(&a, context.stream), "attention"); });
    }

    // 4. output projection + residual; advances the device cache length by `length`
    issue(observer, "output_residual", static_cast<double>(d * d) * (out.w_bf16 ? 2 : 4), [p = out, &context](bool repeat) {
        dlk_gemv_params q = p;
        if (repeat) q.bump_position = nullptr; // a timing repeat leaves the device length alone
        hip_check(dlk_gemv(&q, context.stream), "output projection");
    });

    // 5. gate/up projection: fused RMSNorm prologue and SiLU(gate) * up epilogue; 6. down projection + residual.
    // Workspaces are attached down, gate/up, down: a buffer grows only when a launch needs more than it holds, so
    // after the first two both launches' needs are met and the last attach hands the down launch current
    // pointers without moving the gate/up launch's.  When both take the tiled (prefill) path, gate/up writes its
    // rows already split for the down launch, which then skips its own split pass.
    dlk_gemv_params down{};
    {
        int db = 0;
        dlk_gemv_params p = gemv_params(ws.activation.data<float>(), rows, F, DLK_EPI_RESIDUAL);
        p.nseg = 1;
        p.w[0] = weight_data(ff.down().weight(), db, "down");
        p.seg_rows[0] = static_cast<int>(d);
        p.w_bf16 = db;
        p.y = x_out;
        p.ldy = d;
        p.residual = ws.hidden.data<float>();
        p.ldres = d;
        ws.attach_workspace(p, device);
        down = p;
    }
    {
        int gb = 0, ub = 0, nb = 0;
        dlk_gemv_params p = gemv_params(ws.hidden.data<float>(), rows, d, DLK_EPI_SWIGLU);
        p.apply_norm = 1;
        p.norm_weight = norm_data(layer.feedforward_norm(), nb);
        p.norm_bf16 = nb;
        p.epsilon = static_cast<float>(layer.feedforward_norm().epsilon());
        p.nseg = 2;
        p.w[0] = weight_data(ff.gate().weight(), gb, "gate");
        p.w[1] = weight_data(ff.up().weight(), ub, "up");
        if (gb != ub) throw std::invalid_argument("gate and up projections must share one dtype");
        p.seg_rows[0] = p.seg_rows[1] = static_cast<int>(F);
        p.w_bf16 = gb;
        p.y = static_cast<float*>(mutable_data(ws.activation));
        p.ldy = F;
        ws.attach_workspace(p, device);
        ws.attach_workspace(down, device);
        const int64_t down_stage = dlk_gemv_stage_bytes(&down);
        if (p.stage && dlk_gemv_stage_bytes(&p) > 0 && down.stage && down_stage > 0 && F % 32 == 0) {
            if (!ws.stage_ffn.defined() || ws.stage_ffn.numel() * 4 < down_stage || !(ws.stage_ffn.device() == device))
                ws.stage_ffn = empty_tensor({(down_stage + 3) / 4}, DType::f32, device);
            p.stage_out = mutable_data(ws.stage_ffn);
            down.stage = p.stage_out;
            down.stage_bytes = ws.stage_ffn.numel() * 4;
            down.stage_ready = 1;
        }
        if (dlk_gemv_uses_rows(&p)) p.w_tiles[0] = ws.tiles_of(ff.gate().weight(), &ff.up().weight(), context.stream);
        if (dlk_gemv_uses_rows(&down)) down.w_tiles[0] = ws.tiles_of(ff.down().weight(), nullptr, context.stream);
        issue(observer, "gate_up_silu", static_cast<double>(2 * F * d) * (gb ? 2 : 4),
              [p, &context](bool) { hip_check(dlk_gemv(&p, context.stream), "gate/up projection"); });
    }
    issue(observer, "down_residual", static_cast<double>(F * d) * (down.w_bf16 ? 2 : 4),
          [p = down, &context](bool) { hip_check(dlk_gemv(&p, context.stream), "down projection"); });
    cache.advance(length);
}

} // namespace dl::detail
