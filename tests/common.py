"""Shared test helpers: one seeded model evaluated by the CPU oracle (the checker) and by the GPU library.

The oracle's synthetic weights (tests' and bench's common definition, oracle.synthesize_weights) are loaded
into the library's modules through the C ABI: Embedding from tokens.weight, TransformerDecoder from the
decoder.* entries (its RoPE buffers stay the library's own), Linear head from output.weight.
"""
from __future__ import annotations

import sys

import numpy as np

import ctorch_amd as ct
import oracle


class GpuLM:
    """kv_dtype: the decoder's K/V storage (None: the default f32, as the reference stores it; ct.BF16: the
    opt-in)."""

    def __init__(self, cfg: oracle.ModelConfig, weights: dict[str, np.ndarray], kv_dtype=None):
        dtype = ct.BF16 if cfg.dtype == "bf16" else ct.F32
        gpu = ct.device("gpu")
        self.cfg = cfg
        self.decoder = ct.transformer_decoder(cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden,
                                              cfg.context, dtype, gpu, cfg.rope_base, kv_dtype=kv_dtype)
        if cfg.lora_rank:
            ct.check(ct.lib().dl_transformer_decoder_attach_lora(self.decoder.handle, cfg.lora_rank, cfg.lora_alpha,
                                                                 1, 1))
        state = {}
        for name, value in weights.items():
            if name.startswith("decoder."):
                state[name[len("decoder."):]] = value
        current = self.decoder.state()
        for name, tensor in current.items():
            state.setdefault(name, tensor)
        dtypes = {n: (ct.BF16 if v.dtype == np.uint16 else None) for n, v in state.items() if isinstance(v, np.ndarray)}
        self.decoder.load_state(state, dtypes)
        self.embedding = ct.embedding_from(ct.Tensor.from_numpy(weights["tokens.weight"], dtype, gpu))
        self.head = ct.linear_from(ct.Tensor.from_numpy(weights["output.weight"], dtype, gpu))
        self.lm = ct.DecoderLM(self.embedding, self.decoder, self.head)

    def cache(self) -> ct.DecoderCache:
        return ct.DecoderCache(self.decoder)

    def generate(self, prompt, steps, temperature=0.0, key=(0, 0), use_graph=True, cache=None):
        return self.lm.generate(prompt, cache or self.cache(), steps, temperature, key, use_graph)

    def logits(self, ids, cache):
        return self.lm.logits(ids, cache)


def build_pair(cfg: oracle.ModelConfig, root=(1234, 0), scale: float = 0.02, weights=None, kv_dtype=None):
    """The oracle with the reference's f32 K/V cache, and the GPU model (f32 K/V unless kv_dtype is ct.BF16)."""
    weights = weights if weights is not None else oracle.synthesize_weights(cfg, root, scale)
    return oracle.OracleLM(cfg, weights, kv_bf16=False), GpuLM(cfg, weights, kv_dtype)


KV_DTYPES = {"f32": None, "bf16": ct.BF16}


def seed_prefix(ref_cache, gpu_cache, layer, keys, values, kv_dtype):
    """Writes a seeded prefix into both caches through KVCache::append: bf16-exact values, stored on the GPU in
    the cache's dtype (f32 by default, bf16 for the opt-in) and as f32 in the oracle's cache."""
    kb, vb = oracle.bf16_encode(keys), oracle.bf16_encode(values)
    kf, vf = oracle.bf16_decode(kb), oracle.bf16_decode(vb)
    gpu = ct.device("gpu")
    if kv_dtype == ct.BF16:
        gpu_cache.append(layer, ct.Tensor.from_numpy(kb, ct.BF16, gpu), ct.Tensor.from_numpy(vb, ct.BF16, gpu))
    else:
        gpu_cache.append(layer, ct.Tensor.from_numpy(kf, ct.F32, gpu), ct.Tensor.from_numpy(vf, ct.F32, gpu))
    ref_cache.fill(layer, keys.shape[2], kf, vf)


def say(msg):
    """Progress lines of the GPU tests (flushed: a long case names itself before it runs)."""
    print(msg, flush=True)
    sys.stdout.flush()


def rel_err(got: np.ndarray, want: np.ndarray) -> float:
    """max |got - want| / max |want| over the whole array (the f32 logit criterion)."""
    return float(np.max(np.abs(got.astype(np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))


def one_block_prefix(ref_cache, gpu_cache, layers, batch, kv_heads, length, head_dim, key, kv_dtype):
    """The same seeded N(0, 1) K and V block (bf16-exact values) in every layer: appended to the GPU cache in its
    dtype and written into the oracle's f32 cache."""
    k = oracle.randn(oracle.fold_in(key, 0), batch * kv_heads * length * head_dim)
    v = oracle.randn(oracle.fold_in(key, 1), batch * kv_heads * length * head_dim)
    kb = oracle.bf16_encode(k).reshape(batch, kv_heads, length, head_dim)
    vb = oracle.bf16_encode(v).reshape(batch, kv_heads, length, head_dim)
    del k, v
    kf, vf = oracle.bf16_decode(kb), oracle.bf16_decode(vb)
    gpu = ct.device("gpu")
    if kv_dtype == ct.BF16:
        gk, gv = ct.Tensor.from_numpy(kb, ct.BF16, gpu), ct.Tensor.from_numpy(vb, ct.BF16, gpu)
    else:
        gk, gv = ct.Tensor.from_numpy(kf, ct.F32, gpu), ct.Tensor.from_numpy(vf, ct.F32, gpu)
    for layer in range(layers):
        # each layer gets its own copy of the block (an append copies into the layer's storage)
        gpu_cache.append(layer, gk, gv)
        ref_cache.fill(layer, length, kf, vf)


def greedy_steps(ref, gpu, rc, gc, ids, steps, label):
    """`steps` eager decode steps of the GPU model and the oracle from the same ids, each step's logits within the
    bf16 tolerance; the next ids are the oracle's greedy choice (so both caches see the same history)."""
    for step in range(steps):
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        gap = float(np.max(np.abs(got - want)))
        say(f"  {label} step {step}: max|d| {gap:.3g} (max |logit| {np.max(np.abs(want)):.3g})")
        assert gap <= 2e-2, (label, step)
        ids = want.argmax(-1).reshape(-1, 1)
    return ids
