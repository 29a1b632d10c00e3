"""GPU parity at the full shapes of BASELINE's configs C3, C4 and C5, against the CPU oracle with the reference's
f32 K/V cache, through the C ABI.  (C1 and C2 run in test_gpu_parity.py.)

  C3  1B bf16 decoder, batch 32, each sequence holding 2048 cached positions of seeded random K/V (the bf16 cache
      opt-in, as BASELINE sizes this regime), 2 decode steps;
  C4  8B-width layers (d 4096, 32/8 heads, head dim 128, SwiGLU 14336, RoPE base 500000), batch 8 over 32768
      cached positions (bf16 opt-in): two full-width layers against the oracle, and the whole 32-layer model
      (weights drawn on the device) with the graph-replayed token loop equal to the eager one;
  C5  1B bf16 decoder with unmerged LoRA (rank 16, alpha 32) on q and v: a 2 x 512 prefill (tiled matrix-core
      projections, matrix-core causal attention over the f32 cache) and decode steps against the oracle, and the
      full 4 x 4096 prefill in two chunks equal to one chunk.

Tolerance: bf16 logits within 2e-2 max-abs of the oracle.  The seeded prefixes hold bf16-exact values, so both
caches start identical and only the K/V appended by the decode steps are rounded by the bf16 opt-in.
"""
import sys

import numpy as np
import pytest

import ctorch_amd as ct
import oracle
from common import build_pair, greedy_steps, one_block_prefix, rel_err

pytestmark = pytest.mark.gpu
GPU = ct.device("gpu")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.lib()
    oracle.set_threads(16)


# ------------------------------------------------------------------------------------------ C3
def test_c3_1b_batch_32_over_a_2048_token_prefix():
    say("case: C3 1B bf16, batch 32, 2048-token seeded prefix in the bf16 cache, 2 decode steps")
    cfg = oracle.ModelConfig(vocab=32000, layers=16, dimensions=2048, heads=32, kv_heads=8, hidden=5632,
                             context=2048 + 8, dtype="bf16")
    ref, gpu = build_pair(cfg, root=(3030, 0), kv_dtype=ct.BF16)
    B, P = 32, 2048
    rc, gc = ref.make_cache(B), gpu.cache()
    one_block_prefix(rc, gc, cfg.layers, B, cfg.kv_heads, P, cfg.head_dim, (3131, 0), ct.BF16)
    assert gc.length == P
    ids = oracle.random_ids((3232, 0), B, cfg.vocab).reshape(B, 1)
    greedy_steps(ref, gpu, rc, gc, ids, 2, "C3")


def test_1b_width_batch_20_splits_the_swiglu_launch_into_row_parts_of_16_and_4():
    say("case: 1B widths, 2 layers, batch 20: gate/up over 88 tile groups in row parts of 16 and 4 rows")
    cfg = oracle.ModelConfig(vocab=1000, layers=2, dimensions=2048, heads=32, kv_heads=8, hidden=5632, context=16,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(3434, 0))
    B = 20
    prompt = oracle.random_ids((3535, 0), B * 5, cfg.vocab).reshape(B, 5)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2
    greedy_steps(ref, gpu, rc, gc, want.argmax(-1).reshape(B, 1), 3, "batch 20")


# ------------------------------------------------------------------------------------------ C4
C4_WIDTH = dict(vocab=32000, dimensions=4096, heads=32, kv_heads=8, hidden=14336, rope_base=500000.0, dtype="bf16")


def test_c4_two_8b_width_layers_batch_8_over_a_32768_token_prefix():
    say("case: C4 8B-width layers (2 of 32), batch 8, 32768-token seeded prefix in the bf16 cache, 2 decode steps")
    cfg = oracle.ModelConfig(layers=2, context=32768 + 8, **C4_WIDTH)
    ref, gpu = build_pair(cfg, root=(4040, 0), kv_dtype=ct.BF16)
    B, P = 8, 32768
    rc, gc = ref.make_cache(B), gpu.cache()
    one_block_prefix(rc, gc, cfg.layers, B, cfg.kv_heads, P, cfg.head_dim, (4141, 0), ct.BF16)
    ids = oracle.random_ids((4242, 0), B, cfg.vocab).reshape(B, 1)
    greedy_steps(ref, gpu, rc, gc, ids, 2, "C4")


def device_lm(cfg: oracle.ModelConfig, root, kv_dtype=None):
    """The full model with seeded weights drawn on the device (slot s: scale * randn(fold_in(root, s)) in bf16; the
    norm weights keep their default of ones; LoRA up matrices 1e-3 * randn)."""
    decoder = ct.transformer_decoder(cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                                     ct.BF16, GPU, cfg.rope_base, kv_dtype=kv_dtype)
    if cfg.lora_rank:
        ct.check(ct.lib().dl_transformer_decoder_attach_lora(decoder.handle, cfg.lora_rank, cfg.lora_alpha, 1, 1))
    state, embedding, head = {}, None, None
    for slot, (name, shape) in enumerate(oracle.parameter_names(cfg)):
        if name.endswith("norm.weight") or name == "decoder.normalization.weight":
            continue
        w = ct.normal(ct.fold_in(root, slot), shape, 1e-3 if name.endswith("_adapter.up.weight") else 0.02, ct.BF16,
                      GPU)
        if name == "tokens.weight":
            embedding = w
        elif name == "output.weight":
            head = w
        else:
            state[name[len("decoder."):]] = w
    for name, tensor in decoder.state().items():
        state.setdefault(name, tensor)
    decoder.load_state(state)
    return decoder, ct.DecoderLM(ct.embedding_from(embedding), decoder, ct.linear_from(head))


def test_c4_full_32_layer_model_graph_replay_equals_eager():
    say("case: C4 full 8B model (32 layers, weights drawn on the device), batch 8 over a 32768-token bf16 prefix: "
        "graph-replayed greedy loop == eager loop")
    cfg = oracle.ModelConfig(layers=32, context=32768 + 16, **C4_WIDTH)
    decoder, lm = device_lm(cfg, (88, 0), kv_dtype=ct.BF16)
    B, P, hd = 8, 32768, cfg.head_dim
    cache = ct.DecoderCache(decoder)
    for layer in range(cfg.layers):
        k = ct.normal(ct.fold_in((4343, 0), 2 * layer), [B, cfg.kv_heads, P, hd], 1.0, ct.BF16, GPU)
        v = ct.normal(ct.fold_in((4343, 0), 2 * layer + 1), [B, cfg.kv_heads, P, hd], 1.0, ct.BF16, GPU)
        cache.append(layer, k, v)
        del k, v
    ids = oracle.random_ids((4444, 0), B, cfg.vocab).reshape(B, 1)
    t1, l1 = lm.generate(ids, cache, 4, 0.0, (0, 0), True)
    cache.truncate(P)
    t2, l2 = lm.generate(ids, cache, 4, 0.0, (0, 0), False)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
    assert np.all(np.isfinite(l1))
    # the first step's logits from lm_logits (eager, splits sized for the live length) agree with the loop's ids
    cache.truncate(P)
    first = lm.logits(ids, cache)
    assert np.array_equal(first.argmax(-1), t1[:, 0])


# ------------------------------------------------------------------------------------------ C5
C5 = oracle.ModelConfig(vocab=32000, layers=16, dimensions=2048, heads=32, kv_heads=8, hidden=5632, context=512 + 8,
                        dtype="bf16", lora_rank=16, lora_alpha=32.0)


def test_c5_1b_lora_prefill_2x512_and_decode_against_the_oracle():
    say("case: C5 1B bf16 + LoRA r16 a32 on q/v, prefill 2 x 512 (tiled projections, matrix-core attention over the "
        "f32 cache), then 2 decode steps")
    ref, gpu = build_pair(C5, root=(5050, 0))
    B, P = 2, 512
    prompt = oracle.random_ids((5151, 0), B * P, C5.vocab).reshape(B, P)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    gap = float(np.max(np.abs(got - want)))
    say(f"  C5 prefill: max|d| {gap:.3g}, rel {rel_err(got, want):.3g}")
    assert gap <= 2e-2
    greedy_steps(ref, gpu, rc, gc, want.argmax(-1).reshape(B, 1), 2, "C5 decode")


def test_c5_full_4x4096_prefill_in_two_chunks_equals_one_chunk():
    say("case: C5 full prefill 4 x 4096 (weights drawn on the device): one chunk vs two chunks of 2048, then the "
        "graph-replayed decode equals the eager one")
    cfg = oracle.ModelConfig(vocab=32000, layers=16, dimensions=2048, heads=32, kv_heads=8, hidden=5632,
                             context=4096 + 16, dtype="bf16", lora_rank=16, lora_alpha=32.0)
    decoder, lm = device_lm(cfg, (555, 0))
    B, P = 4, 4096
    prompt = oracle.random_ids((5252, 0), B * P, cfg.vocab).reshape(B, P)
    whole = ct.DecoderCache(decoder)
    full = lm.logits(prompt, whole)
    parts = ct.DecoderCache(decoder)
    lm.logits(prompt[:, :2048], parts)
    chunked = lm.logits(prompt[:, 2048:], parts)
    say(f"  one chunk vs two: rel {rel_err(chunked, full):.3g}")
    assert np.all(np.isfinite(full)) and rel_err(chunked, full) <= 1e-4
    ids = full.argmax(-1).reshape(B, 1)
    t1, l1 = lm.generate(ids, whole, 4, 0.0, (0, 0), True)
    whole.truncate(P)
    t2, l2 = lm.generate(ids, whole, 4, 0.0, (0, 0), False)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
