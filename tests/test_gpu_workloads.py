"""GPU parity at BASELINE's full workload lengths, against the CPU oracle with the reference's f32 K/V cache, through
the C ABI.  The reference's decode loop (src/nn/decoder.cpp:121-142, driven by examples/decoder_generate.cpp:26-31)
runs these lengths; the shorter checks of test_gpu_parity.py and test_gpu_configs.py pin every kernel, these pin
the graph-replayed token loop that bench.py times, over whole requests.

  C2  1B bf16, 128-token prompt, 256 greedy steps replayed from the HIP graph: the loop's last logits against the
      oracle teacher-forced over the 383-position history, and every generated id a maximum of the oracle's logits
      at its position (to the tolerance);
  C3  1B bf16, batch 32 over a 2048-position seeded prefix (the bf16 cache opt-in), 16 graph-replayed steps: the
      last logits and every id against the teacher-forced oracle, and the graph-replayed loop equal to the eager
      one bit for bit;
  C5  1B bf16 with unmerged LoRA (rank 16, alpha 32) on q and v: a 1 x 4096 prefill (tiled matrix-core projections,
      causal attention over the f32 cache) against the oracle's last-position logits, then 8 decode steps.

Tolerance: bf16 logits within 2e-2 max-abs of the oracle; a generated id's oracle logit within 4e-2 of that
position's maximum (twice the logit tolerance: the GPU's own maximum may sit that far from the oracle's)."""
import numpy as np
import pytest

import ctorch_amd as ct
import oracle
from common import build_pair, greedy_steps, one_block_prefix, say

pytestmark = pytest.mark.gpu

LOGIT_TOL = 2e-2
NEAR_MAX = 4e-2
ONE_B = dict(vocab=32000, layers=16, dimensions=2048, heads=32, kv_heads=8, hidden=5632, dtype="bf16")


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.lib()
    oracle.set_threads(16)


def check_history(want, tokens, label):
    """want [steps, V]: the oracle's logits at each step's position; tokens [steps]: the GPU's ids."""
    for step, tok in enumerate(tokens):
        assert want[step, tok] >= want[step].max() - NEAR_MAX, (label, step, int(tok))


def test_c2_256_graph_replayed_greedy_steps_track_the_teacher_forced_oracle():
    say("case: C2 full request: 1B bf16, 128-token prompt, 256 greedy steps from the HIP graph, f32 cache")
    cfg = oracle.ModelConfig(context=128 + 256 + 8, **ONE_B)
    ref, gpu = build_pair(cfg, root=(2030, 0))
    prompt = oracle.random_ids((2031, 0), 128, cfg.vocab).reshape(1, 128)
    tokens, last = gpu.generate(prompt, 256)  # graph-replayed from step 2 on
    assert tokens.shape == (1, 256) and np.all(np.isfinite(last))
    history = np.concatenate([prompt, tokens[:, :-1]], 1)  # the 383 positions the last step has seen
    want = ref.logits(history, ref.make_cache(1))[0, 127:]
    gap = float(np.max(np.abs(last[0] - want[-1])))
    say(f"  last step (383 cached positions): max|d| {gap:.3g}")
    assert gap <= LOGIT_TOL
    check_history(want, tokens[0], "C2")


def test_c3_batch_32_16_graph_replayed_steps_against_the_oracle_and_the_eager_loop():
    say("case: C3 full shape: 1B bf16, batch 32 over a 2048-position seeded prefix (bf16 cache), 16 greedy steps "
        "from the HIP graph, then the same 16 eagerly")
    B, P, steps = 32, 2048, 16
    cfg = oracle.ModelConfig(context=P + steps + 8, **ONE_B)
    ref, gpu = build_pair(cfg, root=(3040, 0), kv_dtype=ct.BF16)
    rc, gc = ref.make_cache(B), gpu.cache()
    one_block_prefix(rc, gc, cfg.layers, B, cfg.kv_heads, P, cfg.head_dim, (3141, 0), ct.BF16)
    ids = oracle.random_ids((3242, 0), B, cfg.vocab).reshape(B, 1)
    tokens, last = gpu.generate(ids, steps, cache=gc)
    assert tokens.shape == (B, steps) and np.all(np.isfinite(last))
    history = np.concatenate([ids, tokens[:, :-1]], 1)  # each sequence's 16 new positions after the prefix
    want = ref.logits(history, rc)
    gap = float(np.max(np.abs(last - want[:, -1])))
    say(f"  last step ({P + steps - 1} cached positions): max|d| {gap:.3g}")
    assert gap <= LOGIT_TOL
    for b in range(B):
        check_history(want[b], tokens[b], f"C3 sequence {b}")
    # the eager loop over the same request: same kernels with the same key runs (the attention's per-wave runs
    # depend on the cache capacity only through a 256-key rounding that both lengths share), so the same bits
    gc.truncate(P)
    eager_tokens, eager_last = gpu.generate(ids, steps, use_graph=False, cache=gc)
    assert np.array_equal(eager_tokens, tokens)
    assert np.array_equal(eager_last, last)


@pytest.mark.timeout(900)
def test_c5_1x4096_lora_prefill_and_8_decode_steps_against_the_oracle():
    say("case: C5 full prompt: 1B bf16 + LoRA r16 a32 on q/v, prefill 1 x 4096 (f32 cache), then 8 greedy steps")
    P = 4096
    cfg = oracle.ModelConfig(context=P + 16, lora_rank=16, lora_alpha=32.0, **ONE_B)
    ref, gpu = build_pair(cfg, root=(5060, 0))
    prompt = oracle.random_ids((5161, 0), P, cfg.vocab).reshape(1, P)
    rc, gc = ref.make_cache(1), gpu.cache()
    got = gpu.logits(prompt, gc)
    want = ref.last_logits(prompt, rc)
    gap = float(np.max(np.abs(got - want)))
    say(f"  prefill last position: max|d| {gap:.3g} (max |logit| {np.max(np.abs(want)):.3g})")
    assert gap <= LOGIT_TOL
    assert gc.length == rc.length == P
    greedy_steps(ref, gpu, rc, gc, want.argmax(-1).reshape(1, 1), 8, "C5 decode")
