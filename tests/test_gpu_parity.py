"""GPU parity of the decoder token loop against the CPU oracle, through the C ABI.

Tolerances:
  f32 configs   logits max|d| / max|ref| <= 1e-4 per compared tensor, greedy ids identical;
  bf16 configs  logits max-abs <= 2e-2 (bf16 weights, f32 accumulation), always against the oracle with the
                reference's f32 K/V cache; the GPU keeps f32 K/V by default and bf16 K/V where a test
                parametrises the opt-in (kv="bf16");
  sampling      ids bit-identical given identical logits and key.
"""
import sys

import numpy as np
import pytest

import ctorch_amd as ct
import oracle
from common import KV_DTYPES, GpuLM, build_pair, greedy_steps, rel_err, seed_prefix

pytestmark = pytest.mark.gpu
GPU = ct.device("gpu")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.lib()
    oracle.set_threads(16)


# ------------------------------------------------------------------------------------------ C1 (f32)
C1 = oracle.ModelConfig(vocab=256, layers=4, dimensions=256, heads=8, kv_heads=2, hidden=688, context=160, dtype="f32")


def test_c1_greedy_128_tokens_identical_and_logits_within_1e4():
    say("case: C1 tiny f32, 32-byte prompt, 128 greedy tokens")
    ref, gpu = build_pair(C1, root=(101, 0))
    prompt = oracle.random_ids((202, 0), 32, 256).reshape(1, 32)
    want_tokens, want_last = ref.generate(prompt, 128)
    got_tokens, got_last = gpu.generate(prompt, 128, use_graph=True)
    assert np.array_equal(got_tokens, want_tokens)
    assert rel_err(got_last, want_last) <= 1e-4
    eager_tokens, eager_last = gpu.generate(prompt, 128, use_graph=False)
    assert np.array_equal(eager_tokens, got_tokens)
    assert np.array_equal(eager_last, got_last)  # graph replay is the eager step, bit for bit


def test_c1_stepwise_logits_and_cache_lengths():
    say("case: C1 stepwise logits through lm_logits")
    ref, gpu = build_pair(C1, root=(103, 0))
    ids = oracle.random_ids((204, 0), 2 * 12, 256).reshape(2, 12)
    rc, gc = ref.make_cache(2), gpu.cache()
    for chunk in (ids[:, :5], ids[:, 5:6], ids[:, 6:7], ids[:, 7:12]):
        want = ref.logits(chunk, rc)[:, -1]
        got = gpu.logits(chunk, gc)
        assert rel_err(got, want) <= 1e-4
        assert gc.length == rc.length


def test_decoder_api_chunked_equals_full_and_capacity_rollback():
    say("case: dl_transformer_decoder_decode chunked vs full, capacity error")
    cfg = oracle.ModelConfig(vocab=64, layers=2, dimensions=64, heads=4, kv_heads=2, hidden=96, context=16, dtype="f32")
    ref, gpu = build_pair(cfg, root=(17, 0), scale=0.2)
    x = np.random.default_rng(10).standard_normal((2, 6, 64)).astype(np.float32)
    want = ref.decode(x, ref.make_cache(2))
    cache = gpu.cache()
    a = ct.decode(gpu.decoder, ct.Tensor.from_numpy(x[:, :2], ct.F32, GPU), cache).numpy()
    b = ct.decode(gpu.decoder, ct.Tensor.from_numpy(x[:, 2:], ct.F32, GPU), cache).numpy()
    full = ct.decode(gpu.decoder, ct.Tensor.from_numpy(x, ct.F32, GPU), gpu.cache()).numpy()
    assert cache.length == 6
    assert rel_err(np.concatenate([a, b], 1), want) <= 1e-5
    assert np.max(np.abs(np.concatenate([a, b], 1) - full)) <= 1e-5
    cache.truncate(2)
    assert cache.length == 2
    again = ct.decode(gpu.decoder, ct.Tensor.from_numpy(x[:, 2:], ct.F32, GPU), cache).numpy()
    assert np.max(np.abs(again - b)) <= 1e-6
    # a chunk that exceeds the capacity fails and leaves every layer at the prefix
    with pytest.raises(ct.DLError, match="capacity"):
        ct.decode(gpu.decoder, ct.Tensor.from_numpy(np.ones((2, 11, 64), np.float32), ct.F32, GPU), cache)
    assert cache.length == 6


# ------------------------------------------------------------------------------------------ bf16
def test_bf16_model_logits_within_2e2_and_graph_equals_eager():
    say("case: bf16 2-layer d=512 model, prompt 20 + 24 greedy steps")
    cfg = oracle.ModelConfig(vocab=1000, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1376, context=64,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(31, 0), scale=0.05)
    prompt = oracle.random_ids((32, 0), 3 * 20, cfg.vocab).reshape(3, 20)
    rc, gc = ref.make_cache(3), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2
    t1, l1 = gpu.generate(prompt, 24, 1.0, (5, 6), use_graph=True)
    t2, l2 = gpu.generate(prompt, 24, 1.0, (5, 6), use_graph=False)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
    # the last sampled id is the oracle's Gumbel-max draw on the same logits and key
    key = oracle.fold_in((5, 6), 23)
    assert np.array_equal(oracle.sample(l1, 1.0, key), t1[:, -1])


def test_sampler_is_bit_exact_against_the_oracle():
    say("case: dl_sample greedy and Gumbel-max, ties and NaN rows")
    rng = np.random.default_rng(4)
    logits = (rng.standard_normal((6, 32000)) * 3).astype(np.float32)
    logits[1, 100:110] = 50.0          # ties: the first index wins
    logits[2, 7] = np.nan               # NaN wins
    logits[3] = np.round(logits[3])     # many ties under noise
    t = ct.Tensor.from_numpy(logits, ct.F32, GPU)
    for temperature, key in ((0.0, (0, 0)), (1.0, (11, 12)), (0.7, (2**63 + 5, 3)), (1e-3, (9, 9))):
        out = ct.sample(t, temperature, key).numpy()
        assert np.array_equal(out, oracle.sample(logits, temperature, key)), (temperature, key)
    greedy = ct.argmax(t, 1).numpy()
    assert np.array_equal(greedy, [oracle.argmax_row(r) for r in logits])


# ------------------------------------------------------------------------------------------ operators
def G(array, dtype=None):
    return ct.Tensor.from_numpy(array, dtype, GPU)


def test_grouped_query_attention_keep_mask_matches_the_oracle():
    """dl_grouped_query_attention with an explicit keep mask (reference include/dl/ops.h:149-153,
    src/ops/attention.cpp:48-50,156-183): a bool mask broadcast to [B, H, L, S], a dropped key's score -inf before
    the softmax, and a row that keeps no key NaN (the reference softmax of an all -inf row).  Random masks at
    several broadcast shapes, over f32 and bf16 K/V, one and several positions, key splits merged by the combine
    launch, head sizes 2 to 128, masks on the GPU and on the host; against the oracle (pinned to torch float64
    SDPA with the same mask)."""
    say("case: dl_grouped_query_attention with keep masks")
    rng = np.random.default_rng(15)
    cases = [  # B, H, KV, L, S, hd, mask shape
        (2, 8, 2, 1, 200, 64, (2, 8, 1, 200)), (2, 8, 2, 1, 200, 64, (200,)), (2, 8, 2, 5, 70, 64, (5, 70)),
        (2, 8, 2, 5, 70, 64, (2, 1, 5, 70)), (1, 32, 8, 1, 2100, 64, (1, 32, 1, 2100)),
        (3, 4, 4, 7, 33, 128, (3, 4, 7, 33)), (2, 4, 1, 6, 90, 32, (1, 4, 6, 1)), (2, 8, 2, 3, 40, 16, (3, 40)),
        (2, 4, 2, 4, 20, 2, (2, 4, 4, 20)), (1, 2, 1, 3, 150, 8, (3, 150)), (8, 8, 2, 1, 3000, 64, (8, 1, 1, 3000)),
    ]
    for B, H, KV, L, S, hd, mshape in cases:
        qq = rng.standard_normal((B, H, L, hd)).astype(np.float32)
        kk = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
        vv = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
        mask = rng.random(mshape) < 0.7
        if mask.size // mshape[-1] > 1:
            mask.reshape(-1, mshape[-1])[-1] = False  # a row (or the rows it broadcasts to) that keeps no key
        kb, vb = oracle.bf16_encode(kk), oracle.bf16_encode(vv)
        for kv_dtype in (ct.F32, ct.BF16):
            k_in = kk if kv_dtype == ct.F32 else kb
            v_in = vv if kv_dtype == ct.F32 else vb
            kf = kk if kv_dtype == ct.F32 else oracle.bf16_decode(kb)
            vf = vv if kv_dtype == ct.F32 else oracle.bf16_decode(vb)
            want = oracle.attention(qq, kf, vf, keep_mask=mask)
            for where in (GPU, ct.device("cpu")):
                m = ct.Tensor.from_numpy(mask, ct.BOOL, where)
                got = ct.grouped_query_attention(G(qq), G(k_in, kv_dtype), G(v_in, kv_dtype), m).numpy()
                case = (B, H, KV, L, S, hd, mshape, kv_dtype)
                assert np.array_equal(np.isnan(got), np.isnan(want)), case
                live = ~np.isnan(want)
                assert np.max(np.abs(got[live] - want[live])) <= 2e-5, case
        # a mask of all True equals no mask
        full = ct.Tensor.from_numpy(np.ones(mshape, bool), ct.BOOL, GPU)
        got = ct.grouped_query_attention(G(qq), G(kk), G(vv), full).numpy()
        assert np.max(np.abs(got - oracle.attention(qq, kk, vv))) <= 2e-5
    qq = rng.standard_normal((2, 8, 3, 64)).astype(np.float32)
    kk = rng.standard_normal((2, 2, 9, 64)).astype(np.float32)
    with pytest.raises(ct.DLError, match="must be bool"):
        ct.grouped_query_attention(G(qq), G(kk), G(kk), G(np.ones((3, 9), np.float32)))
    with pytest.raises(ct.DLError, match="does not broadcast"):
        ct.grouped_query_attention(G(qq), G(kk), G(kk), ct.Tensor.from_numpy(np.ones((4, 9), bool), ct.BOOL, GPU))


def test_operators_match_the_oracle():
    say("case: dl_linear / dl_rms_norm / dl_embedding / dl_rotary_embedding / dl_grouped_query_attention")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((5, 2048)).astype(np.float32)
    w = (rng.standard_normal((300, 2048)) * 0.02).astype(np.float32)
    wb = oracle.bf16_encode(w)
    for weight, dtype in ((w, ct.F32), (wb, ct.BF16)):
        y = ct.linear(G(x), G(weight, dtype)).numpy()
        assert rel_err(y, oracle.linear(x, weight)) <= 1e-5
    # several rows over bf16 weights with 16-row tiles take the matrix cores: activations split into bf16
    # hi + lo (each product carries ~2^-17 relative error), so the bound is the f32 logit tolerance, 1e-4
    # (runs of 1..2 staged chunks take the up-front variant: 2 at (3, 80, 512); longer runs the double-buffered
    # loop: 3 chunks at (3, 16, 768), 4 at (20, 96, 512), an odd count at (9, 80, 1792); at most four
    # 16-row tiles over up to 32 rows and K a multiple of 512 take the few-tile kernel: (20, 32, 512), (3, 48, 1024),
    # (32, 64, 2048))
    for rows, n, k in ((5, 320, 2048), (37, 64, 512), (64, 48, 4096), (3, 16, 768), (20, 96, 512), (3, 80, 512),
                       (9, 80, 1792), (20, 32, 512), (3, 48, 1024), (32, 64, 2048)):
        xx = rng.standard_normal((rows, k)).astype(np.float32)
        ww = oracle.bf16_encode((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        yy = ct.linear(G(xx), G(ww, ct.BF16)).numpy()
        assert rel_err(yy, oracle.linear(xx, ww)) <= 1e-4, (rows, n, k)
    # K not a multiple of the vector chunk takes the generic kernel
    xs = rng.standard_normal((3, 13)).astype(np.float32)
    ws = rng.standard_normal((7, 13)).astype(np.float32)
    assert rel_err(ct.linear(G(xs), G(ws)).numpy(), oracle.linear(xs, ws)) <= 1e-5
    g = rng.standard_normal(2048).astype(np.float32)
    y = ct.rms_norm(G(x), [2048], G(g), 1e-5).numpy()
    assert rel_err(y, oracle.rms_norm(x, g, 1e-5)) <= 1e-5
    table = oracle.bf16_encode(rng.standard_normal((50, 64)).astype(np.float32))
    ids = np.array([[3, 49, 0], [7, 7, 12]], np.int64)
    e = ct.embedding(G(ids), G(table, ct.BF16))
    assert e.dtype == ct.BF16 and np.array_equal(e.numpy(), table[ids])
    with pytest.raises(ct.DLError, match="out of range"):
        ct.embedding(G(np.array([50], np.int64)), G(table, ct.BF16))
    c, s = oracle.rope_tables(64, 9)
    q = rng.standard_normal((2, 3, 9, 64)).astype(np.float32)
    y = ct.rotary_embedding(G(q), G(c), G(s)).numpy()
    want = oracle.rope(q.transpose(0, 2, 1, 3).reshape(18, 3, 64), c, s, np.repeat(np.arange(9)[None], 2, 0).reshape(-1))
    assert np.max(np.abs(y - want.reshape(2, 9, 3, 64).transpose(0, 2, 1, 3))) <= 1e-6
    for L, S in ((1, 200), (3, 70)):
        qq = rng.standard_normal((2, 8, L, 64)).astype(np.float32)
        kk = rng.standard_normal((2, 2, S, 64)).astype(np.float32)
        vv = rng.standard_normal((2, 2, S, 64)).astype(np.float32)
        y = ct.grouped_query_attention(G(qq), G(kk), G(vv)).numpy()
        assert np.max(np.abs(y - oracle.attention(qq, kk, vv, -1))) <= 1e-5
    # one position over few bf16 keys: the matrix-core kernel in one work-group of 256 or 512 keys; past it the
    # keys split and the combine launch merges the partials (query heads per KV head: 4, 8, 16 and 1)
    for S, hd, heads in ((1, 64, 8), (64, 64, 8), (200, 64, 8), (257, 64, 8), (700, 64, 16), (300, 128, 8),
                         (1500, 64, 8), (1100, 64, 2), (300, 64, 32), (90, 128, 32)):
        qq = rng.standard_normal((2, heads, 1, hd)).astype(np.float32)
        kb = oracle.bf16_encode(rng.standard_normal((2, 2, S, hd)).astype(np.float32))
        vb = oracle.bf16_encode(rng.standard_normal((2, 2, S, hd)).astype(np.float32))
        y = ct.grouped_query_attention(G(qq), G(kb, ct.BF16), G(vb, ct.BF16)).numpy()
        want = oracle.attention(qq, oracle.bf16_decode(kb), oracle.bf16_decode(vb), -1)
        assert np.max(np.abs(y - want)) <= 2e-5, (S, hd, heads)
        # the same keys and values held as f32: the matrix-core kernel with the cache split into bf16 hi + lo
        yf = ct.grouped_query_attention(G(qq), G(oracle.bf16_decode(kb)), G(oracle.bf16_decode(vb))).numpy()
        assert np.max(np.abs(yf - want)) <= 2e-5, ("f32", S, hd, heads)
    # many keys in all: key runs per wave over f32 and bf16 K/V; 256 (sequence, KV head) pairs take a work-group
    # each (32 sequences x 8 KV heads)
    for B, KV, S, hd, heads in ((8, 2, 2100, 64, 8), (8, 2, 1500, 128, 8), (8, 2, 3000, 64, 2), (32, 8, 200, 64, 32),
                                (32, 8, 150, 128, 32)):
        qq = rng.standard_normal((B, heads, 1, hd)).astype(np.float32)
        kk = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
        vv = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
        want = oracle.attention(qq, kk, vv, -1)
        assert np.max(np.abs(ct.grouped_query_attention(G(qq), G(kk), G(vv)).numpy() - want)) <= 2e-5, (S, hd)
        kb, vb = oracle.bf16_encode(kk), oracle.bf16_encode(vv)
        want = oracle.attention(qq, oracle.bf16_decode(kb), oracle.bf16_decode(vb), -1)
        y = ct.grouped_query_attention(G(qq), G(kb, ct.BF16), G(vb, ct.BF16)).numpy()
        assert np.max(np.abs(y - want)) <= 2e-5, ("bf16", B, S, hd)
    # several positions without a keep mask see every key (no causal window), over either K/V dtype
    for L, S, hd in ((20, 40, 64), (33, 33, 128)):
        qq = rng.standard_normal((2, 8, L, hd)).astype(np.float32)
        kk = rng.standard_normal((2, 2, S, hd)).astype(np.float32)
        vv = rng.standard_normal((2, 2, S, hd)).astype(np.float32)
        want = oracle.attention(qq, kk, vv, -1)
        assert np.max(np.abs(ct.grouped_query_attention(G(qq), G(kk), G(vv)).numpy() - want)) <= 2e-5, (L, S)
        kb, vb = oracle.bf16_encode(kk), oracle.bf16_encode(vv)
        want = oracle.attention(qq, oracle.bf16_decode(kb), oracle.bf16_decode(vb), -1)
        y = ct.grouped_query_attention(G(qq), G(kb, ct.BF16), G(vb, ct.BF16)).numpy()
        assert np.max(np.abs(y - want)) <= 2e-5, ("bf16", L, S)


# ------------------------------------------------------------------------------------------ seeded prefix
@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_batched_decode_over_a_seeded_prefix(kv):
    say(f"case: B=4 decode over a 150-token seeded {kv} K/V prefix (the C3 route at small scale)")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=256, heads=8, kv_heads=2, hidden=512, context=200,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(41, 0), scale=0.05, kv_dtype=KV_DTYPES[kv])
    B, P, hd = 4, 150, cfg.head_dim
    rc, gc = ref.make_cache(B), gpu.cache()
    for layer in range(cfg.layers):
        k = oracle.randn(oracle.fold_in((77, 0), 2 * layer), B * 2 * P * hd).reshape(B, 2, P, hd)
        v = oracle.randn(oracle.fold_in((77, 0), 2 * layer + 1), B * 2 * P * hd).reshape(B, 2, P, hd)
        seed_prefix(rc, gc, layer, k, v, KV_DTYPES[kv])
    assert gc.length == P
    ids = oracle.random_ids((78, 0), B, cfg.vocab).reshape(B, 1)
    for step in range(3):
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2, step
        ids = want.argmax(-1).reshape(B, 1)


def test_batched_decode_on_matrix_cores():
    say("case: B=6 bf16 decode, d=512 (projections on the matrix cores, key-split with a reduce launch)")
    cfg = oracle.ModelConfig(vocab=1000, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1376, context=48,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(47, 0), scale=0.05)
    B = 6
    prompt = oracle.random_ids((48, 0), B * 5, cfg.vocab).reshape(B, 5)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2
    ids = want.argmax(-1).reshape(B, 1)
    for step in range(4):  # single-position steps: 6 activation rows per projection
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2, step
        ids = want.argmax(-1).reshape(B, 1)
    # those steps took the route where the attention finishes the key-split QKV projection (no reduce launch)
    assert "qkv_split" in {x["name"] for x in gpu.lm.profile(ids, gc, 1)}
    t1, l1 = gpu.generate(prompt, 10, 1.0, (3, 4), use_graph=True)
    t2, l2 = gpu.generate(prompt, 10, 1.0, (3, 4), use_graph=False)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)
    assert np.array_equal(oracle.sample(l1, 1.0, oracle.fold_in((3, 4), 9)), t1[:, -1])


def test_batched_decode_of_48_sequences_on_four_activation_tiles():
    # 33-64 rows per launch: four 16-row activation tiles, the last 16 rows past the batch (masked), through the
    # deep pipeline at K = 512 and 1536 and the LM head at 64-wide chunks
    say("case: B=48 bf16 decode, d=512 (four activation tiles per projection launch)")
    cfg = oracle.ModelConfig(vocab=1024, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1536, context=32,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(49, 0), scale=0.05)
    B = 48
    prompt = oracle.random_ids((50, 0), B * 6, cfg.vocab).reshape(B, 6)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2
    greedy_steps(ref, gpu, rc, gc, want.argmax(-1).reshape(B, 1), 3, "B=48")
    t1, l1 = gpu.generate(prompt, 8, 0.0, (0, 0), use_graph=True)
    t2, l2 = gpu.generate(prompt, 8, 0.0, (0, 0), use_graph=False)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


def test_batched_decode_without_the_repacked_weight_copies_gives_the_same_bits_and_frees_them():
    # dl_decoder_lm_set_weight_repack(0): batched decode reads the weights as stored, and the repacked copies held
    # so far go back to the pool (at least gate/up and down of every layer: widths the matrix-core path takes)
    say("case: B=8 bf16 decode with the weight repack on, off and on again")
    cfg = oracle.ModelConfig(vocab=1024, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1536, context=64,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(47, 0), scale=0.05)
    prompt = oracle.random_ids((48, 0), 8 * 16, cfg.vocab).reshape(8, 16)
    t1, l1 = gpu.generate(prompt, 12)  # repack on (the default): the copies are built on the first batched step
    held = ct.memory_stats().used_bytes
    gpu.lm.set_weight_repack(False)
    freed = held - ct.memory_stats().used_bytes
    assert freed >= cfg.layers * 3 * cfg.hidden * cfg.dimensions * 2, freed
    t2, l2 = gpu.generate(prompt, 12)
    assert np.array_equal(t2, t1) and np.array_equal(l2, l1)
    gpu.lm.set_weight_repack(True)
    t3, l3 = gpu.generate(prompt, 12)
    assert np.array_equal(t3, t1) and np.array_equal(l3, l1)
    history = np.concatenate([prompt, t1[:, :-1]], 1)
    want = ref.logits(history, ref.make_cache(8))[:, -1]
    assert np.max(np.abs(l1 - want)) <= 2e-2


def test_batched_decode_reads_weights_loaded_after_its_repacked_copies_were_built():
    say("case: B=4 bf16 decode (repacked projection weights), then new decoder weights loaded, decode again")
    cfg = oracle.ModelConfig(vocab=1000, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1024, context=32,
                             dtype="bf16")
    first = oracle.synthesize_weights(cfg, (51, 0), 0.05)
    ref, gpu = build_pair(cfg, weights=first)
    B = 4
    prompt = oracle.random_ids((52, 0), B * 3, cfg.vocab).reshape(B, 3)

    def decode(ref_model):
        rc, gc = ref_model.make_cache(B), gpu.cache()
        ids = prompt
        for step in range(4):  # the prompt, then single-position steps (the batched matrix-core route)
            want = ref_model.logits(ids, rc)[:, -1]
            got = gpu.logits(ids, gc)
            assert np.max(np.abs(got - want)) <= 2e-2, step
            ids = want.argmax(-1).reshape(B, 1)

    decode(ref)
    # the decoder's weights change in place; the embedding and the head stay
    second = oracle.synthesize_weights(cfg, (53, 0), 0.05)
    merged = {n: (second[n] if n.startswith("decoder.") else v) for n, v in first.items()}
    state = {n[len("decoder."):]: v for n, v in merged.items() if n.startswith("decoder.")}
    dtypes = {n: (ct.BF16 if v.dtype == np.uint16 else None) for n, v in state.items()}
    for name, tensor in gpu.decoder.state().items():
        state.setdefault(name, tensor)
    gpu.decoder.load_state(state, dtypes)
    decode(oracle.OracleLM(cfg, merged, kv_bf16=False))


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_head_dim_128_batched_decode_over_a_long_prefix(kv):
    say(f"case: B=8 decode, head dim 128, RoPE base 500000, 1000-token seeded {kv} prefix (the C4 route, small)")
    cfg = oracle.ModelConfig(vocab=1000, layers=2, dimensions=1024, heads=8, kv_heads=2, hidden=2048, context=1024,
                             dtype="bf16", rope_base=500000.0)
    ref, gpu = build_pair(cfg, root=(51, 0), scale=0.03, kv_dtype=KV_DTYPES[kv])
    B, P, hd = 8, 1000, cfg.head_dim
    rc, gc = ref.make_cache(B), gpu.cache()
    for layer in range(cfg.layers):
        k = oracle.randn(oracle.fold_in((81, 0), 2 * layer), B * 2 * P * hd).reshape(B, 2, P, hd)
        v = oracle.randn(oracle.fold_in((81, 0), 2 * layer + 1), B * 2 * P * hd).reshape(B, 2, P, hd)
        seed_prefix(rc, gc, layer, k, v, KV_DTYPES[kv])
    ids = oracle.random_ids((82, 0), B, cfg.vocab).reshape(B, 1)
    for step in range(3):
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2, step
        ids = want.argmax(-1).reshape(B, 1)
    # 4 key splits of 16 (sequence, KV head) pairs: the attention finishes the key-split QKV projection
    assert "qkv_split" in {x["name"] for x in gpu.lm.profile(ids, gc, 1)}
    gc.truncate(P)
    t1, l1 = gpu.generate(ids, 6, 0.0, (0, 0), use_graph=True, cache=gc)
    gc.truncate(P)
    t2, l2 = gpu.generate(ids, 6, 0.0, (0, 0), use_graph=False, cache=gc)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_decode_over_split_keys_merges_partials(kv):
    say(f"case: B=2 decode over a 600-token {kv} prefix, head dim 64, 4 query heads per KV head (key splits)")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=512, context=640,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(43, 0), scale=0.05, kv_dtype=KV_DTYPES[kv])
    B, P, hd = 2, 600, cfg.head_dim
    rc, gc = ref.make_cache(B), gpu.cache()
    for layer in range(cfg.layers):
        k = oracle.randn(oracle.fold_in((79, 0), 2 * layer), B * 2 * P * hd).reshape(B, 2, P, hd)
        v = oracle.randn(oracle.fold_in((79, 0), 2 * layer + 1), B * 2 * P * hd).reshape(B, 2, P, hd)
        seed_prefix(rc, gc, layer, k, v, KV_DTYPES[kv])
    ids = oracle.random_ids((80, 0), B, cfg.vocab).reshape(B, 1)
    for step in range(3):  # eager steps: split count from the live length, partials merged by the combine launch
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2, step
        ids = want.argmax(-1).reshape(B, 1)
    # the graph-replayed token loop (splits sized for the capacity, chunks past the length idle) equals eager
    gc.truncate(P)
    t1, l1 = gpu.generate(ids, 12, 0.0, (0, 0), use_graph=True, cache=gc)
    gc.truncate(P)
    t2, l2 = gpu.generate(ids, 12, 0.0, (0, 0), use_graph=False, cache=gc)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("batch,prefix", [(2, 1024), (4, 1024), (4, 1064)])
def test_cache_rows_past_the_length_never_reach_the_decode(batch, prefix, kv):
    # The key-split decode attention requests a wave's first K/V tile before it reads the device length, so the
    # tile holds the cache rows past the length.  Those rows are filled with NaN here (appended, then the cache
    # truncated back).  With a 1024-token prefix a wave's run starts at the new position, so its first tile is the
    # new key and 31 NaN rows; with 1064 that wave's second tile, read through a range that ends at the length,
    # holds 9 live keys.  Batch 2 projects QKV on the vector path, batch 4 in key slices that the attention
    # finishes.
    say(f"case: B={batch} decode over a {prefix}-token {kv} prefix with NaN cache rows past the length")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=512, context=1152,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(44, 0), scale=0.05, kv_dtype=KV_DTYPES[kv])
    B, P, hd, stale = batch, prefix, cfg.head_dim, 40
    rc, gc = ref.make_cache(B), gpu.cache()
    dev = ct.device("gpu")
    if KV_DTYPES[kv] == ct.BF16:
        nan = ct.Tensor.from_numpy(np.full((B, 2, stale, hd), 0x7FC0, np.uint16), ct.BF16, dev)
    else:
        nan = ct.Tensor.from_numpy(np.full((B, 2, stale, hd), np.nan, np.float32), ct.F32, dev)
    for layer in range(cfg.layers):
        k = oracle.randn(oracle.fold_in((85, 0), 2 * layer), B * 2 * P * hd).reshape(B, 2, P, hd)
        v = oracle.randn(oracle.fold_in((85, 0), 2 * layer + 1), B * 2 * P * hd).reshape(B, 2, P, hd)
        seed_prefix(rc, gc, layer, k, v, KV_DTYPES[kv])
        gc.append(layer, nan, nan)
    gc.truncate(P)
    ids = oracle.random_ids((86, 0), B, cfg.vocab).reshape(B, 1)
    steps = 8
    tokens, last = gpu.generate(ids, steps, 0.0, (0, 0), use_graph=False, cache=gc)
    assert np.all(np.isfinite(last))
    history = np.concatenate([ids, tokens[:, :-1]], 1)
    want = ref.logits(history, rc)
    assert np.max(np.abs(last - want[:, -1])) <= 2e-2
    for b in range(B):
        for step in range(steps):
            assert want[b, step, tokens[b, step]] >= want[b, step].max() - 4e-2, (b, step)
    # the graph-replayed loop over the same request (rows P + 8 .. P + 39 still NaN) gives the same bits
    gc.truncate(P)
    graph_tokens, graph_last = gpu.generate(ids, steps, 0.0, (0, 0), use_graph=True, cache=gc)
    assert np.array_equal(graph_tokens, tokens) and np.array_equal(graph_last, last)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("dimensions,heads,kv_heads", [(512, 8, 2), (512, 8, 4), (512, 8, 8), (1024, 8, 2)])
def test_streaming_decode_attention_over_many_keys(dimensions, heads, kv_heads, kv):
    # B * KV * prefix >= 32768 keys in all: one-position steps give each wave of the matrix-core kernel its own
    # run of keys (key splits merged by the combine launch)
    B, P = 8, 2100
    say(f"case: streaming decode attention, d={dimensions} heads={heads}/{kv_heads}, B={B}, {P}-token {kv} prefix")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=dimensions, heads=heads, kv_heads=kv_heads, hidden=512,
                             context=P + 24, dtype="bf16")
    assert B * kv_heads * P >= 32768
    ref, gpu = build_pair(cfg, root=(61, 0), scale=0.04, kv_dtype=KV_DTYPES[kv])
    hd = cfg.head_dim
    rc, gc = ref.make_cache(B), gpu.cache()
    for layer in range(cfg.layers):
        k = oracle.randn(oracle.fold_in((83, 0), 2 * layer), B * kv_heads * P * hd).reshape(B, kv_heads, P, hd)
        v = oracle.randn(oracle.fold_in((83, 0), 2 * layer + 1), B * kv_heads * P * hd).reshape(B, kv_heads, P, hd)
        seed_prefix(rc, gc, layer, k, v, KV_DTYPES[kv])
    ids = oracle.random_ids((84, 0), B, cfg.vocab).reshape(B, 1)
    for step in range(3):
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2, step
        ids = want.argmax(-1).reshape(B, 1)
    # graph replay (splits sized for the capacity, chunks past the length idle) equals eager
    gc.truncate(P)
    t1, l1 = gpu.generate(ids, 8, 0.0, (0, 0), use_graph=True, cache=gc)
    gc.truncate(P)
    t2, l2 = gpu.generate(ids, 8, 0.0, (0, 0), use_graph=False, cache=gc)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_prefill_on_tiled_matrix_cores_with_lora_and_causal_attention(kv):
    say(f"case: bf16 prefill B=2 x 2048, d=1024 (tiled projections + matrix-core causal attention), LoRA q/v, {kv} K/V")
    cfg = oracle.ModelConfig(vocab=512, layers=1, dimensions=1024, heads=16, kv_heads=4, hidden=2816, context=2056,
                             dtype="bf16", lora_rank=16, lora_alpha=32.0)
    weights = oracle.synthesize_weights(cfg, (61, 0), 0.03)
    # non-unit norm weights so the fused norm-weight path is exercised; bf16 values, since a bf16 decoder keeps
    # its norm weights in bf16 (the reference creates every parameter in the module's dtype)
    for i, name in enumerate(n for n in weights if n.endswith("norm.weight")):
        g = (1.0 + 0.2 * oracle.randn((63, i), cfg.dimensions)).astype(np.float32)
        weights[name] = oracle.bf16_decode(oracle.bf16_encode(g))
    ref, gpu = build_pair(cfg, weights=weights, kv_dtype=KV_DTYPES[kv])
    # the bf16 opt-in is also held to the oracle that rounds its K/V the same way, at the f32-cache bound
    same = oracle.OracleLM(cfg, weights, kv_bf16=True) if kv == "bf16" else ref
    B, P = 2, 2048
    prompt = oracle.random_ids((62, 0), B * P, cfg.vocab).reshape(B, P)
    rc, sc, gc = ref.make_cache(B), same.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    near = same.logits(prompt, sc)[:, -1] if same is not ref else want
    got = gpu.logits(prompt, gc)
    say(f"  prefill logits: max|d| {np.max(np.abs(got - want)):.3g}, rel {rel_err(got, want):.3g}; "
        f"vs the same-K/V oracle rel {rel_err(got, near):.3g}")
    # bf16 criterion (2e-2 max-abs) against the reference's f32 cache; the hi + lo activations (and hi + lo
    # K/V of an f32 cache) keep the gap to the oracle with the same K/V storage far below it
    assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, near) <= 5e-4
    ids = want.argmax(-1).reshape(B, 1)
    for step in range(2):  # decode over the 2048 keys the tiled QKV epilogue wrote
        want = ref.logits(ids, rc)[:, -1]
        near = same.logits(ids, sc)[:, -1] if same is not ref else want
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, near) <= 5e-4, step
        ids = want.argmax(-1).reshape(B, 1)
    # two chunks of 1024 (the second attends with an offset) equal the single chunk
    full = gpu.logits(prompt, gpu.cache())
    chunked_cache = gpu.cache()
    gpu.logits(prompt[:, :1024], chunked_cache)
    chunked = gpu.logits(prompt[:, 1024:], chunked_cache)
    assert rel_err(chunked, full) <= 1e-4
    # a truncated cache prefilled again from position 1500 (548 rows: the batched projection path, attention
    # with an offset) equals the single chunk
    chunked_cache.truncate(1500)
    again = gpu.logits(prompt[:, 1500:], chunked_cache)
    assert rel_err(again, full) <= 1e-4


def test_prefill_of_four_sequences_takes_the_tiled_projection_in_groups_of_four_row_blocks():
    # 4 x 2048 rows are 32 row blocks of 256: each XCD takes a band of 4 and walks it in one group of 4 row blocks
    # (the C5 order); two chunks of 1024 per sequence (16 row blocks, groups of 2) must give the same logits, and
    # the 8 (sequence, KV head) pairs take the prefill attention's one-XCD-per-pair order
    say("case: bf16 prefill B=4 x 2048, d=512, LoRA q/v, f32 K/V: tiled projections in groups of 4 row blocks")
    cfg = oracle.ModelConfig(vocab=512, layers=1, dimensions=512, heads=8, kv_heads=2, hidden=1536, context=2056,
                             dtype="bf16", lora_rank=16, lora_alpha=32.0)
    ref, gpu = build_pair(cfg, root=(64, 0), scale=0.03)
    B, P = 4, 2048
    prompt = oracle.random_ids((65, 0), B * P, cfg.vocab).reshape(B, P)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    got = gpu.logits(prompt, gc)
    say(f"  prefill logits: max|d| {np.max(np.abs(got - want)):.3g}, rel {rel_err(got, want):.3g}")
    assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4
    ids = want.argmax(-1).reshape(B, 1)
    for step in range(2):  # decode over the keys the tiled QKV epilogue wrote
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4, step
        ids = want.argmax(-1).reshape(B, 1)
    full = gpu.logits(prompt, gpu.cache())
    chunked_cache = gpu.cache()
    gpu.logits(prompt[:, :1024], chunked_cache)
    chunked = gpu.logits(prompt[:, 1024:], chunked_cache)
    assert rel_err(chunked, full) <= 1e-4


@pytest.mark.parametrize("rank,batch", [(8, 4), (16, 4), (16, 16), (32, 4), (16, 32)])
def test_decode_with_lora_down_rows_folded_into_the_qkv_launch(rank, batch):
    # a decode step of 4..16 rows takes the few-row matrix-core QKV kernel, which at ranks 4..16 applies the LoRA
    # down rows in its own key loop (rank 8: half the operand rows repeat and the up operand is zero past the
    # rank); rank 32, and 32 rows (the key-split kernel), keep the separate down launch.  The prompt's prefill
    # (more rows) takes the separate launch.
    say(f"case: bf16 decode B={batch}, d=512, LoRA q/v rank {rank} (up weights 0.05 randn), f32 K/V")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=1024, context=64,
                             dtype="bf16", lora_rank=rank, lora_alpha=2.0 * rank)
    weights = oracle.synthesize_weights(cfg, (71, rank), 0.03)
    ups = sorted(n for n in weights if "adapter.up" in n)
    # up weights far above the synthesizer's 1e-3 randn, so the adapters move the logits well past the bound
    for i, name in enumerate(ups):
        weights[name] = oracle.bf16_encode(0.05 * oracle.randn((72, i), weights[name].size)).reshape(weights[name].shape)
    ref, gpu = build_pair(cfg, weights=weights)
    plain = oracle.OracleLM(cfg, {n: (np.zeros_like(v) if n in ups else v) for n, v in weights.items()})
    P = 20
    prompt = oracle.random_ids((73, rank), batch * P, cfg.vocab).reshape(batch, P)
    rc, pc, gc = ref.make_cache(batch), plain.make_cache(batch), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    plain.logits(prompt, pc)
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4
    ids = want.argmax(-1).reshape(batch, 1)
    for step in range(3):
        want = ref.logits(ids, rc)[:, -1]
        without = plain.logits(ids, pc)[:, -1]
        got = gpu.logits(ids, gc)
        say(f"  step {step}: max|d| {np.max(np.abs(got - want)):.3g}, rel {rel_err(got, want):.3g}; "
            f"the adapters' share rel {rel_err(without, want):.3g}")
        assert rel_err(without, want) >= 20 * 5e-4, step  # a dropped or halved adapter term fails the bound
        assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4, step
        ids = want.argmax(-1).reshape(batch, 1)
    # graph replay of the decode equals eager
    gc.truncate(P + 3)
    t1, l1 = gpu.generate(ids, 4, 0.0, (0, 0), use_graph=True, cache=gc)
    gc.truncate(P + 3)
    t2, l2 = gpu.generate(ids, 4, 0.0, (0, 0), use_graph=False, cache=gc)
    assert np.array_equal(t1, t2) and np.array_equal(l1, l2)


def test_tiled_prefill_with_lora_and_a_partial_qkv_column_block():
    # d = 256, 8/2 heads of 32: the QKV projection has 24 weight tiles, one full column block of 16 and one of 8,
    # which runs the tiled kernel's checked products and its LoRA epilogue on the missing tiles' slots
    say("case: bf16 prefill B=2 x 512, d=256 (QKV 384 columns: a partial column block), LoRA q/v rank 16, f32 K/V")
    cfg = oracle.ModelConfig(vocab=256, layers=2, dimensions=256, heads=8, kv_heads=2, hidden=512, context=520,
                             dtype="bf16", lora_rank=16, lora_alpha=32.0)
    weights = oracle.synthesize_weights(cfg, (77, 0), 0.05)
    ups = sorted(n for n in weights if "adapter.up" in n)
    for i, name in enumerate(ups):
        weights[name] = oracle.bf16_encode(0.05 * oracle.randn((78, i), weights[name].size)).reshape(weights[name].shape)
    ref, gpu = build_pair(cfg, weights=weights)
    plain = oracle.OracleLM(cfg, {n: (np.zeros_like(v) if n in ups else v) for n, v in weights.items()})
    B, P = 2, 512
    prompt = oracle.random_ids((79, 0), B * P, cfg.vocab).reshape(B, P)
    rc, gc = ref.make_cache(B), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    without = plain.logits(prompt, plain.make_cache(B))[:, -1]
    got = gpu.logits(prompt, gc)
    say(f"  prefill logits: max|d| {np.max(np.abs(got - want)):.3g}, rel {rel_err(got, want):.3g}; "
        f"the adapters' share rel {rel_err(without, want):.3g}")
    assert rel_err(without, want) >= 20 * 5e-4
    assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4
    ids = want.argmax(-1).reshape(B, 1)
    for step in range(2):  # decode over the keys the tiled QKV epilogue wrote
        want = ref.logits(ids, rc)[:, -1]
        got = gpu.logits(ids, gc)
        assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4, step
        ids = want.argmax(-1).reshape(B, 1)


@pytest.mark.parametrize("batch", [4, 16])
def test_decode_with_lora_folded_at_the_c5_width(batch):
    # the C5 layer (d = 2048, 32/8 heads, F = 5632, rank 16): each of the QKV launch's 16 waves takes 128 keys, four
    # k steps of the down rows in one batch of loads
    say(f"case: bf16 decode B={batch}, one C5-width layer, LoRA q/v rank 16 (up weights 0.05 randn), f32 K/V")
    cfg = oracle.ModelConfig(vocab=512, layers=1, dimensions=2048, heads=32, kv_heads=8, hidden=5632, context=40,
                             dtype="bf16", lora_rank=16, lora_alpha=32.0)
    weights = oracle.synthesize_weights(cfg, (74, batch), 0.02)
    ups = sorted(n for n in weights if "adapter.up" in n)
    for i, name in enumerate(ups):
        weights[name] = oracle.bf16_encode(0.05 * oracle.randn((75, i), weights[name].size)).reshape(weights[name].shape)
    ref, gpu = build_pair(cfg, weights=weights)
    plain = oracle.OracleLM(cfg, {n: (np.zeros_like(v) if n in ups else v) for n, v in weights.items()})
    P = 12
    prompt = oracle.random_ids((76, batch), batch * P, cfg.vocab).reshape(batch, P)
    rc, pc, gc = ref.make_cache(batch), plain.make_cache(batch), gpu.cache()
    want = ref.logits(prompt, rc)[:, -1]
    plain.logits(prompt, pc)
    got = gpu.logits(prompt, gc)
    assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4
    ids = want.argmax(-1).reshape(batch, 1)
    for step in range(3):
        want = ref.logits(ids, rc)[:, -1]
        without = plain.logits(ids, pc)[:, -1]
        got = gpu.logits(ids, gc)
        say(f"  step {step}: max|d| {np.max(np.abs(got - want)):.3g}, rel {rel_err(got, want):.3g}; "
            f"the adapters' share rel {rel_err(without, want):.3g}")
        assert rel_err(without, want) >= 20 * 5e-4, step
        assert np.max(np.abs(got - want)) <= 2e-2 and rel_err(got, want) <= 5e-4, step
        ids = want.argmax(-1).reshape(batch, 1)


def test_graph_decode_at_a_capacity_far_above_the_length_ignores_stale_workspace_memory():
    # graph replay sizes the key splits for the cache capacity, so most splits hold no keys and never write their
    # partial output rows; the merge must not read them.  The pool is first filled with NaN blocks and released, so
    # the workspaces the decode allocates next are likely to reuse NaN-holding memory.
    say("case: f32-cache decode at capacity 4096 over a 20-token prompt after NaN-filled pool blocks were released")
    cfg = oracle.ModelConfig(vocab=512, layers=2, dimensions=512, heads=8, kv_heads=2, hidden=512, context=4096,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(45, 0), scale=0.05)
    stale = [G(np.full(n, np.nan, np.float32)) for n in (1 << 14, 1 << 16, 1 << 18, 1 << 20) for _ in range(8)]
    ct.synchronize()
    del stale
    prompt = oracle.random_ids((46, 0), 20, cfg.vocab).reshape(1, 20)
    tokens, last = gpu.generate(prompt, 12, use_graph=True)
    assert np.all(np.isfinite(last))
    history = np.concatenate([prompt, tokens[:, :-1]], 1)
    teacher = ref.logits(history, ref.make_cache(1))[0, -1]
    assert np.max(np.abs(last[0] - teacher)) <= 2e-2


# ------------------------------------------------------------------------------------------ C2 shape
def test_c2_1b_bf16_128_token_prompt_and_16_steps_against_the_f32_cache_oracle():
    say("case: C2 1B bf16 (16 layers, d=2048, 32/8 heads, F=5632, V=32000), 128-token prompt + 16 greedy steps, "
        "then 4 sampled steps at temperature 1")
    cfg = oracle.ModelConfig(vocab=32000, layers=16, dimensions=2048, heads=32, kv_heads=8, hidden=5632, context=176,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(2024, 1))
    prompt = oracle.random_ids((2025, 0), 128, cfg.vocab).reshape(1, 128)
    # the GPU's own greedy history, every step's logits kept (eager steps through lm_logits)
    gc = gpu.cache()
    logits = [gpu.logits(prompt, gc)]
    ids = [int(logits[-1].argmax())]
    for _ in range(15):
        logits.append(gpu.logits(np.array([[ids[-1]]], np.int64), gc))
        ids.append(int(logits[-1].argmax()))
    # teacher-forced oracle over the same history, with the reference's f32 K/V cache
    history = np.concatenate([prompt, np.array([ids[:-1]], np.int64)], 1)
    want = ref.logits(history, ref.make_cache(1))[0, 127:]
    got = np.concatenate(logits, 0)
    gaps = np.max(np.abs(got - want), axis=1)
    say(f"  max|d| per step: first {gaps[0]:.3g}, last {gaps[-1]:.3g}, worst {gaps.max():.3g}")
    assert gaps.max() <= 2e-2
    for step in range(16):  # each greedy id is a maximum of the oracle's logits up to the tolerance
        assert want[step, ids[step]] >= want[step].max() - 4e-2, step
    # the graph-replayed token loop reproduces the eager history and its last logits
    tokens, last = gpu.generate(prompt, 16)
    assert np.array_equal(tokens[0], ids) and np.max(np.abs(last[0] - got[-1])) <= 1e-5
    # temperature 1.0 with an explicit key: at every step the device sampler draws the oracle's Gumbel-max id
    # from the same logits and fold_in(key, step), and the logits along the sampled history stay within the
    # tolerance of the teacher-forced oracle
    key = (99, 1)
    sc = gpu.cache()
    step_logits = gpu.logits(prompt, sc)
    drawn, sampled_logits = [], []
    for step in range(4):
        k = oracle.fold_in(key, step)
        draw = ct.sample(G(step_logits), 1.0, k).numpy()
        assert np.array_equal(draw, oracle.sample(step_logits, 1.0, k)), step
        drawn.append(int(draw[0]))
        sampled_logits.append(step_logits)
        step_logits = gpu.logits(draw.reshape(1, 1), sc)
    history = np.concatenate([prompt, np.array([drawn[:-1]], np.int64)], 1)
    want = ref.logits(history, ref.make_cache(1))[0, 127:]
    assert np.max(np.abs(np.concatenate(sampled_logits, 0) - want)) <= 2e-2
    # the graph-replayed loop samples on the device the same way: its last id is the oracle's draw on its last
    # logits
    sampled, last = gpu.generate(prompt, 4, 1.0, key)
    assert np.array_equal(oracle.sample(last, 1.0, oracle.fold_in(key, 3)), sampled[:, -1])


# ------------------------------------------------------------------------------------------ cache wire format
@pytest.mark.parametrize("dtype,kv", [("f32", "f32"), ("bf16", "f32"), ("bf16", "bf16")])
def test_cache_state_export_matches_the_oracle_and_import_continues_the_decode(dtype, kv):
    say(f"case: {dtype} model, {kv} cache exported as past_key_i / past_value_i after a 9-token prompt, imported, "
        f"2 more steps")
    cfg = oracle.ModelConfig(vocab=256, layers=2, dimensions=256, heads=8, kv_heads=2, hidden=512, context=32,
                             dtype=dtype)
    ref, gpu = build_pair(cfg, root=(61, 0), scale=0.05, kv_dtype=KV_DTYPES[kv])
    prompt = oracle.random_ids((62, 0), 2 * 9, cfg.vocab).reshape(2, 9)
    rc, gc = ref.make_cache(2), gpu.cache()
    ref.logits(prompt, rc)
    gpu.logits(prompt, gc)
    state = {name: t.numpy() for name, t in gc.state().items()}
    assert sorted(state) == sorted(f"past_{kind}_{i}" for i in range(cfg.layers) for kind in ("key", "value"))
    for i in range(cfg.layers):
        for kind, want in (("key", rc.keys[i]), ("value", rc.values[i])):
            got = state[f"past_{kind}_{i}"]
            assert got.shape == (2, cfg.kv_heads, 9, cfg.head_dim)
            if kv == "f32":  # K/V of an f32 or bf16 model, stored as computed
                assert rel_err(got, want[:, :, :9]) <= 1e-4, (kind, i)
            else:  # the bf16 opt-in rounds each stored value (and layer 1's inputs saw rounded K/V of layer 0)
                assert np.max(np.abs(got - want[:, :, :9])) <= 2e-2, (kind, i)
    copy = gpu.cache()
    copy.load_state(gpu.decoder, state)
    assert copy.length == 9
    assert all(np.array_equal(t.numpy(), state[n]) for n, t in copy.state().items())
    ids = oracle.random_ids((63, 0), 2, cfg.vocab).reshape(2, 1)
    for step in range(2):
        a = gpu.logits(ids, gc)
        b = gpu.logits(ids, copy)
        assert np.array_equal(a, b), step  # the same cache contents give the same decode, bit for bit
        ids = a.argmax(-1).reshape(2, 1)


# ------------------------------------------------------------------------------------------ device migration
def test_decoder_built_on_the_host_moves_to_the_gpu_and_its_memory_returns_to_the_pool():
    say("case: f32 decoder loaded on the host, Module::to(gpu), decode vs oracle, pool statistics and trim")
    cfg = oracle.ModelConfig(vocab=64, layers=2, dimensions=128, heads=4, kv_heads=2, hidden=256, context=16,
                             dtype="f32")
    weights = oracle.synthesize_weights(cfg, (71, 0), 0.1)
    ref = oracle.OracleLM(cfg, weights)
    dec = ct.transformer_decoder(cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                                 ct.F32, ct.device("cpu"), cfg.rope_base)
    state = {name[len("decoder."):]: value for name, value in weights.items() if name.startswith("decoder.")}
    for name, tensor in dec.state().items():
        state.setdefault(name, tensor)
    dec.load_state(state)
    weight_bytes = sum(v.nbytes for v in state.values() if isinstance(v, np.ndarray))
    ct.release_unused()
    before = ct.memory_stats()
    dec.to(GPU)
    moved = ct.memory_stats()
    assert moved.used_bytes - before.used_bytes >= weight_bytes
    x = np.random.default_rng(12).standard_normal((2, 5, cfg.dimensions)).astype(np.float32)
    want = ref.decode(x, ref.make_cache(2))
    got = ct.decode(dec, G(x), ct.DecoderCache(dec)).numpy()
    assert rel_err(got, want) <= 1e-5
    del dec
    ct.release_unused()
    after = ct.memory_stats()
    assert after.used_bytes <= moved.used_bytes - weight_bytes
    assert after.reserved_bytes <= moved.reserved_bytes and after.peak_used_bytes >= moved.used_bytes
    ct.reset_peak_stats()
    reset = ct.memory_stats()
    assert reset.peak_used_bytes < moved.used_bytes  # HIP restarts the high-water marks at zero
    block = G(np.zeros(1 << 18, np.float32))
    assert ct.memory_stats().peak_used_bytes >= reset.used_bytes + block.numpy().nbytes
    keep = after.release_threshold
    ct.set_release_threshold(1 << 20)
    assert ct.memory_stats().release_threshold == 1 << 20
    ct.set_release_threshold(keep)
    assert ct.memory_stats().release_threshold == keep


# ------------------------------------------------------------------------------------------ forward without a cache
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_forward_without_a_cache_over_a_sequence_the_reference_would_block(dtype):
    # TransformerDecoder::forward (reference src/nn/decoder.cpp:116-120) runs causal attention over the whole
    # input; at B=1, H=8, S=2048 the reference splits the queries into blocks of (8 Mi / (B*H*S)) = 512 rows
    # (src/ops/attention.cpp:59-63), which leaves the result unchanged.
    say(f"case: {dtype} TransformerDecoder::forward on [1, 2048, 256], no cache, vs the oracle's prefill")
    cfg = oracle.ModelConfig(vocab=64, layers=2, dimensions=256, heads=8, kv_heads=2, hidden=512, context=2048,
                             dtype=dtype)
    ref, gpu = build_pair(cfg, root=(81, 0), scale=0.05)
    x = np.random.default_rng(13).standard_normal((1, 2048, cfg.dimensions)).astype(np.float32)
    want = ref.decode(x, ref.make_cache(1))
    got = gpu.decoder.forward(G(x)).numpy()
    assert got.shape == want.shape
    if dtype == "f32":
        assert rel_err(got, want) <= 1e-4
    else:
        assert np.max(np.abs(got - want)) <= 2e-2
    again = gpu.decoder.forward(G(x)).numpy()
    assert np.array_equal(again, got)  # no state is kept between calls


# ------------------------------------------------------------------------------------------ tensor archives
def test_gpu_decoder_state_saved_to_an_archive_loads_into_a_fresh_gpu_decoder(tmp_path):
    say("case: bf16 GPU decoder state -> .ct archive -> fresh GPU decoder, decode bit for bit")
    cfg = oracle.ModelConfig(vocab=256, layers=2, dimensions=256, heads=8, kv_heads=2, hidden=512, context=32,
                             dtype="bf16")
    ref, gpu = build_pair(cfg, root=(91, 0), scale=0.05)
    path = tmp_path / "decoder.ct"
    ct.save_state(str(path), gpu.decoder.state())  # device tensors are copied to the host by the save
    loaded = ct.load_state(str(path))
    assert all(t.info.device.type == ct.CPU for t in loaded.values())
    fresh = ct.transformer_decoder(cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.context,
                                   ct.BF16, GPU, cfg.rope_base)
    fresh.load_state(loaded)
    x = np.random.default_rng(14).standard_normal((2, 6, cfg.dimensions)).astype(np.float32)
    a = ct.decode(gpu.decoder, G(x), ct.DecoderCache(gpu.decoder)).numpy()
    b = ct.decode(fresh, G(x), ct.DecoderCache(fresh)).numpy()
    assert np.array_equal(a, b)
    assert np.max(np.abs(a - ref.decode(x, ref.make_cache(2)))) <= 2e-2
