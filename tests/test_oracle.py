"""Pins the CPU oracle before it is trusted as the parity checker (CPU only).

Each check is chosen so that a plausible restatement mistake (dropped term, wrong index, wrong
rounding order, swapped operand) fails it: published known-answer vectors, closed forms evaluated
independently in float64 (numpy / torch / scipy), invariants from the reference's own tests
(tests/state.cpp:55-75), and brute force on tiny inputs.
"""
import math

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.filterwarnings("ignore::RuntimeWarning")


@pytest.fixture(scope="module", autouse=True)
def _lib():
    oracle.lib()
    oracle.set_threads(4)


# ------------------------------------------------------------------------------------------ Philox
# Random123 kat_vectors, philox4x32-10: (counter[4], key[2]) -> output[4].  The reference packs the
# counter as (index lo, index hi, stream lo, stream hi) and the key as (seed lo, seed hi)
# (src/core/philox.h:26-29).
KATS = [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
]


@pytest.mark.parametrize("counter,key,expected", KATS)
def test_philox_known_answers(counter, key, expected):
    index = counter[0] | (counter[1] << 32)
    stream = counter[2] | (counter[3] << 32)
    seed = key[0] | (key[1] << 32)
    assert oracle.philox(seed, index, stream) == expected


def test_fold_in_packs_philox_block_and_split_labels_differ():
    root = (0x1234_5678_9ABC_DEF0, 42)
    keys = {oracle.fold_in(root, i) for i in range(64)}
    assert len(keys) == 64
    x, y, z, w = oracle.philox(root[0], 7, root[1])
    assert oracle.fold_in(root, 7) == (x | (y << 32), z | (w << 32))


def test_unit_interval_endpoints():
    L = oracle.lib()
    assert L.orc_unit_f32(0, 0) == 0.0
    assert L.orc_unit_f32(0, 1) == 2.0 ** -24
    assert L.orc_unit_f32(0xFFFFFFFF, 0) == (2 ** 24 - 1) * 2.0 ** -24
    assert L.orc_unit_f64(0, 0, 1) == 2.0 ** -53
    assert L.orc_unit_f64(0xFFFFFFFF, 0xFFFFFFFF, 0) == (2 ** 53 - 1) * 2.0 ** -53


def test_keyed_normal_is_box_muller_of_the_philox_words():
    key = (99, 3)
    z = oracle.randn(key, 512)
    for i in range(0, 512, 37):
        x, _, zz, _ = oracle.philox(key[0], i, key[1])
        u1 = ((x >> 8) + 1) * 2.0 ** -24
        u2 = (zz >> 8) * 2.0 ** -24
        expected = math.sqrt(-2.0 * math.log(u1)) * math.cos(2 * math.pi * u2)
        assert abs(z[i] - expected) <= 2e-6 * max(1.0, abs(expected))
    big = oracle.randn((5, 0), 1 << 20)
    assert abs(big.mean()) < 5e-3 and abs(big.var() - 1.0) < 5e-3


def test_keyed_uniform_range_and_ids():
    u = oracle.uniform((3, 1), 100000, -2.0, 5.0)
    assert u.min() >= -2.0 and u.max() < 5.0 and abs(u.mean() - 1.5) < 0.05
    ids = oracle.random_ids((3, 1), 100000, 256)
    assert ids.min() == 0 and ids.max() == 255
    counts = np.bincount(ids, minlength=256)
    assert counts.min() > 300


# ------------------------------------------------------------------------------------------ bf16
def test_bf16_exhaustive_round_trip():
    bits = np.arange(1 << 16, dtype=np.uint16)
    values = oracle.bf16_decode(bits)
    back = oracle.bf16_encode(values)
    nan = np.isnan(values)
    assert np.array_equal(back[~nan], bits[~nan])
    assert np.array_equal(back[nan], bits[nan] | 0x40)  # NaN is quieted (half.h:45)


def test_bf16_encode_matches_torch_rne():
    rng = np.random.default_rng(0)
    raw = rng.integers(0, 1 << 32, size=1 << 18, dtype=np.uint64).astype(np.uint32)
    ties = (rng.integers(0, 1 << 16, size=4096, dtype=np.uint32) << 16) | 0x8000  # exact halfway cases
    x = np.concatenate([raw, ties]).view(np.float32)
    x = x[~np.isnan(x)]
    expected = torch.from_numpy(x.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(oracle.bf16_encode(x), expected)
    assert oracle.bf16_encode(np.array([1.0 + 2 ** -8], np.float32))[0] == 0x3F80  # tie -> even (down)
    assert oracle.bf16_encode(np.array([1.0 + 3 * 2 ** -8], np.float32))[0] == 0x3F82  # tie -> even (up)


# ------------------------------------------------------------------------------------------ RoPE
@pytest.mark.parametrize("hd,base", [(32, 10000.0), (64, 10000.0), (128, 500000.0)])
def test_rope_tables_closed_form(hd, base):
    cap = 4096
    c, s = oracle.rope_tables(hd, cap, base)
    p = np.arange(cap, dtype=np.float64)[:, None]
    freq = base ** (-2.0 * np.arange(hd // 2) / hd)
    angle = p * freq
    # f32 error budget: the exponent argument x = i*factor carries ~2|x| ulp (factor and product
    # roundings), exp adds one more, the angle product one more; cos/sin add ~1 ulp of the result
    x = np.abs(np.log(freq))
    rel = (2 * x + 3) * 2.0 ** -24
    tol = 1.5 * angle * rel + 2e-7
    assert np.all(np.abs(c - np.cos(angle)) <= tol)
    assert np.all(np.abs(s - np.sin(angle)) <= tol)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_rope_rotates_interleaved_pairs():
    rng = np.random.default_rng(1)
    hd, cap = 64, 128
    c, s = oracle.rope_tables(hd, cap)
    x = rng.standard_normal((5, 3, hd)).astype(np.float32)
    pos = np.array([0, 1, 17, 64, 127])
    y = oracle.rope(x, c, s, pos)
    assert np.array_equal(y[0], x[0])  # position 0 is the identity
    # interleaved pairs (2i, 2i+1) keep their norm and rotate by the table angle
    xe, xo = x[..., 0::2].astype(np.float64), x[..., 1::2].astype(np.float64)
    ye, yo = y[..., 0::2], y[..., 1::2]
    cc, ss = c[pos][:, None, :].astype(np.float64), s[pos][:, None, :].astype(np.float64)
    assert np.allclose(ye, xe * cc - xo * ss, atol=1e-6)
    assert np.allclose(yo, xe * ss + xo * cc, atol=1e-6)
    assert np.allclose(np.hypot(ye, yo), np.hypot(xe, xo), rtol=1e-6)


# ------------------------------------------------------------------------------------------ blocks
def test_rms_norm_closed_form():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((7, 2048)) * 3).astype(np.float32)
    w = rng.standard_normal(2048).astype(np.float32)
    y = oracle.rms_norm(x, w, 1e-5)
    xd = x.astype(np.float64)
    ref = xd / np.sqrt((xd * xd).mean(-1, keepdims=True) + 1e-5) * w
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) < 1.2e-7  # one f32 rounding of a double value
    z = oracle.rms_norm(np.zeros((1, 8), np.float32), None, 1e-5)
    assert np.all(z == 0)


def test_linear_accumulates_in_f32_sequentially():
    # (1e8 + 1) rounds back to 1e8 in f32, so the sequential f32 chain gives 1 where float64 gives 2
    x = np.array([[1e8, 1.0, -1e8, 1.0]], np.float32)
    w = np.ones((1, 4), np.float32)
    assert oracle.linear(x, w)[0, 0] == 1.0
    # reversing k flips which terms cancel: the chain is ((1 - 1e8) + 1) + 1e8 = 0 in f32
    assert oracle.linear(x[:, ::-1].copy(), w)[0, 0] == 0.0


def test_linear_exact_on_integers_and_close_on_random():
    rng = np.random.default_rng(3)
    xi = rng.integers(-8, 8, size=(3, 300)).astype(np.float32)
    wi = rng.integers(-8, 8, size=(37, 300)).astype(np.float32)
    assert np.array_equal(oracle.linear(xi, wi), (xi.astype(np.int64) @ wi.astype(np.int64).T).astype(np.float32))
    x = rng.standard_normal((4, 2048)).astype(np.float32)
    w = (rng.standard_normal((513, 2048)) * 0.02).astype(np.float32)
    wb = oracle.bf16_encode(w)
    ref = x.astype(np.float64) @ oracle.bf16_decode(wb).astype(np.float64).T
    assert np.max(np.abs(oracle.linear(x, wb) - ref)) < 1e-4
    ref32 = x.astype(np.float64) @ w.astype(np.float64).T
    assert np.max(np.abs(oracle.linear(x, w) - ref32)) < 1e-4


def test_linear_is_thread_count_invariant():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((2, 1024)).astype(np.float32)
    w = rng.standard_normal((1001, 1024)).astype(np.float32)
    oracle.set_threads(1)
    a = oracle.linear(x, w)
    oracle.set_threads(7)
    b = oracle.linear(x, w)
    oracle.set_threads(4)
    assert np.array_equal(a, b)


def test_softmax_rules():
    from scipy.special import softmax
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(1000) * 4).astype(np.float32)
    assert np.allclose(oracle.softmax_row(x), softmax(x.astype(np.float64)), rtol=1e-5, atol=1e-9)
    masked = x.copy()
    masked[600:] = -np.inf
    y = oracle.softmax_row(masked)
    assert np.all(y[600:] == 0.0)  # trailing -inf truncated to exact zero (reduction.cpp:176-180)
    assert np.allclose(y[:600], softmax(x[:600].astype(np.float64)), rtol=1e-5, atol=1e-9)
    assert oracle.softmax_row(np.array([3.5], np.float32))[0] == 1.0
    assert np.all(np.isnan(oracle.softmax_row(np.array([1.0, np.nan, 2.0], np.float32))))


def test_argmax_brute_force():
    rng = np.random.default_rng(6)
    for _ in range(400):
        n = int(rng.integers(1, 12))
        x = rng.integers(-3, 3, size=n).astype(np.float32)  # many ties
        if rng.random() < 0.3:
            x[rng.integers(0, n, size=int(rng.integers(1, 3)))] = np.nan
        if rng.random() < 0.2:
            x[rng.integers(0, n)] = -np.inf
        assert oracle.argmax_row(x) == int(np.argmax(x))  # numpy: first max, first NaN


def test_silu_closed_form():
    for v in [-80.0, -20.0, -1.5, -1e-3, 0.0, 1e-3, 0.7, 5.0, 30.0, 90.0]:
        expected = v / (1.0 + math.exp(-v))
        assert abs(oracle.silu(v) - expected) <= 2e-7 * max(1.0, abs(expected))


@pytest.mark.parametrize("L,first", [(1, 9), (5, 0), (4, 6)])
def test_grouped_attention_vs_torch_float64(L, first):
    rng = np.random.default_rng(7)
    B, H, KV, hd = 2, 8, 2, 32
    S = first + L
    q = rng.standard_normal((B, H, L, hd)).astype(np.float32)
    k = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
    v = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
    out = oracle.attention(q, k, v, causal_first=first)
    G = H // KV
    kk = torch.from_numpy(k).double().repeat_interleave(G, dim=1)  # query head h reads KV head h // G
    vv = torch.from_numpy(v).double().repeat_interleave(G, dim=1)
    qq = torch.from_numpy(q).double()
    mask = torch.arange(S)[None, :] <= (first + torch.arange(L))[:, None]
    ref = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=mask).numpy()
    assert np.max(np.abs(out - ref)) < 2e-6


@pytest.mark.parametrize("mask_shape", [(2, 8, 5, 13), (2, 1, 5, 13), (5, 13), (13,), (2, 8, 1, 13), (1, 1, 1, 1),
                                        (1, 8, 5, 1)])
def test_masked_grouped_attention_vs_torch_float64(mask_shape):
    """The keep mask of grouped_query_attention (reference src/ops/attention.cpp:48-50,156-183): broadcast to
    [B, H, L, S], a dropped key's score -inf before the softmax.  Rows that keep a key are pinned against torch's
    float64 SDPA with the same boolean attn_mask; a row that keeps none comes out NaN, which is what the
    reference's softmax of an all -inf row gives (exp(-inf - -inf)), and what torch's explicit softmax gives too
    (its SDPA returns 0 there instead, so those rows are pinned against the explicit form)."""
    rng = np.random.default_rng(11)
    B, H, KV, L, S, hd = 2, 8, 2, 5, 13, 32
    q = rng.standard_normal((B, H, L, hd)).astype(np.float32)
    k = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
    v = rng.standard_normal((B, KV, S, hd)).astype(np.float32)
    mask = rng.random(mask_shape) < 0.6
    if mask.size // mask_shape[-1] > 1:
        mask.reshape(-1, mask_shape[-1])[0] = False  # one row (or every row it broadcasts to) keeps no key
    out = oracle.attention(q, k, v, keep_mask=mask)
    G = H // KV
    kk = torch.from_numpy(k).double().repeat_interleave(G, dim=1)
    vv = torch.from_numpy(v).double().repeat_interleave(G, dim=1)
    qq = torch.from_numpy(q).double()
    mm = torch.from_numpy(np.broadcast_to(mask, (B, H, L, S)).copy())
    sdpa = torch.nn.functional.scaled_dot_product_attention(qq, kk, vv, attn_mask=mm).numpy()
    scores = (qq @ kk.transpose(-1, -2)) / math.sqrt(hd)
    explicit = (torch.softmax(scores.masked_fill(~mm, float("-inf")), -1) @ vv).numpy()
    kept = mm.any(-1).numpy()
    if kept.any():
        assert np.max(np.abs(out[kept] - sdpa[kept])) < 2e-6
    assert np.isnan(explicit[~kept]).all() and np.isnan(out[~kept]).all()
    if mask.all():
        assert np.array_equal(out, oracle.attention(q, k, v))


# ------------------------------------------------------------------------------------------ sampler
def test_portable_log_matches_libm():
    rng = np.random.default_rng(8)
    xs = np.concatenate([rng.random(2000), rng.random(500) * 1e-300, np.exp(rng.uniform(-700, 700, 2000)),
                         [1.0, 2.0, 0.5, 1.4142135623730951, 1.4142135623730954, 5e-324, 2.0 ** -1074 * 3]])
    for x in xs:
        if x <= 0:
            continue
        got, exp = oracle.log(float(x)), math.log(float(x))
        assert abs(got - exp) <= 4 * math.ulp(exp) + 1e-300, (x, got, exp)
    assert oracle.log(1.0) == 0.0


def test_sampler_low_temperature_is_argmax_and_ties_keep_first():
    rng = np.random.default_rng(9)
    logits = rng.standard_normal((6, 300)).astype(np.float32)
    got = oracle.sample(logits, 1e-6, (11, 0))
    assert np.array_equal(got, logits.argmax(-1))
    assert np.array_equal(oracle.sample(logits, 0.0, (11, 0)), logits.argmax(-1))
    nan_row = logits[:1].copy()
    nan_row[0, 17] = np.nan
    assert oracle.sample(nan_row, 1.0, (1, 2))[0] == 17


def test_sampler_frequencies_follow_softmax():
    logits = np.array([[0.0, 1.0, -1.0, 2.0, 0.5, -3.0, 1.5, 0.25]], np.float32)
    T = 1.3
    p = np.exp(logits[0] / T) / np.exp(logits[0] / T).sum()
    n = 20000
    counts = np.zeros(8)
    root = (2024, 7)
    for s in range(n):
        counts[oracle.sample(logits, T, oracle.fold_in(root, s))[0]] += 1
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 30.0  # 7 dof; p-value ~1e-4


# ------------------------------------------------------------------------------------------ decoder
def _tiny(dtype="f32", layers=2, lora=0):
    return oracle.ModelConfig(vocab=64, layers=layers, dimensions=32, heads=4, kv_heads=2, hidden=48,
                              context=16, dtype=dtype, lora_rank=lora, lora_alpha=4.0)


def test_decoder_chunked_equals_full_and_rollback():
    cfg = _tiny()
    lm = oracle.OracleLM(cfg, oracle.synthesize_weights(cfg, (17, 0), scale=0.2))
    rng = np.random.default_rng(10)
    x = rng.standard_normal((2, 6, 32)).astype(np.float32)
    full = lm.decode(x, lm.make_cache(2))
    cache = lm.make_cache(2)
    a = lm.decode(x[:, :2], cache)
    b = lm.decode(x[:, 2:], cache)
    assert np.max(np.abs(np.concatenate([a, b], 1) - full)) < 2e-6  # state.cpp:58-63
    cache.truncate(2)
    assert cache.lengths == [2, 2]
    # too-small last-layer capacity: the failing chunk rolls every layer back (state.cpp:66-70)
    small = lm.make_cache(2)
    small.structs[1].capacity = 2
    lm.decode(x[:, :1], small)
    with pytest.raises(ValueError):
        lm.decode(x[:, 1:3], small)
    assert small.lengths == [1, 1]


def _torch_decoder(cfg, w, ids, kv_round=None):
    """Float64 restatement with torch primitives (an independent check of structure and indices).  kv_round, if
    given, is applied to the rotated keys and the values before attention (the bf16 cache opt-in)."""
    d, H, KV, hd = cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.head_dim
    dec = (lambda a: torch.from_numpy(oracle.bf16_decode(a)).double()) if cfg.dtype == "bf16" else \
        (lambda a: torch.from_numpy(np.asarray(a, np.float32)).double())
    x = dec(w["tokens.weight"])[torch.from_numpy(ids)]
    B, L = ids.shape
    c, s = oracle.rope_tables(hd, cfg.context, cfg.rope_base)
    c, s = torch.from_numpy(c[:L]).double(), torch.from_numpy(s[:L]).double()

    def rope(t):  # t [B, L, heads, hd], interleaved pairs
        e, o = t[..., 0::2], t[..., 1::2]
        cc, ss = c[None, :, None, :], s[None, :, None, :]
        return torch.stack([e * cc - o * ss, e * ss + o * cc], -1).reshape(t.shape)

    def norm(t, weight):
        return torch.nn.functional.rms_norm(t, (d,), torch.from_numpy(weight).double(), eps=cfg.epsilon)

    for i in range(cfg.layers):
        p = f"decoder.layer{i}."
        h = norm(x, w[p + "attention_norm.weight"])
        q = rope((h @ dec(w[p + "attention.query.weight"]).T).reshape(B, L, H, hd)).transpose(1, 2)
        k = rope((h @ dec(w[p + "attention.key.weight"]).T).reshape(B, L, KV, hd)).transpose(1, 2)
        v = (h @ dec(w[p + "attention.value.weight"]).T).reshape(B, L, KV, hd).transpose(1, 2)
        if kv_round is not None:
            k, v = kv_round(k), kv_round(v)
        k = k.repeat_interleave(H // KV, 1)
        v = v.repeat_interleave(H // KV, 1)
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
        x = x + a.transpose(1, 2).reshape(B, L, d) @ dec(w[p + "attention.output.weight"]).T
        h = norm(x, w[p + "feedforward_norm.weight"])
        g = h @ dec(w[p + "feedforward.gate.weight"]).T
        u = h @ dec(w[p + "feedforward.up.weight"]).T
        x = x + (torch.nn.functional.silu(g) * u) @ dec(w[p + "feedforward.down.weight"]).T
    x = norm(x, w["decoder.normalization.weight"])
    return (x @ dec(w["output.weight"]).T).numpy()


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_decoder_lm_vs_torch_float64(dtype):
    cfg = _tiny(dtype)
    w = oracle.synthesize_weights(cfg, (21, 0), scale=0.2)
    lm = oracle.OracleLM(cfg, w, kv_bf16=False)
    ids = oracle.random_ids((5, 0), 2 * 9, cfg.vocab).reshape(2, 9)
    got = lm.logits(ids, lm.make_cache(2))
    ref = _torch_decoder(cfg, w, ids)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-5


def test_bf16_cache_mode_vs_torch_float64_with_rounded_keys_and_values():
    # kv_bf16=True (the product's bf16 cache opt-in) rounds every stored key and value to bf16 (RNE) and reads
    # them back; the restatement rounds its own float64 K/V through torch's bf16 conversion.  The reference's f32
    # cache (kv_bf16=False) differs from that restatement by far more than the bound, and so would a mode that
    # rounded only K or only V.
    cfg = _tiny("bf16")
    w = oracle.synthesize_weights(cfg, (22, 0), scale=0.3)
    ids = oracle.random_ids((6, 0), 2 * 9, cfg.vocab).reshape(2, 9)
    to_bf16 = lambda t: t.to(torch.bfloat16).double()
    rounded = _torch_decoder(cfg, w, ids, kv_round=to_bf16)
    bound = 2e-5 * np.max(np.abs(rounded))
    got = oracle.OracleLM(cfg, w, kv_bf16=True)
    gap = np.max(np.abs(got.logits(ids, got.make_cache(2)) - rounded))
    assert gap < bound, gap
    plain = oracle.OracleLM(cfg, w, kv_bf16=False)
    assert np.max(np.abs(plain.logits(ids, plain.make_cache(2)) - rounded)) > 10 * bound
    for only in ("k", "v"):
        half = _torch_decoder_partial_round(cfg, w, ids, only)
        assert np.max(np.abs(half - rounded)) > 10 * bound, only


def _torch_decoder_partial_round(cfg, w, ids, only):
    calls = {"n": 0}

    def round_one(t):  # called for k then v in every layer: round only the chosen one
        which = "k" if calls["n"] % 2 == 0 else "v"
        calls["n"] += 1
        return t.to(torch.bfloat16).double() if which == only else t
    return _torch_decoder(cfg, w, ids, kv_round=round_one)


def test_generate_greedy_is_consistent_with_stepwise_logits():
    cfg = _tiny("f32")
    lm = oracle.OracleLM(cfg, oracle.synthesize_weights(cfg, (3, 0), scale=0.3))
    prompt = oracle.random_ids((8, 0), 3, cfg.vocab).reshape(1, 3)
    tokens, _ = lm.generate(prompt, 5)
    seq = prompt[0].tolist()
    for t in range(5):
        logits = lm.logits(np.array([seq]), lm.make_cache(1))  # full recompute
        seq.append(int(np.argmax(logits[0, -1])))
        assert seq[-1] == tokens[0, t]


def test_lora_adapter_equals_merged_weight():
    cfg = _tiny("f32", layers=1, lora=4)
    w = oracle.synthesize_weights(cfg, (31, 0), scale=0.2)
    for n in list(w):
        if n.endswith("_adapter.up.weight"):
            w[n] = (w[n] * 200).astype(np.float32)  # make the adapter contribution visible
    lm = oracle.OracleLM(cfg, w)
    merged = dict(w)
    scale = cfg.lora_alpha / cfg.lora_rank
    for proj in ("query", "value"):
        p = f"decoder.layer0.attention.{proj}"
        B = w[f"decoder.layer0.attention.{proj}_adapter.up.weight"].astype(np.float64)
        A = w[f"decoder.layer0.attention.{proj}_adapter.down.weight"].astype(np.float64)
        merged[p + ".weight"] = (w[p + ".weight"] + scale * (B @ A)).astype(np.float32)
    plain_cfg = _tiny("f32", layers=1)
    plain = oracle.OracleLM(plain_cfg, {k: v for k, v in merged.items() if "_adapter" not in k})
    ids = oracle.random_ids((9, 0), 7, cfg.vocab).reshape(1, 7)
    a = lm.logits(ids, lm.make_cache(1))
    b = plain.logits(ids, plain.make_cache(1))
    assert np.max(np.abs(a - b)) < 1e-5
    base = oracle.OracleLM(plain_cfg, {k: v for k, v in w.items() if "_adapter" not in k})
    assert np.max(np.abs(a - base.logits(ids, base.make_cache(1)))) > 1e-3  # the adapter is not a no-op


def test_last_logits_is_the_last_position_of_the_full_logits():
    """OracleLM.last_logits runs the same C path as logits (embedding rows, orc_decoder_decode, orc_linear) with the
    head restricted to each sequence's last row: the same bits as the last position of logits, for f32 and bf16
    models, from an empty cache and from a cache that already holds a prefix."""
    for dtype in ("f32", "bf16"):
        cfg = oracle.ModelConfig(vocab=300, layers=2, dimensions=128, heads=4, kv_heads=2, hidden=256, context=40,
                                 dtype=dtype, lora_rank=4 if dtype == "bf16" else 0, lora_alpha=8.0)
        lm = oracle.OracleLM(cfg, oracle.synthesize_weights(cfg, (21, 0)))
        ids = oracle.random_ids((22, 0), 3 * 17, cfg.vocab).reshape(3, 17)
        a, b = lm.make_cache(3), lm.make_cache(3)
        assert np.array_equal(lm.last_logits(ids[:, :9], a), lm.logits(ids[:, :9], b)[:, -1])
        assert np.array_equal(lm.last_logits(ids[:, 9:], a), lm.logits(ids[:, 9:], b)[:, -1])
        assert a.length == b.length == 17
