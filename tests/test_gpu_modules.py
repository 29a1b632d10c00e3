"""GPU checks of the module entries and integer paths outside the fused token step, through the C ABI:

  dl_lora_linear_create / dl_lora_linear_merge   LoRALinear::forward against the oracle, and the reference's invariant
                                                 adapter(x) == merged()(x) (tests/state.cpp:71-75);
  dl_swiglu_create                               SwiGLU::forward (src/nn/decoder.cpp:11-16) against the oracle;
  dl_grouped_query_attention_create              GroupedQueryAttention::forward (causal, no cache) against the oracle;
  dl_rotary_embedding_create / _forward          RoPE at an offset against the oracle's tables and rotation;
  dl_tensordot                                   against numpy in float64;
  dl_astype on the GPU                           the bf16 codec (include/dl/half.h:43-47, 60-66) bit for bit against the
                                                 oracle over 2^24 random words, every tie class, NaN, Inf, subnormals,
                                                 and all 2^16 bf16 values back to f32;
  dl_uniform_with_key / dl_normal_with_key       keyed device randomness against the oracle (src/kernels/cpu/random.cpp:
                                                 52-83): uniform bit for bit; normal through the device's logf/cosf.
"""
import ctypes as C
import sys

import numpy as np
import pytest

import ctorch_amd as ct
import oracle
from common import rel_err

pytestmark = pytest.mark.gpu
GPU = ct.device("gpu")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def G(array, dtype=None):
    return ct.Tensor.from_numpy(array, dtype, GPU)


def module(fn, *args):
    return ct.Module(ct._new(fn, *args))


def load(mod, values, dtypes=None):
    current = mod.state()
    state = dict(values)
    for name, tensor in current.items():
        state.setdefault(name, tensor)
    mod.load_state(state, dtypes)


def astype(t, dtype):
    """dl_astype; `t` stays referenced by the caller for the duration of the call."""
    return ct.Tensor(ct._new(ct.lib().dl_astype, t.handle, dtype))


def silu(v):
    return np.vectorize(oracle.silu, otypes=[np.float32])(v)


# ------------------------------------------------------------------------------------------ LoRALinear
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_lora_linear_forward_and_merged_weight(dtype):
    say(f"case: LoRALinear ({dtype}) forward vs oracle, adapter(x) == merged()(x)")
    rng = np.random.default_rng(21)
    n, k, r, alpha = 96, 256, 8, 16.0
    wt = ct.BF16 if dtype == "bf16" else ct.F32
    w = (rng.standard_normal((n, k)) * 0.05).astype(np.float32)
    a = (rng.standard_normal((r, k)) * 0.05).astype(np.float32)
    b = (rng.standard_normal((n, r)) * 0.05).astype(np.float32)
    if dtype == "bf16":
        w, a, b = oracle.bf16_encode(w), oracle.bf16_encode(a), oracle.bf16_encode(b)
    base = ct.linear_from(G(w, wt))
    adapter = module(ct.lib().dl_lora_linear_create, base.handle, r, alpha)
    state = adapter.state()
    assert list(state) == ["weight", "down.weight", "up.weight"]  # the reference's registration order
    assert not np.any(state["up.weight"].numpy())                   # up starts at zero
    load(adapter, {"down.weight": a, "up.weight": b}, {"down.weight": wt, "up.weight": wt})
    x = rng.standard_normal((5, k)).astype(np.float32)
    got = adapter.forward(G(x)).numpy()
    want = oracle.linear(x, w) + np.float32(alpha / r) * oracle.linear(oracle.linear(x, a), b)
    # 5 rows over bf16 weights take the matrix cores (activations split hi + lo): the f32 logit bound
    assert rel_err(got, want) <= 1e-4
    merged = module(ct.lib().dl_lora_linear_merge, adapter.handle)
    merged_w = merged.state()["weight"]
    assert merged_w.dtype == wt
    # merged() = W + (alpha/r) B A accumulated in f32 and rounded once to W's dtype
    to32 = oracle.bf16_decode if dtype == "bf16" else (lambda v: v)
    exact = to32(w).astype(np.float64) + (alpha / r) * (to32(b).astype(np.float64) @ to32(a).astype(np.float64))
    got_w = to32(merged_w.numpy())
    assert np.max(np.abs(got_w - exact)) <= (2.0 ** -8 * np.max(np.abs(exact)) if dtype == "bf16" else 1e-6)
    y_merged = merged.forward(G(x)).numpy()
    # the invariant of tests/state.cpp:71-75: the adapter equals its merged Linear (up to the merged weight's rounding)
    assert np.max(np.abs(y_merged - got)) <= (2e-2 if dtype == "bf16" else 1e-5) * np.max(np.abs(got))
    assert abs(float(np.sum(y_merged)) - float(np.sum(got))) <= (1e-2 if dtype == "bf16" else 1e-4) * np.sum(np.abs(got))


# ------------------------------------------------------------------------------------------ SwiGLU
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_swiglu_module_matches_the_oracle(dtype):
    say(f"case: SwiGLU module ({dtype}) via dl_swiglu_create")
    rng = np.random.default_rng(22)
    d, F = 512, 1376
    wt = ct.BF16 if dtype == "bf16" else ct.F32
    mod = module(ct.lib().dl_swiglu_create, d, F, 0, ct.options(wt, GPU))
    assert list(mod.state()) == ["gate.weight", "up.weight", "down.weight"]
    ws = {n: (rng.standard_normal(s) * 0.04).astype(np.float32) for n, s in
          (("gate.weight", (F, d)), ("up.weight", (F, d)), ("down.weight", (d, F)))}
    if dtype == "bf16":
        ws = {n: oracle.bf16_encode(v) for n, v in ws.items()}
    load(mod, ws, {n: wt for n in ws})
    x = rng.standard_normal((3, 7, d)).astype(np.float32)
    got = mod.forward(G(x)).numpy()
    h = silu(oracle.linear(x, ws["gate.weight"])) * oracle.linear(x, ws["up.weight"])
    want = oracle.linear(h, ws["down.weight"])
    assert got.shape == (3, 7, d) and rel_err(got, want) <= 1e-4


# ------------------------------------------------------------------------------------------ GQA module
@pytest.mark.parametrize("heads,kv_heads,hd", [(8, 2, 64), (4, 4, 32), (16, 4, 128)])
def test_grouped_query_attention_module_forward_matches_the_oracle(heads, kv_heads, hd):
    say(f"case: GroupedQueryAttention module forward, {heads}/{kv_heads} heads, head dim {hd}")
    rng = np.random.default_rng(23)
    d = heads * hd
    B, L = 2, 37
    mod = module(ct.lib().dl_grouped_query_attention_create, d, heads, kv_heads, 64, ct.options(ct.F32, GPU))
    names = ["query.weight", "key.weight", "value.weight", "output.weight"]
    assert [n for n in mod.state() if n.endswith("weight")] == names
    shapes = {"query.weight": (d, d), "key.weight": (kv_heads * hd, d), "value.weight": (kv_heads * hd, d),
              "output.weight": (d, d)}
    ws = {n: (rng.standard_normal(s) * (1.0 / np.sqrt(d))).astype(np.float32) for n, s in shapes.items()}
    load(mod, ws)
    x = rng.standard_normal((B, L, d)).astype(np.float32)
    got = mod.forward(G(x)).numpy()
    c, s = oracle.rope_tables(hd, 64)
    pos = np.tile(np.arange(L), B)
    q = oracle.rope(oracle.linear(x, ws["query.weight"]).reshape(B * L, heads, hd), c, s, pos)
    k = oracle.rope(oracle.linear(x, ws["key.weight"]).reshape(B * L, kv_heads, hd), c, s, pos)
    v = oracle.linear(x, ws["value.weight"]).reshape(B * L, kv_heads, hd)
    to_bhld = lambda t, h: t.reshape(B, L, h, hd).transpose(0, 2, 1, 3)
    att = oracle.attention(to_bhld(q, heads), to_bhld(k, kv_heads), to_bhld(v, kv_heads), 0)
    want = oracle.linear(att.transpose(0, 2, 1, 3).reshape(B, L, d), ws["output.weight"])
    # 37 positions take the matrix-core prefill attention where it serves the head layout (f32 K/V split hi + lo)
    assert rel_err(got, want) <= 1e-4


# ------------------------------------------------------------------------------------------ RoPE module
def test_rotary_embedding_module_at_an_offset():
    say("case: RotaryEmbedding module (head dim 64, capacity 40, base 500000) forward at offset 11")
    mod = module(ct.lib().dl_rotary_embedding_create, 64, 40, 500000.0, ct.options(ct.F32, GPU))
    st = mod.state()
    c, s = oracle.rope_tables(64, 40, 500000.0)
    assert np.array_equal(st["cosine"].numpy(), c) and np.array_equal(st["sine"].numpy(), s)
    rng = np.random.default_rng(24)
    x = rng.standard_normal((2, 3, 9, 64)).astype(np.float32)
    gx = G(x)  # held: a handle taken from a temporary would be released before the call
    got = ct.Tensor(ct._new(ct.lib().dl_rotary_embedding_forward, mod.handle, gx.handle, 11)).numpy()
    pos = np.tile(np.arange(11, 20), 2 * 3)
    want = oracle.rope(x.reshape(54, 1, 64), c, s, pos).reshape(2, 3, 9, 64)
    assert np.max(np.abs(got - want)) <= 1e-6
    with pytest.raises(ct.DLError, match="RoPE positions"):
        ct.Tensor(ct._new(ct.lib().dl_rotary_embedding_forward, mod.handle, gx.handle, 32))


# ------------------------------------------------------------------------------------------ tensordot
def test_tensordot_matches_numpy():
    say("case: dl_tensordot over one and two contracted axes")
    rng = np.random.default_rng(25)
    a = rng.standard_normal((4, 6, 8)).astype(np.float32)
    b = rng.standard_normal((8, 6, 5)).astype(np.float32)
    ga, gb = G(a), G(b)
    for axes_a, axes_b in (([2], [0]), ([1, 2], [1, 0])):
        got = ct.Tensor(ct._new(ct.lib().dl_tensordot, ga.handle, gb.handle, ct._shape(axes_a),
                                ct._shape(axes_b))).numpy()
        want = np.tensordot(a.astype(np.float64), b.astype(np.float64), (axes_a, axes_b))
        assert got.shape == want.shape and np.max(np.abs(got - want)) <= 1e-5 * np.max(np.abs(want))


# ------------------------------------------------------------------------------------------ bf16 codec
def test_device_bf16_codec_is_bit_exact():
    say("case: f32 -> bf16 on the GPU over 2^24 random words and the edge classes; bf16 -> f32 over all 2^16")
    rng = np.random.default_rng(26)
    words = rng.integers(0, 2 ** 32, size=1 << 24, dtype=np.uint64).astype(np.uint32)
    edges = []
    for hi in (0x0000, 0x0001, 0x3F80, 0x3F81, 0x7F7F, 0x7F80, 0x7FC0, 0x8000, 0x8001, 0xFF7F, 0xFF80, 0xFFC0, 0x007F):
        for lo in (0x0000, 0x0001, 0x7FFF, 0x8000, 0x8001, 0xFFFF):  # exact, below, tie, above the half
            edges.append((hi << 16) | lo)
    edges += [0x7F800001, 0x7FBFFFFF, 0xFF800001, 0x7FFFFFFF, 0x00000001, 0x807FFFFF, 0x7F7FFFFF]  # sNaN, qNaN, subnormal, max
    words = np.concatenate([words, np.array(edges, np.uint32)])
    values = words.view(np.float32)
    gv = G(values)
    got = astype(gv, ct.BF16).numpy()
    want = oracle.bf16_encode(values)
    mismatch = np.flatnonzero(got != want)
    assert mismatch.size == 0, [hex(int(words[i])) for i in mismatch[:8]]
    every = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    ge = G(every, ct.BF16)
    back = astype(ge, ct.F32).numpy()
    assert np.array_equal(back.view(np.uint32), oracle.bf16_decode(every).view(np.uint32))


# ------------------------------------------------------------------------------------------ keyed randomness
def test_keyed_device_randomness_against_the_oracle():
    say("case: dl_uniform_with_key bit for bit; dl_normal_with_key (weights) against the oracle")
    key = ct.fold_in((1234, 0), 7)
    count = 1 << 20
    u = ct.Tensor(ct._new(ct.lib().dl_uniform_with_key, ct.RandomKey(*key), ct._shape([count]), -2.0, 3.0,
                          ct.options(ct.F32, GPU))).numpy()
    assert np.array_equal(u.view(np.uint32), oracle.uniform(key, count, -2.0, 3.0).view(np.uint32))
    # Box-Muller through the device's logf/cosf: f32 values within a few ulps of the host's libm, so the bf16
    # weights agree except where an f32 value sits next to a bf16 rounding boundary (one bf16 ulp there)
    shape = (1024, 1024)
    g32 = ct.normal(key, shape, 0.02, ct.F32, GPU).numpy()
    w32 = oracle.normal_weights(key, shape, 0.02, oracle.F32)
    assert np.all(np.abs(g32 - w32) <= 2.0 ** -19 * np.abs(w32) + 1e-6 * 0.02)
    gb = ct.normal(key, shape, 0.02, ct.BF16, GPU).numpy()
    wb = oracle.normal_weights(key, shape, 0.02, oracle.BF16)
    diff = gb != wb
    say(f"  bf16 weights differing from the host's: {int(diff.sum())} of {gb.size}")
    assert diff.mean() <= 1e-3
    a, b = oracle.bf16_decode(gb[diff]), oracle.bf16_decode(wb[diff])
    assert np.all(np.abs(a - b) <= 2.0 ** -7 * np.maximum(np.abs(a), np.abs(b)) + 1e-9)  # one bf16 ulp
