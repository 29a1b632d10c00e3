"""CPU checks of the KV-cache wire format adapter (dl_decoder_cache_state / dl_decoder_cache_load_state): the
layout of the reference's ONNX decoder export, past_key_i / past_value_i as f32 [batch, kv_heads, length,
head_dim] per layer (reference extensions/onnx/src/decoder.cpp:64-69, docs/onnx.md:68-113).  Caches of a
decoder built on the host hold host storage, so no GPU is used; the GPU test of the same entries continues a
decode from an imported cache."""
import numpy as np
import pytest

import ctorch_amd as ct
import oracle


def past_state(rng, layers, batch, kv_heads, length, head_dim, prefix="past_"):
    out = {}
    for i in range(layers):
        out[f"{prefix}key_{i}"] = rng.standard_normal((batch, kv_heads, length, head_dim)).astype(np.float32)
        out[f"{prefix}value_{i}"] = rng.standard_normal((batch, kv_heads, length, head_dim)).astype(np.float32)
    return out


def bf16_round(x):
    return oracle.bf16_decode(oracle.bf16_encode(x))


def test_cache_state_round_trips_in_the_decoder_cache_dtype():
    rng = np.random.default_rng(5)
    # the default cache dtype is f32 for f32 and bf16 models alike (the reference's cache takes linear's f32
    # output dtype, src/nn/kv_cache.cpp:16-21); bf16 storage is an explicit opt-in and rounds the imported values
    for dtype, kv_dtype, rounding in ((ct.BF16, None, lambda x: x), (ct.BF16, ct.BF16, bf16_round),
                                      (ct.F32, None, lambda x: x), (ct.F32, ct.BF16, bf16_round)):
        dec = ct.transformer_decoder(2, 64, 4, 2, 96, 24, dtype, ct.device("cpu"), kv_dtype=kv_dtype)
        assert ct.cache_dtype(dec) == (ct.F32 if kv_dtype is None else kv_dtype)
        cache = ct.DecoderCache(dec)
        past = past_state(rng, 2, 3, 2, 5, 16)
        cache.load_state(dec, past)
        assert cache.length == 5
        out = cache.state()
        assert list(out) == ["past_key_0", "past_value_0", "past_key_1", "past_value_1"]
        for name, want in past.items():
            got = out[name]
            assert got.dtype == ct.F32 and got.shape == want.shape
            assert np.array_equal(got.numpy(), rounding(want)), name


def test_cache_state_accepts_onnx_outputs_and_replaces_the_contents():
    rng = np.random.default_rng(6)
    dec = ct.transformer_decoder(2, 64, 4, 2, 96, 24, ct.F32, ct.device("cpu"))
    cache = ct.DecoderCache(dec)
    cache.load_state(dec, past_state(rng, 2, 1, 2, 7, 16))
    present = past_state(rng, 2, 2, 2, 4, 16, prefix="present_")  # an ONNX session's outputs, another batch
    cache.load_state(dec, present)
    assert cache.length == 4
    out = cache.state()
    for i in range(2):
        assert np.array_equal(out[f"past_key_{i}"].numpy(), present[f"present_key_{i}"])
        assert np.array_equal(out[f"past_value_{i}"].numpy(), present[f"present_value_{i}"])


def test_cache_state_errors_leave_the_cache_unchanged():
    rng = np.random.default_rng(7)
    dec = ct.transformer_decoder(2, 64, 4, 2, 96, 24, ct.F32, ct.device("cpu"))
    cache = ct.DecoderCache(dec)
    good = past_state(rng, 2, 1, 2, 5, 16)
    cache.load_state(dec, good)
    missing = {k: v for k, v in good.items() if not k.endswith("_1")}
    with pytest.raises(ct.DLError, match="past_key_1"):
        cache.load_state(dec, missing)
    wrong_heads = past_state(rng, 2, 1, 4, 5, 16)
    with pytest.raises(ct.DLError, match="kv_heads"):
        cache.load_state(dec, wrong_heads)
    uneven = dict(good)
    uneven["past_key_1"] = rng.standard_normal((1, 2, 6, 16)).astype(np.float32)
    uneven["past_value_1"] = rng.standard_normal((1, 2, 6, 16)).astype(np.float32)
    with pytest.raises(ct.DLError, match="share batch and length"):
        cache.load_state(dec, uneven)
    too_long = past_state(rng, 2, 1, 2, 25, 16)
    with pytest.raises(ct.DLError, match="capacity"):
        cache.load_state(dec, too_long)
    twice = dict(good)
    twice["present_key_0"] = good["past_key_0"]
    with pytest.raises(ct.DLError, match="twice"):
        cache.load_state(dec, twice)
    assert cache.length == 5
    out = cache.state()
    for name, want in good.items():
        assert np.array_equal(out[name].numpy(), want), name
    with pytest.raises(ct.DLError, match="no keys yet"):
        ct.DecoderCache(dec).state()


def test_cache_state_is_a_snapshot_of_a_full_f32_cache():
    # at full capacity (and with one sequence and one KV head) the valid prefix is contiguous storage
    rng = np.random.default_rng(8)
    dec = ct.transformer_decoder(1, 32, 2, 1, 48, 6, ct.F32, ct.device("cpu"))
    cache = ct.DecoderCache(dec)
    first = past_state(rng, 1, 1, 1, 6, 16)
    cache.load_state(dec, first)
    exported = cache.state()
    cache.truncate(0)  # rewrite the same storage in place
    other = past_state(rng, 1, 1, 1, 6, 16)
    cache.append(0, ct.Tensor.from_numpy(other["past_key_0"], ct.F32, ct.device("cpu")),
                 ct.Tensor.from_numpy(other["past_value_0"], ct.F32, ct.device("cpu")))
    assert np.array_equal(cache.state()["past_key_0"].numpy(), other["past_key_0"])
    for name, want in first.items():
        assert np.array_equal(exported[name].numpy(), want), name


def test_decode_refuses_a_cache_whose_value_storage_differs_before_any_launch():
    """KV storage takes its shape and dtype from its first append, separately for keys and values (as the
    reference's does).  The fused decode writes and reads both with the layer's layout, so a cache whose value
    storage differs in dtype or head size must be refused on the host before anything is launched: here the
    decoder lives on the host, and the refusal must come from the cache check, not from the missing GPU."""
    cpu = ct.device("cpu")
    rng = np.random.default_rng(9)
    dec = ct.transformer_decoder(2, 64, 4, 2, 96, 24, ct.F32, cpu)
    x = ct.Tensor.from_numpy(rng.standard_normal((1, 1, 64)).astype(np.float32), ct.F32, cpu)
    key = rng.standard_normal((1, 2, 3, 16)).astype(np.float32)
    mixed_dtype = (ct.Tensor.from_numpy(key, ct.F32, cpu), ct.Tensor.from_numpy(oracle.bf16_encode(key), ct.BF16, cpu))
    wide_value = (ct.Tensor.from_numpy(key, ct.F32, cpu),
                  ct.Tensor.from_numpy(rng.standard_normal((1, 2, 3, 32)).astype(np.float32), ct.F32, cpu))
    for k, v in (mixed_dtype, wide_value):
        cache = ct.DecoderCache(dec)
        for layer in range(2):
            cache.append(layer, k, v)
        with pytest.raises(ct.DLError, match="KV cache shape, dtype or device changed"):
            ct.decode(dec, x, cache)
        assert cache.length == 3
    # a consistent cache passes the check and fails only where compute begins (no host compute path)
    cache = ct.DecoderCache(dec)
    for layer in range(2):
        cache.append(layer, ct.Tensor.from_numpy(key, ct.F32, cpu), ct.Tensor.from_numpy(key, ct.F32, cpu))
    with pytest.raises(ct.DLError) as raised:
        ct.decode(dec, x, cache)
    assert "KV cache" not in str(raised.value)
