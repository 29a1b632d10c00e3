"""CPU checks of the C ABI boundary: the library loads, exports every entry the public C headers declare,
and its host-side logic (handles, state names, RoPE tables, keyed randomness, bf16 codec, error reporting)
matches the reference semantics.  Nothing here launches a GPU kernel."""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

import ctorch_amd as ct
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
C_HEADERS = ["c_api.h", "decoder_c_api.h", "generate_c_api.h"]


def declared_entries():
    names = []
    for header in C_HEADERS:
        text = open(os.path.join(ROOT, "include", "dl", header)).read()
        names += re.findall(r"DL_API\s+[\w\s\*]+?\b(dl_\w+)\s*\(", text)
    return names


def test_library_exports_every_declared_entry():
    lib = ct.lib()
    names = declared_entries()
    assert len(names) > 70
    exported = subprocess.run(["nm", "-D", "--defined-only", ct.LIB_PATH], capture_output=True, text=True,
                              check=True).stdout
    exported = set(re.findall(r"\bT (dl_\w+)", exported))
    missing = [n for n in names if n not in exported]
    assert not missing, missing
    for n in names:
        assert hasattr(lib, n)
    # the Python mirror declares a signature for each of them
    assert set(names) == set(ct.SIGNATURES), set(names) ^ set(ct.SIGNATURES)


def test_version_and_error_channel():
    lib = ct.lib()
    assert b"gfx950" in lib.dl_version()
    out = C.c_void_p()
    # a NULL module is an error with a message, and the output slot is cleared
    assert lib.dl_module_forward(None, None, C.byref(out)) == 1
    assert out.value is None
    assert "NULL" in ct.last_error()
    # success clears the thread's error text
    t = ct.Tensor.from_numpy(np.arange(3, dtype=np.float32), ct.F32, ct.device("cpu"))
    assert ct.last_error() == ""
    assert t.shape == (3,)


def test_host_round_trip_casts_and_views():
    x = (np.arange(24, dtype=np.float32) * 0.37 - 3).reshape(2, 3, 4)
    t = ct.Tensor.from_numpy(x, ct.F32, ct.device("cpu"))
    assert np.array_equal(t.numpy(), x)
    b = ct.Tensor(ct._new(ct.lib().dl_astype, t.handle, ct.BF16))
    assert np.array_equal(b.numpy(), oracle.bf16_encode(x))
    n = ct.Tensor(ct._new(ct.lib().dl_narrow, t.handle, 1, 1, 2))
    assert np.array_equal(n.numpy(), x[:, 1:3])
    s = ct.Tensor(ct._new(ct.lib().dl_select, t.handle, 2, -1))
    assert np.array_equal(s.numpy(), x[:, :, -1])
    r = ct.Tensor(ct._new(ct.lib().dl_reshape, n.handle, ct._shape([4, 4])))
    assert np.array_equal(r.numpy(), x[:, 1:3].reshape(4, 4))
    ids = ct.Tensor.from_numpy(np.array([5, -7], np.int64), ct.I64, ct.device("cpu"))
    assert np.array_equal(ids.numpy(), [5, -7])


def test_keyed_randomness_matches_the_oracle_bit_for_bit():
    key = (0x1234_5678_9ABC_DEF0, 77)
    for label in (0, 1, 2**40 + 3):
        assert ct.fold_in(key, label) == oracle.fold_in(key, label)
    split = (ct.RandomKey * 3)()
    ct.lib().dl_random_split(ct.RandomKey(*key), 3, split)
    assert [(k.seed, k.stream) for k in split] == [oracle.fold_in(key, i) for i in range(3)]
    u = ct.Tensor(ct._new(ct.lib().dl_uniform_with_key, ct.RandomKey(*key), ct._shape([4096]), -2.0, 5.0,
                          ct.options(ct.F32, ct.device("cpu"))))
    assert np.array_equal(u.numpy(), oracle.uniform(key, 4096, -2.0, 5.0))
    z = ct.Tensor(ct._new(ct.lib().dl_randn_with_key, ct.RandomKey(*key), ct._shape([4096]),
                          ct.options(ct.F32, ct.device("cpu"))))
    assert np.array_equal(z.numpy(), oracle.randn(key, 4096))
    w = ct.normal(key, [64, 32], 0.02, ct.BF16, ct.device("cpu"))
    assert np.array_equal(w.numpy(), oracle.normal_weights(key, (64, 32), 0.02, oracle.BF16))


def test_decoder_state_names_and_rope_tables_match_the_reference_layout():
    dec = ct.transformer_decoder(2, 64, 4, 2, 96, 40, ct.BF16, ct.device("cpu"), rope_base=500000.0)
    state = dec.state()
    names = list(state)
    layer = ["attention.query.weight", "attention.key.weight", "attention.value.weight", "attention.output.weight",
             "feedforward.gate.weight", "feedforward.up.weight", "feedforward.down.weight",
             "attention_norm.weight", "feedforward_norm.weight"]
    params = [f"layer{i}.{n}" for i in range(2) for n in layer] + ["normalization.weight"]
    buffers = [f"layer{i}.attention.rotary.{n}" for i in range(2) for n in ("cosine", "sine")]
    assert names == params + buffers  # parameters in registration order, then buffers
    assert state["layer0.attention.key.weight"].shape == (2 * 16, 64)
    assert state["layer0.attention.query.weight"].dtype == ct.BF16
    c, s = oracle.rope_tables(16, 40, 500000.0)
    assert state["layer1.attention.rotary.cosine"].dtype == ct.F32  # tables use the accumulation dtype
    assert np.array_equal(state["layer1.attention.rotary.cosine"].numpy(), c)
    assert np.array_equal(state["layer1.attention.rotary.sine"].numpy(), s)
    assert np.array_equal(state["layer0.attention_norm.weight"].numpy(), np.full(64, 0x3F80, np.uint16))


def test_load_state_writes_values_and_rejects_bad_shapes():
    dec = ct.transformer_decoder(1, 32, 4, 2, 48, 16, ct.F32, ct.device("cpu"))
    state = {n: t.numpy() for n, t in dec.state().items()}
    w = np.arange(32 * 32, dtype=np.float32).reshape(32, 32) / 100
    state["layer0.attention.query.weight"] = w
    dec.load_state(state)
    assert np.array_equal(dec.state()["layer0.attention.query.weight"].numpy(), w)
    bad = dict(state)
    bad["layer0.attention.query.weight"] = w[:16]
    with pytest.raises(ct.DLError, match="shape"):
        dec.load_state(bad)
    missing = dict(state)
    del missing["normalization.weight"]
    with pytest.raises(ct.DLError, match="missing"):
        dec.load_state(missing)


def test_constructor_and_cache_errors_follow_the_reference():
    out = C.c_void_p()
    opts = ct.options(ct.F32, ct.device("cpu"))
    assert ct.lib().dl_transformer_decoder_create(1, 30, 4, 2, 8, 16, opts, C.byref(out)) == 1
    assert "divide evenly" in ct.last_error()
    assert ct.lib().dl_transformer_decoder_create(0, 32, 4, 2, 8, 16, opts, C.byref(out)) == 1
    assert "at least one layer" in ct.last_error()
    dec = ct.transformer_decoder(2, 32, 4, 2, 48, 16, ct.F32, ct.device("cpu"))
    cache = ct.DecoderCache(dec)
    assert cache.length == 0
    with pytest.raises(ct.DLError, match="existing prefix"):
        cache.truncate(1)
    cache.clear()
    # GPU arithmetic on CPU tensors is refused before any device call
    x = ct.Tensor.from_numpy(np.ones((1, 2, 32), np.float32), ct.F32, ct.device("cpu"))
    with pytest.raises(ct.DLError, match="GPU only"):
        ct.decode(dec, x, cache)
    assert cache.length == 0


def test_noalloc_attention_refuses_partials_beyond_its_scratch_before_any_device_call():
    # B*H*L * splits * (D + 2) floats above 2 Mi: refused before any pointer is read or any HIP call is made, so
    # this runs without a GPU.  128 (sequence, KV head) pairs over 100000 keys split the keys (98 splits of 1024):
    # 512 rows * 98 * 130 floats.  (From 256 pairs up a work-group takes each pair whole and nothing is split.)
    dummy = C.c_void_p(16)  # never dereferenced: the size check comes first
    status = ct.lib().dl_grouped_query_attention_noalloc(dummy, dummy, dummy, ct.BF16, 16, 32, 8, 1, 100000, 128,
                                                         dummy, 0)
    assert status != 0 and "scratch" in ct.last_error(), ct.last_error()
    # NULL pointers are refused whatever the shape
    status = ct.lib().dl_grouped_query_attention_noalloc(None, dummy, dummy, ct.BF16, 1, 1, 1, 1, 1, 64, dummy, 0)
    assert status != 0 and "NULL" in ct.last_error()
