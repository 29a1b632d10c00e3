"""The allocation-free attention entry (dl_grouped_query_attention_noalloc): through the C ABI, on device pointers
the caller owns, against dl_grouped_query_attention on the same inputs, bit for bit (the same kernels and key
splits; only the partials' home differs), on two calls in a row (the second smaller, reusing the scratch that
the first left behind), and with the device pool's used bytes unchanged by the calls.  (The refusal of shapes
whose partials exceed the scratch is a host-side check, tested on the CPU in test_abi.py.)"""
import sys

import numpy as np
import pytest

import ctorch_amd as ct

pytestmark = pytest.mark.gpu
GPU = ct.device("gpu")


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def data(t):
    return ct.lib().dl_tensor_data(t.handle)


def reference_and_noalloc(rng, B, H, KV, L, S, D, kv_dtype):
    q = rng.standard_normal((B, H, L, D)).astype(np.float32)
    k = rng.standard_normal((B, KV, S, D)).astype(np.float32)
    v = rng.standard_normal((B, KV, S, D)).astype(np.float32)
    if kv_dtype == ct.BF16:  # bf16 bits of the same values (round to nearest even on the host)
        k = (k.view(np.uint32) + 0x7FFF + ((k.view(np.uint32) >> 16) & 1) >> 16).astype(np.uint16)
        v = (v.view(np.uint32) + 0x7FFF + ((v.view(np.uint32) >> 16) & 1) >> 16).astype(np.uint16)
    gq, gk, gv = (ct.Tensor.from_numpy(q, None, GPU), ct.Tensor.from_numpy(k, kv_dtype, GPU),
                  ct.Tensor.from_numpy(v, kv_dtype, GPU))
    want = ct.grouped_query_attention(gq, gk, gv).numpy()          # [B, H, L, D]
    q_rows = ct.Tensor.from_numpy(np.ascontiguousarray(q.transpose(0, 2, 1, 3)), None, GPU)  # [B, L, H, D]
    out = ct.Tensor.from_numpy(np.full((B, L, H, D), np.nan, np.float32), None, GPU)
    ct.synchronize()
    before = ct.memory_stats().used_bytes
    ct.check(ct.lib().dl_grouped_query_attention_noalloc(data(q_rows), data(gk), data(gv), kv_dtype, B, H, KV, L, S,
                                                          D, data(out), 0))
    ct.synchronize()
    after = ct.memory_stats().used_bytes
    got = out.numpy().transpose(0, 2, 1, 3)
    return want, got, before, after


def test_noalloc_attention_equals_the_allocating_entry_on_two_calls():
    rng = np.random.default_rng(31)
    # first call: 4 key splits of 768 keys (f32 K/V); sets up the device's scratch address
    say("case: noalloc attention B=4 H=32 KV=8 L=1 S=3000 D=64 f32 (matrix-core kernel, 4 key splits)")
    want, got, before, after = reference_and_noalloc(rng, 4, 32, 8, 1, 3000, 64, ct.F32)
    assert np.array_equal(got, want)
    # second call, smaller: 2 splits over bf16 K/V, on top of the first call's partials
    say("case: noalloc attention B=2 H=32 KV=8 L=1 S=700 D=64 bf16 (matrix-core kernel, 2 key splits)")
    want, got, before, after = reference_and_noalloc(rng, 2, 32, 8, 1, 700, 64, ct.BF16)
    assert np.array_equal(got, want)
    assert after == before  # the call allocated nothing from the pool
    say("case: noalloc attention several positions, head dim 128, f32")
    want, got, before, after = reference_and_noalloc(rng, 2, 8, 2, 3, 300, 128, ct.F32)
    assert np.array_equal(got, want) and after == before
