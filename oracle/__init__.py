"""ctypes bindings for the CPU oracle (liboracle.so) — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg import this
package, and only as the checker.  The product (``ctorch_amd``) never imports it.

Besides the raw bindings this module holds the harness's synthetic-model definition: the LM
wrapper's parameter order (embedding ``tokens``, ``decoder.layer{i}...``, ``decoder.normalization``,
``output``; depth-first registration order as in src/nn/module.cpp:54-73 of the reference) and the
seeded weights ``W_s = 0.02 * randn(fold_in(root, s))`` for every Embedding/Linear/LoRA slot ``s``.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
F32, BF16 = 0, 5

_lib = None


def build() -> None:
    import subprocess
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run __graft_entry__.build())")
        _lib = C.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


_p = C.c_void_p
_i64 = C.c_int64
_u64 = C.c_uint64
_f64 = C.c_double


class Config(C.Structure):
    _fields_ = [("vocab", _i64), ("layers", _i64), ("dimensions", _i64), ("heads", _i64), ("kv_heads", _i64),
                ("hidden", _i64), ("context", _i64), ("rope_base", _f64), ("epsilon", _f64), ("wdtype", C.c_int),
                ("kv_bf16", C.c_int), ("lora_rank", _i64), ("lora_alpha", _f64)]


class Layer(C.Structure):
    _fields_ = [(n, _p) for n in ("query", "key", "value", "output", "gate", "up", "down", "attention_norm",
                                  "feedforward_norm", "cosine", "sine", "query_down", "query_up", "value_down",
                                  "value_up")]


class Model(C.Structure):
    _fields_ = [("config", Config), ("embedding", _p), ("layers", C.POINTER(Layer)), ("normalization", _p),
                ("head", _p)]


class Cache(C.Structure):
    _fields_ = [("key", _p), ("value", _p), ("batch", _i64), ("capacity", _i64), ("length", _i64)]


def _declare(L):
    L.orc_set_threads.argtypes = [C.c_int]
    L.orc_philox.argtypes = [_u64, _u64, _u64, _p]
    L.orc_fold_in.argtypes = [_u64, _u64, _u64, _p]
    L.orc_unit_f32.argtypes = [C.c_uint32, C.c_int]
    L.orc_unit_f32.restype = C.c_float
    L.orc_unit_f64.argtypes = [C.c_uint32, C.c_uint32, C.c_int]
    L.orc_unit_f64.restype = _f64
    L.orc_uniform_f32.argtypes = [_u64, _u64, _i64, _f64, _f64, _p]
    L.orc_randn_f32.argtypes = [_u64, _u64, _i64, _p]
    L.orc_random_ids.argtypes = [_u64, _u64, _i64, _i64, _p]
    L.orc_bf16_encode.argtypes = [C.c_float]
    L.orc_bf16_encode.restype = C.c_uint16
    L.orc_bf16_encode_n.argtypes = [_p, _i64, _p]
    L.orc_bf16_decode_n.argtypes = [_p, _i64, _p]
    L.orc_normal_weights.argtypes = [_u64, _u64, _i64, _f64, C.c_int, _p]
    L.orc_rope_tables.argtypes = [_i64, _i64, _f64, _p, _p]
    L.orc_rms_norm.argtypes = [_p, _i64, _i64, _p, _f64, _p]
    L.orc_linear.argtypes = [_p, _i64, _i64, _p, C.c_int, _i64, _p]
    L.orc_rope.argtypes = [_p, _i64, _i64, _i64, _p, _p, _p]
    L.orc_softmax_row.argtypes = [_p, _i64, _p]
    L.orc_argmax_row.argtypes = [_p, _i64]
    L.orc_argmax_row.restype = _i64
    L.orc_silu.argtypes = [C.c_float]
    L.orc_silu.restype = C.c_float
    L.orc_attention.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]
    L.orc_attention_masked.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p, _p]
    L.orc_log.argtypes = [_f64]
    L.orc_log.restype = _f64
    L.orc_gumbel.argtypes = [_u64, _u64, _u64]
    L.orc_gumbel.restype = _f64
    L.orc_sample_row.argtypes = [_p, _i64, _f64, _u64, _u64, _i64]
    L.orc_sample_row.restype = _i64
    L.orc_decoder_decode.argtypes = [C.POINTER(Model), _p, _i64, _i64, C.POINTER(Cache), _p]
    L.orc_lm_logits.argtypes = [C.POINTER(Model), _p, _i64, _i64, C.POINTER(Cache), _p]
    L.orc_generate.argtypes = [C.POINTER(Model), _p, _i64, _i64, _i64, _f64, _u64, _u64, C.POINTER(Cache), _p, _p]


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def set_threads(n: int) -> None:
    lib().orc_set_threads(int(n))


# ---------------------------------------------------------------------------- keyed randomness
def philox(seed: int, index: int, stream: int = 0) -> tuple[int, int, int, int]:
    out = np.zeros(4, np.uint32)
    lib().orc_philox(seed, index, stream, _ptr(out))
    return tuple(int(v) for v in out)


def fold_in(key: tuple[int, int], label: int) -> tuple[int, int]:
    out = np.zeros(2, np.uint64)
    lib().orc_fold_in(key[0], key[1], label, _ptr(out))
    return int(out[0]), int(out[1])


def uniform(key, count: int, low: float, high: float) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().orc_uniform_f32(key[0], key[1], count, low, high, _ptr(out))
    return out


def randn(key, count: int) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib().orc_randn_f32(key[0], key[1], count, _ptr(out))
    return out


def random_ids(key, count: int, vocab: int) -> np.ndarray:
    out = np.empty(count, np.int64)
    lib().orc_random_ids(key[0], key[1], count, vocab, _ptr(out))
    return out


def normal_weights(key, shape, scale: float, dtype: int) -> np.ndarray:
    count = int(np.prod(shape))
    out = np.empty(count, np.uint16 if dtype == BF16 else np.float32)
    lib().orc_normal_weights(key[0], key[1], count, scale, dtype, _ptr(out))
    return out.reshape(shape)


# ---------------------------------------------------------------------------- codec + blocks
def bf16_encode(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_bf16_encode_n(_ptr(x), x.size, _ptr(out))
    return out


def bf16_decode(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_decode_n(_ptr(b), b.size, _ptr(out))
    return out


def rope_tables(head_dim: int, capacity: int, base: float = 10000.0):
    c = np.empty((capacity, head_dim // 2), np.float32)
    s = np.empty((capacity, head_dim // 2), np.float32)
    lib().orc_rope_tables(head_dim, capacity, base, _ptr(c), _ptr(s))
    return c, s


def rms_norm(x: np.ndarray, weight: np.ndarray | None, eps: float = 1e-5) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    width = x.shape[-1]
    w = None if weight is None else np.ascontiguousarray(weight, np.float32)
    out = np.empty_like(x)
    lib().orc_rms_norm(_ptr(x), x.size // width, width, _ptr(w), eps, _ptr(out))
    return out


def linear(x: np.ndarray, w: np.ndarray) -> np.ndarray:
    """y = x W^T; w is f32 [out,in] or bf16 bits (uint16) [out,in]."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w)
    dtype = BF16 if w.dtype == np.uint16 else F32
    if dtype == F32:
        w = w.astype(np.float32, copy=False)
    rows = x.size // x.shape[-1]
    out = np.empty(x.shape[:-1] + (w.shape[0],), np.float32)
    lib().orc_linear(_ptr(x), rows, x.shape[-1], _ptr(w), dtype, w.shape[0], _ptr(out))
    return out


def rope(x: np.ndarray, cosine: np.ndarray, sine: np.ndarray, positions: np.ndarray) -> np.ndarray:
    """x [rows, heads, hd] (copied); row r uses table row positions[r]."""
    y = np.array(x, np.float32, copy=True, order="C")
    pos = np.ascontiguousarray(positions, np.int64)
    lib().orc_rope(_ptr(y), y.shape[0], y.shape[1], y.shape[2], _ptr(np.ascontiguousarray(cosine)),
                   _ptr(np.ascontiguousarray(sine)), _ptr(pos))
    return y


def softmax_row(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    lib().orc_softmax_row(_ptr(x), x.size, _ptr(out))
    return out


def argmax_row(x: np.ndarray) -> int:
    x = np.ascontiguousarray(x, np.float32)
    return int(lib().orc_argmax_row(_ptr(x), x.size))


def silu(v: float) -> float:
    return float(lib().orc_silu(v))


def attention(q, k, v, causal_first: int = -1, keep_mask=None) -> np.ndarray:
    """q [B,H,L,hd]; k,v [B,KV,S,hd] (contiguous); returns [B,H,L,hd].  keep_mask: bool array broadcastable to
    [B,H,L,S] (numpy rules, as the reference's where), False dropping a key from the softmax."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    B, H, L, hd = q.shape
    KV, S = k.shape[1], k.shape[2]
    out = np.empty_like(q)
    if keep_mask is None:
        lib().orc_attention(_ptr(q), _ptr(k), _ptr(v), B, H, KV, L, S, S, hd, causal_first, _ptr(out))
        return out
    mask = np.ascontiguousarray(np.asarray(keep_mask, dtype=bool)).view(np.uint8)
    if mask.ndim > 4:
        raise ValueError("keep mask rank above 4")
    shape = (1,) * (4 - mask.ndim) + mask.shape
    mask = mask.reshape(shape)
    strides = []
    for axis, (size, want) in enumerate(zip(shape, (B, H, L, S))):
        if size not in (1, want):
            raise ValueError(f"keep mask {shape} does not broadcast to {(B, H, L, S)}")
        strides.append(0 if size == 1 else mask.strides[axis])
    st = np.array(strides, dtype=np.int64)
    lib().orc_attention_masked(_ptr(q), _ptr(k), _ptr(v), B, H, KV, L, S, S, hd, causal_first, _ptr(mask), _ptr(st),
                               _ptr(out))
    return out


def log(x: float) -> float:
    return float(lib().orc_log(x))


def gumbel(key, index: int) -> float:
    return float(lib().orc_gumbel(key[0], key[1], index))


def sample(logits: np.ndarray, temperature: float, key) -> np.ndarray:
    """logits [B, V] -> [B] int64, Gumbel-max with noise index b*V+i under `key`."""
    logits = np.ascontiguousarray(logits, np.float32)
    B, V = logits.shape
    out = np.empty(B, np.int64)
    for b in range(B):
        out[b] = lib().orc_sample_row(_ptr(logits[b]), V, temperature, key[0], key[1], b)
    return out


# ---------------------------------------------------------------------------- synthetic decoder LM
@dataclass
class ModelConfig:
    vocab: int
    layers: int
    dimensions: int
    heads: int
    kv_heads: int
    hidden: int
    context: int
    rope_base: float = 10000.0
    dtype: str = "bf16"        # "f32" or "bf16" for every projection / embedding / head
    lora_rank: int = 0
    lora_alpha: float = 1.0
    epsilon: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.dimensions // self.heads


def parameter_names(cfg: ModelConfig) -> list[tuple[str, tuple[int, ...]]]:
    """The LM wrapper's named_parameters() order (depth-first registration order)."""
    d, H, KV, F, V = cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden, cfg.vocab
    hd = d // H
    names = [("tokens.weight", (V, d))]
    for i in range(cfg.layers):
        p = f"decoder.layer{i}."
        names += [(p + "attention.query.weight", (H * hd, d)), (p + "attention.key.weight", (KV * hd, d)),
                  (p + "attention.value.weight", (KV * hd, d)), (p + "attention.output.weight", (d, H * hd))]
        if cfg.lora_rank:
            r = cfg.lora_rank
            names += [(p + "attention.query_adapter.down.weight", (r, d)), (p + "attention.query_adapter.up.weight", (H * hd, r)),
                      (p + "attention.value_adapter.down.weight", (r, d)), (p + "attention.value_adapter.up.weight", (KV * hd, r))]
        names += [(p + "feedforward.gate.weight", (F, d)), (p + "feedforward.up.weight", (F, d)),
                  (p + "feedforward.down.weight", (d, F)), (p + "attention_norm.weight", (d,)),
                  (p + "feedforward_norm.weight", (d,))]
    names += [("decoder.normalization.weight", (d,)), ("output.weight", (V, d))]
    return names


def synthesize_weights(cfg: ModelConfig, root=(1234, 0), scale: float = 0.02) -> dict[str, np.ndarray]:
    """Seeded weights: slot s draws 0.02*randn(fold_in(root, s)) (RNE to bf16 for bf16 models).
    Norm weights keep their module default of ones; LoRA up (B) draws 1e-3*randn.  Adapter names follow the product's extension
    (``attention.{query,value}_adapter.{down,up}.weight``)."""
    dtype = BF16 if cfg.dtype == "bf16" else F32
    out = {}
    for slot, (name, shape) in enumerate(parameter_names(cfg)):
        if name.endswith("norm.weight") or name == "decoder.normalization.weight":
            out[name] = np.ones(shape, np.float32)
            continue
        s = 1e-3 if name.endswith("_adapter.up.weight") else scale
        out[name] = normal_weights(fold_in(root, slot), shape, s, dtype)
    return out


class OracleLM:
    """Embedding -> TransformerDecoder -> untied head, evaluated by the CPU oracle."""

    def __init__(self, cfg: ModelConfig, weights: dict[str, np.ndarray], kv_bf16: bool = False):
        """kv_bf16=False keeps the reference's f32 cache (src/nn/kv_cache.cpp:16-21: the cache takes the dtype
        of linear's f32 output); True rounds every appended key and value to bf16, the product's opt-in."""
        self.cfg = cfg
        self.w = {k: np.ascontiguousarray(v) for k, v in weights.items()}
        self.kv_bf16 = bool(kv_bf16)
        hd = cfg.head_dim
        self.tables = []
        for i in range(cfg.layers):
            c = self.w.get(f"decoder.layer{i}.attention.rotary.cosine")
            s = self.w.get(f"decoder.layer{i}.attention.rotary.sine")
            if c is None:
                c, s = rope_tables(hd, cfg.context, cfg.rope_base)
            self.tables.append((np.ascontiguousarray(c, np.float32), np.ascontiguousarray(s, np.float32)))
        self._layers = (Layer * cfg.layers)()
        for i in range(cfg.layers):
            p = f"decoder.layer{i}."
            L = self._layers[i]
            for f, n in (("query", "attention.query"), ("key", "attention.key"), ("value", "attention.value"),
                         ("output", "attention.output"), ("gate", "feedforward.gate"), ("up", "feedforward.up"),
                         ("down", "feedforward.down")):
                setattr(L, f, _ptr(self.w[p + n + ".weight"]))
            for f in ("attention_norm", "feedforward_norm"):
                self.w[p + f + ".weight"] = np.ascontiguousarray(self.w[p + f + ".weight"], np.float32)
                setattr(L, f, _ptr(self.w[p + f + ".weight"]))
            L.cosine, L.sine = _ptr(self.tables[i][0]), _ptr(self.tables[i][1])
            if cfg.lora_rank:
                L.query_down = _ptr(self.w[p + "attention.query_adapter.down.weight"])
                L.query_up = _ptr(self.w[p + "attention.query_adapter.up.weight"])
                L.value_down = _ptr(self.w[p + "attention.value_adapter.down.weight"])
                L.value_up = _ptr(self.w[p + "attention.value_adapter.up.weight"])
        self.w["decoder.normalization.weight"] = np.ascontiguousarray(self.w["decoder.normalization.weight"], np.float32)
        self.model = Model()
        self.model.config = Config(cfg.vocab, cfg.layers, cfg.dimensions, cfg.heads, cfg.kv_heads, cfg.hidden,
                                   cfg.context, cfg.rope_base, cfg.epsilon, BF16 if cfg.dtype == "bf16" else F32,
                                   int(self.kv_bf16), cfg.lora_rank, cfg.lora_alpha)
        self.model.embedding = _ptr(self.w["tokens.weight"])
        self.model.layers = self._layers
        self.model.normalization = _ptr(self.w["decoder.normalization.weight"])
        self.model.head = _ptr(self.w["output.weight"])

    # caches -------------------------------------------------------------------------------
    def make_cache(self, batch: int, capacity: int | None = None) -> "OracleCache":
        return OracleCache(self.cfg, batch, capacity or self.cfg.context)

    # evaluation ---------------------------------------------------------------------------
    def decode(self, x: np.ndarray, cache: "OracleCache") -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        B, L, d = x.shape
        out = np.empty_like(x)
        st = lib().orc_decoder_decode(C.byref(self.model), _ptr(x), B, L, cache.structs, _ptr(out))
        if st:
            raise ValueError(f"oracle decode failed with status {st}")
        return out

    def logits(self, ids: np.ndarray, cache: "OracleCache") -> np.ndarray:
        ids = np.ascontiguousarray(ids, np.int64)
        B, L = ids.shape
        out = np.empty((B, L, self.cfg.vocab), np.float32)
        st = lib().orc_lm_logits(C.byref(self.model), _ptr(ids), B, L, cache.structs, _ptr(out))
        if st:
            raise ValueError(f"oracle lm failed with status {st}")
        return out

    def last_logits(self, ids: np.ndarray, cache: "OracleCache") -> np.ndarray:
        """logits(ids, cache)[:, -1] without the head over the other positions: the embedding rows, the decoder
        (orc_decoder_decode, final RMSNorm included, as orc_lm_logits runs them), then the head on each sequence's
        last row only (orc_linear)."""
        ids = np.ascontiguousarray(ids, np.int64)
        B, L = ids.shape
        if ids.min() < 0 or ids.max() >= self.cfg.vocab:
            raise ValueError("token id out of range")
        table = self.w["tokens.weight"]
        x = bf16_decode(table[ids]) if self.cfg.dtype == "bf16" else np.asarray(table[ids], np.float32)
        features = self.decode(x, cache)
        return linear(np.ascontiguousarray(features[:, -1]), self.w["output.weight"])

    def generate(self, prompt: np.ndarray, steps: int, temperature: float = 0.0, key=(0, 0),
                 cache: "OracleCache | None" = None):
        prompt = np.ascontiguousarray(prompt, np.int64)
        B, P = prompt.shape
        cache = cache or self.make_cache(B)
        tokens = np.empty((B, steps), np.int64)
        last = np.empty((B, self.cfg.vocab), np.float32)
        st = lib().orc_generate(C.byref(self.model), _ptr(prompt), B, P, steps, temperature, key[0], key[1],
                                cache.structs, _ptr(tokens), _ptr(last))
        if st:
            raise ValueError(f"oracle generate failed with status {st}")
        return tokens, last


class OracleCache:
    def __init__(self, cfg: ModelConfig, batch: int, capacity: int):
        hd = cfg.head_dim
        self.keys = [np.zeros((batch, cfg.kv_heads, capacity, hd), np.float32) for _ in range(cfg.layers)]
        self.values = [np.zeros((batch, cfg.kv_heads, capacity, hd), np.float32) for _ in range(cfg.layers)]
        self.structs = (Cache * cfg.layers)()
        for i in range(cfg.layers):
            self.structs[i] = Cache(_ptr(self.keys[i]), _ptr(self.values[i]), batch, capacity, 0)

    @property
    def lengths(self) -> list[int]:
        return [int(s.length) for s in self.structs]

    @property
    def length(self) -> int:
        return int(self.structs[0].length)

    def truncate(self, length: int) -> None:
        for s in self.structs:
            if length < 0 or length > s.length:
                raise IndexError("truncate must keep an existing prefix")
            s.length = length

    def fill(self, layer: int, length: int, key_values: np.ndarray, value_values: np.ndarray) -> None:
        """Write a prefix directly (the KVCache::append route for a seeded random prefix)."""
        self.keys[layer][:, :, :length] = key_values
        self.values[layer][:, :, :length] = value_values
        self.structs[layer].length = length
