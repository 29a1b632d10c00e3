"""ctypes binding of libctorch_amd.so, the MI355X build of Ctorch's decoder token loop.

The library's boundary is the reference's C17 surface (``include/dl/c_api.h``, ``include/dl/decoder_c_api.h``)
plus the on-device token loop extension (``include/dl/generate_c_api.h``).  This module mirrors that surface
for Python callers (tests, bench): thin handle classes over the same entry points, with the same argument
meaning and error behaviour (a ``DL_ERROR`` status raises ``DLError`` carrying ``dl_last_error()``).

There is no CPU compute path: if the shared library is missing, ``lib()`` raises.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libctorch_amd.so")

F32, F64, I64, BOOL, F16, BF16 = 0, 1, 2, 3, 4, 5
CPU, GPU = 0, 1
_NP = {F32: np.float32, F64: np.float64, I64: np.int64, BOOL: np.bool_, F16: np.uint16, BF16: np.uint16}


class DLError(RuntimeError):
    pass


class Shape(C.Structure):
    _fields_ = [("data", C.POINTER(C.c_int64)), ("size", C.c_size_t)]


class Device(C.Structure):
    _fields_ = [("type", C.c_int), ("index", C.c_int32)]


class TensorOptions(C.Structure):
    _fields_ = [("dtype", C.c_int), ("device", Device), ("requires_grad", C.c_int32)]


class TensorInfo(C.Structure):
    _fields_ = [("dtype", C.c_int), ("device", Device), ("numel", C.c_int64), ("contiguous", C.c_int32),
                ("requires_grad", C.c_int32), ("leaf", C.c_int32)]


class RandomKey(C.Structure):
    _fields_ = [("seed", C.c_uint64), ("stream", C.c_uint64)]


class MemoryStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("used_bytes", "reserved_bytes", "peak_used_bytes", "peak_reserved_bytes",
                                          "release_threshold")]


class KernelTiming(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("launches", C.c_int64), ("total_ms", C.c_double), ("bytes", C.c_double)]


_p = C.c_void_p
_pp = C.POINTER(C.c_void_p)
_st = C.c_int
_i64 = C.c_int64
_i32 = C.c_int32
_f64 = C.c_double

# name -> (restype, argtypes); every entry the headers declare
SIGNATURES = {
    "dl_version": (C.c_char_p, []),
    "dl_last_error": (C.c_char_p, []),
    "dl_default_tensor_options": (TensorOptions, []),
    "dl_tensor_release": (None, [_p]),
    "dl_tensor_retain": (_st, [_p, _pp]),
    "dl_tensor_get_info": (TensorInfo, [_p]),
    "dl_tensor_shape": (Shape, [_p]),
    "dl_tensor_strides": (Shape, [_p]),
    "dl_tensor_data": (_p, [_p]),
    "dl_tensor_nbytes": (C.c_size_t, [_p]),
    "dl_tensor_copy_to_host": (_st, [_p, _p]),
    "dl_from_host": (_st, [_p, Shape, TensorOptions, _pp]),
    "dl_full": (_st, [Shape, _f64, TensorOptions, _pp]),
    "dl_zeros": (_st, [Shape, TensorOptions, _pp]),
    "dl_ones": (_st, [Shape, TensorOptions, _pp]),
    "dl_clone": (_st, [_p, _pp]),
    "dl_contiguous": (_st, [_p, _pp]),
    "dl_astype": (_st, [_p, C.c_int, _pp]),
    "dl_to": (_st, [_p, Device, _pp]),
    "dl_reshape": (_st, [_p, Shape, _pp]),
    "dl_select": (_st, [_p, _i64, _i64, _pp]),
    "dl_narrow": (_st, [_p, _i64, _i64, _i64, _pp]),
    "dl_argmax": (_st, [_p, _i64, _i32, _pp]),
    "dl_linear": (_st, [_p, _p, _p, _pp]),
    "dl_embedding": (_st, [_p, _p, _pp]),
    "dl_rms_norm": (_st, [_p, Shape, _p, C.POINTER(_f64), _pp]),
    "dl_synchronize": (_st, [Device]),
    "dl_gpu_memory_get_stats": (_st, [_i32, C.POINTER(MemoryStats)]),
    "dl_gpu_memory_set_release_threshold": (_st, [_i32, C.c_uint64]),
    "dl_gpu_memory_reset_peak_stats": (_st, [_i32]),
    "dl_gpu_memory_release_unused": (_st, [_i32]),
    "dl_cuda_memory_get_stats": (_st, [_i32, C.POINTER(MemoryStats)]),
    "dl_cuda_memory_set_release_threshold": (_st, [_i32, C.c_uint64]),
    "dl_cuda_memory_reset_peak_stats": (_st, [_i32]),
    "dl_cuda_memory_release_unused": (_st, [_i32]),
    "dl_grad_enabled": (_i32, []),
    "dl_random_fold_in": (RandomKey, [RandomKey, C.c_uint64]),
    "dl_random_split": (None, [RandomKey, C.c_size_t, C.POINTER(RandomKey)]),
    "dl_uniform_with_key": (_st, [RandomKey, Shape, _f64, _f64, TensorOptions, _pp]),
    "dl_randn_with_key": (_st, [RandomKey, Shape, TensorOptions, _pp]),
    "dl_module_release": (None, [_p]),
    "dl_module_retain": (_st, [_p, _pp]),
    "dl_linear_create": (_st, [_i64, _i64, _i32, TensorOptions, _pp]),
    "dl_linear_from_tensors": (_st, [_p, _p, _pp]),
    "dl_embedding_create": (_st, [_i64, _i64, TensorOptions, _pp]),
    "dl_embedding_from_tensor": (_st, [_p, _pp]),
    "dl_rms_norm_create": (_st, [Shape, C.POINTER(_f64), _i32, TensorOptions, _pp]),
    "dl_module_forward": (_st, [_p, _p, _pp]),
    "dl_module_to": (_st, [_p, Device]),
    "dl_module_parameters": (_st, [_p, _pp]),
    "dl_module_state": (_st, [_p, _pp]),
    "dl_module_load_state": (_st, [_p, _p]),
    "dl_state_release": (None, [_p]),
    "dl_state_size": (C.c_size_t, [_p]),
    "dl_state_name": (C.c_char_p, [_p, C.c_size_t]),
    "dl_state_tensor": (_st, [_p, C.c_size_t, _pp]),
    "dl_state_create": (_st, [C.POINTER(C.c_char_p), C.POINTER(_p), C.c_size_t, _pp]),
    "dl_state_save": (_st, [C.c_char_p, _p]),
    "dl_state_load": (_st, [C.c_char_p, _pp]),
    # decoder_c_api.h
    "dl_tensordot": (_st, [_p, _p, Shape, Shape, _pp]),
    "dl_rotary_embedding": (_st, [_p, _p, _p, _pp]),
    "dl_grouped_query_attention": (_st, [_p, _p, _p, _p, _pp]),
    "dl_grouped_query_attention_noalloc": (_st, [_p, _p, _p, C.c_int, _i64, _i64, _i64, _i64, _i64, _i64, _p, _i32]),
    "dl_swiglu_create": (_st, [_i64, _i64, _i32, TensorOptions, _pp]),
    "dl_lora_linear_create": (_st, [_p, _i64, _f64, _pp]),
    "dl_lora_linear_merge": (_st, [_p, _pp]),
    "dl_rotary_embedding_create": (_st, [_i64, _i64, _f64, TensorOptions, _pp]),
    "dl_rotary_embedding_forward": (_st, [_p, _p, _i64, _pp]),
    "dl_grouped_query_attention_create": (_st, [_i64, _i64, _i64, _i64, TensorOptions, _pp]),
    "dl_transformer_decoder_create": (_st, [_i64, _i64, _i64, _i64, _i64, _i64, TensorOptions, _pp]),
    "dl_decoder_cache_create": (_st, [_p, _pp]),
    "dl_decoder_cache_release": (None, [_p]),
    "dl_decoder_cache_clear": (_st, [_p]),
    "dl_decoder_cache_truncate": (_st, [_p, _i64]),
    "dl_decoder_cache_length": (_st, [_p, C.POINTER(_i64)]),
    "dl_transformer_decoder_decode": (_st, [_p, _p, _p, _pp]),
    "dl_transformer_decoder_create_with_base": (_st, [_i64, _i64, _i64, _i64, _i64, _i64, _f64, TensorOptions, _pp]),
    "dl_transformer_decoder_attach_lora": (_st, [_p, _i64, _f64, _i32, _i32]),
    "dl_decoder_cache_append": (_st, [_p, _i64, _p, _p]),
    "dl_transformer_decoder_set_cache_dtype": (_st, [_p, C.c_int]),
    "dl_transformer_decoder_cache_dtype": (_st, [_p, C.POINTER(C.c_int)]),
    "dl_decoder_cache_state": (_st, [_p, _pp]),
    "dl_decoder_cache_load_state": (_st, [_p, _p, _p]),
    # generate_c_api.h
    "dl_decoder_lm_create": (_st, [_p, _p, _p, _pp]),
    "dl_decoder_lm_release": (None, [_p]),
    "dl_decoder_lm_logits": (_st, [_p, _p, _p, _pp]),
    "dl_decoder_lm_generate": (_st, [_p, _p, _p, _i64, _f64, RandomKey, _i32, _pp, _pp]),
    "dl_decoder_lm_benchmark": (_st, [_p, _p, _p, _i64, _i64, _f64, RandomKey, _i32, C.POINTER(_f64), _pp]),
    "dl_decoder_lm_profile": (_st, [_p, _p, _p, _i64, C.POINTER(KernelTiming), C.c_size_t, C.POINTER(C.c_size_t)]),
    "dl_decoder_lm_set_weight_repack": (_st, [_p, _i32]),
    "dl_sample": (_st, [_p, _f64, RandomKey, _pp]),
    "dl_normal_with_key": (_st, [RandomKey, Shape, _f64, TensorOptions, _pp]),
    "dl_timer_create": (_st, [Device, _pp]),
    "dl_timer_release": (None, [_p]),
    "dl_timer_start": (_st, [_p]),
    "dl_timer_stop": (_st, [_p, C.POINTER(_f64)]),
    "dl_gpu_copy_bandwidth": (_st, [_i32, C.c_uint64, _i32, C.POINTER(_f64)]),
}

_lib = None


def build() -> None:
    """Compiles libctorch_amd.so in-tree (hipcc for the gfx950 kernels, g++ for the C++20 host layers)."""
    subprocess.run(["make", "-s", "-j8", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"ctorch_amd: {LIB_PATH} is not built (run __graft_entry__.build()); "
                               "there is no CPU fallback")
        handle = C.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().dl_last_error().decode()


def check(status: int) -> None:
    if status != 0:
        raise DLError(last_error())


def _shape(dims) -> Shape:
    arr = (C.c_int64 * len(dims))(*[int(d) for d in dims])
    s = Shape(arr, len(dims))
    s._keep = arr  # keep the array alive with the struct
    return s


def device(kind: str = "gpu", index: int = 0) -> Device:
    return Device(GPU if kind == "gpu" else CPU, index)


def memory_stats(index: int = 0) -> MemoryStats:
    """dl_gpu_memory_get_stats: the device pool's used / reserved bytes and their peaks."""
    out = MemoryStats()
    check(lib().dl_gpu_memory_get_stats(index, C.byref(out)))
    return out


def set_release_threshold(bytes_: int, index: int = 0) -> None:
    """dl_gpu_memory_set_release_threshold: free bytes above this go back to the device at synchronisation."""
    check(lib().dl_gpu_memory_set_release_threshold(index, bytes_))


def reset_peak_stats(index: int = 0) -> None:
    """dl_gpu_memory_reset_peak_stats: restarts both peaks (from zero, as HIP does)."""
    check(lib().dl_gpu_memory_reset_peak_stats(index))


def release_unused(index: int = 0) -> None:
    """dl_gpu_memory_release_unused: returns the pool's free blocks to the device."""
    check(lib().dl_gpu_memory_release_unused(index))


def options(dtype: int = F32, dev: Device | None = None) -> TensorOptions:
    return TensorOptions(dtype, dev if dev is not None else device("gpu"), 0)


class Tensor:
    """Owned dl_tensor handle."""

    def __init__(self, handle):
        self.handle = C.c_void_p(handle) if not isinstance(handle, C.c_void_p) else handle

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.dl_tensor_release(self.handle)
            self.handle = None

    @staticmethod
    def from_numpy(array: np.ndarray, dtype: int | None = None, dev: Device | None = None) -> "Tensor":
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.float64): F64, np.dtype(np.int64): I64,
                     np.dtype(np.bool_): BOOL, np.dtype(np.uint16): BF16}[array.dtype]
        shape = array.shape  # np.ascontiguousarray turns a rank-0 array into rank 1
        array = np.ascontiguousarray(array, _NP[dtype])
        out = C.c_void_p()
        check(lib().dl_from_host(array.ctypes.data_as(C.c_void_p), _shape(shape), options(dtype, dev),
                                 C.byref(out)))
        return Tensor(out)

    @property
    def info(self) -> TensorInfo:
        return lib().dl_tensor_get_info(self.handle)

    @property
    def shape(self) -> tuple[int, ...]:
        s = lib().dl_tensor_shape(self.handle)
        return tuple(s.data[i] for i in range(s.size))

    @property
    def dtype(self) -> int:
        return self.info.dtype

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, _NP[self.dtype])
        check(lib().dl_tensor_copy_to_host(self.handle, out.ctypes.data_as(C.c_void_p)))
        return out

    def to(self, dev: Device) -> "Tensor":
        out = C.c_void_p()
        check(lib().dl_to(self.handle, dev, C.byref(out)))
        return Tensor(out)


def _new(fn, *args) -> C.c_void_p:
    out = C.c_void_p()
    check(fn(*args, C.byref(out)))
    return out


class Module:
    """Owned dl_module handle."""

    def __init__(self, handle):
        self.handle = handle

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.dl_module_release(self.handle)
            self.handle = None

    def to(self, dev: Device) -> "Module":
        check(lib().dl_module_to(self.handle, dev))
        return self

    def forward(self, x: Tensor) -> Tensor:
        return Tensor(_new(lib().dl_module_forward, self.handle, x.handle))

    def state(self) -> dict[str, Tensor]:
        st = _new(lib().dl_module_state, self.handle)
        try:
            out = {}
            for i in range(lib().dl_state_size(st)):
                name = lib().dl_state_name(st, i).decode()
                out[name] = Tensor(_new(lib().dl_state_tensor, st, i))
            return out
        finally:
            lib().dl_state_release(st)

    def load_state(self, values: dict[str, np.ndarray | Tensor], dtypes: dict[str, int] | None = None) -> None:
        names, tensors = [], []
        for name, value in values.items():
            if not isinstance(value, Tensor):
                dt = (dtypes or {}).get(name)
                value = Tensor.from_numpy(value, dt, device("cpu"))
            names.append(name)
            tensors.append(value)
        c_names = (C.c_char_p * len(names))(*[n.encode() for n in names])
        c_tensors = (C.c_void_p * len(tensors))(*[t.handle.value for t in tensors])
        st = _new(lib().dl_state_create, c_names, c_tensors, len(names))
        try:
            check(lib().dl_module_load_state(self.handle, st))
        finally:
            lib().dl_state_release(st)


def _state_handle(values: dict[str, np.ndarray | Tensor], dtypes: dict[str, int] | None = None) -> C.c_void_p:
    names, tensors = [], []
    for name, value in values.items():
        if not isinstance(value, Tensor):
            value = Tensor.from_numpy(value, (dtypes or {}).get(name), device("cpu"))
        names.append(name)
        tensors.append(value)
    c_names = (C.c_char_p * len(names))(*[n.encode() for n in names])
    c_tensors = (C.c_void_p * len(tensors))(*[t.handle.value for t in tensors])
    return _new(lib().dl_state_create, c_names, c_tensors, len(names))


def save_state(path: str, values: dict[str, np.ndarray | Tensor], dtypes: dict[str, int] | None = None) -> None:
    """dl_state_save: the named tensors as a version-1 Ctorch tensor archive (`.ct`)."""
    st = _state_handle(values, dtypes)
    try:
        check(lib().dl_state_save(str(path).encode(), st))
    finally:
        lib().dl_state_release(st)


def load_state(path: str) -> dict[str, Tensor]:
    """dl_state_load: the archive's named tensors, on the CPU, in file order."""
    st = _new(lib().dl_state_load, str(path).encode())
    try:
        return {lib().dl_state_name(st, i).decode(): Tensor(_new(lib().dl_state_tensor, st, i))
                for i in range(lib().dl_state_size(st))}
    finally:
        lib().dl_state_release(st)


def transformer_decoder(layers, dimensions, heads, kv_heads, hidden, context, dtype=F32, dev=None,
                        rope_base: float = 10000.0, kv_dtype: int | None = None) -> Module:
    """TransformerDecoder; kv_dtype (F32 default, or BF16) is the K/V storage dtype of its decode."""
    opts = options(dtype, dev if dev is not None else device("cpu"))
    if rope_base == 10000.0:
        module = Module(_new(lib().dl_transformer_decoder_create, layers, dimensions, heads, kv_heads, hidden, context,
                             opts))
    else:
        module = Module(_new(lib().dl_transformer_decoder_create_with_base, layers, dimensions, heads, kv_heads, hidden,
                             context, rope_base, opts))
    if kv_dtype is not None:
        check(lib().dl_transformer_decoder_set_cache_dtype(module.handle, kv_dtype))
    return module


def cache_dtype(decoder: Module) -> int:
    out = C.c_int()
    check(lib().dl_transformer_decoder_cache_dtype(decoder.handle, C.byref(out)))
    return out.value


def embedding_from(weight: Tensor) -> Module:
    return Module(_new(lib().dl_embedding_from_tensor, weight.handle))


def linear_from(weight: Tensor, bias: Tensor | None = None) -> Module:
    return Module(_new(lib().dl_linear_from_tensors, weight.handle, bias.handle if bias else None))


class DecoderCache:
    def __init__(self, decoder: Module):
        self.handle = _new(lib().dl_decoder_cache_create, decoder.handle)

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.dl_decoder_cache_release(self.handle)
            self.handle = None

    @property
    def length(self) -> int:
        n = C.c_int64()
        check(lib().dl_decoder_cache_length(self.handle, C.byref(n)))
        return n.value

    def truncate(self, length: int) -> None:
        check(lib().dl_decoder_cache_truncate(self.handle, length))

    def clear(self) -> None:
        check(lib().dl_decoder_cache_clear(self.handle))

    def state(self) -> dict[str, Tensor]:
        """dl_decoder_cache_state: past_key_i / past_value_i, f32 [B, KV, length, hd] (the ONNX wire format)."""
        st = _new(lib().dl_decoder_cache_state, self.handle)
        try:
            return {lib().dl_state_name(st, i).decode(): Tensor(_new(lib().dl_state_tensor, st, i))
                    for i in range(lib().dl_state_size(st))}
        finally:
            lib().dl_state_release(st)

    def load_state(self, decoder: "Module", values: dict[str, np.ndarray | Tensor]) -> None:
        """dl_decoder_cache_load_state: replaces the cache's contents with past_* (or present_*) tensors."""
        st = _state_handle(values)
        try:
            check(lib().dl_decoder_cache_load_state(decoder.handle, self.handle, st))
        finally:
            lib().dl_state_release(st)

    def append(self, layer: int, key: Tensor, value: Tensor) -> None:
        check(lib().dl_decoder_cache_append(self.handle, layer, key.handle, value.handle))


def decode(decoder: Module, x: Tensor, cache: DecoderCache) -> Tensor:
    return Tensor(_new(lib().dl_transformer_decoder_decode, decoder.handle, x.handle, cache.handle))


class DecoderLM:
    """Embedding -> TransformerDecoder -> head with the whole token step on the GPU."""

    def __init__(self, embedding: Module, decoder: Module, head: Module):
        self.modules = (embedding, decoder, head)
        self.handle = _new(lib().dl_decoder_lm_create, embedding.handle, decoder.handle, head.handle)

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.dl_decoder_lm_release(self.handle)
            self.handle = None

    def logits(self, ids: np.ndarray, cache: DecoderCache) -> np.ndarray:
        t = Tensor.from_numpy(np.ascontiguousarray(ids, np.int64), I64, device("cpu"))
        return Tensor(_new(lib().dl_decoder_lm_logits, self.handle, t.handle, cache.handle)).numpy()

    def generate(self, prompt: np.ndarray, cache: DecoderCache, steps: int, temperature: float = 0.0,
                 key=(0, 0), use_graph: bool = True, host: bool = True):
        t = Tensor.from_numpy(np.ascontiguousarray(prompt, np.int64), I64, device("cpu"))
        tokens, last = C.c_void_p(), C.c_void_p()
        check(lib().dl_decoder_lm_generate(self.handle, t.handle, cache.handle, steps, temperature,
                                           RandomKey(key[0], key[1]), int(use_graph), C.byref(tokens),
                                           C.byref(last)))
        tokens, last = Tensor(tokens), Tensor(last)
        return (tokens.numpy(), last.numpy()) if host else (tokens, last)

    def benchmark(self, prompt: np.ndarray, cache: DecoderCache, warmup: int, timed: int, temperature: float = 0.0,
                  key=(0, 0), use_graph: bool = True) -> tuple[float, np.ndarray]:
        t = Tensor.from_numpy(np.ascontiguousarray(prompt, np.int64), I64, device("cpu"))
        ms, tokens = C.c_double(), C.c_void_p()
        check(lib().dl_decoder_lm_benchmark(self.handle, t.handle, cache.handle, warmup, timed, temperature,
                                            RandomKey(key[0], key[1]), int(use_graph), C.byref(ms), C.byref(tokens)))
        return ms.value, Tensor(tokens).numpy()

    def profile(self, ids: np.ndarray, cache: DecoderCache, rounds: int) -> list[dict]:
        """Per kernel class: its launches of one step repeated `rounds` times back to back (HIP events)."""
        t = Tensor.from_numpy(np.ascontiguousarray(ids, np.int64), I64, device("cpu"))
        out = (KernelTiming * 32)()
        n = C.c_size_t()
        check(lib().dl_decoder_lm_profile(self.handle, t.handle, cache.handle, rounds, out, 32, C.byref(n)))
        return [{"name": out[i].name.decode(), "launches": out[i].launches, "total_ms": out[i].total_ms,
                 "bytes": out[i].bytes} for i in range(n.value)]

    def set_weight_repack(self, enabled: bool) -> None:
        """Whether batched decode reads a repacked second copy of every bf16 weight (off: the copies are dropped)."""
        check(lib().dl_decoder_lm_set_weight_repack(self.handle, int(enabled)))


class Timer:
    def __init__(self, index: int = 0):
        self.handle = _new(lib().dl_timer_create, device("gpu", index))

    def __del__(self):
        if getattr(self, "handle", None) and _lib is not None:
            _lib.dl_timer_release(self.handle)
            self.handle = None

    def start(self) -> None:
        check(lib().dl_timer_start(self.handle))

    def stop(self) -> float:
        ms = C.c_double()
        check(lib().dl_timer_stop(self.handle, C.byref(ms)))
        return ms.value


def normal(key, shape, scale: float, dtype: int = BF16, dev: Device | None = None) -> Tensor:
    return Tensor(_new(lib().dl_normal_with_key, RandomKey(*key), _shape(shape), scale, options(dtype, dev)))


def fold_in(key, label: int) -> tuple[int, int]:
    k = lib().dl_random_fold_in(RandomKey(*key), label)
    return k.seed, k.stream


def synchronize(index: int = 0) -> None:
    check(lib().dl_synchronize(device("gpu", index)))


def copy_bandwidth(nbytes: int, iterations: int = 20, index: int = 0) -> float:
    gbps = C.c_double()
    check(lib().dl_gpu_copy_bandwidth(index, nbytes, iterations, C.byref(gbps)))
    return gbps.value


# ---------------------------------------------------------------------------------------------- operators
# Each wrapper holds its Tensor arguments for the duration of the call (a bare `.handle` of a temporary would
# be released by the wrapper's destructor before the library reads it).
def linear(x: Tensor, weight: Tensor, bias: Tensor | None = None) -> Tensor:
    return Tensor(_new(lib().dl_linear, x.handle, weight.handle, bias.handle if bias is not None else None))


def rms_norm(x: Tensor, normalized_shape, weight: Tensor | None = None, epsilon: float | None = None) -> Tensor:
    eps = C.c_double(epsilon) if epsilon is not None else None
    return Tensor(_new(lib().dl_rms_norm, x.handle, _shape(normalized_shape),
                       weight.handle if weight is not None else None, C.byref(eps) if eps is not None else None))


def embedding(ids: Tensor, weight: Tensor) -> Tensor:
    return Tensor(_new(lib().dl_embedding, ids.handle, weight.handle))


def argmax(x: Tensor, axis: int, keepdim: bool = False) -> Tensor:
    return Tensor(_new(lib().dl_argmax, x.handle, axis, int(keepdim)))


def sample(logits: Tensor, temperature: float, key) -> Tensor:
    return Tensor(_new(lib().dl_sample, logits.handle, temperature, RandomKey(*key)))


def rotary_embedding(x: Tensor, cosine: Tensor, sine: Tensor) -> Tensor:
    return Tensor(_new(lib().dl_rotary_embedding, x.handle, cosine.handle, sine.handle))


def grouped_query_attention(q: Tensor, k: Tensor, v: Tensor, keep_mask: Tensor | None = None) -> Tensor:
    return Tensor(_new(lib().dl_grouped_query_attention, q.handle, k.handle, v.handle,
                       keep_mask.handle if keep_mask is not None else None))
