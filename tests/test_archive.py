"""CPU checks of the tensor archive entries dl_state_save / dl_state_load (reference include/dl/c_api.h:647-648,
include/dl/io.h:15-18, src/io/checkpoint.cpp:17-114): the version-1 `.ct` byte layout, pinned by a known-answer
byte string, by a golden archive written with an encoder that shares no code with the library
(tests/golden/make_archive.py), and by a reader that follows the reference's own independent one
(examples/comparison/compare.py:19-33).  No GPU is used: archives hold CPU tensors."""
import os
import struct

import numpy as np
import pytest

import ctorch_amd as ct

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FORMATS = {0: "<f4", 1: "<f8", 2: "<i8", 3: "?", 4: "<u2", 5: "<u2"}


def read_archive(path):
    """name -> (dtype code, array), decoded with struct/numpy only (compare.py:19-33, plus codes 4 and 5)."""
    out = {}
    with open(path, "rb") as f:
        def u64():
            return struct.unpack("<Q", f.read(8))[0]
        assert f.read(8) == b"CTORCH\x00\x01"
        for _ in range(u64()):
            name = f.read(u64()).decode()
            code = f.read(1)[0]
            shape = tuple(u64() for _ in range(u64()))
            dtype = np.dtype(FORMATS[code])
            count = int(np.prod(shape, dtype=np.int64)) if shape else 1
            out[name] = (code, np.frombuffer(f.read(count * dtype.itemsize), dtype).copy().reshape(shape))
        assert f.read() == b""
    return out


def sample_state():
    rng = np.random.default_rng(7)
    return {
        "a.weight": (ct.F32, rng.standard_normal((5, 3)).astype(np.float32)),
        "b": (ct.F64, np.array(2.5)),
        "ids": (ct.I64, np.array([[1, -2], [3, 2**40]], dtype=np.int64)),
        "flags": (ct.BOOL, np.array([True, False, True])),
        "h": (ct.F16, np.array([0x3C00, 0x8001], dtype=np.uint16)),
        "w.bf16": (ct.BF16, np.array([0x3F80, 0xFFC1, 0x0000], dtype=np.uint16)),
        "none": (ct.F32, np.zeros((0, 4), dtype=np.float32)),
    }


def test_known_answer_bytes(tmp_path):
    path = tmp_path / "one.ct"
    ct.save_state(str(path), {"w": np.array([1.0, -2.0], np.float32)})
    want = bytes.fromhex(
        "4354 4f52 4348 0001"          # "CTORCH\0\1"
        "0100 0000 0000 0000"          # one entry
        "0100 0000 0000 0000 77"       # name length 1, "w"
        "00"                           # dtype f32
        "0100 0000 0000 0000"          # rank 1
        "0200 0000 0000 0000"          # dim 2
        "0000 803f 0000 00c0")         # 1.0, -2.0 little-endian
    assert path.read_bytes() == want


def test_golden_archive_loads_with_its_names_dtypes_and_bits():
    loaded = ct.load_state(os.path.join(GOLDEN, "archive_v1.ct"))
    ref = np.load(os.path.join(GOLDEN, "archive_v1.npz"))
    names = [str(n) for n in ref["names"]]
    assert list(loaded) == names  # file order
    for i, name in enumerate(names):
        tensor, want = loaded[name], ref[f"value{i}"]
        assert tensor.dtype == int(ref["codes"][i])
        assert tensor.shape == want.shape
        got = tensor.numpy()
        assert got.tobytes() == np.ascontiguousarray(want, got.dtype).tobytes(), name


def test_saved_archive_matches_the_independent_reader_and_round_trips(tmp_path):
    state = sample_state()
    path = tmp_path / "state.ct"
    ct.save_state(str(path), {n: a for n, (_, a) in state.items()}, {n: c for n, (c, _) in state.items()})
    decoded = read_archive(path)
    assert list(decoded) == list(state)
    for name, (code, array) in state.items():
        got_code, got = decoded[name]
        assert got_code == code and got.shape == array.shape
        assert got.tobytes() == np.ascontiguousarray(array, FORMATS[code]).tobytes(), name
    loaded = ct.load_state(str(path))
    for name, (code, array) in state.items():
        assert loaded[name].dtype == code and loaded[name].numpy().tobytes() == array.tobytes(), name
    # saving what was loaded reproduces the file byte for byte
    again = tmp_path / "again.ct"
    ct.save_state(str(again), loaded)
    assert again.read_bytes() == path.read_bytes()


def test_golden_archive_is_rewritten_byte_for_byte(tmp_path):
    loaded = ct.load_state(os.path.join(GOLDEN, "archive_v1.ct"))
    out = tmp_path / "copy.ct"
    ct.save_state(str(out), loaded)
    assert out.read_bytes() == open(os.path.join(GOLDEN, "archive_v1.ct"), "rb").read()


def test_bad_header_truncation_and_missing_files_raise(tmp_path):
    good = tmp_path / "good.ct"
    ct.save_state(str(good), {"x": np.arange(6, dtype=np.float32)})
    data = good.read_bytes()
    bad = tmp_path / "bad.ct"
    bad.write_bytes(b"CTORCH\x00\x02" + data[8:])
    with pytest.raises(ct.DLError, match="unsupported Ctorch checkpoint format"):
        ct.load_state(str(bad))
    cut = tmp_path / "cut.ct"
    cut.write_bytes(data[:-3])
    with pytest.raises(ct.DLError, match="truncated"):
        ct.load_state(str(cut))
    with pytest.raises(ct.DLError):
        ct.load_state(str(tmp_path / "absent.ct"))
    code = tmp_path / "code.ct"
    code.write_bytes(data[:8 + 8 + 8 + 1] + b"\x09" + data[8 + 8 + 8 + 1 + 1:])
    with pytest.raises(ct.DLError, match="dtype"):
        ct.load_state(str(code))


def test_save_replaces_the_target_only_when_complete(tmp_path):
    path = tmp_path / "model.ct"
    ct.save_state(str(path), {"x": np.ones(3, np.float32)})
    first = path.read_bytes()
    with pytest.raises(ct.DLError):
        ct.save_state(str(tmp_path / "missing-dir" / "model.ct"), {"x": np.ones(3, np.float32)})
    assert path.read_bytes() == first
    ct.save_state(str(path), {"x": np.zeros(2, np.float32)})
    assert read_archive(path)["x"][1].tolist() == [0.0, 0.0]
    assert sorted(os.listdir(tmp_path)) == ["model.ct"]  # no temporary file is left behind


def test_decoder_state_round_trips_through_an_archive(tmp_path):
    dec = ct.transformer_decoder(2, 64, 4, 2, 96, 24, ct.BF16, ct.device("cpu"))
    state = {n: t.numpy() for n, t in dec.state().items()}
    rng = np.random.default_rng(3)
    for name in state:
        if name.endswith(".weight"):
            state[name] = rng.integers(0, 2**16, size=state[name].shape, dtype=np.uint16)
    dtypes = {n: t.dtype for n, t in dec.state().items()}
    dec.load_state(state, dtypes)
    path = tmp_path / "decoder.ct"
    ct.save_state(str(path), dec.state())
    fresh = ct.transformer_decoder(2, 64, 4, 2, 96, 24, ct.BF16, ct.device("cpu"))
    fresh.load_state(ct.load_state(str(path)))
    for name, tensor in fresh.state().items():
        assert tensor.numpy().tobytes() == dec.state()[name].numpy().tobytes(), name
