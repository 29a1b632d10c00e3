"""Writes tests/golden/archive_v1.ct and archive_v1.npz: a small state in Ctorch's version-1 tensor archive format,
encoded here with `struct` from the format description alone (header b"CTORCH\\x00\\x01", little-endian u64 entry
count, per entry a u64 name length + name, u8 dtype code, u64 rank, u64 dims, contiguous little-endian values;
reference src/io/checkpoint.cpp:17-114, src/io/archive.h:14-45, and the reference's own independent reader
examples/comparison/compare.py:19-33).  The .npz holds the same arrays (bf16 as uint16 bit patterns) with their
dtype codes, so the library's loader can be checked against an encoder it shares no code with.

Run from the repository root: python tests/golden/make_archive.py
"""
import os
import struct

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
CODES = {"f32": (0, "<f4"), "f64": (1, "<f8"), "i64": (2, "<i8"), "bool": (3, "?"), "f16": (4, "<u2"),
         "bf16": (5, "<u2")}


def entries():
    rng = np.random.default_rng(2024)
    return [
        ("layer0.attention.query.weight", "f32", rng.standard_normal((3, 4)).astype(np.float32)),
        ("scalar", "f64", np.array(-1.25e-300, dtype=np.float64)),  # rank 0
        ("ids", "i64", np.array([0, -1, 2**62, -(2**63)], dtype=np.int64)),
        ("mask", "bool", np.array([[True, False], [False, True]])),
        ("half", "f16", np.array([0x3C00, 0x7C00, 0xFE00], dtype=np.uint16)),  # 1, +inf, a NaN (bit patterns)
        ("weight.bf16", "bf16", np.array([[0x3F80, 0xBF80, 0x0001], [0x7F80, 0x7FC0, 0x8000]], dtype=np.uint16)),
        ("empty", "f32", np.zeros((2, 0, 3), dtype=np.float32)),
        ("名前", "f32", np.array([3.5], dtype=np.float32)),  # UTF-8 name bytes
    ]


def encode(items):
    out = bytearray(b"CTORCH\x00\x01")
    out += struct.pack("<Q", len(items))
    for name, kind, array in items:
        code, fmt = CODES[kind]
        raw = name.encode()
        out += struct.pack("<Q", len(raw)) + raw
        out += struct.pack("<B", code)
        out += struct.pack("<Q", array.ndim)
        for dim in array.shape:
            out += struct.pack("<Q", dim)
        out += np.ascontiguousarray(array, dtype=fmt).tobytes()
    return bytes(out)


def main():
    items = entries()
    with open(os.path.join(HERE, "archive_v1.ct"), "wb") as f:
        f.write(encode(items))
    arrays = {f"value{i}": a for i, (_, _, a) in enumerate(items)}
    np.savez(os.path.join(HERE, "archive_v1.npz"), names=np.array([n for n, _, _ in items]),
             codes=np.array([CODES[k][0] for _, k, _ in items], dtype=np.int64), **arrays)


if __name__ == "__main__":
    main()
