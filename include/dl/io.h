#pragma once
// Tensor archives (`.ct` files).  Mirrors the state-dict part of include/dl/io.h:15-18 (reference): save and load
// of named tensors in the reference's version-1 archive format (src/io/checkpoint.cpp:17-114,
// src/io/archive.h:14-45), so checkpoints written by either library load in the other.
//
// Layout, little-endian throughout: the 8-byte header "CTORCH\0\1"; u64 entry count; per entry a u64 name
// length and the name's bytes, a u8 dtype code (DType order: f32, f64, i64, bool, f16, bf16), a u64 rank, one u64
// per dimension, and the contiguous element bytes.  Training checkpoints (optimizer, loader, RNG state) are not
// part of the decoder token loop and are not provided.

#include "dl/nn.h"

#include <filesystem>
#include <span>

namespace dl::io {

/// Writes `state` (names, dtype, shape, contiguous values; device tensors are copied to the host first).  The
/// bytes go to a temporary file beside `path` that replaces `path` only once it is complete, so a failed write
/// leaves an existing `path` as it was (reference src/io/output_file.cpp:14-41).
DL_API void save(const std::filesystem::path& path, std::span<const NamedTensor> state);

/// Reads an archive into CPU tensors; throws std::runtime_error for another format or a truncated file.
DL_API StateDict load(const std::filesystem::path& path);

} // namespace dl::io
