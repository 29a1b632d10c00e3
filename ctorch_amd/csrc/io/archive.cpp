// Tensor archive reader and writer (see include/dl/io.h for the format).  Integers are encoded byte by byte
// in little-endian order, so the files do not depend on the host's byte order; element bytes are swapped on a
// big-endian host, as the reference does (src/io/checkpoint.cpp:19-27).
#include "dl/io.h"

#include "dl/tensor.h"

#include <algorithm>
#include <array>
#include <atomic>
#include <bit>
#include <chrono>
#include <cstring>
#include <fstream>
#include <limits>
#include <stdexcept>
#include <string>
#include <vector>

namespace dl::io {
namespace {

constexpr std::array<char, 8> kHeader{'C', 'T', 'O', 'R', 'C', 'H', 0, 1};
constexpr std::uint64_t kMaxRank = 64;

void put_u64(std::ostream& out, std::uint64_t value) {
    char bytes[8];
    for (int i = 0; i < 8; ++i) bytes[i] = static_cast<char>((value >> (8 * i)) & 0xff);
    out.write(bytes, 8);
}

std::uint64_t get_u64(std::istream& in) {
    unsigned char bytes[8];
    in.read(reinterpret_cast<char*>(bytes), 8);
    std::uint64_t value = 0;
    for (int i = 0; i < 8; ++i) value |= static_cast<std::uint64_t>(bytes[i]) << (8 * i);
    return value;
}

void swap_elements(char* bytes, std::size_t count, std::size_t width) {
    if constexpr (std::endian::native == std::endian::big) {
        for (std::size_t i = 0; i < count; ++i) std::reverse(bytes + i * width, bytes + (i + 1) * width);
    }
}

void write_entry(std::ostream& out, const std::string& name, const Tensor& tensor) {
    if (!tensor.defined()) throw std::invalid_argument("save: undefined tensor '" + name + "'");
    put_u64(out, name.size());
    out.write(name.data(), static_cast<std::streamsize>(name.size()));
    const char code = static_cast<char>(tensor.dtype());
    out.write(&code, 1);
    put_u64(out, static_cast<std::uint64_t>(tensor.ndim()));
    for (Index dim : tensor.shape()) put_u64(out, static_cast<std::uint64_t>(dim));
    const Tensor dense = tensor.to(Device::cpu()).contiguous();
    const std::size_t width = element_size(dense.dtype());
    const std::size_t count = static_cast<std::size_t>(dense.numel());
    if (count == 0) return;
    const char* first = dense.data<char>();
    if constexpr (std::endian::native == std::endian::big) {
        std::vector<char> copy(first, first + count * width);
        swap_elements(copy.data(), count, width);
        out.write(copy.data(), static_cast<std::streamsize>(copy.size()));
    } else {
        out.write(first, static_cast<std::streamsize>(count * width));
    }
}

NamedTensor read_entry(std::istream& in) {
    const std::uint64_t length = get_u64(in);
    if (length > (std::uint64_t(1) << 20)) throw std::runtime_error("corrupt Ctorch archive: name length");
    std::string name(static_cast<std::size_t>(length), '\0');
    in.read(name.data(), static_cast<std::streamsize>(length));
    char code = 0;
    in.read(&code, 1);
    if (static_cast<unsigned char>(code) > static_cast<unsigned char>(DType::bf16))
        throw std::runtime_error("corrupt Ctorch archive: dtype code " + std::to_string(static_cast<int>(code)));
    const DType dtype = static_cast<DType>(code);
    const std::uint64_t rank = get_u64(in);
    if (rank > kMaxRank) throw std::runtime_error("corrupt Ctorch archive: rank");
    Shape shape(static_cast<std::size_t>(rank));
    std::uint64_t count = 1;
    for (auto& dim : shape) {
        const std::uint64_t value = get_u64(in);
        if (value > static_cast<std::uint64_t>(std::numeric_limits<Index>::max()) ||
            (value != 0 && count > std::numeric_limits<std::uint64_t>::max() / 16 / value))
            throw std::runtime_error("corrupt Ctorch archive: shape");
        dim = static_cast<Index>(value);
        count *= value;
    }
    const std::size_t width = element_size(dtype);
    std::vector<char> bytes(static_cast<std::size_t>(count) * width);
    in.read(bytes.data(), static_cast<std::streamsize>(bytes.size()));
    swap_elements(bytes.data(), static_cast<std::size_t>(count), width);
    return {std::move(name), detail::from_host(bytes.data(), std::move(shape), dtype, false, Device::cpu())};
}

// A temporary file in the target's directory that replaces the target on commit and is removed otherwise.
class ReplacingFile {
public:
    explicit ReplacingFile(const std::filesystem::path& path) : path_(path), temporary_(path) {
        static std::atomic<unsigned long long> sequence{0};
        const auto tick = std::chrono::steady_clock::now().time_since_epoch().count();
        temporary_ += ".tmp." + std::to_string(tick) + "." + std::to_string(sequence++);
        stream_.exceptions(std::ios::failbit | std::ios::badbit);
        stream_.open(temporary_, std::ios::binary | std::ios::trunc);
    }
    ~ReplacingFile() {
        stream_.exceptions(std::ios::goodbit);
        if (stream_.is_open()) stream_.close();
        if (!temporary_.empty()) {
            std::error_code ignored;
            std::filesystem::remove(temporary_, ignored);
        }
    }
    ReplacingFile(const ReplacingFile&) = delete;
    ReplacingFile& operator=(const ReplacingFile&) = delete;
    std::ofstream& stream() { return stream_; }
    void commit() {
        stream_.close();
        std::filesystem::rename(temporary_, path_);
        temporary_.clear();
    }

private:
    std::filesystem::path path_, temporary_;
    std::ofstream stream_;
};

} // namespace

void save(const std::filesystem::path& path, std::span<const NamedTensor> state) {
    ReplacingFile file(path);
    auto& out = file.stream();
    out.write(kHeader.data(), kHeader.size());
    put_u64(out, state.size());
    for (const auto& [name, tensor] : state) write_entry(out, name, tensor);
    file.commit();
}

StateDict load(const std::filesystem::path& path) {
    std::ifstream in;
    in.exceptions(std::ios::failbit | std::ios::badbit);
    try {
        in.open(path, std::ios::binary);
        std::array<char, 8> header{};
        in.read(header.data(), header.size());
        if (header != kHeader) throw std::runtime_error("unsupported Ctorch checkpoint format");
        const std::uint64_t count = get_u64(in);
        StateDict state;
        state.reserve(static_cast<std::size_t>(std::min<std::uint64_t>(count, 1 << 16)));
        for (std::uint64_t i = 0; i < count; ++i) state.push_back(read_entry(in));
        return state;
    } catch (const std::ios_base::failure&) {
        throw std::runtime_error("cannot read Ctorch archive " + path.string() + ": missing or truncated");
    }
}

} // namespace dl::io
