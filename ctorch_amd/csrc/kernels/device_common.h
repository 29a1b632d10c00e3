// Device helpers shared by the kernels: bf16 codec, Philox4x32-10, the portable Gumbel noise, wave64
// reductions and the argmax preference rule.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "kernels/kernels.h"

namespace dlk {

constexpr int kWave = 64;
/// Buffer descriptor word 3 for raw (untyped) buffer access on gfx9-family GPUs.
constexpr int kBufferFlags = 0x00020000;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }
__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Every 64-byte line of a kernel's argument block (BYTES of explicit arguments, then the line of the implicit
// ones the runtime appends: grid and group sizes) requested at once, at entry.  The compiler loads each argument
// where it is first used, so the lines of a large parameter struct arrive in several dependent scalar round trips
// (a branch's operand, then the next block's pointers, ...), and between the steps of a decode the weight stream
// has evicted them from the caches; touched together here they cost one round trip, and the later loads hit.
template <int EXPLICIT>
__device__ __forceinline__ void touch_kernargs() {
    constexpr int LINES = ((EXPLICIT + 7) / 8 * 8 + 64 + 63) / 64;
    static_assert(LINES <= 10, "one operand per line below");
    typedef const __attribute__((address_space(4))) uint32_t KernargWord;
    KernargWord* words = (KernargWord*)__builtin_amdgcn_kernarg_segment_ptr();
    // one word of each line, all consumed by a single statement: a scalar load's result waits for every scalar
    // load in flight, so one use point keeps them in one round trip
    uint32_t v[10];
#pragma unroll
    for (int i = 0; i < 10; ++i) v[i] = words[16 * (i < LINES ? i : LINES - 1)];
    __asm__ volatile("" ::"s"(v[0]), "s"(v[1]), "s"(v[2]), "s"(v[3]), "s"(v[4]), "s"(v[5]), "s"(v[6]), "s"(v[7]),
                     "s"(v[8]), "s"(v[9]));
}

// wait until at most n vector-memory operations of this wave are outstanding (lgkm and exp counts untouched)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16-byte global->LDS DMA: this lane's 16 bytes at base + offset land at LDS offset lds_base + 16 * lane (base
// and lds_base wave-uniform).  Issued as inline asm so that the compiler's own wait insertion does not see it
// (it would drain every DMA in flight before each LDS read): the caller waits for it explicitly (wait_vm) before
// the work-group barrier that publishes the LDS data.  The compiler's own waits for its loads stay correct (the
// count of operations issued after a load only grows with the DMAs, so they wait longer, never shorter).
__device__ __forceinline__ void dma16(const void* base, uint32_t offset, uint32_t lds_base) {
    // M0 (the LDS destination) is reserved by the compiler: saved and restored around the DMA
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %3\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(offset), "s"(base), "s"(lds_base)
                 : "memory");
}

__device__ __forceinline__ uint32_t lds_offset(const void* p) {
    return static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p));
}

/// f32 -> bf16, round to nearest even, NaN quieted (reference include/dl/half.h:43-47).
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    const uint32_t b = __float_as_uint(v);
    if ((b & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((b >> 16) | 0x40u);
    return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

/// Philox4x32-10 with counter (index lo, index hi, stream lo, stream hi) and key (seed lo, seed hi)
/// (reference src/core/philox.h:26-38).
__device__ __forceinline__ void philox(uint64_t seed, uint64_t index, uint64_t stream, uint32_t out[4]) {
    uint32_t c0 = static_cast<uint32_t>(index), c1 = static_cast<uint32_t>(index >> 32);
    uint32_t c2 = static_cast<uint32_t>(stream), c3 = static_cast<uint32_t>(stream >> 32);
    uint32_t k0 = static_cast<uint32_t>(seed), k1 = static_cast<uint32_t>(seed >> 32);
#pragma unroll
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = static_cast<uint64_t>(c0) * 0xd2511f53u;
        const uint64_t p1 = static_cast<uint64_t>(c2) * 0xcd9e8d57u;
        const uint32_t n0 = static_cast<uint32_t>(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = static_cast<uint32_t>(p0 >> 32) ^ c3 ^ k1;
        c1 = static_cast<uint32_t>(p1);
        c3 = static_cast<uint32_t>(p0);
        c0 = n0;
        c2 = n2;
        k0 += 0x9e3779b9u;
        k1 += 0xbb67ae85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

/// fold_in(key, label): the Philox block of (seed, label, stream) packed into a new (seed, stream)
/// (reference src/core/random.cpp:14-18).
__device__ __forceinline__ void fold_in(uint64_t seed, uint64_t stream, uint64_t label, uint64_t& out_seed,
                                        uint64_t& out_stream) {
    uint32_t b[4];
    philox(seed, label, stream, b);
    out_seed = static_cast<uint64_t>(b[0]) | (static_cast<uint64_t>(b[1]) << 32);
    out_stream = static_cast<uint64_t>(b[2]) | (static_cast<uint64_t>(b[3]) << 32);
}

/// Natural log of a positive finite double from IEEE add/sub/mul/div only (no contraction), so that the
/// host restatement evaluates identical bits: x = m 2^e, m in [sqrt(1/2), sqrt(2)), log m = 2 atanh(s),
/// s = (m-1)/(m+1), odd series to s^23, ln 2 split in a high and a low part.
__device__ __noinline__ double portable_log(double x) {
#pragma clang fp contract(off)
    uint64_t bits = __double_as_longlong(x);
    int64_t exponent = static_cast<int64_t>((bits >> 52) & 0x7ff);
    if (exponent == 0) {
        x = x * 0x1p54;
        bits = __double_as_longlong(x);
        exponent = static_cast<int64_t>((bits >> 52) & 0x7ff) - 54;
    }
    exponent -= 1023;
    const uint64_t mantissa_bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m = __longlong_as_double(static_cast<long long>(mantissa_bits));
    if (m > 1.4142135623730951) { m = m * 0.5; exponent += 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double t = s * s;
    double p = 1.0 / 23.0;
    p = p * t + 1.0 / 21.0;
    p = p * t + 1.0 / 19.0;
    p = p * t + 1.0 / 17.0;
    p = p * t + 1.0 / 15.0;
    p = p * t + 1.0 / 13.0;
    p = p * t + 1.0 / 11.0;
    p = p * t + 1.0 / 9.0;
    p = p * t + 1.0 / 7.0;
    p = p * t + 1.0 / 5.0;
    p = p * t + 1.0 / 3.0;
    p = p * t + 1.0;
    const double log_m = 2.0 * s * p;
    const double e = static_cast<double>(exponent);
    return e * 6.93147180369123816490e-01 + (e * 1.90821492927058770002e-10 + log_m);
}

/// Gumbel noise g = -log(-log u), u = ((53-bit Philox value >> 1) + 0.5) * 2^-52 strictly inside (0, 1).
__device__ __forceinline__ double gumbel(uint64_t seed, uint64_t stream, uint64_t index) {
    uint32_t b[4];
    philox(seed, index, stream, b);
    const uint64_t bits = (static_cast<uint64_t>(b[0] >> 5) << 26) | (b[1] >> 6);
    const double u = (static_cast<double>(bits >> 1) + 0.5) * 0x1p-52;
    return -portable_log(-portable_log(u));
}

/// Sampling score: the logit for greedy, logit / T + Gumbel noise otherwise (no contraction).
__device__ __forceinline__ double sample_score(float logit, int mode, double temperature, uint64_t seed,
                                               uint64_t stream, uint64_t index) {
#pragma clang fp contract(off)
    if (mode != 2) return static_cast<double>(logit);
    const double scaled = static_cast<double>(logit) / temperature;
    return scaled + gumbel(seed, stream, index);
}

/// argmax preference (reference src/kernels/cpu/reduction.cpp:141-145): a NaN beats everything and the
/// first NaN wins; otherwise the larger value, ties to the lower index.
__device__ __forceinline__ bool prefer(double a, int64_t ia, double b, int64_t ib) {
    const bool an = a != a, bn = b != b;
    if (an || bn) return an && (!bn || ia < ib);
    if (a != b) return a > b;
    return ia < ib;
}

// Wave64 all-reductions without LDS: DPP steps reduce each row of 16 lanes (pair, quad, half-row, row; every
// lane ends with its row's value), then the four row values are read into scalars and combined.  The result
// is wave-uniform and identical in every lane.  All 64 lanes must be active.
template <typename Op>
__device__ __forceinline__ float wave_reduce(float v, Op op) {
    constexpr int kQuadSwap1 = 0xB1; // quad_perm [1, 0, 3, 2]
    constexpr int kQuadSwap2 = 0x4E; // quad_perm [2, 3, 0, 1]
    constexpr int kHalfMirror = 0x141;
    constexpr int kRowMirror = 0x140;
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v = op(v, dpp(v, std::integral_constant<int, kQuadSwap1>{}));
    v = op(v, dpp(v, std::integral_constant<int, kQuadSwap2>{}));
    v = op(v, dpp(v, std::integral_constant<int, kHalfMirror>{}));
    v = op(v, dpp(v, std::integral_constant<int, kRowMirror>{}));
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return op(op(r0, r1), op(r2, r3));
}

__device__ __forceinline__ float wave_sum(float v) {
    return wave_reduce(v, [](float a, float b) { return a + b; });
}
__device__ __forceinline__ float wave_max(float v) {
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}

} // namespace dlk
