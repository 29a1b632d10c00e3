// Small kernels of the token loop and of the tensor API: strided copy/cast, fill, embedding gather,
// standalone RMSNorm / RoPE / argmax, two-phase sampling, keyed Philox generation, a generic linear for
// shapes the GEMV does not take, and a streaming copy for the bandwidth probe.
#include "kernels/device_common.h"

#include <algorithm>

namespace dlk {
namespace {

constexpr int kThreads = 256;

__device__ __forceinline__ double load_as_double(const void* base, int dtype, int64_t i) {
    switch (dtype) {
    case DLK_F32: return static_cast<const float*>(base)[i];
    case DLK_F64: return static_cast<const double*>(base)[i];
    case DLK_I64: return static_cast<double>(static_cast<const int64_t*>(base)[i]);
    case DLK_BOOL: return static_cast<const uint8_t*>(base)[i] ? 1.0 : 0.0;
    default: return bf16_to_f32(static_cast<const uint16_t*>(base)[i]);
    }
}

__device__ __forceinline__ void store_from_double(void* base, int dtype, int64_t i, double v) {
    switch (dtype) {
    case DLK_F32: static_cast<float*>(base)[i] = static_cast<float>(v); break;
    case DLK_F64: static_cast<double*>(base)[i] = v; break;
    case DLK_I64: static_cast<int64_t*>(base)[i] = static_cast<int64_t>(v); break;
    case DLK_BOOL: static_cast<uint8_t*>(base)[i] = v != 0.0; break;
    default: static_cast<uint16_t*>(base)[i] = f32_to_bf16(static_cast<float>(v)); break;
    }
}

struct CopyShape {
    int64_t shape[8], src_strides[8], dst_strides[8];
    int rank;
};

// Same-dtype copies move raw elements (exact for every type, i64 included); casts go through double, which
// is exact for every f32/bf16/f64 value and for i64 magnitudes below 2^53.
__global__ void copy_kernel(const void* src, int src_dtype, void* dst, int dst_dtype, CopyShape s, int64_t count) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t linear = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; linear < count; linear += stride) {
        int64_t rem = linear, so = 0, d = 0;
        for (int a = s.rank - 1; a >= 0; --a) {
            const int64_t i = rem % s.shape[a];
            rem /= s.shape[a];
            so += i * s.src_strides[a];
            d += i * s.dst_strides[a];
        }
        if (src_dtype == dst_dtype) {
            switch (src_dtype) {
            case DLK_F32: static_cast<float*>(dst)[d] = static_cast<const float*>(src)[so]; break;
            case DLK_F64: case DLK_I64: static_cast<int64_t*>(dst)[d] = static_cast<const int64_t*>(src)[so]; break;
            case DLK_BOOL: static_cast<uint8_t*>(dst)[d] = static_cast<const uint8_t*>(src)[so]; break;
            default: static_cast<uint16_t*>(dst)[d] = static_cast<const uint16_t*>(src)[so]; break;
            }
        } else if (src_dtype == DLK_I64 && dst_dtype == DLK_F64) {
            static_cast<double*>(dst)[d] = static_cast<double>(static_cast<const int64_t*>(src)[so]);
        } else if (src_dtype == DLK_BF16 && dst_dtype == DLK_F32) {
            // the bf16 codec on the bits (include/dl/half.h:60-66): a signalling NaN keeps its payload, which a
            // round trip through double would quiet
            static_cast<uint32_t*>(dst)[d] = static_cast<uint32_t>(static_cast<const uint16_t*>(src)[so]) << 16;
        } else if (src_dtype == DLK_F32 && dst_dtype == DLK_BF16) {
            static_cast<uint16_t*>(dst)[d] = f32_to_bf16(static_cast<const float*>(src)[so]);
        } else {
            store_from_double(dst, dst_dtype, d, load_as_double(src, src_dtype, so));
        }
    }
}

__global__ void fill_kernel(void* dst, int dtype, int64_t count, double value) {
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
        store_from_double(dst, dtype, i, value);
}

__global__ void embedding_kernel(const int64_t* ids, const void* weight, int weight_dtype, int64_t vocabulary,
                                 int64_t width, void* out, int out_dtype, int32_t* error_flag) {
    const int64_t row = blockIdx.x;
    const int64_t id = ids[row];
    const bool valid = id >= 0 && id < vocabulary;
    if (!valid && error_flag && threadIdx.x == 0) *error_flag = 1;
    for (int64_t i = threadIdx.x; i < width; i += blockDim.x) {
        const int64_t o = row * width + i;
        if (!valid) { store_from_double(out, out_dtype, o, 0.0); continue; }
        const int64_t w = id * width + i;
        if (weight_dtype == out_dtype) {
            if (out_dtype == DLK_BF16) static_cast<uint16_t*>(out)[o] = static_cast<const uint16_t*>(weight)[w];
            else if (out_dtype == DLK_F32) static_cast<float*>(out)[o] = static_cast<const float*>(weight)[w];
            else store_from_double(out, out_dtype, o, load_as_double(weight, weight_dtype, w));
        } else {
            store_from_double(out, out_dtype, o, load_as_double(weight, weight_dtype, w));
        }
    }
}

__global__ __launch_bounds__(kThreads) void rms_norm_kernel(const float* x, int64_t width, const void* weight,
                                                            int weight_bf16, float epsilon, float* y) {
    __shared__ float sums[kThreads / kWave];
    const float* row = x + static_cast<int64_t>(blockIdx.x) * width;
    float s = 0.0f;
    for (int64_t i = threadIdx.x; i < width; i += kThreads) s += row[i] * row[i];
    s = wave_sum(s);
    if (threadIdx.x % kWave == 0) sums[threadIdx.x / kWave] = s;
    __syncthreads();
    float total = 0.0f;
    for (int w = 0; w < kThreads / kWave; ++w) total += sums[w];
    const float inv = rsqrtf(total / static_cast<float>(width) + epsilon);
    float* out = y + static_cast<int64_t>(blockIdx.x) * width;
    for (int64_t i = threadIdx.x; i < width; i += kThreads) {
        const float v = row[i] * inv;
        if (!weight) out[i] = v;
        else out[i] = v * (weight_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(weight)[i])
                                       : static_cast<const float*>(weight)[i]);
    }
}

__global__ void rope_kernel(const float* x, int64_t outer, int64_t length, int64_t dim, const float* cosine,
                            const float* sine, float* y) {
    const int64_t half = dim / 2;
    const int64_t pairs = outer * length * half;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < pairs; i += stride) {
        const int64_t pair = i % half, row = i / half, l = row % length;
        const float e = x[row * dim + 2 * pair], o = x[row * dim + 2 * pair + 1];
        const float c = cosine[l * half + pair], s = sine[l * half + pair];
        y[row * dim + 2 * pair] = e * c - o * s;
        y[row * dim + 2 * pair + 1] = e * s + o * c;
    }
}

// Greedy or Gumbel-max candidates: block (row, part) scans a contiguous slice of the row.
__global__ __launch_bounds__(kThreads) void sample_partials_kernel(const float* logits, int64_t n, int mode,
                                                                   double temperature, uint64_t key_seed,
                                                                   uint64_t key_stream, const int64_t* key_label,
                                                                   dlk_sample_partial* partial, int blocks) {
    __shared__ double best_score[kThreads];
    __shared__ int64_t best_index[kThreads];
    const int64_t row = blockIdx.y;
    const int part = blockIdx.x;
    uint64_t seed = key_seed, stream = key_stream;
    if (key_label) fold_in(key_seed, key_stream, static_cast<uint64_t>(*key_label), seed, stream);
    const int64_t per = (n + blocks - 1) / blocks;
    const int64_t begin = part * per, end = min(n, begin + per);
    double best = 0.0;
    int64_t index = -1;
    for (int64_t i = begin + threadIdx.x; i < end; i += kThreads) {
        const double s = sample_score(logits[row * n + i], mode, temperature, seed, stream,
                                      static_cast<uint64_t>(row * n + i));
        if (index < 0 || prefer(s, i, best, index)) { best = s; index = i; }
    }
    best_score[threadIdx.x] = best;
    best_index[threadIdx.x] = index;
    __syncthreads();
    for (int width = kThreads / 2; width > 0; width >>= 1) {
        if (threadIdx.x < width) {
            const int64_t j = best_index[threadIdx.x + width];
            if (j >= 0) {
                const double s = best_score[threadIdx.x + width];
                const int64_t i = best_index[threadIdx.x];
                if (i < 0 || prefer(s, j, best_score[threadIdx.x], i)) {
                    best_score[threadIdx.x] = s;
                    best_index[threadIdx.x] = j;
                }
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        dlk_sample_partial out;
        out.score = best_score[0];
        out.index = best_index[0];
        partial[row * blocks + part] = out;
    }
}

constexpr int kFinalizeThreads = 256;
// One work-group per row: the row's candidates reduce with the preference rule (associative and commutative on
// distinct indices, so the reduction order does not change the result; wave shuffles, then LDS), the
// chosen id is written out, and its embedding row becomes the next step's input.  With `advance` (one row) the
// work-group also advances the step counter; several rows leave that to step_advance_kernel, launched after,
// so that no work-group reads the counter after another has written it.
__global__ __launch_bounds__(kFinalizeThreads) void sample_finalize_kernel(
    const dlk_sample_partial* partial, int blocks, int64_t* out, int64_t* next_ids, int64_t* tokens,
    int64_t token_stride, int64_t* step, int advance, const void* embedding, int embedding_dtype, int64_t width,
    float* x) {
    __shared__ double wave_score[kFinalizeThreads / kWave];
    __shared__ int64_t wave_index[kFinalizeThreads / kWave];
    __shared__ int64_t chosen;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t row = blockIdx.x;
    const int64_t column = step ? *step : 0;
    double best = 0.0;
    int64_t index = -1;
    for (int i = threadIdx.x; i < blocks; i += kFinalizeThreads) {
        const dlk_sample_partial c = partial[row * blocks + i];
        if (c.index < 0) continue;
        if (index < 0 || prefer(c.score, c.index, best, index)) { best = c.score; index = c.index; }
    }
    for (int offset = kWave / 2; offset > 0; offset >>= 1) {
        const double s = __shfl_xor(best, offset, kWave);
        const int64_t j = __shfl_xor(index, offset, kWave);
        if (j >= 0 && (index < 0 || prefer(s, j, best, index))) { best = s; index = j; }
    }
    if (lane == 0) { wave_score[wave] = best; wave_index[wave] = index; }
    __syncthreads();
    if (threadIdx.x == 0) {
        double b = 0.0;
        int64_t bi = -1;
        for (int w = 0; w < kFinalizeThreads / kWave; ++w) {
            const int64_t j = wave_index[w];
            if (j >= 0 && (bi < 0 || prefer(wave_score[w], j, b, bi))) { b = wave_score[w]; bi = j; }
        }
        chosen = bi;
        if (out) out[row] = bi;
        if (next_ids) next_ids[row] = bi;
        if (tokens) tokens[row * token_stride + column] = bi;
    }
    __syncthreads();
    if (embedding && x) {
        const int64_t id = chosen < 0 ? 0 : chosen;
        for (int64_t i = threadIdx.x; i < width; i += kFinalizeThreads)
            x[row * width + i] = embedding_dtype == DLK_BF16
                                     ? bf16_to_f32(static_cast<const uint16_t*>(embedding)[id * width + i])
                                     : static_cast<const float*>(embedding)[id * width + i];
    }
    if (advance && step && threadIdx.x == 0) *step = column + 1;
}

__global__ void step_advance_kernel(int64_t* step) { *step += 1; }

// First maximum of one row per work-group (NaN first, ties to the lower index), reference
// src/kernels/cpu/reduction.cpp:128-151.
__global__ __launch_bounds__(kThreads) void argmax_kernel(const float* x, int64_t n, int64_t* out) {
    __shared__ double best_score[kThreads];
    __shared__ int64_t best_index[kThreads];
    const float* row = x + static_cast<int64_t>(blockIdx.x) * n;
    double best = 0.0;
    int64_t index = -1;
    for (int64_t i = threadIdx.x; i < n; i += kThreads) {
        const double s = row[i];
        if (index < 0 || prefer(s, i, best, index)) { best = s; index = i; }
    }
    best_score[threadIdx.x] = best;
    best_index[threadIdx.x] = index;
    __syncthreads();
    for (int width = kThreads / 2; width > 0; width >>= 1) {
        if (threadIdx.x < width) {
            const int64_t j = best_index[threadIdx.x + width];
            if (j >= 0) {
                const double s = best_score[threadIdx.x + width];
                const int64_t i = best_index[threadIdx.x];
                if (i < 0 || prefer(s, j, best_score[threadIdx.x], i)) {
                    best_score[threadIdx.x] = s;
                    best_index[threadIdx.x] = j;
                }
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = best_index[0];
}

// Keyed uniform / normal (reference src/kernels/cpu/random.cpp:52-83 and cuda/random.cu:16-29): element i
// uses Philox(seed, i, stream); uniform = low + (high - low) * ((x >> 8) * 2^-24); normal is Box-Muller on
// words 0 and 2 with the first unit open at zero.
__global__ void random_kernel(uint64_t seed, uint64_t stream, int64_t count, int mode, float low, float high,
                              float scale, void* out, int out_dtype) {
#pragma clang fp contract(off)
    const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += step) {
        uint32_t b[4];
        philox(seed, static_cast<uint64_t>(i), stream, b);
        float value;
        if (mode == 0) {
            const float u = static_cast<float>(b[0] >> 8) * 0x1p-24f;
            value = low + (high - low) * u;
        } else {
            const float u1 = (static_cast<float>(b[0] >> 8) + 1.0f) * 0x1p-24f;
            const float u2 = static_cast<float>(b[2] >> 8) * 0x1p-24f;
            const float radius = sqrtf(-2.0f * logf(u1));
            value = radius * cosf(6.2831853071795864769f * u2);
            value = value * scale;
        }
        if (out_dtype == DLK_BF16) static_cast<uint16_t*>(out)[i] = f32_to_bf16(value);
        else static_cast<float*>(out)[i] = value;
    }
}

__global__ void linear_generic_kernel(const float* x, int64_t rows, int64_t K, const void* w, int w_dtype, int64_t N,
                                      const void* bias, int bias_dtype, float* y) {
    const int64_t total = rows * N;
    const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
        const int64_t r = i / N, n = i % N;
        float acc = 0.0f;
        for (int64_t k = 0; k < K; ++k)
            acc += x[r * K + k] * static_cast<float>(load_as_double(w, w_dtype, n * K + k));
        if (bias) acc += static_cast<float>(load_as_double(bias, bias_dtype, n));
        y[i] = acc;
    }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(kThreads) void stream_copy_kernel(const u32x4* src, u32x4* dst, uint64_t count) {
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
    for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < count; i += stride)
        __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

int grid_for(int64_t count) {
    const int64_t blocks = (count + kThreads - 1) / kThreads;
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(blocks, 8192)));
}

int status() { return static_cast<int>(hipGetLastError()); }
hipStream_t as_stream(dlh_stream s) { return reinterpret_cast<hipStream_t>(s); }

} // namespace
} // namespace dlk

using dlk::as_stream;
using dlk::grid_for;
using dlk::kThreads;

extern "C" {

int dlk_copy(const void* src, int src_dtype, const int64_t* src_strides, void* dst, int dst_dtype,
             const int64_t* dst_strides, const int64_t* shape, int rank, dlh_stream stream) {
    if (rank < 0 || rank > 8) return static_cast<int>(hipErrorInvalidValue);
    dlk::CopyShape s{};
    s.rank = rank;
    int64_t count = 1;
    for (int a = 0; a < rank; ++a) {
        s.shape[a] = shape[a];
        s.src_strides[a] = src_strides[a];
        s.dst_strides[a] = dst_strides[a];
        count *= shape[a];
    }
    if (count == 0) return 0;
    hipLaunchKernelGGL(dlk::copy_kernel, dim3(grid_for(count)), dim3(kThreads), 0, as_stream(stream), src, src_dtype,
                       dst, dst_dtype, s, count);
    return dlk::status();
}

int dlk_fill(void* dst, int dtype, int64_t count, double value, dlh_stream stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(dlk::fill_kernel, dim3(grid_for(count)), dim3(kThreads), 0, as_stream(stream), dst, dtype, count,
                       value);
    return dlk::status();
}

int dlk_embedding(const int64_t* ids, int64_t count, const void* weight, int weight_dtype, int64_t vocabulary,
                  int64_t width, void* out, int out_dtype, int32_t* error_flag, dlh_stream stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(dlk::embedding_kernel, dim3(static_cast<unsigned>(count)), dim3(kThreads), 0, as_stream(stream),
                       ids, weight, weight_dtype, vocabulary, width, out, out_dtype, error_flag);
    return dlk::status();
}

int dlk_rms_norm(const float* x, int64_t rows, int64_t width, const void* weight, int weight_bf16, float epsilon,
                 float* y, dlh_stream stream) {
    if (rows == 0) return 0;
    hipLaunchKernelGGL(dlk::rms_norm_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, as_stream(stream), x,
                       width, weight, weight_bf16, epsilon, y);
    return dlk::status();
}

int dlk_rope(const float* x, int64_t outer, int64_t length, int64_t dim, const float* cosine, const float* sine,
             float* y, dlh_stream stream) {
    const int64_t pairs = outer * length * (dim / 2);
    if (pairs == 0) return 0;
    hipLaunchKernelGGL(dlk::rope_kernel, dim3(grid_for(pairs)), dim3(kThreads), 0, as_stream(stream), x, outer, length,
                       dim, cosine, sine, y);
    return dlk::status();
}

int dlk_sample_blocks(int64_t n) {
    return static_cast<int>(std::max<int64_t>(1, std::min<int64_t>(64, (n + 2047) / 2048)));
}

int dlk_sample_partials(const float* logits, int64_t rows, int64_t n, int mode, double temperature, uint64_t key_seed,
                        uint64_t key_stream, const int64_t* key_label, dlk_sample_partial* partial, int blocks,
                        dlh_stream stream) {
    if (rows == 0) return 0;
    hipLaunchKernelGGL(dlk::sample_partials_kernel, dim3(blocks, static_cast<unsigned>(rows)), dim3(kThreads), 0,
                       as_stream(stream), logits, n, mode, temperature, key_seed, key_stream, key_label, partial, blocks);
    return dlk::status();
}

int dlk_sample_finalize(const dlk_sample_partial* partial, int64_t rows, int blocks, int64_t* out, int64_t* next_ids,
                        int64_t* tokens, int64_t token_stride, int64_t* step, const void* embedding,
                        int embedding_dtype, int64_t width, float* x, dlh_stream stream) {
    if (rows <= 0) return 0;
    const int advance = rows == 1;
    hipLaunchKernelGGL(dlk::sample_finalize_kernel, dim3(static_cast<unsigned>(rows)), dim3(dlk::kFinalizeThreads), 0,
                       as_stream(stream), partial, blocks, out, next_ids, tokens, token_stride, step, advance,
                       embedding, embedding_dtype, width, x);
    int status = dlk::status();
    if (status == 0 && !advance && step) {
        hipLaunchKernelGGL(dlk::step_advance_kernel, dim3(1), dim3(1), 0, as_stream(stream), step);
        status = dlk::status();
    }
    return status;
}

int dlk_argmax(const float* x, int64_t rows, int64_t n, int64_t* out, dlh_stream stream) {
    if (n <= 0) return static_cast<int>(hipErrorInvalidValue);
    if (rows == 0) return 0;
    hipLaunchKernelGGL(dlk::argmax_kernel, dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, as_stream(stream), x,
                       n, out);
    return dlk::status();
}

int dlk_random(uint64_t seed, uint64_t stream_bits, int64_t count, int mode, double low, double high, double scale,
               void* out, int out_dtype, dlh_stream stream) {
    if (count == 0) return 0;
    hipLaunchKernelGGL(dlk::random_kernel, dim3(grid_for(count)), dim3(kThreads), 0, as_stream(stream), seed,
                       stream_bits, count, mode, static_cast<float>(low), static_cast<float>(high),
                       static_cast<float>(scale), out, out_dtype);
    return dlk::status();
}

int dlk_linear_generic(const float* x, int64_t rows, int64_t K, const void* w, int w_dtype, int64_t N,
                       const void* bias, int bias_dtype, float* y, dlh_stream stream) {
    const int64_t total = rows * N;
    if (total == 0) return 0;
    hipLaunchKernelGGL(dlk::linear_generic_kernel, dim3(grid_for(total)), dim3(kThreads), 0, as_stream(stream), x, rows,
                       K, w, w_dtype, N, bias, bias_dtype, y);
    return dlk::status();
}

int dlk_stream_copy(const void* src, void* dst, uint64_t bytes, dlh_stream stream) {
    if (bytes % 16 != 0) return static_cast<int>(hipErrorInvalidValue);
    const uint64_t count = bytes / 16;
    hipLaunchKernelGGL(dlk::stream_copy_kernel, dim3(2048), dim3(kThreads), 0, as_stream(stream),
                       static_cast<const dlk::u32x4*>(src), static_cast<dlk::u32x4*>(dst), count);
    return dlk::status();
}

} // extern "C"
