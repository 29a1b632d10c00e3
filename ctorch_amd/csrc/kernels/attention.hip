// Split-K grouped-query decode attention (see dlk_attention_params in kernels.h).
//
// Grid (key split, query-row block, b * KV + kv head).  A work-group serves up to kRowsMax query rows of one
// KV head: the H/KV query heads that share it, for one or more new positions.  It walks its key range in
// tiles of T keys: the K and V tiles are loaded from HBM once (coalesced 16-byte loads, the next tile
// prefetched into registers while the current one is used) and staged in LDS with a padded row stride, so
// every query head of the group reuses them.  Scores use one lane per key, softmax is online (running max and
// sum per row, wave64 reductions), P*V uses one lane per head-dim column.  With one split the work-group
// writes the normalised output; otherwise it writes (o, max, sum) partials that attention_combine merges in a
// second launch (the kernel boundary orders them: no device-scope fence, whose L2 write-back across the XCDs
// costs microseconds per work-group).
#include "kernels/device_common.h"

#include <algorithm>
#include <mutex>
#include <type_traits>

namespace dlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kRowsMax = 16;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

template <typename KT> struct KvTraits;
template <> struct KvTraits<uint16_t> {
    __device__ static __forceinline__ float at(const uint32_t* row, int d) {
        const uint32_t w = row[d >> 1];
        return (d & 1) ? bf16_hi(w) : bf16_lo(w);
    }
};
template <> struct KvTraits<float> {
    __device__ static __forceinline__ float at(const uint32_t* row, int d) { return __uint_as_float(row[d]); }
};

template <typename KT, int HD, int T>
__global__ __launch_bounds__(kThreads) void attention_kernel(const dlk_attention_params p) {
    constexpr int ES = sizeof(KT);
    constexpr int ROW_WORDS = HD * ES / 4 + 1;            // padded LDS row: odd word stride, no bank conflicts
    constexpr int CHUNKS_PER_ROW = HD * ES / 16;          // 16-byte chunks per K/V row
    constexpr int TILE_CHUNKS = T * CHUNKS_PER_ROW;
    constexpr int LOADS = (TILE_CHUNKS + kThreads - 1) / kThreads;
    constexpr int DCOLS = (HD + kWave - 1) / kWave;       // head-dim columns per lane in P*V
    constexpr int RPW = kRowsMax / kWaves;                // rows per wave

    __shared__ uint32_t k_tile[T * ROW_WORDS];
    __shared__ uint32_t v_tile[T * ROW_WORDS];
    __shared__ float q_tile[kRowsMax][HD];
    __shared__ float p_tile[kRowsMax][T];

    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    const int split = blockIdx.x, row_block = blockIdx.y;
    const int b = blockIdx.z / p.KV, kvh = blockIdx.z % p.KV;
    const int G = p.H / p.KV;
    const int rows_total = G * p.L;
    const int row0 = row_block * kRowsMax;
    const int rows = min(kRowsMax, rows_total - row0);
    const int64_t first = p.position ? *p.position : p.first_host;
    const int64_t S = first + p.L;

    // query row r of this block -> (l, g): rows are ordered l-major so a block spans few positions
    auto row_l = [&](int r) { return (row0 + r) / G; };
    auto row_h = [&](int r) { return kvh * G + (row0 + r) % G; };

    int64_t k_begin = static_cast<int64_t>(split) * p.chunk;
    int64_t k_end = min(S, k_begin + p.chunk);
    if (p.causal) k_end = min(k_end, first + row_l(rows - 1) + 1);

    const size_t head_base = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity;
    const KT* kbase = static_cast<const KT*>(p.k) + head_base * HD;
    const KT* vbase = static_cast<const KT*>(p.v) + head_base * HD;

    // q rows (scaled once) into LDS
    for (int i = t; i < rows * HD; i += kThreads) {
        const int r = i / HD, d = i % HD;
        const int64_t m = static_cast<int64_t>(b) * p.L + row_l(r);
        q_tile[r][d] = p.q[m * p.ldq + static_cast<int64_t>(row_h(r)) * HD + d] * p.scale;
    }

    float m_run[RPW], l_run[RPW], o_acc[RPW][DCOLS];
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        m_run[j] = -INFINITY;
        l_run[j] = 0.0f;
#pragma unroll
        for (int c = 0; c < DCOLS; ++c) o_acc[j][c] = 0.0f;
    }

    u32x4 k_next[LOADS], v_next[LOADS];
    auto load_tile = [&](int64_t tile0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int chunk = t + i * kThreads;
            const int key = chunk / CHUNKS_PER_ROW, part = chunk % CHUNKS_PER_ROW;
            const int64_t kk = tile0 + key;
            if (chunk < TILE_CHUNKS && kk < k_end) {
                const size_t offset = static_cast<size_t>(kk) * HD * ES + static_cast<size_t>(part) * 16;
                k_next[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(kbase) + offset);
                v_next[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(vbase) + offset);
            } else {
                k_next[i] = u32x4{0u, 0u, 0u, 0u};
                v_next[i] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&]() {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int chunk = t + i * kThreads;
            if (chunk < TILE_CHUNKS) {
                const int key = chunk / CHUNKS_PER_ROW, part = chunk % CHUNKS_PER_ROW;
                uint32_t* kd = k_tile + key * ROW_WORDS + part * 4;
                uint32_t* vd = v_tile + key * ROW_WORDS + part * 4;
                kd[0] = k_next[i].x; kd[1] = k_next[i].y; kd[2] = k_next[i].z; kd[3] = k_next[i].w;
                vd[0] = v_next[i].x; vd[1] = v_next[i].y; vd[2] = v_next[i].z; vd[3] = v_next[i].w;
            }
        }
    };

    if (k_begin < k_end) load_tile(k_begin);
    for (int64_t tile0 = k_begin; tile0 < k_end; tile0 += T) {
        __syncthreads(); // previous tile fully consumed (and q_tile written before the first tile)
        store_tile();
        __syncthreads();
        if (tile0 + T < k_end) load_tile(tile0 + T); // in flight while this tile is used

#pragma unroll
        for (int j = 0; j < RPW; ++j) {
            const int r = wave + j * kWaves;
            if (r >= rows) break;
            // scores: lane = key
            float s = -INFINITY;
            const int64_t kk = tile0 + lane;
            int64_t limit = k_end;
            if (p.causal) limit = min(limit, first + row_l(r) + 1);
            if (lane < T && kk < limit) {
                const uint32_t* krow = k_tile + lane * ROW_WORDS;
                float acc = 0.0f;
#pragma unroll
                for (int d = 0; d < HD; ++d) acc += q_tile[r][d] * KvTraits<KT>::at(krow, d);
                s = acc;
                if (p.keep_mask && !p.keep_mask[b * p.mask_stride[0] + row_h(r) * p.mask_stride[1] +
                                                row_l(r) * p.mask_stride[2] + kk * p.mask_stride[3]])
                    s = -INFINITY;
            }
            const float tile_max = wave_max(s);
            const float m_new = fmaxf(m_run[j], tile_max);
            float pr = 0.0f, alpha = 1.0f;
            if (m_new != -INFINITY) {
                pr = s == -INFINITY ? 0.0f : expf(s - m_new);
                alpha = m_run[j] == -INFINITY ? 0.0f : expf(m_run[j] - m_new);
            }
            const float tile_sum = wave_sum(pr);
            l_run[j] = l_run[j] * alpha + tile_sum;
            m_run[j] = m_new;
            if (lane < T) p_tile[r][lane] = pr;
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            // P*V: lane = head-dim column
#pragma unroll
            for (int c = 0; c < DCOLS; ++c) {
                const int d = lane + c * kWave;
                float acc = o_acc[j][c] * alpha;
                if (d < HD) {
#pragma unroll 8
                    for (int key = 0; key < T; ++key)
                        acc += p_tile[r][key] * KvTraits<KT>::at(v_tile + key * ROW_WORDS, d);
                }
                o_acc[j][c] = acc;
            }
        }
    }

    // write results: the normalised output with one split, else (o, max, sum) partials for the combine pass
#pragma unroll
    for (int j = 0; j < RPW; ++j) {
        const int r = wave + j * kWaves;
        if (r >= rows) break;
        const int l = row_l(r), h = row_h(r);
        const int64_t m = static_cast<int64_t>(b) * p.L + l;
        if (p.splits == 1) {
            // a masked row that kept no key: NaN, as the reference's softmax over an all -inf row
            const float inv = l_run[j] > 0.0f ? 1.0f / l_run[j] : p.keep_mask ? __builtin_nanf("") : 0.0f;
#pragma unroll
            for (int c = 0; c < DCOLS; ++c) {
                const int d = lane + c * kWave;
                if (d < HD) p.out[m * p.ldo + static_cast<int64_t>(h) * HD + d] = o_acc[j][c] * inv;
            }
        } else {
            const int64_t prow = (static_cast<int64_t>(b) * p.H + h) * p.L + l;
            const int64_t slot = prow * p.splits + split;
#pragma unroll
            for (int c = 0; c < DCOLS; ++c) {
                const int d = lane + c * kWave;
                if (d < HD) p.partial_o[slot * HD + d] = o_acc[j][c];
            }
            if (lane == 0) {
                p.partial_ml[slot * 2] = m_run[j];
                p.partial_ml[slot * 2 + 1] = l_run[j];
            }
        }
    }
}

// One work-group per (b, h, l) row merges its split partials: the global maximum first, then each thread takes
// one head-dim column and every (512 / HD)-th split, and the column groups add up in LDS in a fixed order.  A
// thread loads four of its splits at a time (the last group clamped to a valid split and discarded), so their
// loads are in flight together; dead splits are dropped by selection, never by a branch around the loads.
constexpr int kCombineThreads = 512;

template <int HD>
__global__ __launch_bounds__(kCombineThreads) void attention_combine(const dlk_attention_params p) {
    constexpr int GROUPS = kCombineThreads / HD;
    constexpr int WAVES = kCombineThreads / kWave;
    constexpr int U = 4; // splits per thread in flight
    __shared__ float wave_max_s[WAVES];
    __shared__ float acc_s[GROUPS][HD];
    __shared__ float total_s[GROUPS];
    const int64_t prow = blockIdx.x; // (b * H + h) * L + l
    const int t = threadIdx.x, lane = t % kWave;
    const int64_t l = prow % p.L, h = (prow / p.L) % p.H, b = prow / (static_cast<int64_t>(p.L) * p.H);
    const float* ml = p.partial_ml + prow * p.splits * 2;
    float maximum = -INFINITY;
    for (int s = t; s < p.splits; s += kCombineThreads)
        if (ml[2 * s + 1] > 0.0f) maximum = fmaxf(maximum, ml[2 * s]);
    maximum = wave_max(maximum);
    if (lane == 0) wave_max_s[t / kWave] = maximum;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < WAVES; ++w) maximum = fmaxf(maximum, wave_max_s[w]);
    const int d = t % HD, group = t / HD;
    float acc = 0.0f, total = 0.0f;
    for (int s0 = group; s0 < p.splits; s0 += U * GROUPS) {
        float ms[U], ls[U], o[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int s = min(s0 + u * GROUPS, p.splits - 1);
            ms[u] = ml[2 * s];
            ls[u] = ml[2 * s + 1];
            o[u] = p.partial_o[(prow * p.splits + s) * HD + d];
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            // a split without keys has weight 0 and an unwritten partial_o row: it must not enter the sum (0 * a
            // stale NaN or Inf would), so it is selected away
            const bool live = s0 + u * GROUPS < p.splits && ls[u] > 0.0f && ms[u] != -INFINITY;
            const float w = live ? expf(ms[u] - maximum) : 0.0f;
            total += live ? w * ls[u] : 0.0f;
            acc += live ? w * o[u] : 0.0f;
        }
    }
    acc_s[group][d] = acc;
    if (d == 0) total_s[group] = total;
    __syncthreads();
    if (group == 0) {
        float sum = 0.0f, weight = 0.0f;
#pragma unroll
        for (int g = 0; g < GROUPS; ++g) {
            sum += acc_s[g][d];
            weight += total_s[g];
        }
        const float inv = weight > 0.0f ? 1.0f / weight : p.keep_mask ? __builtin_nanf("") : 0.0f;
        p.out[(b * p.L + l) * p.ldo + h * HD + d] = sum * inv;
    }
}

// ------------------------------------------------------------------------------------------ small heads
// Head sizes below 16 (the reference's tiny test decoders: tests/c_api.c:31 builds one with head size 2).  Not a hot
// path: one wave per (query row, key split); lane = key within each 64-key step, the scores and the weighted V
// columns reduced over the wave, online softmax across the steps.  Writes the output, or (o, max, sum) partials
// for attention_combine when the keys are split.
template <typename KT, int HD>
__global__ __launch_bounds__(kWave) void attention_small(const dlk_attention_params p) {
    const int lane = threadIdx.x;
    const int64_t prow = blockIdx.x; // (b * H + h) * L + l
    const int split = blockIdx.y;
    const int l = static_cast<int>(prow % p.L), h = static_cast<int>((prow / p.L) % p.H);
    const int b = static_cast<int>(prow / (static_cast<int64_t>(p.L) * p.H));
    const int kvh = h / (p.H / p.KV);
    const int64_t first = p.position ? *p.position : p.first_host;
    const int64_t S = first + p.L;
    const int64_t visible = p.causal ? min(S, first + l + 1) : S;
    const int64_t k_begin = static_cast<int64_t>(split) * p.chunk;
    const int64_t k_end = min(visible, k_begin + p.chunk);
    const float* qrow = p.q + (static_cast<int64_t>(b) * p.L + l) * p.ldq + static_cast<int64_t>(h) * HD;
    float q[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) q[d] = qrow[d] * p.scale;
    const size_t head = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity;
    const KT* kbase = static_cast<const KT*>(p.k) + head * HD;
    const KT* vbase = static_cast<const KT*>(p.v) + head * HD;
    auto value = [](const KT* row, int d) {
        if constexpr (sizeof(KT) == 2) return bf16_to_f32(reinterpret_cast<const uint16_t*>(row)[d]);
        else return static_cast<float>(row[d]);
    };
    float m = -INFINITY, total = 0.0f, o[HD];
#pragma unroll
    for (int d = 0; d < HD; ++d) o[d] = 0.0f;
    const unsigned char* keep =
        p.keep_mask ? p.keep_mask + b * p.mask_stride[0] + h * p.mask_stride[1] + l * p.mask_stride[2] : nullptr;
    for (int64_t k0 = k_begin; k0 < k_end; k0 += kWave) {
        const int64_t key = k0 + lane;
        // a live key the mask keeps (without a mask every step holds one, so m_new is finite)
        const bool live = key < k_end && (!keep || keep[key * p.mask_stride[3]]);
        float s = -INFINITY;
        if (live) {
            s = 0.0f;
#pragma unroll
            for (int d = 0; d < HD; ++d) s += q[d] * value(kbase + key * HD, d);
        }
        const float m_new = fmaxf(m, wave_max(s));
        const float alpha = m == -INFINITY ? 0.0f : expf(m - m_new);
        const float pr = live ? expf(s - m_new) : 0.0f;
        total = total * alpha + wave_sum(pr);
#pragma unroll
        for (int d = 0; d < HD; ++d) o[d] = o[d] * alpha + wave_sum(live ? pr * value(vbase + key * HD, d) : 0.0f);
        m = m_new;
    }
    if (lane != 0) return;
    if (p.splits == 1) {
        float* out = p.out + (static_cast<int64_t>(b) * p.L + l) * p.ldo + static_cast<int64_t>(h) * HD;
#pragma unroll
        for (int d = 0; d < HD; ++d) out[d] = total > 0.0f ? o[d] / total : keep ? __builtin_nanf("") : 0.0f;
    } else {
        const int64_t slot = prow * p.splits + split;
#pragma unroll
        for (int d = 0; d < HD; ++d) p.partial_o[slot * HD + d] = o[d];
        p.partial_ml[slot * 2] = m;
        p.partial_ml[slot * 2 + 1] = total;
    }
}

template <typename KT, int HD>
int launch_small(const dlk_attention_params& p, hipStream_t stream) {
    const int64_t rows = static_cast<int64_t>(p.B) * p.H * p.L;
    hipLaunchKernelGGL((attention_small<KT, HD>), dim3(static_cast<unsigned>(rows), p.splits), dim3(kWave), 0, stream,
                       p);
    int status = static_cast<int>(hipGetLastError());
    if (status != 0 || p.splits == 1 || p.partials_only) return status;
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(rows)), dim3(kCombineThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

template <int HD>
int launch_combine(const dlk_attention_params& p, hipStream_t stream) {
    const int64_t combine_rows = static_cast<int64_t>(p.B) * p.H * p.L;
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(combine_rows)), dim3(kCombineThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

template <typename KT, int HD>
int launch(const dlk_attention_params& p, hipStream_t stream) {
    // 64-key tiles; f32 K/V with 128-wide heads use 32-key tiles to keep the LDS footprint under 64 KB
    constexpr int T = sizeof(KT) * HD > 256 ? 32 : 64;
    const int G = p.H / p.KV;
    const int row_blocks = (G * p.L + kRowsMax - 1) / kRowsMax;
    dim3 grid(p.splits, row_blocks, p.B * p.KV);
    hipLaunchKernelGGL((attention_kernel<KT, HD, T>), grid, dim3(kThreads), 0, stream, p);
    int status = static_cast<int>(hipGetLastError());
    if (status != 0 || p.splits == 1 || p.partials_only) return status;
    const int64_t combine_rows = static_cast<int64_t>(p.B) * p.H * p.L;
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(combine_rows)), dim3(kCombineThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

} // namespace
} // namespace dlk

// Key-split partials of the allocation-free attention entry: a fixed array in device memory, one copy per GPU the
// library runs on, held until the process ends.  Host code never passes the array's name to a kernel (on the host
// it is only a stand-in for the symbol): dlk_attention_scratch resolves each device's own address once, with that
// device current, and the launches take that address.
static __device__ __align__(256) float scratch[DLK_ATTENTION_SCRATCH_FLOATS];

extern "C" int dlk_attention_scratch(int device, float** address) {
    constexpr int kDevicesMax = 64;
    static std::mutex mutex;
    static float* addresses[kDevicesMax] = {};
    if (!address || device < 0 || device >= kDevicesMax) return static_cast<int>(hipErrorInvalidValue);
    std::lock_guard<std::mutex> lock(mutex);
    if (!addresses[device]) {
        int current = 0;
        hipError_t status = hipGetDevice(&current);
        if (status != hipSuccess) return static_cast<int>(status);
        if (current != device && (status = hipSetDevice(device)) != hipSuccess) return static_cast<int>(status);
        void* found = nullptr;
        status = hipGetSymbolAddress(&found, HIP_SYMBOL(scratch));
        if (current != device) {
            const hipError_t restored = hipSetDevice(current);
            if (status == hipSuccess) status = restored;
        }
        if (status != hipSuccess) return static_cast<int>(status);
        if (!found) return static_cast<int>(hipErrorInvalidSymbol);
        addresses[device] = static_cast<float*>(found);
    }
    *address = addresses[device];
    return 0;
}

extern "C" int dlk_attention(const dlk_attention_params* params, dlh_stream stream_handle) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    const dlk_attention_params& p = *params;
    if (p.B <= 0 || p.L <= 0 || p.KV <= 0 || p.H % p.KV != 0 || p.splits <= 0 || p.chunk <= 0 ||
        (p.splits > 1 && (!p.partial_o || !p.partial_ml)) || (p.splits > 1 && p.chunk % 64 != 0))
        return static_cast<int>(hipErrorInvalidValue);
    // a keep mask is applied by the general and small-head kernels, which serve non-causal attention
    if (p.keep_mask && (p.causal || p.qkv_partial || p.stage_out || p.kv_split)) return static_cast<int>(hipErrorInvalidValue);
    // the QKV projection's partials are finished only by the matrix kernel
    if (p.qkv_partial && (p.stage_out || !dlk_attention_matrix_eligible(&p))) return static_cast<int>(hipErrorInvalidValue);
    // the staged output exists only on the prefill kernel
    if (p.stage_out) {
        if (!dlk_attention_prefill_eligible(&p) || (p.H * p.hd) % 32 != 0 ||
            reinterpret_cast<uintptr_t>(p.stage_out) % 16 != 0)
            return static_cast<int>(hipErrorInvalidValue);
        return dlk_attention_prefill(&p, stream_handle);
    }
    // one position on the matrix cores, then the merge of its key splits
    if (dlk_attention_matrix_eligible(&p)) {
        const int status = dlk_attention_matrix_decode(&p, stream_handle);
        if (status != 0 || p.splits == 1 || p.partials_only) return status;
        return p.hd == 64 ? dlk::launch_combine<64>(p, stream) : dlk::launch_combine<128>(p, stream);
    }
    if (dlk_attention_prefill_eligible(&p)) return dlk_attention_prefill(&p, stream_handle);
    if (p.hd < 16) {
        switch (p.hd) {
        case 2: return p.kv_bf16 ? dlk::launch_small<uint16_t, 2>(p, stream) : dlk::launch_small<float, 2>(p, stream);
        case 4: return p.kv_bf16 ? dlk::launch_small<uint16_t, 4>(p, stream) : dlk::launch_small<float, 4>(p, stream);
        case 8: return p.kv_bf16 ? dlk::launch_small<uint16_t, 8>(p, stream) : dlk::launch_small<float, 8>(p, stream);
        default: return static_cast<int>(hipErrorInvalidValue);
        }
    }
    if (p.kv_bf16) {
        switch (p.hd) {
        case 16: return dlk::launch<uint16_t, 16>(p, stream);
        case 32: return dlk::launch<uint16_t, 32>(p, stream);
        case 64: return dlk::launch<uint16_t, 64>(p, stream);
        case 128: return dlk::launch<uint16_t, 128>(p, stream);
        default: return static_cast<int>(hipErrorInvalidValue);
        }
    }
    switch (p.hd) {
    case 16: return dlk::launch<float, 16>(p, stream);
    case 32: return dlk::launch<float, 32>(p, stream);
    case 64: return dlk::launch<float, 64>(p, stream);
    case 128: return dlk::launch<float, 128>(p, stream);
    default: return static_cast<int>(hipErrorInvalidValue);
    }
}
