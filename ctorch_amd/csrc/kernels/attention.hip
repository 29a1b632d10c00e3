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
constexpr int kDecodeChunkMax = 16 * kWave; // keys per work-group of the decode kernel, at most
static_assert(kDecodeChunkMax == DLK_DECODE_CHUNK_MAX, "decode chunk");
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
            const float inv = l_run[j] > 0.0f ? 1.0f / l_run[j] : 0.0f;
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
// one head-dim column and every (256 / HD)-th split, and the column groups add up in LDS in a fixed order.
template <int HD>
__global__ __launch_bounds__(kThreads) void attention_combine(const dlk_attention_params p) {
    constexpr int GROUPS = kThreads / HD;
    __shared__ float wave_max_s[kWaves];
    __shared__ float acc_s[GROUPS][HD];
    __shared__ float total_s[GROUPS];
    const int64_t prow = blockIdx.x; // (b * H + h) * L + l
    const int t = threadIdx.x, lane = t % kWave;
    const int64_t l = prow % p.L, h = (prow / p.L) % p.H, b = prow / (static_cast<int64_t>(p.L) * p.H);
    const float* ml = p.partial_ml + prow * p.splits * 2;
    float maximum = -INFINITY;
    for (int s = t; s < p.splits; s += kThreads)
        if (ml[2 * s + 1] > 0.0f) maximum = fmaxf(maximum, ml[2 * s]);
    maximum = wave_max(maximum);
    if (lane == 0) wave_max_s[t / kWave] = maximum;
    __syncthreads();
    maximum = fmaxf(fmaxf(wave_max_s[0], wave_max_s[1]), fmaxf(wave_max_s[2], wave_max_s[3]));
    const int d = t % HD, group = t / HD;
    float acc = 0.0f, total = 0.0f;
    for (int s = group; s < p.splits; s += GROUPS) {
        const float ms = ml[2 * s], ls = ml[2 * s + 1];
        // a split without keys has weight 0 and an unwritten partial_o row: it must not enter the sum (0 * a
        // stale NaN or Inf would)
        if (!(ls > 0.0f && ms != -INFINITY)) continue;
        const float w = expf(ms - maximum);
        total += w * ls;
        acc += w * p.partial_o[(prow * p.splits + s) * HD + d];
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
        const float inv = weight > 0.0f ? 1.0f / weight : 0.0f;
        p.out[(b * p.L + l) * p.ldo + h * HD + d] = sum * inv;
    }
}

// ------------------------------------------------------------------------------------------ decode
// One new position per sequence (L = 1) over bf16 or f32 K/V, G = H/KV query heads per KV head.  A work-group of W
// waves takes one (sequence, KV head, key chunk of 64 W keys); each wave one 64-key tile of the chunk, loaded
// straight into registers when the kernel starts (no dependency precedes them): the K rows with one lane per
// key for the scores, the V rows with one lane per CPL head-dim columns for P*V (two bf16 columns per 32-bit
// load, four f32 columns per 16-byte load).  The scaled q rows are broadcast from LDS.  Each wave normalises its
// tile on its own (max, exp, sum); the W waves merge through LDS.  A single chunk writes the output; with
// several, each writes (o, max, sum) partials (empty ones a zero weight) and attention_combine merges them in
// fixed order in the next launch.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

/// The head-dim values of one 16-byte piece of a K/V row: 8 bf16 or 4 f32.
template <typename KT>
__device__ __forceinline__ void unpack16(const u32x4 w, float (&f)[16 / sizeof(KT)]) {
    if constexpr (sizeof(KT) == 2) {
        f[0] = bf16_lo(w.x); f[1] = bf16_hi(w.x); f[2] = bf16_lo(w.y); f[3] = bf16_hi(w.y);
        f[4] = bf16_lo(w.z); f[5] = bf16_hi(w.z); f[6] = bf16_lo(w.w); f[7] = bf16_hi(w.w);
    } else {
        f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y); f[2] = __uint_as_float(w.z);
        f[3] = __uint_as_float(w.w);
    }
}

template <typename KT> struct DecodeV;
template <> struct DecodeV<uint16_t> { // two bf16 columns per lane, one 32-bit load
    static constexpr int CPL = 2;
    using Word = uint32_t;
    __device__ static __forceinline__ Word load(__amdgpu_buffer_rsrc_t r, int offset, int soffset) {
        return __builtin_amdgcn_raw_buffer_load_b32(r, offset, soffset, 0);
    }
    __device__ static __forceinline__ void unpack(Word w, float (&f)[CPL]) { f[0] = bf16_lo(w); f[1] = bf16_hi(w); }
};
template <> struct DecodeV<float> { // four f32 columns per lane, one 16-byte load
    static constexpr int CPL = 4;
    using Word = u32x4;
    __device__ static __forceinline__ Word load(__amdgpu_buffer_rsrc_t r, int offset, int soffset) {
        return __builtin_amdgcn_raw_buffer_load_b128(r, offset, soffset, 0);
    }
    __device__ static __forceinline__ void unpack(Word w, float (&f)[CPL]) {
        f[0] = __uint_as_float(w.x); f[1] = __uint_as_float(w.y); f[2] = __uint_as_float(w.z);
        f[3] = __uint_as_float(w.w);
    }
};

template <typename KT, int HD, int G, int W>
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(1, 2))) void attention_decode(
    const dlk_attention_params p) {
    constexpr int kThreads = W * kWave;
    constexpr int ES = sizeof(KT);
    constexpr int DPC = 16 / ES;      // head-dim values per 16-byte piece
    constexpr int KCH = HD / DPC;     // 16-byte pieces of a K row
    constexpr int CPL = DecodeV<KT>::CPL;
    constexpr int DL = HD / CPL;      // lanes per V row
    constexpr int KP = kWave / DL;    // keys per V load instruction
    constexpr int VL = kWave / KP;    // V loads per lane for a 64-key tile
    constexpr int QN = (G * HD + kThreads - 1) / kThreads;
    static_assert(DL <= kWave && kWave % DL == 0, "a V row must fit one wave");
    using VWord = typename DecodeV<KT>::Word;
    __shared__ float q_s[G][HD];
    __shared__ float p_s[W][kWave][G];
    __shared__ float m_s[W][G], l_s[W][G];
    __shared__ float o_s[W][G][HD];

    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int split = blockIdx.x;
    const int bk = blockIdx.y; // b * KV + kv head
    const int b = bk / p.KV, kvh = bk % p.KV;
    const int64_t first = p.position ? *p.position : p.first_host;
    const int64_t S = first + 1;
    const int active = static_cast<int>((S + p.chunk - 1) / p.chunk);

    if (split >= active) {
        // no keys here: the combine pass gives this slot zero weight
        if (t < G) {
            const int64_t slot = (static_cast<int64_t>(b) * p.H + kvh * G + t) * p.splits + split;
            p.partial_ml[slot * 2] = -INFINITY;
            p.partial_ml[slot * 2 + 1] = 0.0f;
        }
        return;
    }
    const int64_t k_begin = static_cast<int64_t>(split) * p.chunk;
    const int64_t k_end = min(S, k_begin + p.chunk);
    const int64_t key0 = k_begin + static_cast<int64_t>(kWave) * wave;
    const size_t head = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity;
    const KT* kbase = static_cast<const KT*>(p.k) + head * HD;
    const KT* vbase = static_cast<const KT*>(p.v) + head * HD;

    // q first, then K and V (vector loads complete in issue order: the q wait never covers K/V).  Keys past
    // the chunk end are clamped to its last key; their scores are masked.
    float qv[QN];
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        const int idx = min(t + i * kThreads, G * HD - 1);
        qv[i] = p.q[static_cast<int64_t>(b) * p.ldq + static_cast<int64_t>(kvh * G) * HD + idx];
    }
    // buffer loads over this wave's tile: offsets are immediates or scalars, and rows past the chunk end read
    // as zero (their scores are masked below)
    u32x4 kr[KCH];
    VWord vr[VL];
    {
        const int bytes = static_cast<int>(max<int64_t>(0, k_end - key0)) * HD * ES;
        const __amdgpu_buffer_rsrc_t kres =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(kbase + key0 * HD), 0, bytes, kBufferFlags);
        const __amdgpu_buffer_rsrc_t vres =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<KT*>(vbase + key0 * HD), 0, bytes, kBufferFlags);
        const int krow = lane * HD * ES;
#pragma unroll
        for (int c = 0; c < KCH; ++c) kr[c] = __builtin_amdgcn_raw_buffer_load_b128(kres, krow + c * 16, 0, 0);
        __builtin_amdgcn_sched_barrier(0); // K is issued (and so completes) before V: the scores wait for K only
        const int vlane = (lane / DL) * HD * ES + (lane % DL) * CPL * ES;
#pragma unroll
        for (int j = 0; j < VL; ++j) vr[j] = DecodeV<KT>::load(vres, vlane, j * KP * HD * ES);
    }
#pragma unroll
    for (int i = 0; i < QN; ++i) {
        const int idx = t + i * kThreads;
        if (idx < G * HD) (&q_s[0][0])[idx] = qv[i] * p.scale;
    }
    lds_barrier();

    // scores: lane = key.  The q values of piece c + 1 are read from LDS (broadcast) while piece c is used: a
    // batch of G DPC reads in flight instead of one read at a time.
    constexpr int Q4 = DPC / 4; // float4 reads of q per piece and head
    const bool valid = key0 + lane < k_end;
    float sc[G];
#pragma unroll
    for (int g = 0; g < G; ++g) sc[g] = 0.0f;
    float4 qc[G][Q4], qn[G][Q4];
    auto read_q = [&](int c, float4 (&dst)[G][Q4]) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < Q4; ++j) dst[g][j] = *reinterpret_cast<const float4*>(&q_s[g][c * DPC + 4 * j]);
    };
    read_q(0, qc);
#pragma unroll
    for (int c = 0; c < KCH; ++c) {
        if (c + 1 < KCH) read_q(c + 1, qn);
        __builtin_amdgcn_sched_barrier(0);
        float kf[DPC];
        unpack16<KT>(kr[c], kf);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float part = 0.0f;
#pragma unroll
            for (int j = 0; j < Q4; ++j) {
                const float4 qa = qc[g][j];
                part += qa.x * kf[4 * j] + qa.y * kf[4 * j + 1] + qa.z * kf[4 * j + 2] + qa.w * kf[4 * j + 3];
            }
            sc[g] += part;
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < Q4; ++j) qc[g][j] = qn[g][j];
    }
    // the wave's softmax over its tile
    float m_w[G], l_w[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m_w[g] = wave_max(valid ? sc[g] : -INFINITY);
        const float pr = valid ? expf(sc[g] - m_w[g]) : 0.0f;
        l_w[g] = wave_sum(pr);
        p_s[wave][lane][g] = pr;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront", "local");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront", "local");

    // P*V: lane = (column group lane % DL, key class lane / DL); the P values of the next PB keys are read from
    // LDS while the current ones are used
    constexpr int PB = HD * G > 256 ? 4 : 8; // smaller batches keep the widest variants under 256 registers
    static_assert(VL % PB == 0, "P batches");
    float o[G][CPL];
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int c = 0; c < CPL; ++c) o[g][c] = 0.0f;
    float pc[PB][G], pn[PB][G];
    auto read_p = [&](int j0, float (&dst)[PB][G]) {
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            const int kl = (j0 + i) * KP + lane / DL;
            if constexpr (G % 4 == 0) {
#pragma unroll
                for (int g = 0; g < G; g += 4) {
                    const float4 v4 = *reinterpret_cast<const float4*>(&p_s[wave][kl][g]);
                    dst[i][g] = v4.x;
                    dst[i][g + 1] = v4.y;
                    dst[i][g + 2] = v4.z;
                    dst[i][g + 3] = v4.w;
                }
            } else {
#pragma unroll
                for (int g = 0; g < G; ++g) dst[i][g] = p_s[wave][kl][g];
            }
        }
    };
    read_p(0, pc);
#pragma unroll
    for (int j0 = 0; j0 < VL; j0 += PB) {
        if (j0 + PB < VL) read_p(j0 + PB, pn);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < PB; ++i) {
            float vf[CPL];
            DecodeV<KT>::unpack(vr[j0 + i], vf);
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int c = 0; c < CPL; ++c) o[g][c] += pc[i][g] * vf[c];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < PB; ++i)
#pragma unroll
            for (int g = 0; g < G; ++g) pc[i][g] = pn[i][g];
    }
#pragma unroll
    for (int off = DL; off < kWave; off <<= 1)
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < CPL; ++c) o[g][c] += __shfl_xor(o[g][c], off, kWave);

    // merge the W waves
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            m_s[wave][g] = m_w[g];
            l_s[wave][g] = l_w[g];
        }
    }
    if (lane < DL) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int c = 0; c < CPL; ++c) o_s[wave][g][CPL * lane + c] = o[g][c];
    }
    lds_barrier();
    for (int idx = t; idx < G * HD; idx += kThreads) {
        const int g = idx / HD, d = idx % HD, h = kvh * G + g;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, m_s[w][g]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            if (m_s[w][g] == -INFINITY) continue;
            const float wt = expf(m_s[w][g] - M);
            L += wt * l_s[w][g];
            O += wt * o_s[w][g][d];
        }
        if (p.splits == 1) {
            p.out[static_cast<int64_t>(b) * p.ldo + static_cast<int64_t>(h) * HD + d] = O * (1.0f / L);
        } else {
            const int64_t slot = (static_cast<int64_t>(b) * p.H + h) * p.splits + split;
            p.partial_o[slot * HD + d] = O;
            if (d == 0) {
                p.partial_ml[slot * 2] = M;
                p.partial_ml[slot * 2 + 1] = L;
            }
        }
    }
}

// ------------------------------------------------------------------------------------------ streaming decode
// One new position per sequence (L = 1) over bf16 or f32 K/V, HD 64 or 128, G = H/KV <= 4.  A work-group of four
// waves takes one (sequence, KV head, key chunk); each wave streams its own run of chunk / 4 keys in tiles of TK
// keys, the next tile's K and V requested while the current one is used.  Loads put consecutive lanes on
// consecutive 16-byte pieces, so every load instruction reads 1 KB of whole 128-byte lines: lane l holds the DPL
// dims DPL (l % LPK) .. +DPL of key slot l / LPK (DPL = 8 bf16 or 4 f32 values; LPK = lanes per key row, 8 to 32).
// A score is the sum over the LPK lanes of a key slot (DPP within 16-lane rows, a lane swap across two rows, no
// LDS); its softmax weight is then already in the lanes that hold the same key's V piece, so P*V needs no
// exchange either.  Each lane keeps its own running (max, sum, DPL output dims); the key slots
// merge once at the end (lane exchanges), the four waves through LDS.  A single chunk writes the output;
// otherwise the chunk writes (o, max, sum) partials for attention_combine, as the kernel above.  On MI355X this
// reads C4's 1.07 GB of K/V per layer at 5.0 TB/s (the tile-per-wave kernel: 3.2 TB/s); with few keys in all
// (C2) the tile-per-wave kernel's shorter chain wins, so the host picks by the total key count.
template <int LPK>
__device__ __forceinline__ float group_sum(float v) {
    constexpr int kQuadSwap1 = 0xB1, kQuadSwap2 = 0x4E, kHalfMirror = 0x141, kRowMirror = 0x140;
    auto dpp = [](float x, auto ctrl) {
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), decltype(ctrl)::value, 0xF, 0xF, false));
    };
    v += dpp(v, std::integral_constant<int, kQuadSwap1>{});
    v += dpp(v, std::integral_constant<int, kQuadSwap2>{});
    v += dpp(v, std::integral_constant<int, kHalfMirror>{});
    if constexpr (LPK >= 16) v += dpp(v, std::integral_constant<int, kRowMirror>{});
    if constexpr (LPK == 32) {
        // rows 2i and 2i + 1 exchange their values in registers: both receive the pair's sum
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    return v;
}

template <typename KT, int HD, int G, int TK, int W>
__global__ __launch_bounds__(W * kWave) __attribute__((amdgpu_waves_per_eu(1, 2))) void attention_stream(
    const dlk_attention_params p) {
    constexpr int ES = sizeof(KT);
    constexpr int DPL = 16 / ES;            // head-dim values per lane (one 16-byte piece)
    constexpr int LPK = HD * ES / 16;       // lanes per key row
    constexpr int KPI = kWave / LPK;        // keys per load instruction
    constexpr int NI = TK / KPI;            // load instructions per tile (K, and again V)
    constexpr int ROW = HD * ES;            // bytes per key row
    static_assert(NI >= 1 && TK % KPI == 0, "whole load instructions per tile");
    __shared__ float m_s[W][G], l_s[W][G];
    __shared__ float o_s[W][G][HD];

    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int split = blockIdx.x;
    const int bk = blockIdx.y; // b * KV + kv head
    const int b = bk / p.KV, kvh = bk % p.KV;
    const int64_t first = p.position ? *p.position : p.first_host;
    const int64_t S = first + 1;
    const int active = static_cast<int>((S + p.chunk - 1) / p.chunk);
    if (split >= active) {
        // no keys here: the combine pass gives this slot zero weight
        if (t < G) {
            const int64_t slot = (static_cast<int64_t>(b) * p.H + kvh * G + t) * p.splits + split;
            p.partial_ml[slot * 2] = -INFINITY;
            p.partial_ml[slot * 2 + 1] = 0.0f;
        }
        return;
    }
    const int per_wave = p.chunk / W;
    const int64_t k_end = min(S, static_cast<int64_t>(split) * p.chunk + p.chunk);
    const int64_t w_begin = static_cast<int64_t>(split) * p.chunk + static_cast<int64_t>(wave) * per_wave;
    const int keys = static_cast<int>(max<int64_t>(0, min<int64_t>(k_end, w_begin + per_wave) - w_begin));
    const int tiles = (keys + TK - 1) / TK;
    const int slot_key = lane / LPK, dc = lane % LPK;

    // q: dims DPL dc .. +DPL of the G heads, scaled by scale * log2(e) so that the softmax runs in base 2 (one
    // v_exp_f32 per weight; the maxima are turned back to natural units for the merges)
    float q[G][DPL];
    {
        const float qs = p.scale * 1.4426950408889634f;
        const float* qrow = p.q + static_cast<int64_t>(b) * p.ldq + static_cast<int64_t>(kvh * G) * HD + DPL * dc;
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < DPL; j += 4) {
                const float4 a = *reinterpret_cast<const float4*>(qrow + g * HD + j);
                q[g][j] = a.x * qs; q[g][j + 1] = a.y * qs; q[g][j + 2] = a.z * qs; q[g][j + 3] = a.w * qs;
            }
    }
    // buffer ranges over this wave's keys: rows past them read as zero (their scores are masked)
    const size_t head = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity + w_begin;
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<KT*>(static_cast<const KT*>(p.k) + head * HD), 0, keys * ROW, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<KT*>(static_cast<const KT*>(p.v) + head * HD), 0, keys * ROW, kBufferFlags);
    const int lane_offset = slot_key * ROW + 16 * dc;

    struct Tile {
        u32x4 k[NI], v[NI];
    };
    auto load = [&](int tile, Tile& dst) {
        const int base = tile * TK * ROW + lane_offset;
#pragma unroll
        for (int i = 0; i < NI; ++i) dst.k[i] = __builtin_amdgcn_raw_buffer_load_b128(kres, base + i * KPI * ROW, 0, 0);
#pragma unroll
        for (int i = 0; i < NI; ++i) dst.v[i] = __builtin_amdgcn_raw_buffer_load_b128(vres, base + i * KPI * ROW, 0, 0);
    };

    float m[G], l[G], o[G][DPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < DPL; ++j) o[g][j] = 0.0f;
    }
    auto use = [&](int tile, const Tile& cur) {
        // scores of the lane's NI key slots (identical across the LPK lanes of a slot)
        float sc[NI][G];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            float kf[DPL];
            unpack16<KT>(cur.k[i], kf);
            const bool valid = tile * TK + i * KPI + slot_key < keys;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float part = q[g][0] * kf[0];
#pragma unroll
                for (int j = 1; j < DPL; ++j) part += q[g][j] * kf[j];
                const float total = group_sum<LPK>(part);
                sc[i][g] = valid ? total : -INFINITY;
            }
        }
        // online softmax of the lane's keys, then P*V on the lane's own V pieces
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float tile_max = sc[0][g];
#pragma unroll
            for (int i = 1; i < NI; ++i) tile_max = fmaxf(tile_max, sc[i][g]);
            const float m_new = fmaxf(m[g], tile_max);
            if (m_new == -INFINITY) continue; // no valid key seen yet in this lane's slots
            const float alpha = m[g] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[g] - m_new);
            l[g] *= alpha;
#pragma unroll
            for (int j = 0; j < DPL; ++j) o[g][j] *= alpha;
#pragma unroll
            for (int i = 0; i < NI; ++i) {
                const float pr = sc[i][g] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(sc[i][g] - m_new);
                l[g] += pr;
                float vf[DPL];
                unpack16<KT>(cur.v[i], vf);
#pragma unroll
                for (int j = 0; j < DPL; ++j) o[g][j] += pr * vf[j];
            }
            m[g] = m_new;
        }
    };
    if (tiles > 0) {
        Tile a, c;
        load(0, a);
        // two tiles per iteration so that the buffers are named statically; the next tile is in flight while one
        // is used, and no load sits in a branch inside the loop (the last tile is peeled)
        int tile = 0;
        for (;;) {
            if (tile + 1 >= tiles) { use(tile, a); break; }
            load(tile + 1, c);
            use(tile, a);
            ++tile;
            if (tile + 1 >= tiles) { use(tile, c); break; }
            load(tile + 1, a);
            use(tile, c);
            ++tile;
        }
    }
    // merge the key slots: lanes l and l ^ (LPK, 2 LPK, ...) hold the same dims (symmetric: both lanes get
    // identical values)
#pragma unroll
    for (int off = LPK; off < kWave; off <<= 1) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const float mo = __shfl_xor(m[g], off, kWave);
            const float lo = __shfl_xor(l[g], off, kWave);
            const float mm = fmaxf(m[g], mo);
            const float a = m[g] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m[g] - mm);
            const float c = mo == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mo - mm);
            l[g] = l[g] * a + lo * c;
#pragma unroll
            for (int j = 0; j < DPL; ++j) {
                const float oo = __shfl_xor(o[g][j], off, kWave);
                o[g][j] = o[g][j] * a + oo * c;
            }
            m[g] = mm;
        }
    }
    // merge the four waves (the same LDS merge as the tile-per-wave kernel, maxima in natural units)
    if (lane == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            m_s[wave][g] = m[g] * 0.6931471805599453f;
            l_s[wave][g] = l[g];
        }
    }
    if (lane < LPK) {
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int j = 0; j < DPL; ++j) o_s[wave][g][DPL * dc + j] = o[g][j];
    }
    lds_barrier();
    for (int idx = t; idx < G * HD; idx += W * kWave) {
        const int g = idx / HD, d = idx % HD, h = kvh * G + g;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, m_s[w][g]);
        float L = 0.0f, O = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) {
            if (m_s[w][g] == -INFINITY) continue;
            const float wt = expf(m_s[w][g] - M);
            L += wt * l_s[w][g];
            O += wt * o_s[w][g][d];
        }
        if (p.splits == 1) {
            p.out[static_cast<int64_t>(b) * p.ldo + static_cast<int64_t>(h) * HD + d] = O * (1.0f / L);
        } else {
            const int64_t slot = (static_cast<int64_t>(b) * p.H + h) * p.splits + split;
            p.partial_o[slot * HD + d] = O;
            if (d == 0) {
                p.partial_ml[slot * 2] = M;
                p.partial_ml[slot * 2 + 1] = L;
            }
        }
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
    for (int64_t k0 = k_begin; k0 < k_end; k0 += kWave) {
        const int64_t key = k0 + lane;
        const bool live = key < k_end;
        float s = -INFINITY;
        if (live) {
            s = 0.0f;
#pragma unroll
            for (int d = 0; d < HD; ++d) s += q[d] * value(kbase + key * HD, d);
        }
        const float m_new = fmaxf(m, wave_max(s)); // finite: every step holds at least one live key
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
        for (int d = 0; d < HD; ++d) out[d] = total > 0.0f ? o[d] / total : 0.0f;
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
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(rows)), dim3(kThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

/// Whether the streaming decode kernel serves these heads (bf16 or f32 K/V, HD 64 or 128, G = 1, 2 or 4).
bool stream_heads(int heads, int kv_heads, int hd, int kv_bf16) {
    (void)kv_bf16;
    if (kv_heads <= 0 || heads % kv_heads != 0 || (hd != 64 && hd != 128)) return false;
    const int G = heads / kv_heads;
    return G == 1 || G == 2 || G == 4;
}

// bf16: four waves, tiles of 32 keys at HD 64 and 16 at HD 128 (4 KB of K and of V per tile).  f32: eight waves
// (twice the bytes in flight per work-group), tiles of the same key counts (8 KB of K and of V per tile).
template <typename KT, int HD, int TK = (HD == 64 ? 32 : 16), int W = sizeof(KT) == 4 ? 8 : 4>
int launch_stream(const dlk_attention_params& p, hipStream_t stream) {
    const dim3 grid(p.splits, p.B * p.KV), block(W * kWave);
    switch (p.H / p.KV) {
    case 1: hipLaunchKernelGGL((attention_stream<KT, HD, 1, TK, W>), grid, block, 0, stream, p); break;
    case 2: hipLaunchKernelGGL((attention_stream<KT, HD, 2, TK, W>), grid, block, 0, stream, p); break;
    case 4: hipLaunchKernelGGL((attention_stream<KT, HD, 4, TK, W>), grid, block, 0, stream, p); break;
    default: return static_cast<int>(hipErrorInvalidValue);
    }
    int status = static_cast<int>(hipGetLastError());
    if (status != 0 || p.splits == 1 || p.partials_only) return status;
    const int64_t combine_rows = static_cast<int64_t>(p.B) * p.H;
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(combine_rows)), dim3(kThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

/// Widest work-group (waves) each decode variant runs without register spills: a wave may hold 512 / (W / 4)
/// registers, and the bf16 variants need ~90-210 (HD 64) or ~155-335 (HD 128).  f32 K/V hold twice the K and V
/// bytes per lane (64 + 64 registers at HD 64): at most eight waves, four at G = 8; f32 at HD 128 takes the
/// streaming kernel.
constexpr int decode_waves_max(int hd, int g, bool f32) {
    if (f32) return hd == 64 ? (g <= 4 ? 8 : 4) : 0;
    return hd == 64 ? (g <= 2 ? 16 : 8) : (g <= 2 ? 8 : 4);
}

template <typename KT, int HD, int W>
int launch_decode_w(const dlk_attention_params& p, hipStream_t stream) {
    const dim3 grid(p.splits, p.B * p.KV), block(W * kWave);
    auto go = [&](auto g) {
        constexpr int G = decltype(g)::value;
        if constexpr (W <= decode_waves_max(HD, G, sizeof(KT) == 4) && !(HD == 128 && G > 4)) {
            hipLaunchKernelGGL((attention_decode<KT, HD, G, W>), grid, block, 0, stream, p);
            return static_cast<int>(hipGetLastError());
        }
        return static_cast<int>(hipErrorInvalidValue);
    };
    switch (p.H / p.KV) {
    case 1: return go(std::integral_constant<int, 1>{});
    case 2: return go(std::integral_constant<int, 2>{});
    case 4: return go(std::integral_constant<int, 4>{});
    case 8: return go(std::integral_constant<int, 8>{});
    default: return static_cast<int>(hipErrorInvalidValue);
    }
}

template <typename KT, int HD>
int launch_decode(const dlk_attention_params& p, hipStream_t stream) {
    int status = 0;
    switch (p.chunk / kWave) {
    case 4: status = launch_decode_w<KT, HD, 4>(p, stream); break;
    case 8: status = launch_decode_w<KT, HD, 8>(p, stream); break;
    case 16:
        if constexpr (sizeof(KT) == 2) {
            status = launch_decode_w<KT, HD, 16>(p, stream);
            break;
        }
        return static_cast<int>(hipErrorInvalidValue);
    default: return static_cast<int>(hipErrorInvalidValue);
    }
    if (status != 0 || p.splits == 1 || p.partials_only) return status;
    const int64_t combine_rows = static_cast<int64_t>(p.B) * p.H;
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(combine_rows)), dim3(kThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

/// The decode kernel serves one new position over bf16 K/V with HD 64 (G in {1, 2, 4, 8}) or 128 (G <= 4), or
/// over f32 K/V with HD 64, and chunks of 4, 8 or 16 64-key tiles (one per wave).
int decode_chunk_max(int heads, int kv_heads, int hd, int kv_bf16) {
    if (kv_heads <= 0 || heads % kv_heads != 0 || (hd != 64 && hd != 128)) return 0;
    const int G = heads / kv_heads;
    if (!(G == 1 || G == 2 || G == 4 || (G == 8 && hd == 64))) return 0;
    return decode_waves_max(hd, G, !kv_bf16) * kWave;
}

bool decode_path(const dlk_attention_params& p) {
    const int most = decode_chunk_max(p.H, p.KV, p.hd, p.kv_bf16);
    return p.L == 1 && most > 0 && p.chunk <= most &&
           (p.chunk == 4 * kWave || p.chunk == 8 * kWave || p.chunk == 16 * kWave);
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
    hipLaunchKernelGGL((attention_combine<HD>), dim3(static_cast<unsigned>(combine_rows)), dim3(kThreads), 0, stream, p);
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

extern "C" int dlk_attention_decode_chunk(int heads, int kv_heads, int head_dim, int kv_bf16) {
    return dlk::decode_chunk_max(heads, kv_heads, head_dim, kv_bf16);
}

extern "C" int dlk_attention_stream_decode(int heads, int kv_heads, int head_dim, int kv_bf16) {
    return dlk::stream_heads(heads, kv_heads, head_dim, kv_bf16) ? 1 : 0;
}

extern "C" int dlk_attention(const dlk_attention_params* params, dlh_stream stream_handle) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    const dlk_attention_params& p = *params;
    if (p.B <= 0 || p.L <= 0 || p.KV <= 0 || p.H % p.KV != 0 || p.splits <= 0 || p.chunk <= 0 ||
        (p.splits > 1 && (!p.partial_o || !p.partial_ml)) || (p.splits > 1 && p.chunk % 64 != 0))
        return static_cast<int>(hipErrorInvalidValue);
    if (p.L == 1 && dlk::stream_heads(p.H, p.KV, p.hd, p.kv_bf16) && p.chunk % 128 == 0 &&
        (static_cast<int64_t>(p.B) * p.KV * p.splits * p.chunk >= DLK_STREAM_DECODE_KEYS || !dlk::decode_path(p))) {
        if (p.kv_bf16)
            return p.hd == 64 ? dlk::launch_stream<uint16_t, 64>(p, stream) : dlk::launch_stream<uint16_t, 128>(p, stream);
        return p.hd == 64 ? dlk::launch_stream<float, 64>(p, stream) : dlk::launch_stream<float, 128>(p, stream);
    }
    if (dlk::decode_path(p)) {
        if (p.kv_bf16)
            return p.hd == 64 ? dlk::launch_decode<uint16_t, 64>(p, stream) : dlk::launch_decode<uint16_t, 128>(p, stream);
        return p.hd == 64 ? dlk::launch_decode<float, 64>(p, stream) : static_cast<int>(hipErrorInvalidValue);
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
