// One new position per sequence (L = 1) over a bf16 or f32 K/V cache on the matrix cores: the decode counterpart of
// attention_prefill.hip (see dlk_attention_params in kernels.h).  Replaces, for one new position, the reference's
// grouped_block + attention_weights (src/ops/attention.cpp:59-95, 161-188): scores in f32, softmax with the
// maximum subtracted, P * V, every key of the sequence visible.
//
// The query tile of a work-group is the G = H/KV query heads that share one KV head (columns G..15 of the 16-wide
// tile are zero), so a work-group takes one (key split, sequence, KV head) and its W waves split the keys: each
// wave streams its own run in tiles of 32 keys and keeps its own online softmax; the waves merge in LDS.  Per tile:
//   S^T[16 keys][16 heads] = K[16][HD] * Q[16][HD]^T   (v_mfma_f32_16x16x32_bf16: A = 16 key rows loaded from HBM
//                                                         as they are stored, 16 bytes per lane; B = the query
//                                                         heads split into bf16 hi + lo)
// so lane l holds S[keys 4(l/16) .. +4][head l%16] of each 16-key half; the probabilities of both halves are the
// B operand of
//   O^T[16 d][16 heads] += V^T[16 d][32 keys] * P^T     (A = V^T, transposed through the wave's own LDS tile)
// and the row sums come out of one more product whose A operand is all ones.  Two MFMAs per product (hi and lo)
// keep f32-level accuracy against a bf16 cache; an f32 cache is split into hi and lo as it is loaded and each
// product takes three (Kh Qh + Kh Ql + Kl Qh: the Kl Ql term is below 2^-16 of the product).  The softmax runs
// in base 2 (log2 e folded into the query scale).  Keys past the wave's run read as zero from the buffer range
// and are masked out of the softmax.  One split writes the output; several write (o, max, sum) partials that
// attention_combine merges in the next launch.
//
// The products on the vector ALUs instead (eight lanes per key row, lane-group sums) cost ~600 vector instructions
// per 32-key tile at G = 4, which bound a work-group per CU at ~4 TB/s (measured on MI355X: 32.9 us per layer at
// batch 32 over 2048 bf16 keys, 25.7 us here); this kernel counts ~170 (the softmax, the V transpose, and the
// wave's set-up and merge spread over its tiles) and 18 MFMAs per tile.
#include "kernels/device_common.h"

namespace dlk {
namespace {

constexpr int kTileKeys = 32;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

// bf16 hi and lo parts of eight f32 values (x = hi + lo to ~2^-16; x - hi is exact in f32)
__device__ __forceinline__ void split8(const f32x8 v, bf16x8& hi, bf16x8& lo) {
    const u32x4 h = __builtin_bit_cast(u32x4, __builtin_convertvector(v, bf16x8));
    const f32x8 back = {__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xffff0000u),
                        __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xffff0000u),
                        __uint_as_float(h.z << 16), __uint_as_float(h.z & 0xffff0000u),
                        __uint_as_float(h.w << 16), __uint_as_float(h.w & 0xffff0000u)};
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_convertvector(v - back, bf16x8);
}

// the same for four values, as packed words
__device__ __forceinline__ void split4(const u32x4 w, u32x2& hi, u32x2& lo) {
    const f32x4 v = __builtin_bit_cast(f32x4, w);
    const u32x2 h = __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf16x4));
    const f32x4 back = {__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xffff0000u),
                        __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xffff0000u)};
    hi = h;
    lo = __builtin_bit_cast(u32x2, __builtin_convertvector(v - back, bf16x4));
}

// maximum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (one query head's column): lane swaps in registers
__device__ __forceinline__ float max_over_column(float x) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename KT, int HD, int W, bool FINISH>
__global__ __launch_bounds__(W * kWave) void attention_matrix(const dlk_attention_params p) {
    constexpr bool F32 = sizeof(KT) == 4;
    constexpr int PLANES = F32 ? 2 : 1;      // bf16 planes of the staged V^T: hi (+ lo for an f32 cache)
    constexpr int KS = HD / 32;              // k steps of the score product
    constexpr int DT = HD / 16;              // 16-wide head-dim tiles of the output
    constexpr int KL = F32 ? 2 : 1;          // 16-byte loads per lane per K fragment (8 values)
    constexpr int DPP = 16 / sizeof(KT);     // head-dim values per 16-byte piece
    constexpr int VI = HD / DPP / 4;         // V pieces per lane per key of a pair (64 lanes: 16 pairs x 4 groups)
    constexpr int VSTRIDE = kTileKeys + 4;   // bf16 per staged V^T row: 18 words, so the 64 lanes' stores and
                                             // 8-byte reads spread over the banks
    constexpr int ROW = HD * static_cast<int>(sizeof(KT)); // bytes per key row
    __shared__ __attribute__((aligned(16))) uint16_t vt[W][PLANES][HD * VSTRIDE];
    __shared__ float m_s[W][16], l_s[W][16];
    __shared__ float o_s[W][16][HD];
    __shared__ __attribute__((aligned(16))) float kv_s[2][HD]; // the new K/V row (qkv_partial holder wave)

    const int t = threadIdx.x, lane = t % kWave, q = lane / 16, col = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int split = blockIdx.x;
    const int bk = blockIdx.y;
    const int b = bk / p.KV, kvh = bk % p.KV;
    const int G = p.H / p.KV;
    const int per_wave = p.chunk / W;
    const int64_t w_begin = static_cast<int64_t>(split) * p.chunk + static_cast<int64_t>(wave) * per_wave;
    const size_t head = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity + w_begin;
    KT* const k_base = const_cast<KT*>(static_cast<const KT*>(p.k) + head * HD);
    KT* const v_base = const_cast<KT*>(static_cast<const KT*>(p.v) + head * HD);
    // K fragment (half u, k step st): key 16 u + col, head dims 32 st + 8 q .. +8.  V: key pair kp = col (keys
    // 2 kp, 2 kp + 1), pieces dg = q + 4 i.
    const int k_offset = col * ROW + (8 * q) * static_cast<int>(sizeof(KT));
    const int v_offset = 2 * col * ROW + q * 16;
    struct Tile {
        u32x4 k[2][KS][KL];
        u32x4 v[VI][2];
    };
    auto load = [&](int tile, Tile& dst, __amdgpu_buffer_rsrc_t kres, __amdgpu_buffer_rsrc_t vres) {
        const int base = tile * kTileKeys * ROW;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int st = 0; st < KS; ++st)
#pragma unroll
                for (int e = 0; e < KL; ++e)
                    dst.k[u][st][e] = __builtin_amdgcn_raw_buffer_load_b128(
                        kres, base + k_offset + 16 * u * ROW + (32 * st) * static_cast<int>(sizeof(KT)) + 16 * e, 0, 0);
#pragma unroll
        for (int i = 0; i < VI; ++i)
#pragma unroll
            for (int e = 0; e < 2; ++e)
                dst.v[i][e] = __builtin_amdgcn_raw_buffer_load_b128(vres, base + v_offset + e * ROW + 64 * i, 0, 0);
    };

    // A wave whose run starts below the caller's early_keys requests its first tile (after the query rows, when
    // no QKV partials are to be summed) before the device length arrives: that tile's range is the wave's run
    // within the cache capacity, so its rows past the length hold whatever the cache held (their scores are
    // masked, their values zeroed in use()).  The other waves, and every later tile, read through ranges that end
    // at the length.  Measured on MI355X (A/B, one box), with every wave of four-wave work-groups requesting
    // early: C3 1.181 -> 1.163 ms a step, C4 9.34-9.39 -> 9.29-9.33 ms; with every wave of the one-sequence launch
    // too (C2: eight waves, most past the length) C2 went 550 -> 571 us, which the hint avoids (waves past the
    // known keys fetched cache rows no step had touched).  With the hint: C3 1.176 -> 1.162 ms, C2, C4 and the
    // C5 decode unchanged.
    const bool early = w_begin < p.early_keys;
    Tile a, c;
    float4 xq[KS][2];
    if constexpr (!FINISH) {
        const float* qrow =
            p.q + static_cast<int64_t>(b) * p.ldq + static_cast<int64_t>(kvh * G + min(col, G - 1)) * HD;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            xq[st][0] = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q);
            xq[st][1] = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q + 4);
        }
    }
    if (early) {
        const int room = static_cast<int>(max<int64_t>(0, min<int64_t>(per_wave, p.capacity - w_begin)));
        load(0, a, __builtin_amdgcn_make_buffer_rsrc(k_base, 0, room * ROW, kBufferFlags),
             __builtin_amdgcn_make_buffer_rsrc(v_base, 0, room * ROW, kBufferFlags));
    }

    const int64_t S = (p.position ? *p.position : p.first_host) + 1;
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
    const int64_t k_end = min(S, static_cast<int64_t>(split) * p.chunk + p.chunk);
    const int keys = static_cast<int>(max<int64_t>(0, min<int64_t>(k_end, w_begin + per_wave) - w_begin));
    const int tiles = (keys + kTileKeys - 1) / kTileKeys;

    // buffer ranges over this wave's keys: rows past them read as zero
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(k_base, 0, keys * ROW, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(v_base, 0, keys * ROW, kBufferFlags);
    if (!early && tiles > 0) load(0, a, kres, vres);

    // the query heads of this KV head as the B operand (column col = head kvh G + col), scaled into base 2
    bf16x8 qh[KS], ql[KS];

    f32x4 o[DT], l = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    uint16_t* my_vt = &vt[wave][0][0];

    auto use = [&](int tile, const Tile& cur) {
        // values of keys past the wave's run (the first tile of an early request only: its range did not wait
        // for the length) are zeroed, so that their zero probabilities cannot meet a non-finite value
        const bool cut = early && tile == 0 && keys < kTileKeys;
        const bool live0 = !cut || 2 * col < keys, live1 = !cut || 2 * col + 1 < keys;
        // V^T of the tile into the wave's LDS tile (word = key pair kp of one head-dim row)
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const u32x4 zero = u32x4{0u, 0u, 0u, 0u};
            const u32x4 a = live0 ? cur.v[i][0] : zero, c = live1 ? cur.v[i][1] : zero;
            if constexpr (F32) {
                // piece dg = q + 4 i holds head dims 4 dg .. +4 of keys 2 kp (a) and 2 kp + 1 (c)
                u32x2 h0, l0, h1, l1;
                split4(a, h0, l0);
                split4(c, h1, l1);
                const uint32_t hw[4] = {(h0.x & 0xffffu) | (h1.x << 16), (h0.x >> 16) | (h1.x & 0xffff0000u),
                                        (h0.y & 0xffffu) | (h1.y << 16), (h0.y >> 16) | (h1.y & 0xffff0000u)};
                const uint32_t lw[4] = {(l0.x & 0xffffu) | (l1.x << 16), (l0.x >> 16) | (l1.x & 0xffff0000u),
                                        (l0.y & 0xffffu) | (l1.y << 16), (l0.y >> 16) | (l1.y & 0xffff0000u)};
                const int d0 = 4 * (q + 4 * i);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    reinterpret_cast<uint32_t*>(my_vt)[((d0 + e) * VSTRIDE) / 2 + col] = hw[e];
                    reinterpret_cast<uint32_t*>(my_vt + HD * VSTRIDE)[((d0 + e) * VSTRIDE) / 2 + col] = lw[e];
                }
            } else {
                // piece dg = q + 4 i holds head dims 8 dg .. +8
                const uint32_t aw[4] = {a.x, a.y, a.z, a.w}, cw[4] = {c.x, c.y, c.z, c.w};
                const int d0 = 8 * (q + 4 * i);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    reinterpret_cast<uint32_t*>(my_vt)[((d0 + 2 * e) * VSTRIDE) / 2 + col] =
                        (aw[e] & 0xffffu) | (cw[e] << 16);
                    reinterpret_cast<uint32_t*>(my_vt)[((d0 + 2 * e + 1) * VSTRIDE) / 2 + col] =
                        (aw[e] >> 16) | (cw[e] & 0xffff0000u);
                }
            }
        }
        // scores of both 16-key halves
        f32x4 s[2];
#pragma unroll
        for (int u = 0; u < 2; ++u) {
            s[u] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                if constexpr (F32) {
                    bf16x8 kh, kl;
                    split8(__builtin_bit_cast(f32x8, __builtin_shufflevector(cur.k[u][st][0], cur.k[u][st][1], 0, 1, 2,
                                                                              3, 4, 5, 6, 7)),
                           kh, kl);
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[st], s[u], 0, 0, 0);
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[st], s[u], 0, 0, 0);
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[st], s[u], 0, 0, 0);
                } else {
                    const bf16x8 kf = __builtin_bit_cast(bf16x8, cur.k[u][st][0]);
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qh[st], s[u], 0, 0, 0);
                    s[u] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, ql[st], s[u], 0, 0, 0);
                }
            }
        }
        // online softmax of each head column over the tile's live keys
        float mx = -INFINITY;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (tile * kTileKeys + 16 * u + 4 * q + j >= keys) s[u][j] = -INFINITY;
                mx = fmaxf(mx, s[u][j]);
            }
        mx = max_over_column(mx);
        // every tile holds a live key, so m_new is finite; exp2(-inf) = 0 for the masked keys and the first alpha
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int j = 0; j < 4; ++j) s[u][j] = __builtin_amdgcn_exp2f(s[u][j] - m_new);
        if (!__all(alpha == 1.0f)) {
            l *= alpha;
#pragma unroll
            for (int d = 0; d < DT; ++d) o[d] *= alpha;
        }
        bf16x8 ph, pl;
        split8(f32x8{s[0][0], s[0][1], s[0][2], s[0][3], s[1][0], s[1][1], s[1][2], s[1][3]}, ph, pl);
        l = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, ph, l, 0, 0, 0);
        l = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pl, l, 0, 0, 0);
        // O^T += V^T P^T: lane (d = 16 dt + col, q) supplies V[keys 4 q .. +4 and 16 + 4 q .. +4][d]
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const int at = (16 * dt + col) * VSTRIDE + 4 * q;
            const u32x2 lo4 = *reinterpret_cast<const u32x2*>(my_vt + at);
            const u32x2 hi4 = *reinterpret_cast<const u32x2*>(my_vt + at + 16);
            const bf16x8 a = __builtin_bit_cast(bf16x8, u32x4{lo4.x, lo4.y, hi4.x, hi4.y});
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph, o[dt], 0, 0, 0);
            o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl, o[dt], 0, 0, 0);
            if constexpr (F32) {
                const u32x2 llo4 = *reinterpret_cast<const u32x2*>(my_vt + HD * VSTRIDE + at);
                const u32x2 lhi4 = *reinterpret_cast<const u32x2*>(my_vt + HD * VSTRIDE + at + 16);
                const bf16x8 al = __builtin_bit_cast(bf16x8, u32x4{llo4.x, llo4.y, lhi4.x, lhi4.y});
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, ph, o[dt], 0, 0, 0);
            }
        }
    };
    // The QKV projection's partials, when the projection left them (qkv_partial): every wave finishes the query
    // rows of its KV head's G heads from them, in the projection's reduce order (slices in order, the RMSNorm
    // factor from the summed row squares, RoPE on interleaved pairs at the new position), staged through its own
    // part of o_s (free until the merge).  The one wave whose keys hold the new position (in the last active
    // split's work-group) also finishes the new K/V row: it writes the row into the cache for later steps and
    // puts it in place of what its tile load returned for that key, so no wave waits on the write.
    constexpr bool finish = FINISH; // the launch chooses FINISH = (qkv_partial != NULL)
    const int64_t newest = S - 1;
    const bool holder = finish && split == active - 1 && newest >= w_begin && newest < w_begin + keys;
    const int patch_tile = holder ? static_cast<int>(newest - w_begin) / kTileKeys : -1;
    const int patch_key = holder ? static_cast<int>(newest - w_begin) % kTileKeys : 0;
    {
        const float qs = p.scale * 1.4426950408889634f;
        const float z = col < G ? qs : 0.0f;
        // q rows finished here, from LDS: a path of their own, so that the reads are typed (a pointer that may
        // hold LDS or global addresses would take flat loads)
        auto split_q = [&](const float* qrow) {
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                const float4 x0 = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q);
                const float4 x1 = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q + 4);
                split8(f32x8{x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w} * z, qh[st], ql[st]);
            }
        };
        if constexpr (finish) {
            constexpr int kBatch = 8; // slices requested at once
            constexpr int UNITS = HD / 4; // 4-dim units per head row
            const int width = p.qkv_width;
            const int slice = p.B * width; // floats per slice
            const __amdgpu_buffer_rsrc_t dots = __builtin_amdgcn_make_buffer_rsrc(
                const_cast<float*>(p.qkv_partial), 0, p.qkv_splits * slice * 4, kBufferFlags);
            float f = p.qkv_scale;
            if (p.qkv_norm) {
                const __amdgpu_buffer_rsrc_t sums = __builtin_amdgcn_make_buffer_rsrc(
                    const_cast<float*>(p.qkv_partial) + static_cast<int64_t>(p.qkv_splits) * slice, 0,
                    p.qkv_splits * p.B * 4, kBufferFlags);
                float row[16];
#pragma unroll
                for (int s = 0; s < 16; ++s)
                    row[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sums, (s * p.B + b) * 4, 0, 0));
                float total = 0.0f;
#pragma unroll
                for (int s = 0; s < 16; ++s) total += row[s];
                f = rsqrtf(total / static_cast<float>(p.qkv_K) + p.qkv_epsilon) * p.qkv_scale;
            }
            const float* cosine = p.rope_cos + newest * (HD / 2);
            const float* sine = p.rope_sin + newest * (HD / 2);
            float* stage = &o_s[wave][0][0];
            const int qunits = G * UNITS;
            // round r: lane finishes query unit lane + 64 r (head g, dims d .. +4) and, in round 0 of the holder,
            // K/V unit lane (lanes < UNITS: key dims 4 lane .., then value dims)
            for (int r = 0; r * kWave < qunits; ++r) {
                const int unit = min(lane + kWave * r, qunits - 1);
                const int g = unit / UNITS, d = 4 * (unit % UNITS);
                const int qoff = (b * width + (kvh * G + g) * HD + d) * 4;
                const bool kv = holder && r == 0 && lane < 2 * UNITS;
                const bool key = lane < UNITS;
                const int kd = 4 * (lane % UNITS);
                const int koff = (b * width + p.H * HD + (key ? 0 : p.KV * HD) + kvh * HD + kd) * 4;
                f32x4 qa = f32x4{0.f, 0.f, 0.f, 0.f}, ka = f32x4{0.f, 0.f, 0.f, 0.f};
                for (int s0 = 0; s0 < p.qkv_splits; s0 += kBatch) {
                    u32x4 qp[kBatch], kp[kBatch];
#pragma unroll
                    for (int s = 0; s < kBatch; ++s)
                        qp[s] = __builtin_amdgcn_raw_buffer_load_b128(dots, qoff + (s0 + s) * slice * 4, 0, 0);
                    if (kv) {
#pragma unroll
                        for (int s = 0; s < kBatch; ++s)
                            kp[s] = __builtin_amdgcn_raw_buffer_load_b128(dots, koff + (s0 + s) * slice * 4, 0, 0);
                    }
#pragma unroll
                    for (int s = 0; s < kBatch; ++s) qa += __builtin_bit_cast(f32x4, qp[s]);
                    if (kv) {
#pragma unroll
                        for (int s = 0; s < kBatch; ++s) ka += __builtin_bit_cast(f32x4, kp[s]);
                    }
                }
                // RoPE: even' = e c - o s, odd' = e s + o c on the pairs (d, d + 1), (d + 2, d + 3)
                const float2 qc = *reinterpret_cast<const float2*>(cosine + d / 2);
                const float2 qs2 = *reinterpret_cast<const float2*>(sine + d / 2);
                qa *= f;
                const f32x4 qr = f32x4{qa[0] * qc.x - qa[1] * qs2.x, qa[0] * qs2.x + qa[1] * qc.x,
                                       qa[2] * qc.y - qa[3] * qs2.y, qa[2] * qs2.y + qa[3] * qc.y};
                if (lane + kWave * r < qunits) *reinterpret_cast<f32x4*>(stage + g * HD + d) = qr;
                if (kv) {
                    ka *= f;
                    f32x4 kr = ka;
                    if (key) {
                        const float2 kc = *reinterpret_cast<const float2*>(cosine + kd / 2);
                        const float2 ks = *reinterpret_cast<const float2*>(sine + kd / 2);
                        kr = f32x4{ka[0] * kc.x - ka[1] * ks.x, ka[0] * ks.x + ka[1] * kc.x,
                                   ka[2] * kc.y - ka[3] * ks.y, ka[2] * ks.y + ka[3] * kc.y};
                    }
                    const int64_t index = ((static_cast<int64_t>(b) * p.KV + kvh) * p.capacity + newest) * HD + kd;
                    KT* dst = const_cast<KT*>(static_cast<const KT*>(key ? p.k : p.v)) + index;
                    if constexpr (F32) {
                        *reinterpret_cast<f32x4*>(dst) = kr;
                    } else {
                        // the cache's bf16 values, and the same values for the patch below
                        *reinterpret_cast<u32x2*>(dst) =
                            u32x2{static_cast<uint32_t>(f32_to_bf16(kr[0])) | (static_cast<uint32_t>(f32_to_bf16(kr[1])) << 16),
                                  static_cast<uint32_t>(f32_to_bf16(kr[2])) | (static_cast<uint32_t>(f32_to_bf16(kr[3])) << 16)};
                    }
                    *reinterpret_cast<f32x4*>(&kv_s[key ? 0 : 1][kd]) = kr;
                }
            }
            // the staged rows are read back by the lanes of this wave only (LDS operations of a wave complete in
            // order); the barriers keep the compiler from moving the reads above the writes, and the merge's
            // writes of o_s above the reads
            __asm__ volatile("" ::: "memory");
            split_q(stage + min(col, G - 1) * HD);
            __asm__ volatile("" ::: "memory");
        } else {
            // the query rows were requested before the first tile, so this split waits for them only
#pragma unroll
            for (int st = 0; st < KS; ++st)
                split8(f32x8{xq[st][0].x, xq[st][0].y, xq[st][0].z, xq[st][0].w, xq[st][1].x, xq[st][1].y,
                             xq[st][1].z, xq[st][1].w} * z, qh[st], ql[st]);
        }
    }
    // The holder's new key in its tile's registers (K: lanes col = key % 16 of half key / 16 hold dims
    // 32 st + 8 q ..; V: lanes col = key / 2, member key % 2 hold pieces q + 4 i), in the cache's type.
    auto to_kt = [&](const float* src) -> u32x4 {
        if constexpr (F32) {
            return __builtin_bit_cast(u32x4, *reinterpret_cast<const f32x4*>(src));
        } else {
            u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                w[e] = static_cast<uint32_t>(f32_to_bf16(src[2 * e])) |
                       (static_cast<uint32_t>(f32_to_bf16(src[2 * e + 1])) << 16);
            return w;
        }
    };
    auto patch = [&](int tile, Tile& dst) {
        if (!FINISH || tile != patch_tile) return;
        __asm__ volatile("" ::: "memory"); // the row is read here, not kept in registers through the loop
        const int u = patch_key / 16, kc = patch_key % 16, vc = patch_key / 2, ve = patch_key % 2;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int st = 0; st < KS; ++st)
#pragma unroll
                for (int e = 0; e < KL; ++e) {
                    const u32x4 w = to_kt(&kv_s[0][32 * st + 8 * q + e * DPP]);
                    if (h == u && col == kc) dst.k[h][st][e] = w;
                }
#pragma unroll
        for (int i = 0; i < VI; ++i)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const u32x4 w = to_kt(&kv_s[1][DPP * (q + 4 * i)]);
                if (e == ve && col == vc) dst.v[i][e] = w;
            }
    };
    if (tiles > 0) {
        // two tiles per iteration so that the buffers are named statically; the next tile is in flight while one
        // is used, and no load sits in a branch inside the loop (the last tile is peeled: the new key, the last
        // of its range, is always in the holder's last tile)
        int tile = 0;
        for (;;) {
            if (tile + 1 >= tiles) { patch(tile, a); use(tile, a); break; }
            load(tile + 1, c, kres, vres);
            use(tile, a);
            ++tile;
            if (tile + 1 >= tiles) { patch(tile, c); use(tile, c); break; }
            load(tile + 1, a, kres, vres);
            use(tile, c);
            ++tile;
        }
    }

    // merge the waves: lane holds O[head col][d = 16 dt + 4 q + j], the head's sum in every entry of l, and its
    // running maximum (base 2; natural units for the merge)
    if (col < G) {
        if (q == 0) {
            m_s[wave][col] = m_run * 0.6931471805599453f;
            l_s[wave][col] = l[0];
        }
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) o_s[wave][col][16 * dt + 4 * q + j] = o[dt][j];
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
            if (m_s[w][g] == -INFINITY) continue; // a wave without keys
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

template <typename KT, int HD>
int launch(const dlk_attention_params& p, hipStream_t stream) {
    const dim3 grid(p.splits, p.B * p.KV);
    // one short chunk per (sequence, KV head) (a one-sequence decode: one work-group per KV head) spreads over
    // eight waves; key splits and long runs over four (measured on MI355X: 1B widths, f32 cache, 129 / 257 / 385
    // keys: 6.1 / 7.6 / 10.3 us per layer with eight, 7.9 / 8.4 / 9.2 with four; batch 32 over 2048 bf16 keys:
    // 25.7 us with four, 26.4 with eight; batch 4 over 4100 keys of an f32 cache in 512-key splits: 26.5 us with
    // four, 28.5 with eight, and in 1024-key splits: 23.0 with four, 24.1 with eight)
    if constexpr (HD == 64) {
        if (p.chunk <= 512 && p.splits == 1) {
            if (p.qkv_partial) hipLaunchKernelGGL((attention_matrix<KT, HD, 8, true>), grid, dim3(8 * kWave), 0, stream, p);
            else hipLaunchKernelGGL((attention_matrix<KT, HD, 8, false>), grid, dim3(8 * kWave), 0, stream, p);
            return static_cast<int>(hipGetLastError());
        }
    }
    if (p.qkv_partial) hipLaunchKernelGGL((attention_matrix<KT, HD, 4, true>), grid, dim3(4 * kWave), 0, stream, p);
    else hipLaunchKernelGGL((attention_matrix<KT, HD, 4, false>), grid, dim3(4 * kWave), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

} // namespace
} // namespace dlk

extern "C" int dlk_attention_matrix_heads(int heads, int kv_heads, int head_dim) {
    return kv_heads > 0 && heads % kv_heads == 0 && heads / kv_heads <= 16 && (head_dim == 64 || head_dim == 128);
}

/* Whether dlk_attention_matrix_decode takes these parameters: one position, head dim 64 or 128, at most 16 query
   heads per KV head, key chunks of whole 32-key tiles per wave. */
extern "C" int dlk_attention_matrix_eligible(const dlk_attention_params* p) {
    // the partials are addressed with 32-bit byte offsets (batches of 8 slices run up to 24 slices past the base)
    const bool qkv = !p->qkv_partial ||
                     (p->qkv_splits >= 1 && p->qkv_splits <= 16 && p->rope_cos && p->rope_sin && p->qkv_K > 0 &&
                      p->qkv_width == (p->H + 2 * p->KV) * p->hd &&
                      24LL * p->B * p->qkv_width * 4 <= INT32_MAX);
    return p->L == 1 && !p->keep_mask && dlk_attention_matrix_heads(p->H, p->KV, p->hd) &&
           p->chunk % (4 * dlk::kTileKeys) == 0 &&
           p->ldq % 4 == 0 && qkv &&
           (p->splits == 1 || (p->partial_o && p->partial_ml));
}

/* The attention of one position on the matrix cores (the partials only: the caller launches the merge). */
extern "C" int dlk_attention_matrix_decode(const dlk_attention_params* params, dlh_stream stream_handle) {
    const dlk_attention_params& p = *params;
    if (!dlk_attention_matrix_eligible(&p)) return static_cast<int>(hipErrorInvalidValue);
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    if (p.kv_bf16) return p.hd == 64 ? dlk::launch<uint16_t, 64>(p, stream) : dlk::launch<uint16_t, 128>(p, stream);
    return p.hd == 64 ? dlk::launch<float, 64>(p, stream) : dlk::launch<float, 128>(p, stream);
}
