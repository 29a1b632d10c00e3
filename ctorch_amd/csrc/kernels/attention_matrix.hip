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

template <typename KT, int HD, int W>
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

    const int t = threadIdx.x, lane = t % kWave, q = lane / 16, col = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int split = blockIdx.x;
    const int bk = blockIdx.y;
    const int b = bk / p.KV, kvh = bk % p.KV;
    const int G = p.H / p.KV;
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
    const int per_wave = p.chunk / W;
    const int64_t k_end = min(S, static_cast<int64_t>(split) * p.chunk + p.chunk);
    const int64_t w_begin = static_cast<int64_t>(split) * p.chunk + static_cast<int64_t>(wave) * per_wave;
    const int keys = static_cast<int>(max<int64_t>(0, min<int64_t>(k_end, w_begin + per_wave) - w_begin));
    const int tiles = (keys + kTileKeys - 1) / kTileKeys;

    // the query heads of this KV head as the B operand (column col = head kvh G + col), scaled into base 2
    bf16x8 qh[KS], ql[KS];
    {
        const float qs = p.scale * 1.4426950408889634f;
        const float* qrow = p.q + static_cast<int64_t>(b) * p.ldq + static_cast<int64_t>(kvh * G + min(col, G - 1)) * HD;
#pragma unroll
        for (int st = 0; st < KS; ++st) {
            const float4 a = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q);
            const float4 c = *reinterpret_cast<const float4*>(qrow + 32 * st + 8 * q + 4);
            const float z = col < G ? qs : 0.0f;
            split8(f32x8{a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w} * z, qh[st], ql[st]);
        }
    }

    // buffer ranges over this wave's keys: rows past them read as zero
    const size_t head = (static_cast<size_t>(b) * p.KV + kvh) * p.capacity + w_begin;
    const __amdgpu_buffer_rsrc_t kres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<KT*>(static_cast<const KT*>(p.k) + head * HD), 0, keys * ROW, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<KT*>(static_cast<const KT*>(p.v) + head * HD), 0, keys * ROW, kBufferFlags);
    // K fragment (half u, k step st): key 16 u + col, head dims 32 st + 8 q .. +8.  V: key pair kp = col (keys
    // 2 kp, 2 kp + 1), pieces dg = q + 4 i.
    const int k_offset = col * ROW + (8 * q) * static_cast<int>(sizeof(KT));
    const int v_offset = 2 * col * ROW + q * 16;
    struct Tile {
        u32x4 k[2][KS][KL];
        u32x4 v[VI][2];
    };
    auto load = [&](int tile, Tile& dst) {
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

    f32x4 o[DT], l = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int d = 0; d < DT; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY;
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});
    uint16_t* my_vt = &vt[wave][0][0];

    auto use = [&](int tile, const Tile& cur) {
        // V^T of the tile into the wave's LDS tile (word = key pair kp of one head-dim row)
#pragma unroll
        for (int i = 0; i < VI; ++i) {
            const u32x4 a = cur.v[i][0], c = cur.v[i][1];
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
    // 25.7 us with four, 26.4 with eight; batch 4 over 4100 keys in 512-key splits: 26.5 us with four, 28.5 with
    // eight)
    if constexpr (HD == 64) {
        if (p.chunk <= 512 && p.splits == 1) {
            hipLaunchKernelGGL((attention_matrix<KT, HD, 8>), grid, dim3(8 * kWave), 0, stream, p);
            return static_cast<int>(hipGetLastError());
        }
    }
    hipLaunchKernelGGL((attention_matrix<KT, HD, 4>), grid, dim3(4 * kWave), 0, stream, p);
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
    return p->L == 1 && dlk_attention_matrix_heads(p->H, p->KV, p->hd) && p->chunk % (4 * dlk::kTileKeys) == 0 &&
           p->ldq % 4 == 0 &&
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
