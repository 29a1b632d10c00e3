// Causal grouped-query attention over a prefill chunk on the matrix cores (see dlk_attention_params in
// kernels.h): bf16 or f32 K/V cache, head dim 64 or 128, one split.  Replaces, for L new positions, the query-blocked
// grouped_block + attention_weights of the reference (src/ops/attention.cpp:59-95, 161-188): scores in f32,
// causal rule key <= first + row (:52-57), softmax with the row maximum subtracted, P * V.
//
// Work-group: 4 waves and 128 query rows of one (batch, KV head): the G = H/KV query heads that share the KV
// head times 128/G consecutive positions (row r -> head r / (128/G), position l0 + r % (128/G)); each wave owns
// 32 rows as two 16-row query tiles.  Keys stream in tiles of 64 through LDS (double buffered: the next tile is
// loaded into registers while the current one is used), K as loaded and V transposed, shared by every head of
// the group.  Per tile and query tile:
//   S^T[16 keys][16 queries] = K[16][HD] * Q[16][HD]^T   (v_mfma_f32_16x16x32_bf16; A = K rows from LDS,
//                                                         B = the query rows, split into bf16 hi + lo)
// so lane l holds S[keys 4(l/16) .. +4][query l%16]: the online softmax of query l%16 runs on the lane's own
// values plus one cross-lane maximum, and the probabilities of two adjacent 16-key tiles are already the B
// operand of
//   O^T[16 d][16 queries] += V^T[16 d][32 keys] * P^T     (A = V^T from the transposed LDS tile, in the key
//                                                         order the lane holds; P split into hi + lo)
// Two MFMAs per product (hi and lo) keep f32-level accuracy against the bf16 K and V.  An f32 cache is split the
// same way when it is staged (K = Kh + Kl, V = Vh + Vl, each a bf16 plane in LDS), and each product takes three
// MFMAs: Kh Qh + Kh Ql + Kl Qh (the Kl Ql term is below 2^-16 of the product) and likewise for V^T P^T.  The softmax runs in base 2
// (log2 e folded into the score scale, one v_exp_f32 per score) and masks only the tiles that cross the causal
// diagonal.  The row maxima cross the four lanes of a row with the in-register lane swaps (v_permlane32_swap,
// v_permlane16_swap); the row sums come out of the matrix cores as one more output tile whose A operand is all
// ones, so every lane holds its row's sum with no cross-lane step.  Keys at or past the end of the sequence are
// staged as zeros, so stale cache rows never reach the products.
#include "kernels/device_common.h"

#include <type_traits>

namespace dlk {
namespace {

constexpr int kThreads = 256;
constexpr int kRows = 128;  // query rows per work-group
constexpr int kKeys = 64;   // keys per tile
constexpr int kXcds = 8;    // XCDs of the MI355X: linear work-group id i runs on XCD i % 8
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void split8(const f32x8 v, bf16x8& hi, bf16x8& lo) {
    hi = __builtin_convertvector(v, bf16x8);
    lo = __builtin_convertvector(v - __builtin_convertvector(hi, f32x8), bf16x8);
}

// The same split with the hi values widened back from the packed pairs (low half: << 16, high half: mask), one
// conversion per pair instead of one per value.
__device__ __forceinline__ void split8_pairs(const f32x8 v, bf16x8& hi, bf16x8& lo) {
    const u32x4 h = __builtin_bit_cast(u32x4, __builtin_convertvector(v, bf16x8));
    const f32x8 back = {__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xffff0000u),
                        __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xffff0000u),
                        __uint_as_float(h.z << 16), __uint_as_float(h.z & 0xffff0000u),
                        __uint_as_float(h.w << 16), __uint_as_float(h.w & 0xffff0000u)};
    hi = __builtin_bit_cast(bf16x8, h);
    lo = __builtin_convertvector(v - back, bf16x8);
}

// Maximum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the lanes that hold one query row): the lane-swap
// instructions exchange the two wave halves, then adjacent 16-lane rows, in registers.
__device__ __forceinline__ float max_over_rows(float x) {
    const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    x = fmaxf(__uint_as_float(h[0]), __uint_as_float(h[1]));
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ void block_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// bf16 hi and lo parts of four f32 values (round to nearest even twice: x - hi is exact in f32)
__device__ __forceinline__ void split4(const u32x4 w, u32x2& hi, u32x2& lo) {
    const f32x4 v = __builtin_bit_cast(f32x4, w);
    const bf16x4 h = __builtin_convertvector(v, bf16x4);
    const u32x2 hw = __builtin_bit_cast(u32x2, h);
    const f32x4 back = {__uint_as_float(hw.x << 16), __uint_as_float(hw.x & 0xffff0000u),
                        __uint_as_float(hw.y << 16), __uint_as_float(hw.y & 0xffff0000u)};
    hi = hw;
    lo = __builtin_bit_cast(u32x2, __builtin_convertvector(v - back, bf16x4));
}

// Pre-split K/V tiles of an f32 cache: for each (sequence, KV head) and 64-key tile, the K rows and the V^T rows
// split into bf16 hi and lo planes exactly as the attention kernel stages them in LDS (rows padded to KSTRIDE and
// VSTRIDE; keys at or past the end zero), one tile after another: [B * KV][kv_split_tiles][K hi | K lo | V^T hi |
// V^T lo].  One preparation pass per launch replaces the split that every work-group of a (sequence, KV head)
// would repeat on each tile it reads (C5: 128 work-groups per pair), and the attention copies a tile into LDS
// with the global->LDS DMA, no registers or vector-ALU work on the way.
template <int HD> struct SplitTile {
    // V^T rows of 136 bytes: the paired 8-byte fragment reads (ds_read2_b64, 32 bytes apart) of 16 rows hit no
    // LDS bank twice (measured on MI355X: 144-byte rows cost ~8 conflict cycles per read); each plane is padded
    // to whole 1 KB DMA blocks
    static constexpr int KSTRIDE = HD + 16, VSTRIDE = kKeys + 4;
    static constexpr int KPLANE = kKeys * KSTRIDE * 2, VPLANE = (HD * VSTRIDE * 2 + 1023) / 1024 * 1024; // bytes
    static constexpr int BYTES = 2 * KPLANE + 2 * VPLANE;
    static_assert(KPLANE % 1024 == 0 && VPLANE % 1024 == 0, "whole 1 KB DMA blocks");
};

// The preparation pass: work-group (tile, b * KV + kvh), the thread-to-piece maps of the kernel's own staging.
template <int HD>
__global__ __launch_bounds__(kThreads) void split_kv(const dlk_attention_params p) {
    using T = SplitTile<HD>;
    constexpr int NG = HD / 4;                  // 16-byte pieces (4 floats) per row
    constexpr int LOADS = kKeys * NG / kThreads;
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave, kp = lane % 32;
    const int tile = blockIdx.x, bk = blockIdx.y;
    const int64_t S = (p.position ? *p.position : p.first_host) + p.L;
    if (static_cast<int64_t>(tile) * kKeys >= S) return;
    const float* kbase = static_cast<const float*>(p.k) + static_cast<int64_t>(bk) * p.capacity * HD;
    const float* vbase = static_cast<const float*>(p.v) + static_cast<int64_t>(bk) * p.capacity * HD;
    char* dst = static_cast<char*>(p.kv_split) + (static_cast<int64_t>(bk) * p.kv_split_tiles + tile) * T::BYTES;
    uint16_t* khi = reinterpret_cast<uint16_t*>(dst);
    uint16_t* klo = reinterpret_cast<uint16_t*>(dst + T::KPLANE);
    uint16_t* vhi = reinterpret_cast<uint16_t*>(dst + 2 * T::KPLANE);
    uint16_t* vlo = reinterpret_cast<uint16_t*>(dst + 2 * T::KPLANE + T::VPLANE);
    u32x4 kr[LOADS], vr[LOADS];
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int c = t + kThreads * i, key = c / NG, dg = c % NG;
        const int64_t row = static_cast<int64_t>(tile) * kKeys + key;
        kr[i] = row < S ? *reinterpret_cast<const u32x4*>(kbase + row * HD + 4 * dg) : u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int i = 0; i < LOADS / 2; ++i) {
        const int dg = 2 * wave + lane / 32 + 8 * i;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int64_t row = static_cast<int64_t>(tile) * kKeys + 2 * kp + e;
            vr[2 * i + e] =
                row < S ? *reinterpret_cast<const u32x4*>(vbase + row * HD + 4 * dg) : u32x4{0u, 0u, 0u, 0u};
        }
    }
#pragma unroll
    for (int i = 0; i < LOADS; ++i) {
        const int c = t + kThreads * i, key = c / NG, dg = c % NG;
        u32x2 hi, lo;
        split4(kr[i], hi, lo);
        *reinterpret_cast<u32x2*>(khi + key * T::KSTRIDE + 4 * dg) = hi;
        *reinterpret_cast<u32x2*>(klo + key * T::KSTRIDE + 4 * dg) = lo;
    }
#pragma unroll
    for (int i = 0; i < LOADS / 2; ++i) {
        const int dg = 2 * wave + lane / 32 + 8 * i;
        // key 2 kp's hi (lo) values in the low halves, key 2 kp + 1's in the high halves
        u32x2 h0, l0, h1, l1;
        split4(vr[2 * i], h0, l0);
        split4(vr[2 * i + 1], h1, l1);
        const uint32_t h[4] = {h0.x & 0xffffu, h0.x >> 16, h0.y & 0xffffu, h0.y >> 16};
        const uint32_t hn[4] = {h1.x << 16, h1.x & 0xffff0000u, h1.y << 16, h1.y & 0xffff0000u};
        const uint32_t l[4] = {l0.x & 0xffffu, l0.x >> 16, l0.y & 0xffffu, l0.y >> 16};
        const uint32_t ln[4] = {l1.x << 16, l1.x & 0xffff0000u, l1.y << 16, l1.y & 0xffff0000u};
        uint32_t* col_h = reinterpret_cast<uint32_t*>(vhi + 4 * dg * T::VSTRIDE + 2 * kp);
        uint32_t* col_l = reinterpret_cast<uint32_t*>(vlo + 4 * dg * T::VSTRIDE + 2 * kp);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            col_h[e * (T::VSTRIDE / 2)] = h[e] | hn[e]; // head-dim 4 dg + e
            col_l[e * (T::VSTRIDE / 2)] = l[e] | ln[e];
        }
    }
}

template <typename KT, int HD, bool SPLIT>
__global__ __launch_bounds__(kThreads, sizeof(KT) == 2 ? 2 : 1) void attention_prefill(const dlk_attention_params p) {
    constexpr bool F32 = sizeof(KT) == 4;
    static_assert(!SPLIT || F32, "pre-split tiles exist for an f32 cache");
    constexpr int PLANES = F32 ? 2 : 1;         // staged bf16 planes per tile: hi (+ lo for an f32 cache)
    constexpr int KS = HD / 32;                 // k steps of the score MFMA
    constexpr int DT = HD / 16;                 // 16-wide head-dim tiles of the output
    // bf16 per staged K row: 160 (288) bytes at head dim 64 (128), where the 16-byte fragment reads of 16 rows
    // hit no LDS bank twice (measured on MI355X: a 144- or 272-byte row costs ~4 conflict cycles per read)
    constexpr int KSTRIDE = HD + 16;
    // bf16 per staged V^T row (one head-dim column): the pre-split tile's conflict-free 68, or 72, where the
    // 4-byte transposing stores of the in-kernel staging spread over the banks
    constexpr int VSTRIDE = SPLIT ? SplitTile<HD>::VSTRIDE : kKeys + 8;
    constexpr int VELEMS = SPLIT ? SplitTile<HD>::VPLANE / 2 : HD * VSTRIDE; // bf16 per V^T plane
    constexpr int DPP = 16 / sizeof(KT);        // head-dim values per 16-byte piece
    constexpr int NG = HD / DPP;                // pieces per K (or V) row
    constexpr int LOADS = kKeys * NG / kThreads; // K pieces per thread per tile (and V pieces, in key pairs)
    static_assert(kKeys * NG % kThreads == 0 && LOADS % 2 == 0, "whole loads; V pieces come in key pairs");
    __shared__ __attribute__((aligned(16))) uint16_t ks[PLANES][2][kKeys * KSTRIDE];
    __shared__ __attribute__((aligned(16))) uint16_t vt[PLANES][2][VELEMS];

    const int t = threadIdx.x, lane = t % kWave, q = lane / 16;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int G = p.H / p.KV, per_head = kRows / G;
    const int blocks = (p.L + per_head - 1) / per_head;
    // XCD-aware order: the hardware hands linear work-group id i to XCD i % 8, so with the (sequence, KV head)
    // pairs a multiple of 8, pair j's query blocks all run on XCD j % 8, the next pair of that XCD following once
    // they are done: the XCD's L2 then holds the K/V tiles of one or two pairs, which its work-groups share, not
    // those of every pair
    int qx = static_cast<int>(blockIdx.x), pair = static_cast<int>(blockIdx.y);
    if (gridDim.y % kXcds == 0) {
        const int linear = qx + static_cast<int>(gridDim.x) * pair;
        const int xcd = linear % kXcds, idx = linear / kXcds;
        pair = xcd + kXcds * (idx / static_cast<int>(gridDim.x));
        qx = idx % static_cast<int>(gridDim.x);
    }
    const int qb = blocks - 1 - qx; // the longest key ranges start first
    const int b = pair / p.KV, kvh = pair % p.KV;
    const int first = static_cast<int>(p.position ? *p.position : p.first_host);
    const int S = first + p.L;
    const int l0 = qb * per_head;
    const int key_end = min(first + l0 + per_head, S); // keys any row of this work-group sees
    const int tiles = (key_end + kKeys - 1) / kKeys;
    const int unmasked = (first + l0 + 1) / kKeys;      // tiles every row sees whole
    const float scale2 = p.scale * 1.4426950408889634f; // scores in base 2

    // this lane's two query rows (tile qt: row 32 wave + 16 qt + lane % 16)
    int head[2], pos[2];
    bool valid[2];
    int limit[2]; // last visible key
    bf16x8 qh[2][KS], ql[2][KS];
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        const int r = 32 * wave + 16 * qt + lane % 16;
        head[qt] = kvh * G + r / per_head;
        pos[qt] = l0 + r % per_head;
        valid[qt] = pos[qt] < p.L;
        const int l = min(pos[qt], p.L - 1);
        limit[qt] = min(first + pos[qt], S - 1);
        const float* row = p.q + (static_cast<int64_t>(b) * p.L + l) * p.ldq + static_cast<int64_t>(head[qt]) * HD;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
            const float4 a = *reinterpret_cast<const float4*>(row + 32 * s + 8 * q);
            const float4 c = *reinterpret_cast<const float4*>(row + 32 * s + 8 * q + 4);
            // the score scale (and log2 e) folded into the query before its split: the scores come out in base 2
            split8(f32x8{a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w} * scale2, qh[qt][s], ql[qt][s]);
        }
    }

    // K staging: piece c = t + 256 i -> key c / NG, head-dim group c % NG, stored as loaded (an f32 piece split
    // into its hi and lo planes).  V staging: lane -> key pair kp = lane % 32 and head-dim group 2 wave + lane / 32
    // (+ 8 per pass): the two keys' pieces are transposed into 32-bit words (key pair) of the V^T rows, the 64
    // lanes of a wave hitting 64 banks.
    const KT* kbase = static_cast<const KT*>(p.k) + (static_cast<int64_t>(b) * p.KV + kvh) * p.capacity * HD;
    const KT* vbase = static_cast<const KT*>(p.v) + (static_cast<int64_t>(b) * p.KV + kvh) * p.capacity * HD;
    const int kp = lane % 32;
    u32x4 kr[LOADS], vr[LOADS];
    auto load = [&](int tile) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int c = t + kThreads * i, key = c / NG, dg = c % NG;
            const int row = min(tile * kKeys + key, S - 1); // in bounds; rows past the end are zeroed when staged
            kr[i] = *reinterpret_cast<const u32x4*>(kbase + static_cast<int64_t>(row) * HD + DPP * dg);
        }
#pragma unroll
        for (int i = 0; i < LOADS / 2; ++i) {
            const int dg = 2 * wave + lane / 32 + 8 * i;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int row = min(tile * kKeys + 2 * kp + e, S - 1);
                vr[2 * i + e] = *reinterpret_cast<const u32x4*>(vbase + static_cast<int64_t>(row) * HD + DPP * dg);
            }
        }
    };
    auto stage = [&](int tile, int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int c = t + kThreads * i, key = c / NG, dg = c % NG;
            const bool live = tile * kKeys + key < S;
            const u32x4 w = live ? kr[i] : u32x4{0u, 0u, 0u, 0u};
            if constexpr (F32) {
                u32x2 hi, lo;
                split4(w, hi, lo);
                *reinterpret_cast<u32x2*>(&ks[0][buf][key * KSTRIDE + DPP * dg]) = hi;
                *reinterpret_cast<u32x2*>(&ks[PLANES - 1][buf][key * KSTRIDE + DPP * dg]) = lo;
            } else {
                *reinterpret_cast<u32x4*>(&ks[0][buf][key * KSTRIDE + DPP * dg]) = w;
            }
        }
#pragma unroll
        for (int i = 0; i < LOADS / 2; ++i) {
            const int dg = 2 * wave + lane / 32 + 8 * i;
            const bool live0 = tile * kKeys + 2 * kp < S, live1 = tile * kKeys + 2 * kp + 1 < S;
            const u32x4 v0 = live0 ? vr[2 * i] : u32x4{0u, 0u, 0u, 0u};
            const u32x4 v1 = live1 ? vr[2 * i + 1] : u32x4{0u, 0u, 0u, 0u};
            if constexpr (F32) {
                // key 2 kp's hi (lo) values in the low halves, key 2 kp + 1's in the high halves
                u32x2 h0, l0, h1, l1;
                split4(v0, h0, l0);
                split4(v1, h1, l1);
                const uint32_t h[4] = {h0.x & 0xffffu, h0.x >> 16, h0.y & 0xffffu, h0.y >> 16};
                const uint32_t hn[4] = {h1.x << 16, h1.x & 0xffff0000u, h1.y << 16, h1.y & 0xffff0000u};
                const uint32_t l[4] = {l0.x & 0xffffu, l0.x >> 16, l0.y & 0xffffu, l0.y >> 16};
                const uint32_t ln[4] = {l1.x << 16, l1.x & 0xffff0000u, l1.y << 16, l1.y & 0xffff0000u};
                uint32_t* col_h = reinterpret_cast<uint32_t*>(&vt[0][buf][DPP * dg * VSTRIDE + 2 * kp]);
                uint32_t* col_l = reinterpret_cast<uint32_t*>(&vt[PLANES - 1][buf][DPP * dg * VSTRIDE + 2 * kp]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    col_h[e * (VSTRIDE / 2)] = h[e] | hn[e]; // head-dim 4 dg + e
                    col_l[e * (VSTRIDE / 2)] = l[e] | ln[e];
                }
            } else {
                const uint32_t a[4] = {v0.x, v0.y, v0.z, v0.w}, c[4] = {v1.x, v1.y, v1.z, v1.w};
                uint32_t* col = reinterpret_cast<uint32_t*>(&vt[0][buf][DPP * dg * VSTRIDE + 2 * kp]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    col[(2 * e) * (VSTRIDE / 2)] = (a[e] & 0xffffu) | (c[e] << 16);        // head-dim 8 dg + 2 e
                    col[(2 * e + 1) * (VSTRIDE / 2)] = (a[e] >> 16) | (c[e] & 0xffff0000u); // head-dim 8 dg + 2 e + 1
                }
            }
        }
    };

    // SPLIT: wave w copies plane w of a pre-split tile (K hi, K lo, V^T hi, V^T lo) into LDS buffer buf; the
    // caller waits for its DMAs before the barrier that publishes the buffer
    auto copy = [&](int tile, int buf) {
        if constexpr (SPLIT) {
            using T = SplitTile<HD>;
            static_assert(T::KSTRIDE == KSTRIDE && T::VSTRIDE == VSTRIDE, "one layout");
            const char* src = static_cast<const char*>(p.kv_split) +
                              (static_cast<int64_t>(pair) * p.kv_split_tiles + tile) * T::BYTES +
                              (wave < 2 ? wave * T::KPLANE : 2 * T::KPLANE + (wave - 2) * T::VPLANE);
            const uint32_t lds = lds_offset(wave < 2 ? &ks[wave][buf][0] : &vt[wave - 2][buf][0]);
            const int blocks = (wave < 2 ? T::KPLANE : T::VPLANE) / 1024;
            for (int i = 0; i < blocks; ++i) dma16(src + 1024 * i, 16 * lane, lds + 1024 * i);
        }
    };

    // o: the output accumulators; l: the running row sums, taken by the matrix cores as a ones row of V^T times
    // P^T (every entry of l[qt] holds the sum of the lane's query row, so no cross-lane step is needed)
    f32x4 o[2][DT], l[2];
    float m_run[2] = {-INFINITY, -INFINITY};
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        l[qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int d = 0; d < DT; ++d) o[qt][d] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u});

    // one key tile; MASK: the tile crosses the causal diagonal of some row of the work-group
    auto step = [&](int tile, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int buf = tile & 1;
        if (tile + 1 < tiles) {
            if constexpr (SPLIT) copy(tile + 1, buf ^ 1);
            else load(tile + 1);
        }

        // scores: s[i][qt] = S[keys 64 tile + 16 i + 4 q + j][query row (qt, lane % 16)]
        // the K fragments are read ahead so that the reads overlap: the whole tile at head dim 64, one 16-key
        // block at a time at 128 (whose registers would not hold the whole tile)
        bf16x8 kf[4][KS], kl[4][KS];
        auto read_k = [&](int i) {
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                const int at = (16 * i + lane % 16) * KSTRIDE + 32 * st + 8 * q;
                kf[i][st] = *reinterpret_cast<const bf16x8*>(&ks[0][buf][at]);
                if constexpr (F32) kl[i][st] = *reinterpret_cast<const bf16x8*>(&ks[PLANES - 1][buf][at]);
            }
        };
        if constexpr (HD == 64) {
#pragma unroll
            for (int i = 0; i < 4; ++i) read_k(i);
        }
        f32x4 s[4][2];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (HD != 64) read_k(i);
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) s[i][qt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int st = 0; st < KS; ++st) {
#pragma unroll
                for (int qt = 0; qt < 2; ++qt) {
                    s[i][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i][st], qh[qt][st], s[i][qt], 0, 0, 0);
                    s[i][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[i][st], ql[qt][st], s[i][qt], 0, 0, 0);
                    if constexpr (F32)
                        s[i][qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl[i][st], qh[qt][st], s[i][qt], 0, 0, 0);
                }
            }
        }

        // online softmax per query row (the lane's column; lanes l, l^16, l^32, l^48 share it), in base 2
        bf16x8 ph[2][2], pl[2][2]; // [key block u: tiles 2u, 2u+1][qt]
        auto softmax = [&](int qt) {
            float mx = -INFINITY;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    float v = s[i][qt][j];
                    if constexpr (MASK) {
                        if (tile * kKeys + 16 * i + 4 * q + j > limit[qt]) v = -INFINITY;
                        s[i][qt][j] = v;
                    }
                    mx = fmaxf(mx, v);
                }
            mx = max_over_rows(mx);
            // key 0 is visible to every row, so m_new is finite from the first tile on; exp2(-inf) = 0
            const float m_new = fmaxf(m_run[qt], mx);
            const float alpha = __builtin_amdgcn_exp2f(m_run[qt] - m_new);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) s[i][qt][j] = __builtin_amdgcn_exp2f(s[i][qt][j] - m_new);
            m_run[qt] = m_new;
            // f32 cache: unconditional (alpha = 1 when the maxima stayed), since a branch would split the tile into
            // basic blocks and the scheduler could not put this work under the MFMAs; the bf16 kernels keep the
            // branch, whose registers hold at head dim 128 only with it
            if (F32 || !__all(alpha == 1.0f)) {
                l[qt] *= alpha;
#pragma unroll
                for (int d = 0; d < DT; ++d) o[qt][d] *= alpha;
            }
#pragma unroll
            for (int u = 0; u < 2; ++u)
                split8_pairs(f32x8{s[2 * u][qt][0], s[2 * u][qt][1], s[2 * u][qt][2], s[2 * u][qt][3],
                             s[2 * u + 1][qt][0], s[2 * u + 1][qt][1], s[2 * u + 1][qt][2], s[2 * u + 1][qt][3]},
                       ph[u][qt], pl[u][qt]);
        };
        softmax(0);
        softmax(1);
        // O^T += V^T P^T: lane (d = 16 dt + lane % 16, q) supplies V[keys 32 u + 4 q .. +4, 32 u + 16 + 4 q .. +4][d]
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int qt = 0; qt < 2; ++qt) {
                l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, ph[u][qt], l[qt], 0, 0, 0);
                l[qt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pl[u][qt], l[qt], 0, 0, 0);
            }
        auto v_frag = [&](int plane, int dt, int u) {
            const int at = (16 * dt + lane % 16) * VSTRIDE + 32 * u + 4 * q;
            const u32x2 lo4 = *reinterpret_cast<const u32x2*>(&vt[plane][buf][at]);
            const u32x2 hi4 = *reinterpret_cast<const u32x2*>(&vt[plane][buf][at + 16]);
            return __builtin_bit_cast(bf16x8, u32x4{lo4.x, lo4.y, hi4.x, hi4.y});
        };
        if constexpr (HD == 64) {
            // one key half at a time: its V^T fragments of every head-dim tile are read before its products (a
            // scheduling barrier keeps the reads from sinking to their first use, where each would expose an LDS
            // latency); each o[qt][dt] still takes half 0, then half 1.  At head dim 128 the registers would spill.
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                bf16x8 a[DT], al[DT];
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    a[dt] = v_frag(0, dt, u);
                    if constexpr (F32) al[dt] = v_frag(PLANES - 1, dt, u);
                }
                __builtin_amdgcn_sched_barrier(0);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt)
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt) {
                        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[dt], ph[u][qt], o[qt][dt], 0, 0, 0);
                        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[dt], pl[u][qt], o[qt][dt], 0, 0, 0);
                        if constexpr (F32)
                            o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[dt], ph[u][qt], o[qt][dt], 0, 0, 0);
                    }
            }
        } else {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const bf16x8 a = v_frag(0, dt, u);
                    bf16x8 al;
                    if constexpr (F32) al = v_frag(PLANES - 1, dt, u);
#pragma unroll
                    for (int qt = 0; qt < 2; ++qt) {
                        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, ph[u][qt], o[qt][dt], 0, 0, 0);
                        o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pl[u][qt], o[qt][dt], 0, 0, 0);
                        if constexpr (F32)
                            o[qt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, ph[u][qt], o[qt][dt], 0, 0, 0);
                    }
                }
            }
        }

        if (tile + 1 < tiles) {
            if constexpr (SPLIT) wait_vm<0>();
            else stage(tile + 1, buf ^ 1);
        }
        block_barrier();
    };
    if constexpr (SPLIT) {
        copy(0, 0);
        wait_vm<0>();
    } else {
        load(0);
        stage(0, 0);
    }
    block_barrier();
    for (int tile = 0; tile < min(unmasked, tiles); ++tile) step(tile, std::false_type{});
    for (int tile = unmasked; tile < tiles; ++tile) step(tile, std::true_type{});

    // lane holds O[query row (qt, lane % 16)][d = 16 dt + 4 q + j].  With stage_out the four values go to the
    // projection's staging layout instead (row m = b L + l, k = head HD + d): hi and lo of row m, k step k / 32,
    // lane (m % 16) + 16 ((k % 32) / 8), elements k % 8 .. +4, the split its preparation pass would make
#pragma unroll
    for (int qt = 0; qt < 2; ++qt) {
        if (!valid[qt]) continue;
        const float inv = 1.0f / l[qt][0];
        const int64_t row = static_cast<int64_t>(b) * p.L + pos[qt];
        if (p.stage_out) {
            const int ksteps = p.H * HD / 32;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const int k = head[qt] * HD + 16 * dt + 4 * q;
                const f32x4 v = {o[qt][dt][0] * inv, o[qt][dt][1] * inv, o[qt][dt][2] * inv, o[qt][dt][3] * inv};
                const bf16x4 h = __builtin_convertvector(v, bf16x4);
                const bf16x4 lo = __builtin_convertvector(v - __builtin_convertvector(h, f32x4), bf16x4);
                char* at = static_cast<char*>(p.stage_out) + ((row / 16) * ksteps + k / 32) * 2048 +
                           ((row % 16) + 16 * ((k % 32) / 8)) * 16 + (k % 8) * 2;
                *reinterpret_cast<bf16x4*>(at) = h;
                *reinterpret_cast<bf16x4*>(at + 1024) = lo;
            }
            continue;
        }
        float* out = p.out + row * p.ldo + static_cast<int64_t>(head[qt]) * HD;
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
            *reinterpret_cast<float4*>(out + 16 * dt + 4 * q) =
                make_float4(o[qt][dt][0] * inv, o[qt][dt][1] * inv, o[qt][dt][2] * inv, o[qt][dt][3] * inv);
    }
}

} // namespace
} // namespace dlk

/* Whether dlk_attention takes the matrix-core prefill kernel for these parameters. */
extern "C" int dlk_attention_prefill_eligible(const dlk_attention_params* p) {
    const int G = p->KV > 0 ? p->H / p->KV : 0;
    return p->causal && !p->keep_mask && (p->hd == 64 || p->hd == 128) && p->L >= 16 && G > 0 && dlk::kRows % G == 0 &&
           p->splits == 1 && p->ldq % 4 == 0 && p->ldo % 4 == 0;
}

extern "C" int64_t dlk_attention_split_bytes(const dlk_attention_params* p) {
    if (p->kv_bf16 || !dlk_attention_prefill_eligible(p)) return 0;
    const int64_t tiles = (p->capacity + dlk::kKeys - 1) / dlk::kKeys;
    const int64_t tile = p->hd == 64 ? dlk::SplitTile<64>::BYTES : dlk::SplitTile<128>::BYTES;
    return static_cast<int64_t>(p->B) * p->KV * tiles * tile;
}

extern "C" int dlk_attention_prefill(const dlk_attention_params* params, dlh_stream stream_handle) {
    const dlk_attention_params& p = *params;
    if (!dlk_attention_prefill_eligible(&p)) return static_cast<int>(hipErrorInvalidValue);
    // the pre-split tiles cover every position the cache can hold
    if (p.kv_split && (p.kv_bf16 || static_cast<int64_t>(p.kv_split_tiles) * dlk::kKeys < p.capacity ||
                       reinterpret_cast<uintptr_t>(p.kv_split) % 16 != 0))
        return static_cast<int>(hipErrorInvalidValue);
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    const int per_head = dlk::kRows / (p.H / p.KV);
    const dim3 grid((p.L + per_head - 1) / per_head, p.B * p.KV);
    const dim3 threads(dlk::kThreads);
    if (p.kv_bf16) {
        if (p.hd == 64) hipLaunchKernelGGL((dlk::attention_prefill<uint16_t, 64, false>), grid, threads, 0, stream, p);
        else hipLaunchKernelGGL((dlk::attention_prefill<uint16_t, 128, false>), grid, threads, 0, stream, p);
    } else if (p.kv_split) {
        const dim3 tiles(p.kv_split_tiles, p.B * p.KV);
        if (p.hd == 64) {
            hipLaunchKernelGGL((dlk::split_kv<64>), tiles, threads, 0, stream, p);
            hipLaunchKernelGGL((dlk::attention_prefill<float, 64, true>), grid, threads, 0, stream, p);
        } else {
            hipLaunchKernelGGL((dlk::split_kv<128>), tiles, threads, 0, stream, p);
            hipLaunchKernelGGL((dlk::attention_prefill<float, 128, true>), grid, threads, 0, stream, p);
        }
    } else {
        if (p.hd == 64) hipLaunchKernelGGL((dlk::attention_prefill<float, 64, false>), grid, threads, 0, stream, p);
        else hipLaunchKernelGGL((dlk::attention_prefill<float, 128, false>), grid, threads, 0, stream, p);
    }
    return static_cast<int>(hipGetLastError());
}
