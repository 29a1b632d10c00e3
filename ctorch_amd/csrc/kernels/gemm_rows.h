// Projection over several activation rows (batched decode, M = 3..64 per launch) on the matrix cores, with the
// epilogues of the GEMV (see dlk_gemv_params in kernels.h).
//
// One v_mfma_f32_16x16x32_bf16 computes D[16 weight rows][16 activation rows] += W[16][32] * X[16][32]^T.  Lane
// l supplies A = W[row l%16][k 8*(l/16) .. +8] (16 contiguous bytes of a weight row, so the weights stream from
// HBM in their row-major layout), B = X[row l%16][k 8*(l/16) .. +8], and receives D[rows 4*(l/16) .. +4][l%16].
//
// A work-group is eight waves; each wave owns one tile of 16 weight rows and all activation rows (MT tiles of
// 16).  The activation rows are staged per K-chunk in LDS as bf16 pairs hi + lo (x = hi + lo to ~2^-16), so every
// product is two MFMAs and the result keeps f32-level accuracy against a bf16 weight.  The RMSNorm of the
// activation rows is fused: the staged rows are x * g, the sums of squares accumulate while staging, and the
// per-row factor 1/sqrt(mean x^2 + eps) scales the finished dot products.  A work-group of up to two chunks
// (NC = 2) issues every activation and weight load of its chunks at once, stages them all, and computes: one
// memory round trip.  Longer runs double buffer the chunks in LDS: with repacked weights and a run of 4, 8, 16 or
// 32 chunks (NC = the run) the weights of the next three chunks are in flight while one is used; otherwise
// (NC = 0) the next chunk's activations (into registers) and weights.
//
// Tile rows: generic epilogues take 16 consecutive rows of one weight segment; SwiGLU interleaves gate and up
// (tile row 2j = gate row 8T + j, 2j + 1 = up row 8T + j), so every lane holds (gate, up) pairs and QKV holds
// RoPE pairs (rows 2j, 2j + 1 of a head) in one lane.
#pragma once

#include "kernels/gemv_impl.h"

namespace dlk::gemm {

using gemv::u32x4;
constexpr int kThreads = 512;
constexpr int kWaves = kThreads / kWave;
constexpr int kTile = 16;                       // weight rows per wave tile
constexpr int kMaxRows = 64;                    // activation rows per launch
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

/// k per staged chunk: the smallest the staging map takes (each row's 4-column groups span at most half a
/// work-group).  Shorter chunks pipeline the loads finer against the staging and the products; measured on MI355X
/// (1B widths, A/B on one box): 16 rows 256 -> 128 (gate/up at batch 32 in row parts 16.25 -> 15.55 us a layer,
/// the batch-4 LoRA decode step 1.29 -> 1.24 ms), 32 rows 128 -> 64 (QKV at batch 32 7.35 -> 6.34 us a layer);
/// 512 at 16 rows was slower (gate/up 19.0 us).
constexpr int chunk_k(int mt) { return mt == 1 ? 128 : 64; }
constexpr int lds_stride(int mt) { return chunk_k(mt) + 8; } // bf16 elements per staged row (bank spread)
/// LDS of a work-group: two staged chunks of hi and lo rows (every variant).
constexpr size_t lds_bytes(int mt) { return size_t(2) * 2 * 16 * mt * lds_stride(mt) * 2; }
/// Chunks the deep pipeline keeps in flight ahead of the one in use.  Measured on MI355X (C3 step, A/B on one box):
/// 3 ahead 1.183 ms; 4 (16-row tiles) / 6 (32-row tiles) ahead 1.198-1.210 ms; 5 / 8 ahead 1.214-1.225 ms.
constexpr int kDeepAhead = 3;
/// Variant for a run of `nchunks` chunks: 2 (all loads up front; that many chunks at most), the run length itself
/// (the deep pipeline, unrolled over a run of 4, 8, 16 or 32 chunks; `deep`: repacked weights and 16 or more
/// activation rows per work-group), or 0 for the double-buffered loop.  Measured on MI355X (A/B, one box): at batch
/// 32 (1B) the deep pipeline took the C3 step 1.190-1.204 -> 1.168-1.170 ms (gate/up 15.5 -> 14.9 us, down 11.7-12.2
/// -> 10.9, LM head 30.5-31.1 -> 29.3); at 8 rows (8B, batch 8) the QKV and gate/up launches, already streaming at
/// ~5.6 TB/s, lost 1-1.7 us each, so those keep the loop.  Runs of three or four chunks take a loop, not all loads
/// up front (C3 down projection in 11 key slices of 4 chunks: 11.2 us a layer against 12.7).
constexpr int loop_variant(int nchunks, bool deep) {
    if (nchunks <= 2) return 2;
    if (deep && (nchunks == 4 || nchunks == 8 || nchunks == 16 || nchunks == 32)) return nchunks;
    return 0;
}
/// Most key slices a launch takes (the reduce kernel keeps them all in flight).
constexpr int kMaxSplits = 16;

/// Whether the matrix-core path takes these parameters (host side).
inline bool eligible(const dlk_gemv_params& p) {
    if (!p.w_bf16 || p.M < 3 || p.K % 256 != 0 || p.K < 512) return false;
    if (p.epilogue == DLK_EPI_SWIGLU) return p.seg_rows[0] % 8 == 0;
    for (int s = 0; s < p.nseg; ++s)
        if (p.seg_rows[s] % kTile != 0) return false;
    return true;
}

/// Whether every weight segment of the launch comes repacked in tile order (w_tiles).
inline bool repacked(const dlk_gemv_params& p) {
    const int segs = p.epilogue == DLK_EPI_SWIGLU ? 1 : p.nseg;
    for (int s = 0; s < segs; ++s)
        if (!p.w_tiles[s]) return false;
    return true;
}

/// 16-row weight tiles of a launch.
__host__ __device__ inline int tiles_of(const dlk_gemv_params& p) {
    if (p.epilogue == DLK_EPI_SWIGLU) return p.seg_rows[0] / 8;
    int t = p.seg_rows[0] / kTile;
    if (p.nseg > 1) t += p.seg_rows[1] / kTile;
    if (p.nseg > 2) t += p.seg_rows[2] / kTile;
    return t;
}

inline int blocks_of(const dlk_gemv_params& p) { return (tiles_of(p) + kWaves - 1) / kWaves; }

/// Activation tiles of 16 rows for a launch of `rows` (<= 64) rows.
inline int row_tiles(int rows) { return rows <= 16 ? 1 : rows <= 32 ? 2 : 4; }

/// Key slices of a launch: one, unless the weight tiles leave most CUs idle; then the most slices (each a whole
/// number of chunks; runs of one to four chunks take the up-front variant, longer ones the loop) that keep the
/// launch within 352 work-groups.  Measured on MI355X (1B widths, SwiGLU, weights repacked): at batch 4,
/// 16.4 us at 352 work-groups against 17.3 at 176; at batch 32 two work-groups on a CU streamed slower than
/// one (24.8 us at 352 against 21.0 at 176, row-major weights), and that launch now splits over rows instead.
inline int splits_of(const dlk_gemv_params& p, int rows) {
    if (p.epilogue == DLK_EPI_LOGITS) return 1;
    const int blocks = blocks_of(p);
    if (blocks >= 192) return 1;
    const int chunks = p.K / chunk_k(row_tiles(rows));
    // SwiGLU over at most 16 rows (a small batch's gate/up) within 720 work-groups: at batch 4, 8 slices (704
    // work-groups) 14.6-14.7 us against 15.7 at 4 and 15.9 at 16, the C5 decode step 1.030 -> 1.011 ms (A/B,
    // interleaved runs).  The other launches keep the cap their split counts were measured at.
    const int cap = p.epilogue == DLK_EPI_SWIGLU && rows <= 16 ? 720 : 352;
    int best = 1;
    for (int s = 2; s <= kMaxSplits && blocks * s <= cap; ++s) {
        if (chunks % s == 0) best = s;
    }
    return best;
}

/// Workspace floats of a split launch of `rows` rows: partial dots [S][rows][tiles * 16], then squares [S][rows].
inline int64_t split_floats(const dlk_gemv_params& p, int splits, int rows) {
    return splits <= 1 ? 0 : static_cast<int64_t>(splits) * rows * (tiles_of(p) * kTile + 1);
}

// A wave's tile: segment, first row in the segment, the matrix of tile row i.
struct TileMap {
    int seg, n0, rows;
    const uint16_t *base0, *base1;
};

template <bool SWIGLU>
__device__ __forceinline__ TileMap locate(const dlk_gemv_params& p, int tile) {
    const uint16_t* w0 = static_cast<const uint16_t*>(p.w[0]);
    const uint16_t* w1 = static_cast<const uint16_t*>(p.w[1]);
    const uint16_t* w2 = static_cast<const uint16_t*>(p.w[2]);
    if constexpr (SWIGLU) return {0, tile * 8, p.seg_rows[0], w0, w1};
    const int t0 = p.seg_rows[0] / kTile, t1 = p.nseg > 1 ? p.seg_rows[1] / kTile : 0;
    if (tile < t0 || p.nseg == 1) return {0, tile * kTile, p.seg_rows[0], w0, w0};
    if (tile < t0 + t1 || p.nseg == 2) return {1, (tile - t0) * kTile, p.seg_rows[1], w1, w1};
    return {2, (tile - t0 - t1) * kTile, p.seg_rows[2], w2, w2};
}

// weight row of tile row i (SwiGLU: even rows gate, odd rows up of the same output)
template <bool SWIGLU>
__device__ __forceinline__ const uint16_t* tile_row(const TileMap& t, int i, int K) {
    if constexpr (SWIGLU) return (i & 1 ? t.base1 : t.base0) + static_cast<int64_t>(t.n0 + i / 2) * K;
    return t.base0 + static_cast<int64_t>(t.n0 + i) * K;
}

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4))); // the bf16 operands of v_mfma_f32_16x16x16_bf16

// bf16 hi and lo parts of four values (x = hi + lo to ~2^-16): the hardware's round-to-nearest-even conversion
// packs two values per instruction, and the hi values are widened back from the packed words by shift and mask
__device__ __forceinline__ void split4_bf16(const float (&e)[4], u32x2& hi, u32x2& lo) {
    const f32x4v v = {e[0], e[1], e[2], e[3]};
    const u32x2 h = __builtin_bit_cast(u32x2, __builtin_convertvector(v, bf16x4));
    const f32x4v back = {__uint_as_float(h.x << 16), __uint_as_float(h.x & 0xffff0000u),
                         __uint_as_float(h.y << 16), __uint_as_float(h.y & 0xffff0000u)};
    hi = h;
    lo = __builtin_bit_cast(u32x2, __builtin_convertvector(v - back, bf16x4));
}

// LoRA products of a lane's four tile rows, when the caller computed them (passed by value: a pointer to a
// local array would keep it in scratch memory).
struct LoraProducts {
    float v[4];
    bool set;
};

// Unmerged LoRA of the output pair (n, n + 1): up[n, :] . h and up[n + 1, :] . h over the rank, for a bf16 up
// matrix.  Ranks of 8..32 in steps of 8 issue every load first (16-byte pieces of both up rows and of h; pieces
// past the rank repeat the last one and are not used), so the pair costs one memory round trip instead of one per
// rank entry; other ranks take the scalar loop.
constexpr int kLoraPiecesMax = 4; // rank 32
__device__ __forceinline__ void lora_pair(const dlk_gemv_params& p, const void* up, const float* hrow, int n,
                                          float& de, float& dodd) {
    using Traits = gemv::WeightTraits<uint16_t>;
    const int r = p.lora_rank;
    de = 0.0f;
    dodd = 0.0f;
    if (r % 8 == 0 && r <= 8 * kLoraPiecesMax && gemv::lora_stride(p) % 4 == 0) {
        const int pieces = r / 8;
        const uint16_t* ue = static_cast<const uint16_t*>(up) + static_cast<int64_t>(n) * r;
        u32x4 we[kLoraPiecesMax], wo[kLoraPiecesMax];
        float h[kLoraPiecesMax][8];
#pragma unroll
        for (int s = 0; s < kLoraPiecesMax; ++s) {
            const int k = 8 * min(s, pieces - 1);
            we[s] = *reinterpret_cast<const u32x4*>(ue + k);
            wo[s] = *reinterpret_cast<const u32x4*>(ue + r + k);
            const float4 a = *reinterpret_cast<const float4*>(hrow + k);
            const float4 c = *reinterpret_cast<const float4*>(hrow + k + 4);
            h[s][0] = a.x; h[s][1] = a.y; h[s][2] = a.z; h[s][3] = a.w;
            h[s][4] = c.x; h[s][5] = c.y; h[s][6] = c.z; h[s][7] = c.w;
        }
#pragma unroll
        for (int s = 0; s < kLoraPiecesMax; ++s) {
            if (s >= pieces) break;
            de += Traits::dot(we[s], h[s]);
            dodd += Traits::dot(wo[s], h[s]);
        }
        return;
    }
    for (int j = 0; j < r; ++j) {
        de += Traits::scalar(up, static_cast<int64_t>(n) * r + j) * hrow[j];
        dodd += Traits::scalar(up, static_cast<int64_t>(n + 1) * r + j) * hrow[j];
    }
}

// QKV: the batch and cache position of activation row m, when the caller computed them once for the row
// (they take a 64-bit division).
struct RowPosition {
    int64_t batch, position;
    bool set;
};

// The epilogue of one lane: v[j] = finished dot products of tile rows 4q + j (q = lane / 16) for activation
// row m of the launch.  QKV: lora (if set) holds the unscaled LoRA products up[n, :] . hidden[m, :] of the
// same rows, computed by the caller; otherwise they are computed here.
template <int EPI>
__device__ __forceinline__ void lane_epilogue(const dlk_gemv_params& p, const TileMap& t, int q, int m,
                                              const float (&v)[4], double& best_score, int64_t& best_index,
                                              uint64_t seed, uint64_t stream, LoraProducts lora = {{}, false},
                                              RowPosition where = {0, 0, false}) {
    if constexpr (EPI == DLK_EPI_SWIGLU) {
        const int n = t.n0 + 2 * q;
        p.y[static_cast<int64_t>(m) * p.ldy + n] = gemv::silu(v[0]) * v[1];
        p.y[static_cast<int64_t>(m) * p.ldy + n + 1] = gemv::silu(v[2]) * v[3];
    } else if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        // every operand is loaded before the first store: y may alias them as far as the compiler knows, so a
        // load issued after a store waits for it, and the four outputs would take four memory round trips
        float add[4] = {0.f, 0.f, 0.f, 0.f};
        const bool bias = EPI == DLK_EPI_STORE && p.bias;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = (EPI == DLK_EPI_STORE ? gemv::seg_column(p, t.seg) : 0) + t.n0 + 4 * q + j;
            if constexpr (EPI == DLK_EPI_STORE) {
                if (bias)
                    add[j] = p.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p.bias)[n])
                                         : static_cast<const float*>(p.bias)[n];
            } else {
                add[j] = p.residual[static_cast<int64_t>(m) * p.ldres + n];
            }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = (EPI == DLK_EPI_STORE ? gemv::seg_column(p, t.seg) : 0) + t.n0 + 4 * q + j;
            float out = v[j];
            if (EPI == DLK_EPI_RESIDUAL || bias) out += add[j];
            p.y[static_cast<int64_t>(m) * p.ldy + n] = out;
        }
    } else if constexpr (EPI == DLK_EPI_QKV) {
        const int64_t mg = p.m_base + m;
        const int64_t b = where.set ? where.batch : mg / p.length;
        const int64_t pos = where.set ? where.position : *p.position + mg % p.length;
        const int hd = p.head_dim;
        const float* hidden = t.seg == 0 ? p.lora_hidden[0] : t.seg == 2 ? p.lora_hidden[2] : nullptr;
        const void* lora_up = t.seg == 0 ? p.lora_up[0] : p.lora_up[2];
        // the rotation of both pairs is loaded before any store (see the residual epilogue above)
        float rc[2] = {1.f, 1.f}, rs[2] = {0.f, 0.f};
        if (t.seg < 2) {
#pragma unroll
            for (int pair = 0; pair < 2; ++pair) {
                const int d = (t.n0 + 4 * q + 2 * pair) % hd;
                const int64_t table = pos * (hd / 2) + d / 2;
                rc[pair] = p.cosine[table];
                rs[pair] = p.sine[table];
            }
        }
#pragma unroll
        for (int pair = 0; pair < 2; ++pair) {
            const int n = t.n0 + 4 * q + 2 * pair; // even: the pair (n, n + 1) shares one rotation
            float even = v[2 * pair], odd = v[2 * pair + 1];
            if (hidden && lora.set) {
                even += lora.v[2 * pair] * p.lora_scale;
                odd += lora.v[2 * pair + 1] * p.lora_scale;
            } else if (hidden) {
                // unmerged LoRA: + scale * up[n, :] . hidden[m, :]
                float de, dodd;
                lora_pair(p, lora_up, hidden + mg * gemv::lora_stride(p), n, de, dodd);
                even += de * p.lora_scale;
                odd += dodd * p.lora_scale;
            }
            const int d = n % hd, head = n / hd;
            if (t.seg < 2) {
                // even: x_e c - x_o s ; odd: x_e s + x_o c (interleaved pairs, src/ops/contraction.cpp:44-49)
                const float c = rc[pair], s = rs[pair];
                const float re = even * c - odd * s, ro = even * s + odd * c;
                even = re;
                odd = ro;
            }
            if (t.seg == 0) {
                p.y[mg * p.ldy + n] = even;
                p.y[mg * p.ldy + n + 1] = odd;
            } else {
                const int64_t index = ((b * p.kv_heads + head) * p.cache_capacity + pos) * hd + d;
                void* cache = t.seg == 1 ? p.k_cache : p.v_cache;
                if (p.cache_bf16) {
                    static_cast<uint16_t*>(cache)[index] = f32_to_bf16(even);
                    static_cast<uint16_t*>(cache)[index + 1] = f32_to_bf16(odd);
                } else {
                    static_cast<float*>(cache)[index] = even;
                    static_cast<float*>(cache)[index + 1] = odd;
                }
            }
        }
    } else if constexpr (EPI == DLK_EPI_LOGITS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = t.n0 + 4 * q + j;
            if (p.y) p.y[static_cast<int64_t>(m) * p.ldy + n] = v[j];
            if (p.sample_mode != 0) {
                const int64_t mg = p.m_base + m;
                const double s = sample_score(v[j], p.sample_mode, p.temperature, seed, stream,
                                              static_cast<uint64_t>(mg * t.rows + n));
                if (best_index < 0 || prefer(s, n, best_score, best_index)) {
                    best_score = s;
                    best_index = n;
                }
            }
        }
    }
}

template <int EPI, bool NORM, int MT, int NC>
__global__ __launch_bounds__(kThreads) void gemm_rows(const dlk_gemv_params launch) {
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    constexpr int RM = 16 * MT;            // staged activation rows
    constexpr int KC = chunk_k(MT);        // k per chunk
    constexpr int STRIDE = lds_stride(MT); // bf16 per staged row
    constexpr int STEPS = KC / 32;         // MFMA k-steps per chunk
    constexpr int COLS = KC / 4;           // staging: lanes per row (4 columns each)
    constexpr int ROWS_PER_PASS = kThreads / COLS;
    constexpr int XR = RM / ROWS_PER_PASS; // staging loads per thread per chunk
    static_assert(RM % ROWS_PER_PASS == 0, "staging covers the rows");
    // the dynamic LDS follows the static variables below: their sizes are multiples of 16 bytes, and the
    // alignment is stated, because its 128-bit reads run at half speed or worse when misaligned
    extern __shared__ __attribute__((aligned(16))) uint16_t lds[]; // [2 buffers][hi, lo][RM][STRIDE]
    __shared__ float row_squares[RM];
    __shared__ double pool_score[kWaves][RM];
    __shared__ int64_t pool_index[kWaves][RM];

    // A SwiGLU launch over more rows than one work-group's tiles may be split over the rows instead of the keys
    // (row_parts: part y takes rows RM y .. +RM with all of K; no partials, no reduce launch), as the host
    // splits a launch into 64-row chunks
    dlk_gemv_params p = launch;
    const bool by_rows = SWIGLU && launch.row_parts > 1;
    if (by_rows) {
        const int m0 = static_cast<int>(blockIdx.y) * RM;
        p.M = min(RM, launch.M - m0);
        p.x = launch.x + static_cast<int64_t>(m0) * launch.ldx;
        p.y = launch.y + static_cast<int64_t>(m0) * launch.ldy;
        p.m_base = launch.m_base + m0;
    }
    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int K = p.K, splits = by_rows ? 1 : gridDim.y, slice = K / splits, k_begin = by_rows ? 0 : blockIdx.y * slice;
    const int nchunks = slice / KC;
    const int tiles = tiles_of(p);
    const int my_tile = blockIdx.x * kWaves + wave;
    const bool active = my_tile < tiles;
    // idle waves of the last work-group stream a valid tile (unused) so no load sits in a branch
    const TileMap tm = locate<SWIGLU>(p, min(my_tile, tiles - 1));
    const uint16_t* wrow = tile_row<SWIGLU>(tm, lane % 16, K) + k_begin + 8 * (lane / 16);

    // staging: thread -> (column group c4, rows r0, r0 + ROWS_PER_PASS, ...)
    const int c4 = t % COLS, r0 = t / COLS;
    const bool norm = NORM && p.apply_norm;
    const bool affine = norm && p.norm_weight;
    const int esize = p.norm_bf16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t gres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(affine ? p.norm_weight : static_cast<const void*>(p.x)), 0, affine ? K * esize : 0,
        kBufferFlags);

    auto load_x = [&](int c, float4 (&xr)[XR], u32x4& graw) {
        const int k = k_begin + c * KC + 4 * c4;
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const int m = min(r0 + i * ROWS_PER_PASS, p.M - 1);
            xr[i] = *reinterpret_cast<const float4*>(p.x + static_cast<int64_t>(m) * p.ldx + k);
        }
        if constexpr (NORM) graw = __builtin_amdgcn_raw_buffer_load_b128(gres, k * esize, 0, 0);
    };
    float squares[XR];
#pragma unroll
    for (int i = 0; i < XR; ++i) squares[i] = 0.0f;
    auto stage = [&](int buf, const float4 (&xr)[XR], const u32x4& graw) {
        float g[4] = {1.0f, 1.0f, 1.0f, 1.0f};
        if constexpr (NORM && NC >= 4) {
            // selects, not branches: a load used only inside a branch is sunk into it by the compiler, issued
            // after the loads that follow it in the source, and its wait then drains those too (the deep
            // pipeline's prologue; the other variants measured faster with the branches)
            const float gb[4] = {bf16_lo(graw.x), bf16_hi(graw.x), bf16_lo(graw.y), bf16_hi(graw.y)};
            const float gf[4] = {__uint_as_float(graw.x), __uint_as_float(graw.y), __uint_as_float(graw.z),
                                 __uint_as_float(graw.w)};
#pragma unroll
            for (int i = 0; i < 4; ++i) g[i] = affine ? (p.norm_bf16 ? gb[i] : gf[i]) : 1.0f;
        } else if constexpr (NORM) {
            if (affine) {
                if (p.norm_bf16) {
                    g[0] = bf16_lo(graw.x); g[1] = bf16_hi(graw.x); g[2] = bf16_lo(graw.y); g[3] = bf16_hi(graw.y);
                } else {
                    g[0] = __uint_as_float(graw.x); g[1] = __uint_as_float(graw.y);
                    g[2] = __uint_as_float(graw.z); g[3] = __uint_as_float(graw.w);
                }
            }
        }
        uint16_t* hi = lds + buf * 2 * RM * STRIDE;
        uint16_t* lo = hi + RM * STRIDE;
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            const int m = r0 + i * ROWS_PER_PASS;
            float4 v = xr[i];
            if (m >= p.M) v = make_float4(0.f, 0.f, 0.f, 0.f);
            squares[i] += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
            const float e[4] = {v.x * g[0], v.y * g[1], v.z * g[2], v.w * g[3]};
            u32x2 h, l;
            split4_bf16(e, h, l);
            *reinterpret_cast<u32x2*>(hi + m * STRIDE + 4 * c4) = h;
            *reinterpret_cast<u32x2*>(lo + m * STRIDE + 4 * c4) = l;
        }
    };
    u32x4 wa[STEPS], wb[STEPS];
    // weights row-major (each load instruction reads 16 rows x 64 bytes), or repacked in MFMA tile order
    // (w_tiles: 1 KB per 16-row tile and k step, so each load instruction reads 1 KB contiguous; measured on
    // MI355X: a 1B decode step at batch 32 1.44 -> 1.33 ms, at batch 4 with LoRA 1.54 -> 1.34 ms)
    const uint16_t* wtiles = static_cast<const uint16_t*>(tm.seg == 0   ? p.w_tiles[0]
                                                          : tm.seg == 1 ? p.w_tiles[1]
                                                                        : p.w_tiles[2]);
    const uint16_t* wsrc = wrow;
    int chunk_stride = KC, step_stride = 32;
    if (wtiles) {
        const int local = SWIGLU ? tm.n0 / 8 : tm.n0 / kTile; // the tile within its segment
        wsrc = wtiles + (static_cast<int64_t>(local) * (K / 32) + k_begin / 32) * 512 + 8 * lane;
        chunk_stride = STEPS * 512;
        step_stride = 512;
    }
    auto load_w = [&](int c, u32x4 (&dst)[STEPS]) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s)
            dst[s] = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4*>(wsrc + c * chunk_stride + s * step_stride));
    };
    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buf, const u32x4 (&w)[STEPS]) {
        const uint16_t* hi = lds + buf * 2 * RM * STRIDE;
        const uint16_t* lo = hi + RM * STRIDE;
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
            const bf16x8 a = __builtin_bit_cast(bf16x8, w[s]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const int off = (16 * mt + lane % 16) * STRIDE + 32 * s + 8 * (lane / 16);
                const bf16x8 bh = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(hi + off));
                const bf16x8 bl = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(lo + off));
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh, acc[mt], 0, 0, 0);
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl, acc[mt], 0, 0, 0);
            }
        }
    };

    if constexpr (NC >= 4) {
        // Deep pipeline over a run of exactly NC chunks (the launch reads repacked weights): at step c the loads
        // of chunk c + A (A = kDeepAhead) are issued first, so the weights of c + 1 .. c + A stay in flight while
        // chunk c is used; a chunk's activations are issued before its weights, so waiting for the ones staged
        // next leaves the later weights in flight.  A + 1 register sets rotate with the steps; the run is unrolled
        // whole, so every wait counts exactly the loads issued after the one it needs.
        constexpr int A = kDeepAhead, SETS = A + 1, PRE = A < NC ? A : NC;
        float4 xs[SETS][XR];
        u32x4 gs[SETS], ws[SETS][STEPS];
        // the first chunks' activations, then their weights chunk by chunk, in that order (scheduling barriers
        // keep the compiler from interleaving them): the wait for chunk 0's activations leaves every weight load
        // in flight, and the one for chunk 0's weights those of the later chunks
#pragma unroll
        for (int c = 0; c < PRE; ++c) load_x(c, xs[c], gs[c]);
#pragma unroll
        for (int c = 0; c < PRE; ++c) {
            __builtin_amdgcn_sched_barrier(0);
            load_w(c, ws[c]);
        }
        __builtin_amdgcn_sched_barrier(0);
        stage(0, xs[0], gs[0]);
        gemv::lds_barrier();
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            if (c + A < NC) {
                load_x(c + A, xs[(c + A) % SETS], gs[(c + A) % SETS]);
                load_w(c + A, ws[(c + A) % SETS]);
            }
            compute(c % 2, ws[c % SETS]);
            if (c + 1 < NC) {
                stage((c + 1) % 2, xs[(c + 1) % SETS], gs[(c + 1) % SETS]);
                gemv::lds_barrier();
            }
        }
    } else if constexpr (NC == 2) {
        // every load of the run first (chunks past the run repeat its last chunk: loads stay unconditional, so
        // no branch drains them early), then the staging of the run's chunks into NC buffers and the products
        float4 xs[NC][XR];
        u32x4 gs[NC], ws[NC][STEPS];
#pragma unroll
        for (int c = 0; c < NC; ++c) load_x(min(c, nchunks - 1), xs[c], gs[c]);
#pragma unroll
        for (int c = 0; c < NC; ++c) load_w(min(c, nchunks - 1), ws[c]);
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (c < nchunks) stage(c, xs[c], gs[c]);
        gemv::lds_barrier();
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (c < nchunks) compute(c, ws[c]);
    } else {
        // Invariant at the top of each pair of chunks (c, c + 1): LDS buffer 0 holds chunk c, the registers hold
        // chunk c + 1's activations, and the weights of c (wa) and c + 1 (wb) are loaded or in flight.  Loads in
        // the loop are unconditional (a load on one path of a branch would drain every load at the next wait);
        // the last two or three chunks are peeled.  nchunks >= 2 (the host requires K >= 2 * chunk).
        float4 xr[XR];
        u32x4 graw;
        load_x(0, xr, graw);
        load_w(0, wa);
        stage(0, xr, graw);
        load_x(1, xr, graw);
        load_w(1, wb);
        gemv::lds_barrier();
        int c = 0;
        for (; c + 3 < nchunks; c += 2) {
            compute(0, wa);
            stage(1, xr, graw);
            load_x(c + 2, xr, graw);
            load_w(c + 2, wa);
            gemv::lds_barrier();
            compute(1, wb);
            stage(0, xr, graw);
            load_x(c + 3, xr, graw);
            load_w(c + 3, wb);
            gemv::lds_barrier();
        }
        compute(0, wa);     // chunk c
        stage(1, xr, graw); // chunk c + 1
        if (c + 2 < nchunks) {
            load_x(c + 2, xr, graw);
            load_w(c + 2, wa);
        }
        gemv::lds_barrier();
        compute(1, wb); // chunk c + 1
        if (c + 2 < nchunks) {
            stage(0, xr, graw);
            gemv::lds_barrier();
            compute(0, wa); // chunk c + 2
        }
    }

    // per-row norm factor: every row belongs to one staging pass row, summed across the lanes that staged it
    if (norm) {
#pragma unroll
        for (int i = 0; i < XR; ++i) {
            // lanes t with the same r0 staged disjoint columns of row r0 + i * ROWS_PER_PASS
            float s = squares[i];
            if constexpr (COLS == kWave) {
                s = wave_sum(s);
                if (lane == 0) row_squares[r0 + i * ROWS_PER_PASS] = s;
            } else {
                // COLS = 32 or 16 lanes per row: reduce within the row's lane group
#pragma unroll
                for (int off = COLS / 2; off > 0; off >>= 1) s += __shfl_xor(s, off, kWave);
                if (c4 == 0) row_squares[r0 + i * ROWS_PER_PASS] = s;
            }
        }
    }
    gemv::lds_barrier();

    const int q = lane / 16;
    if (splits > 1) {
        // key slice: raw partial dots and this slice's row sums of squares; gemm_reduce finishes them
        const int64_t width = static_cast<int64_t>(tiles) * kTile;
        float* part = p.split_partial + static_cast<int64_t>(blockIdx.y) * p.M * width;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const int m = 16 * mt + lane % 16;
            if (active && m < p.M)
#pragma unroll
                for (int j = 0; j < 4; ++j) part[m * width + my_tile * kTile + 4 * q + j] = acc[mt][j];
        }
        if (norm && blockIdx.x == 0 && t < p.M)
            p.split_partial[static_cast<int64_t>(splits) * p.M * width + blockIdx.y * p.M + t] = row_squares[t];
        return;
    }

    // epilogue: lane holds D[4q + j][m] of each activation tile
    uint64_t seed = p.key_seed, stream = p.key_stream;
    if constexpr (EPI == DLK_EPI_LOGITS) {
        if (p.sample_mode == 2 && p.key_label)
            fold_in(p.key_seed, p.key_stream, static_cast<uint64_t>(*p.key_label), seed, stream);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + lane % 16;
        double bs = 0.0;
        int64_t bi = -1;
        if (active && m < p.M) {
            const float inv = norm ? rsqrtf(row_squares[m] / static_cast<float>(K) + p.epsilon) : 1.0f;
            const float v[4] = {acc[mt][0] * inv * p.acc_scale, acc[mt][1] * inv * p.acc_scale,
                                acc[mt][2] * inv * p.acc_scale, acc[mt][3] * inv * p.acc_scale};
            lane_epilogue<EPI>(p, tm, q, m, v, bs, bi, seed, stream);
        }
        if constexpr (EPI == DLK_EPI_LOGITS) {
            // the 4 lanes of row m (q = 0..3) -> one candidate; then the 4 waves through LDS
#pragma unroll
            for (int off = 16; off < kWave; off <<= 1) {
                const double os = __shfl_xor(bs, off, kWave);
                const int64_t oi = __shfl_xor(bi, off, kWave);
                if (oi >= 0 && (bi < 0 || prefer(os, oi, bs, bi))) {
                    bs = os;
                    bi = oi;
                }
            }
            if (q == 0) {
                pool_score[wave][m] = bs;
                pool_index[wave][m] = bi;
            }
        }
    }
    if constexpr (EPI == DLK_EPI_LOGITS) {
        if (p.sample_mode != 0) {
            gemv::lds_barrier();
            if (wave == 0) {
                for (int m = lane; m < RM && m < p.M; m += kWave) {
                    double bs = 0.0;
                    int64_t bi = -1;
#pragma unroll
                    for (int w = 0; w < kWaves; ++w) {
                        const int64_t j = pool_index[w][m];
                        if (j >= 0 && (bi < 0 || prefer(pool_score[w][m], j, bs, bi))) {
                            bs = pool_score[w][m];
                            bi = j;
                        }
                    }
                    dlk_sample_partial out;
                    out.score = bs;
                    out.index = bi;
                    p.partial[(p.m_base + m) * p.partial_blocks + blockIdx.x] = out;
                }
            }
        }
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (p.bump_position && blockIdx.x == 0 && t == 0) *p.bump_position += p.bump_count;
    }
}

constexpr int kReduceThreads = 128;

// Second launch of a key-split projection: thread (m, tile, q) sums the S partial dots of tile rows 4q .. 4q+3
// for activation row m in slice order, applies the row's norm factor, and runs the lane epilogue.  All
// kMaxSplits slices' loads are issued at once through buffer ranges that end at the launch's S slices: loads
// past them read zero, and adding +0 after the S slices leaves every sum as the slice-order sum.
template <int EPI, bool NORM>
__global__ __launch_bounds__(kReduceThreads) void gemm_reduce(const dlk_gemv_params p, int splits) {
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    const int tiles = tiles_of(p);
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * kReduceThreads + threadIdx.x;
    const int q = static_cast<int>(idx % 4);
    const int tile = static_cast<int>((idx / 4) % tiles);
    const int m = static_cast<int>(idx / (4 * static_cast<int64_t>(tiles)));
    if (m < p.M) {
        const int width = tiles * kTile;
        const int plane = p.M * width; // floats per slice
        const __amdgpu_buffer_rsrc_t dots = __builtin_amdgcn_make_buffer_rsrc(
            p.split_partial, 0, splits * plane * static_cast<int>(sizeof(float)), kBufferFlags);
        const __amdgpu_buffer_rsrc_t sums = __builtin_amdgcn_make_buffer_rsrc(
            p.split_partial + static_cast<int64_t>(splits) * plane, 0, NORM ? splits * p.M * 4 : 0, kBufferFlags);
        const int offset = (m * width + tile * kTile + 4 * q) * static_cast<int>(sizeof(float));
        u32x4 part[kMaxSplits];
        float row[kMaxSplits];
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s)
            part[s] = __builtin_amdgcn_raw_buffer_load_b128(dots, offset + s * plane * 4, 0, 0);
        if constexpr (NORM) {
#pragma unroll
            for (int s = 0; s < kMaxSplits; ++s)
                row[s] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(sums, (s * p.M + m) * 4, 0, 0));
        }
        float v[4] = {0.f, 0.f, 0.f, 0.f};
        float squares = 0.0f;
#pragma unroll
        for (int s = 0; s < kMaxSplits; ++s) {
            v[0] += __uint_as_float(part[s].x);
            v[1] += __uint_as_float(part[s].y);
            v[2] += __uint_as_float(part[s].z);
            v[3] += __uint_as_float(part[s].w);
            if constexpr (NORM) squares += row[s];
        }
        const float inv = NORM && p.apply_norm ? rsqrtf(squares / static_cast<float>(p.K) + p.epsilon) : 1.0f;
#pragma unroll
        for (int j = 0; j < 4; ++j) v[j] *= inv * p.acc_scale;
        double bs = 0.0;
        int64_t bi = -1;
        lane_epilogue<EPI>(p, locate<SWIGLU>(p, tile), q, m, v, bs, bi, p.key_seed, p.key_stream);
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (p.bump_position && blockIdx.x == 0 && threadIdx.x == 0) *p.bump_position += p.bump_count;
    }
}


// Few weight tiles (a LoRA down projection: rank 16 per adapter) over several rows: one work-group per 16-row
// tile, whose kWideWaves waves split K (K / kWideWaves keys each, every load of the wave issued at once) and merge
// their dot products and row sums of squares in LDS in wave order; the first wave runs the lane epilogue.  One
// launch and one memory round trip, where the key-split kernel would take a split launch and a reduce launch for
// 2 tiles.  Each wave reads its activation fragments straight from memory (bf16 hi + lo in registers): the
// re-read of the activation rows by every work-group is what makes this shape lose at many tiles.
constexpr int kWideWaves = 16;
constexpr int kWideTiles = 4;

/// A residual launch of up to 128 tiles over 17-32 rows and K <= 2048 takes the wide kernel in row parts of 16
/// rows (measured on MI355X, O of the 1B model at batch 32: split + reduce 9.7 us -> 8.8 us)
inline bool wide_parts_eligible(const dlk_gemv_params& p) {
    return p.epilogue == DLK_EPI_RESIDUAL && p.M > 16 && p.M <= 32 && tiles_of(p) <= 128 && p.K <= 2048 &&
           p.K % (32 * kWideWaves) == 0 && p.ldx % 4 == 0;
}

inline bool wide_eligible(const dlk_gemv_params& p) {
    // Also over at most 16 rows and K <= 2048: a residual projection of up to 128 tiles, and a QKV projection of
    // up to 192 with unmerged LoRA (whose partials the attention cannot finish).  Measured on MI355X, the 1B model
    // with LoRA at batch 4: O 8.8 -> 6.3 us, QKV 11.7 -> 9.5 us, the step 1.333 -> 1.25 ms; at 32 rows, or
    // K = 5632, the key-split kernel stays faster.
    const bool lora = p.lora_up[0] || p.lora_up[2];
    const bool small_residual = (p.epilogue == DLK_EPI_RESIDUAL ? tiles_of(p) <= 128
                                 : p.epilogue == DLK_EPI_QKV && lora ? tiles_of(p) <= 192 : false) &&
                                p.M <= 16 && p.K <= 2048;
    return p.epilogue != DLK_EPI_LOGITS && (tiles_of(p) <= kWideTiles || small_residual) && p.M <= 32 &&
           p.K % (32 * kWideWaves) == 0 &&
           p.ldx % 4 == 0;
}

/// A QKV launch on the wide kernel over one activation tile with LoRA down rows (bf16, rank 4..16 in steps of 4,
/// 16-byte aligned rows) folds the down projections into its key loop.
inline bool lora_fold_eligible(const dlk_gemv_params& p) {
    const bool any = p.lora_down[0] || p.lora_down[2];
    const int r = p.lora_rank;
    if (p.epilogue != DLK_EPI_QKV || !any || p.lora_down[1] || p.M > 16 || !p.w_bf16 || p.acc_scale != 1.0f ||
        r < 4 || r > 16 || r % 4 != 0 || !wide_eligible(p))
        return false;
    for (int s = 0; s < 3; s += 2)
        if (p.lora_down[s] && (!p.lora_up[s] || p.lora_hidden[s] || reinterpret_cast<uintptr_t>(p.lora_down[s]) % 16 != 0 ||
                               reinterpret_cast<uintptr_t>(p.lora_up[s]) % 8 != 0))
            return false;
    return true;
}

template <int EPI, bool NORM, int MT>
__global__ __launch_bounds__(kWideWaves * kWave) void gemm_wide(const dlk_gemv_params launch) {
    // row_parts: work-group row y takes rows 16 MT y .. +16 MT of the launch (the length advances once)
    dlk_gemv_params p = launch;
    if (launch.row_parts > 1) {
        const int m0 = static_cast<int>(blockIdx.y) * 16 * MT;
        p.M = min(16 * MT, launch.M - m0);
        p.x = launch.x + static_cast<int64_t>(m0) * launch.ldx;
        p.y = launch.y ? launch.y + static_cast<int64_t>(m0) * launch.ldy : nullptr;
        p.residual = launch.residual ? launch.residual + static_cast<int64_t>(m0) * launch.ldres : nullptr;
        p.m_base = launch.m_base + m0;
        if (blockIdx.y != 0) p.bump_position = nullptr;
    }
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    constexpr int RM = 16 * MT;
    constexpr int D = MT == 1 ? 4 : 2; // k steps per batch of loads (within 128 registers at 16 waves)
    __shared__ float red[kWideWaves][MT][4][kWave];
    __shared__ float sq[kWideWaves][RM];
    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int K = p.K, tile = blockIdx.x;
    const int per = K / kWideWaves, steps = per / 32, kb = wave * per;
    const TileMap tm = locate<SWIGLU>(p, tile);
    const int i16 = lane % 16, g4 = lane / 16;
    // weights row-major (16 rows x 64 bytes per load instruction) or repacked in tile order (w_tiles: 1 KB)
    const uint16_t* wtiles = static_cast<const uint16_t*>(tm.seg == 0   ? p.w_tiles[0]
                                                          : tm.seg == 1 ? p.w_tiles[1]
                                                                        : p.w_tiles[2]);
    const uint16_t* wrow = tile_row<SWIGLU>(tm, i16, K) + kb + 8 * g4;
    int wstep = 32;
    if (wtiles) {
        const int local = SWIGLU ? tm.n0 / 8 : tm.n0 / kTile; // the tile within its segment
        wrow = wtiles + (static_cast<int64_t>(local) * (K / 32) + kb / 32) * 512 + 8 * lane;
        wstep = 512;
    }
    const bool norm = NORM && p.apply_norm;
    const bool affine = norm && p.norm_weight;
    const int esize = p.norm_bf16 ? 2 : 4;
    const __amdgpu_buffer_rsrc_t gres = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(affine ? p.norm_weight : static_cast<const void*>(p.x)), 0, affine ? K * esize : 0,
        kBufferFlags);
    const float* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        xrow[mt] = p.x + static_cast<int64_t>(min(16 * mt + i16, p.M - 1)) * p.ldx + kb + 8 * g4;
    f32x4 acc[MT];
    float squares[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        acc[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        squares[mt] = 0.f;
    }
    // Folded LoRA (QKV over one activation tile, lora_down set for this tile's segment): the down rows (rank <= 16:
    // one 16-row operand, rows past the rank repeat the last one) take the same activation fragments as the
    // weights, into a partial hidden tile H_w[r][m] over this wave's keys.  That accumulator's lane layout (rows
    // 4 (lane / 16) .. +3 of column lane % 16) is the B operand of the 16x16x16 MFMA, so the wave applies the up
    // rows to its own partial (up . H = sum over waves of up . H_w) and adds scale * up . H_w to acc before the
    // merge: no hidden rows in memory and no launch for them.  The norm factor and acc_scale then apply to both.
    constexpr bool FOLD = EPI == DLK_EPI_QKV && MT == 1;
    const uint16_t* drow = nullptr;
    u32x2 up_frag = {0u, 0u};
    f32x4 hacc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (FOLD) {
        const void* down = tm.seg == 0 ? p.lora_down[0] : tm.seg == 2 ? p.lora_down[2] : nullptr;
        if (down) {
            const int rank = p.lora_rank;
            drow = static_cast<const uint16_t*>(down) + static_cast<int64_t>(min(i16, rank - 1)) * K + kb + 8 * g4;
            // up rows n0 + lane % 16, ranks 4 (lane / 16) .. +3 (zero past the rank: the A operand)
            if (4 * g4 < rank)
                up_frag = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(tm.seg == 0 ? p.lora_up[0]
                                                                                                   : p.lora_up[2]) +
                                                          static_cast<int64_t>(tm.n0 + i16) * rank + 4 * g4);
        }
    }
    for (int s0 = 0; s0 < steps; s0 += D) {
        // the batch's loads first (steps past the wave's run repeat its last step and are not used)
        u32x4 wv[D], gv[D][2], dv[D];
        float4 xv[D][MT][2];
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int s = min(s0 + d, steps - 1);
            wv[d] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + wstep * s));
            dv[d] = u32x4{0u, 0u, 0u, 0u};
            if (FOLD && drow) dv[d] = *reinterpret_cast<const u32x4*>(drow + 32 * s);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                xv[d][mt][0] = *reinterpret_cast<const float4*>(xrow[mt] + 32 * s);
                xv[d][mt][1] = *reinterpret_cast<const float4*>(xrow[mt] + 32 * s + 4);
            }
            if constexpr (NORM) {
                const int k = kb + 8 * g4 + 32 * s;
                gv[d][0] = __builtin_amdgcn_raw_buffer_load_b128(gres, k * esize, 0, 0);
                gv[d][1] = __builtin_amdgcn_raw_buffer_load_b128(gres, p.norm_bf16 ? gemv::kOutOfRange : (k + 4) * 4, 0, 0);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (s0 + d >= steps) break;
            float g[8] = {1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f, 1.f};
            if constexpr (NORM) {
                if (affine) {
                    const u32x4 a = gv[d][0], c = gv[d][1];
                    if (p.norm_bf16) {
                        g[0] = bf16_lo(a.x); g[1] = bf16_hi(a.x); g[2] = bf16_lo(a.y); g[3] = bf16_hi(a.y);
                        g[4] = bf16_lo(a.z); g[5] = bf16_hi(a.z); g[6] = bf16_lo(a.w); g[7] = bf16_hi(a.w);
                    } else {
                        g[0] = __uint_as_float(a.x); g[1] = __uint_as_float(a.y); g[2] = __uint_as_float(a.z);
                        g[3] = __uint_as_float(a.w); g[4] = __uint_as_float(c.x); g[5] = __uint_as_float(c.y);
                        g[6] = __uint_as_float(c.z); g[7] = __uint_as_float(c.w);
                    }
                }
            }
            const bf16x8 a = __builtin_bit_cast(bf16x8, wv[d]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                float4 v0 = xv[d][mt][0], v1 = xv[d][mt][1];
                if (16 * mt + i16 >= p.M) v0 = v1 = make_float4(0.f, 0.f, 0.f, 0.f);
                squares[mt] += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w + v1.x * v1.x + v1.y * v1.y +
                               v1.z * v1.z + v1.w * v1.w;
                const float e0[4] = {v0.x * g[0], v0.y * g[1], v0.z * g[2], v0.w * g[3]};
                const float e1[4] = {v1.x * g[4], v1.y * g[5], v1.z * g[6], v1.w * g[7]};
                u32x2 h0, l0, h1, l1;
                split4_bf16(e0, h0, l0);
                split4_bf16(e1, h1, l1);
                const u32x4 hh = {h0.x, h0.y, h1.x, h1.y}, ll = {l0.x, l0.y, l1.x, l1.y};
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, hh), acc[mt], 0, 0, 0);
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, __builtin_bit_cast(bf16x8, ll), acc[mt], 0, 0, 0);
                if (FOLD && drow) {
                    const bf16x8 down = __builtin_bit_cast(bf16x8, dv[d]);
                    hacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(down, __builtin_bit_cast(bf16x8, hh), hacc, 0, 0, 0);
                    hacc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(down, __builtin_bit_cast(bf16x8, ll), hacc, 0, 0, 0);
                }
            }
        }
    }
    if (FOLD && drow) {
        // the partial hidden tile as bf16 hi + lo (to 2^-16 of itself), times the up rows
        const float h[4] = {hacc[0], hacc[1], hacc[2], hacc[3]};
        u32x2 hi, lo;
        split4_bf16(h, hi, lo);
        const s16x4 up = __builtin_bit_cast(s16x4, up_frag);
        f32x4 l = {0.f, 0.f, 0.f, 0.f};
        l = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(up, __builtin_bit_cast(s16x4, hi), l, 0, 0, 0);
        l = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(up, __builtin_bit_cast(s16x4, lo), l, 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[0][j] += p.lora_scale * l[j];
    }
    // merge the waves in wave order
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int j = 0; j < 4; ++j) red[wave][mt][j][lane] = acc[mt][j];
        float s = squares[mt];
        s += __shfl_xor(s, 16, kWave);
        s += __shfl_xor(s, 32, kWave);
        if (g4 == 0) sq[wave][16 * mt + i16] = s;
    }
    gemv::lds_barrier();
    if (wave != 0) return;
    double bs = 0.0;
    int64_t bi = -1;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + i16;
        float v[4] = {0.f, 0.f, 0.f, 0.f}, ss = 0.f;
        for (int w = 0; w < kWideWaves; ++w) {
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] += red[w][mt][j][lane];
            ss += sq[w][m];
        }
        if (m < p.M) {
            const float inv = norm ? rsqrtf(ss / static_cast<float>(K) + p.epsilon) : 1.0f;
            const float out[4] = {v[0] * inv * p.acc_scale, v[1] * inv * p.acc_scale, v[2] * inv * p.acc_scale,
                                  v[3] * inv * p.acc_scale};
            lane_epilogue<EPI>(p, tm, g4, m, out, bs, bi, p.key_seed, p.key_stream);
        }
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (p.bump_position && blockIdx.x == 0 && t == 0) *p.bump_position += p.bump_count;
    }
}

/// The reduce kernel of a key-split launch; {} if none.
template <int EPI>
gemv::Kernel resolve_reduce(const dlk_gemv_params& p) {
    if constexpr (EPI == DLK_EPI_LOGITS) {
        return {};
    } else {
        if (gemv::norm_variant(EPI, p.apply_norm != 0)) {
            if constexpr (EPI != DLK_EPI_RESIDUAL)
                return {reinterpret_cast<const void*>(&gemm_reduce<EPI, true>), 0};
            return {};
        }
        if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL)
            return {reinterpret_cast<const void*>(&gemm_reduce<EPI, false>), 0};
        return {};
    }
}

/// The matrix-core kernel for mt (1, 2 or 4) activation tiles and loop variant nc (loop_variant), or the few-tile
/// kernel (nc = -1, mt 1 or 2); {} if none.
template <int EPI>
gemv::Kernel resolve(const dlk_gemv_params& p, int mt, int nc) {
    auto pick = [&](auto norm) -> gemv::Kernel {
        constexpr bool N = decltype(norm)::value;
        if constexpr (EPI != DLK_EPI_LOGITS) {
            if (nc < 0) {
                if (mt == 1) return {reinterpret_cast<const void*>(&gemm_wide<EPI, N, 1>), 0};
                if (mt == 2) return {reinterpret_cast<const void*>(&gemm_wide<EPI, N, 2>), 0};
                return {};
            }
        }
#define DLK_GEMM_ROWS(MT, NC) {reinterpret_cast<const void*>(&gemm_rows<EPI, N, MT, NC>), lds_bytes(MT)}
        auto by_run = [&](auto mtc) -> gemv::Kernel {
            constexpr int MT = decltype(mtc)::value;
            switch (nc) {
            case 0: return DLK_GEMM_ROWS(MT, 0);
            case 2: return DLK_GEMM_ROWS(MT, 2);
            case 4: return DLK_GEMM_ROWS(MT, 4);
            case 8: return DLK_GEMM_ROWS(MT, 8);
            case 16: return DLK_GEMM_ROWS(MT, 16);
            case 32: return DLK_GEMM_ROWS(MT, 32);
            default: return {};
            }
        };
        switch (mt) {
        case 1: return by_run(std::integral_constant<int, 1>{});
        case 2: return by_run(std::integral_constant<int, 2>{});
        case 4: return by_run(std::integral_constant<int, 4>{});
        default: return {};
        }
#undef DLK_GEMM_ROWS
    };
    if (gemv::norm_variant(EPI, p.apply_norm != 0)) {
        if constexpr (EPI != DLK_EPI_RESIDUAL) return pick(std::true_type{});
        return {};
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) return pick(std::false_type{});
    return {};
}

} // namespace dlk::gemm

dlk::gemv::Kernel dlk_gemm_kernel_store(const dlk_gemv_params& p, int mt, int nc);
dlk::gemv::Kernel dlk_gemm_kernel_residual(const dlk_gemv_params& p, int mt, int nc);
dlk::gemv::Kernel dlk_gemm_kernel_qkv(const dlk_gemv_params& p, int mt, int nc);
dlk::gemv::Kernel dlk_gemm_kernel_swiglu(const dlk_gemv_params& p, int mt, int nc);
dlk::gemv::Kernel dlk_gemm_kernel_logits(const dlk_gemv_params& p, int mt, int nc);
dlk::gemv::Kernel dlk_gemm_reduce_store(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_gemm_reduce_residual(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_gemm_reduce_qkv(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_gemm_reduce_swiglu(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_gemm_reduce_logits(const dlk_gemv_params& p);
