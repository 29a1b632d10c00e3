// Projection over many activation rows (prefill chunks) on the matrix cores, with the epilogues of the GEMV
// (see dlk_gemv_params in kernels.h).  The decode-side kernel (gemm_rows.h) holds every activation row of a
// launch in one work-group and streams each weight row once; here both sides are tiled so that each weight
// tile is reused across 256 activation rows and each activation tile across 256 weight rows.
//
// Two launches.  prepare_rows writes the activation rows, times the fused RMSNorm weight, as bf16 pairs hi + lo
// (x = hi + lo to ~2^-16) into a staging workspace, with the per-row norm factors 1/sqrt(mean x^2 + eps).
// gemm_tiles then multiplies: every product is two MFMAs (hi and lo against the bf16 weight), so the result
// keeps f32-level accuracy, and the norm factor scales the finished dot products.
//
// Work-group: 8 waves (two per SIMD), output tile of 256 weight rows x 256 activation rows; wave (wn, wm) owns
// weight rows 128 wn .. +128 and activation rows 64 wm .. +64 as 8 x 4 v_mfma_f32_16x16x32_bf16 tiles with the
// operand roles of gemm_rows (A = 16 weight rows, B = 16 activation rows; lane l holds D[weight rows 4(l/16) ..
// +4][activation row l%16]), so the lane epilogue is shared.  SwiGLU blocks cover 128 features: 8 gate tiles
// and the 8 up tiles of the same features, a wave owning matching gate and up tiles, so silu(gate) * up pairs
// in the lane's own registers.
//
// Operands reach LDS by the 16-byte global->LDS DMA (lane i of a DMA instruction lands at LDS base + 16 i), in
// fragment order: for each 16-row tile and 32-wide k step the 16 bytes that MFMA lane l needs sit at 16 l, so the
// fragment reads are linear and conflict-free and no register staging is needed.  Two rings are in flight:
// weights two k pairs ahead (issued by waves 0-3), activations one k step ahead (waves 4-7).  The global->LDS
// traffic (48 KB per k step per work-group) and its latency are what bound the kernel, hence the largest tile the
// LDS rings and the registers hold.
//
// Blocks are placed XCD-aware: the hardware hands consecutive work-group ids to the 8 XCDs in turn, so block b
// runs on XCD b % 8, which takes a band of row blocks and walks it in small groups of row blocks column by
// column, so that the work-groups it runs at once share weight and activation slices in its L2.
#pragma once

#include "kernels/gemm_rows.h"

namespace dlk::tiles {

using gemm::bf16x4;
using gemm::bf16x8;
using gemm::f32x4;
using gemv::u32x4;
typedef float f32x8 __attribute__((ext_vector_type(8)));
constexpr int kThreads = 512;                      // 8 waves
constexpr int kWaves = kThreads / kWave;
constexpr int kPrepThreads = 256;                  // prepare_rows: one work-group per 16-row tile and k chunk
constexpr int kPrepChunk = 512;                    // k per prepare_rows work-group
constexpr int kBN = 256;                           // weight rows per work-group (16 tiles of 16)
constexpr int kBM = 256;                           // activation rows per work-group (16 tiles of 16)
constexpr int kActStages = 3;                      // activation ring: k steps of 32
constexpr int kActBytes = (kBM / 16) * 2048;       // one k step of activation fragments (hi, lo)
constexpr int kWeightStages = 2;                   // weight ring: k pairs (64)
constexpr int kWeightPairBytes = (kBN / 16) * 2048; // one k pair of weight fragments
constexpr size_t kLdsBytes = 0;                    // the rings are static LDS
constexpr int kActDma = 2 * (kBM / 16) / (kWaves / 2);   // activation DMA instructions per activation wave per k step
constexpr int kWeightDma = 2 * (kBN / 16) / (kWaves / 2); // weight DMA instructions per weight wave per k pair
static_assert(kActStages * kActBytes + kWeightStages * kWeightPairBytes <= 160 * 1024, "LDS");
constexpr int kMinBlocks = 64;                     // one row block of 256 takes the tiled path only this wide
constexpr int kXcds = 8;
static_assert(kActDma == 8 && kWeightDma == 8, "per wave: four activation tiles (hi, lo), four weight tiles (two halves)");

/// Staging workspace of a launch: the split rows in fragment order, then per-k-chunk sums of squares of each row
/// (f32 [ceil(K / 512)][M]; the norm factor of row m is 1/sqrt(sum over chunks / K + eps), summed in chunk order).
/// Fragment order: for each 16-row tile mt (rows up to M rounded to the 256-row block) and 32-wide k step s,
/// 1 KB of hi then 1 KB of lo, lane l's 16 bytes at 16 l holding row 16 mt + l%16, k 32 s + 8 (l/16) .. +8.  So
/// every activation DMA reads 1 KB contiguous (consecutive lanes, consecutive 16 bytes: whole 128-byte lines
/// per 8 lanes, the pattern the global->LDS path serves fastest).
__host__ __device__ inline int64_t stage_rows(int M) { return (static_cast<int64_t>(M) + 255) / 256 * 256; }
__host__ __device__ inline int prep_chunks(int K) { return (K + kPrepChunk - 1) / kPrepChunk; }
__host__ __device__ inline int64_t stage_bytes(const dlk_gemv_params& p) {
    return stage_rows(p.M) * p.K * 4 + static_cast<int64_t>(prep_chunks(p.K)) * p.M * 4;
}
__host__ __device__ inline const float* stage_squares(const dlk_gemv_params& p) {
    return reinterpret_cast<const float*>(static_cast<const char*>(p.stage) + stage_rows(p.M) * p.K * 4);
}
/// Norm factor of row m (0 <= m < M) from the chunk sums, in chunk order.
__device__ __forceinline__ float stage_inv(const dlk_gemv_params& p, int m) {
    const float* sq = stage_squares(p);
    const int chunks = prep_chunks(p.K);
    float total = 0.0f;
    for (int c = 0; c < chunks; ++c) total += sq[static_cast<int64_t>(c) * p.M + m];
    return rsqrtf(total / static_cast<float>(p.K) + p.epsilon);
}

/// Weight-row blocks of a launch: 16 tiles of 16 rows; SwiGLU: 128 features (8 gate tiles + 8 up tiles).
__host__ __device__ inline int col_blocks(const dlk_gemv_params& p) {
    if (p.epilogue == DLK_EPI_SWIGLU) return (p.seg_rows[0] + 127) / 128;
    return (gemm::tiles_of(p) + 15) / 16;
}
__host__ __device__ inline int row_blocks(const dlk_gemv_params& p) { return (p.M + kBM - 1) / kBM; }

/// Whether the shape suits the tiled path (host side): bf16 weights, whole k pairs, tile-shaped segments, rows
/// that prepare_rows reads as float4, and two or more row blocks (or one with a wide weight): narrower launches of
/// that many rows would take gemm_rows 64 rows at a time, re-streaming the weights and under-filling the device.
inline bool shape_eligible(const dlk_gemv_params& p) {
    if (!p.w_bf16 || p.epilogue == DLK_EPI_LOGITS || p.K % 64 != 0 || p.M < kBM) return false;
    if (p.ldx % 4 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
    if ((p.epilogue == DLK_EPI_STORE || p.epilogue == DLK_EPI_RESIDUAL || p.epilogue == DLK_EPI_SWIGLU) &&
        (p.ldy % 4 != 0 || reinterpret_cast<uintptr_t>(p.y) % 16 != 0)) return false; // 16-byte output stores
    if (p.epilogue == DLK_EPI_RESIDUAL && (p.ldres % 4 != 0 || reinterpret_cast<uintptr_t>(p.residual) % 16 != 0))
        return false;
    if (p.epilogue == DLK_EPI_QKV &&
        (p.head_dim % 4 != 0 || p.ldy % 4 != 0 || reinterpret_cast<uintptr_t>(p.y) % 16 != 0 ||
         reinterpret_cast<uintptr_t>(p.cosine) % 8 != 0 || reinterpret_cast<uintptr_t>(p.sine) % 8 != 0 ||
         reinterpret_cast<uintptr_t>(p.k_cache) % 16 != 0 || reinterpret_cast<uintptr_t>(p.v_cache) % 16 != 0))
        return false; // vector stores of four head-dim entries
    if (static_cast<int64_t>(kBM) * p.K * 2 >= (int64_t(1) << 31)) return false; // 32-bit DMA lane offsets
    for (int s = 0; s < p.nseg; ++s)
        if (p.seg_rows[s] % gemm::kTile != 0) return false;
    return row_blocks(p) >= 2 || col_blocks(p) >= kMinBlocks;
}

/// The tiled path runs when the shape suits it and the caller attached the staging workspace.
inline bool eligible(const dlk_gemv_params& p) {
    return shape_eligible(p) && p.stage && p.stage_bytes >= stage_bytes(p) &&
           reinterpret_cast<uintptr_t>(p.stage) % 16 == 0;
}

// Work-group barrier for the DMA ring: the caller has waited for its own DMA; no fence (a fence over LDS would
// wait for every DMA in flight).  The empty asm keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void ring_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// First weight row of work-group tile T (0..15).  Generic: global tile 16 n_blk + T, located across the
// segments (past the last tile: the last tile).  SwiGLU: T < 8 gate rows, T >= 8 up rows, both of features
// 128 n_blk + 16 (T % 8) (past the last feature: the last 16).
template <bool SWIGLU>
__device__ __forceinline__ const char* tile_base(const dlk_gemv_params& p, int n_blk, int T, int tiles) {
    if constexpr (SWIGLU) {
        const int f = min(128 * n_blk + 16 * (T % 8), p.seg_rows[0] - 16);
        return static_cast<const char*>(p.w[T < 8 ? 0 : 1]) + static_cast<int64_t>(f) * p.K * 2;
    } else {
        const gemm::TileMap tm = gemm::locate<false>(p, min(16 * n_blk + T, tiles - 1));
        return reinterpret_cast<const char*>(tm.base0 + static_cast<int64_t>(tm.n0) * p.K);
    }
}

// Preparation launch: work-group (mt, c) splits rows 16 mt .. +16 over k chunk c (512 wide).  Wave w takes the
// chunk's k steps w, w + 4, ...; lane l (row 16 mt + l % 16, k 32 s + 8 (l / 16) .. +8) writes hi + lo = x * g
// (bf16 pair, the remainder rounded once more) at 16 l of the step's two 1 KB blocks, so every wave writes whole
// 1 KB blocks.  With the norm the work-group writes the chunk's sum of squares of x (f32) for each row.
template <bool NORM>
__global__ __launch_bounds__(kPrepThreads) void prepare_rows(const dlk_gemv_params p) {
    constexpr int kPrepWaves = kPrepThreads / kWave;
    __shared__ float partial[kPrepWaves][16];
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave, K = p.K, nsteps = K / 32;
    const int mt = blockIdx.x, chunk = blockIdx.y, r = lane % 16, q = lane / 16;
    const float* x = p.x + static_cast<int64_t>(min(16 * mt + r, p.M - 1)) * p.ldx; // rows past M repeat the last
    char* tile = static_cast<char*>(p.stage) + static_cast<int64_t>(mt) * nsteps * 2048 + 16 * lane;
    const bool affine = NORM && p.apply_norm && p.norm_weight;
    const int s_end = min(nsteps, (chunk + 1) * (kPrepChunk / 32));
    float squares = 0.0f;
    for (int s = chunk * (kPrepChunk / 32) + wave; s < s_end; s += kPrepWaves) {
        const int k = 32 * s + 8 * q;
        const float4 a = *reinterpret_cast<const float4*>(x + k);
        const float4 b = *reinterpret_cast<const float4*>(x + k + 4);
        f32x8 v = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if constexpr (NORM) {
            const f32x8 v2 = v * v;
            squares += ((v2[0] + v2[1]) + (v2[2] + v2[3])) + ((v2[4] + v2[5]) + (v2[6] + v2[7]));
            if (affine) {
                f32x8 g;
                if (p.norm_bf16) {
                    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.norm_weight) + k);
                    g = f32x8{bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y),
                              bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w)};
                } else {
                    const float4 g0 = *reinterpret_cast<const float4*>(static_cast<const float*>(p.norm_weight) + k);
                    const float4 g1 =
                        *reinterpret_cast<const float4*>(static_cast<const float*>(p.norm_weight) + k + 4);
                    g = f32x8{g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
                }
                v = v * g;
            }
        }
        const bf16x8 h = __builtin_convertvector(v, bf16x8);
        const bf16x8 l = __builtin_convertvector(v - __builtin_convertvector(h, f32x8), bf16x8);
        *reinterpret_cast<bf16x8*>(tile + static_cast<int64_t>(s) * 2048) = h;
        *reinterpret_cast<bf16x8*>(tile + static_cast<int64_t>(s) * 2048 + 1024) = l;
    }
    if constexpr (NORM) {
        if (p.apply_norm) {
            // lanes r, r + 16, r + 32, r + 48 hold four k quarters of row r; then the waves through LDS
            squares += __shfl_xor(squares, 16, kWave);
            squares += __shfl_xor(squares, 32, kWave);
            if (q == 0) partial[wave][r] = squares;
            gemv::lds_barrier();
            const int m = 16 * mt + t;
            if (t < 16 && m < p.M) {
                float total = 0.0f;
#pragma unroll
                for (int w = 0; w < kPrepWaves; ++w) total += partial[w][t];
                const_cast<float*>(stage_squares(p))[static_cast<int64_t>(chunk) * p.M + m] = total;
            }
        }
    }
}

template <int EPI, bool NORM>
__global__ __launch_bounds__(kThreads, 1) void gemm_tiles(const dlk_gemv_params p) {
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    __shared__ __attribute__((aligned(1024))) char wring[kWeightStages][kWeightPairBytes];
    __shared__ __attribute__((aligned(1024))) char xring[kActStages][kActBytes];

    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int K = p.K, nsteps = K / 32;
    const int tiles = gemm::tiles_of(p);
    const int nb = col_blocks(p), total = nb * row_blocks(p);

    // XCD-aware placement: XCD x runs logical tiles [start_x, start_x + count_x).  When the row blocks divide
    // evenly over the XCDs, that range is a band of whole row blocks, and the XCD walks it in groups of GR row
    // blocks, column by column: its 32 resident work-groups then cover 32 / GR weight blocks and GR row blocks, so
    // a k step's weight slice is shared by GR of them and its activation slice by 32 / GR (in row order: weights
    // by none, activations by all 32), and a work-group's share of the L2 misses per k step falls from 17 KB to
    // 8 KB at GR = 4.  Measured (C5 prefill, A/B against two byte-identical builds): 58.4-58.7 -> 57.6-57.8 ms at
    // GR 4 or 2, 57.9-58.3 at 8.
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = blockIdx.x % kXcds, idx = blockIdx.x / kXcds;
    const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
    int n_blk = logical % nb, m_blk = logical / nb;
    const int band_rows = row_blocks(p) % kXcds == 0 ? row_blocks(p) / kXcds : 0;
    const int GR = band_rows % 4 == 0 ? 4 : band_rows % 2 == 0 ? 2 : 1;
    if (band_rows > 0 && GR > 1) {
        const int group = idx / (GR * nb), within = idx % (GR * nb);
        n_blk = within / GR;
        m_blk = band_rows * xcd + group * GR + within % GR;
    }
    const int m_first = m_blk * kBM;

    // Weights: a 64-wide k pair of a 16-row tile is 2 KB of LDS, two halves of 8 rows x 128 bytes; each DMA
    // instruction reads 8 whole 128-byte lines (8 lanes per row), which the global->LDS path serves ~3.7x faster
    // than 16 half lines.  Row R of the tile keeps its 16-byte column g at slot g ^ (R >> 1) (XOR swizzle), so
    // the 16 lanes of an MFMA fragment read (rows 0..15, one column) hit 16 different bank groups.
    //
    // Waves 0-3 issue the weight DMAs and waves 4-7 the activation DMAs, so that each wave's in-order count of
    // loads in flight tracks one stream: a weight wave can wait for pair p while pair p + 1 stays in flight, with
    // no activation request behind it.  Weight wave r fills tiles 4r .. +4 (both halves), activation wave r
    // activation tiles 4r .. +4 (hi and lo).
    const bool weight_wave = wave < kWaves / 2;
    const int role = weight_wave ? wave : wave - kWaves / 2;
    const char* wbase[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) wbase[j] = tile_base<SWIGLU>(p, n_blk, 4 * role + j, tiles);
    uint32_t woff[2]; // per half h: lane i -> row 8 h + i / 8, slot i % 8 <- column (i % 8) ^ ((8 h + i / 8) >> 1)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int R = 8 * h + lane / 8;
        woff[h] = static_cast<uint32_t>(R) * K * 2 + 16 * ((lane % 8) ^ (R >> 1));
    }
    // activation tiles in the staging workspace's fragment order: (tile, step) is 2 KB (hi, lo) at
    // ((tile * nsteps) + step) * 2048 (rows past M hold whatever was there: their results are never stored)
    const char* xbase[4];
#pragma unroll
    for (int h = 0; h < 4; ++h)
        xbase[h] = static_cast<const char*>(p.stage) + static_cast<int64_t>(m_first / 16 + 4 * role + h) * nsteps * 2048;
    const uint32_t xoff = 16 * lane;
    // half H (0, 1) of a weight wave's share of pair `pair`: tiles 4r + 2H, 4r + 2H + 1
    auto issue_weights = [&](int pair, auto half_tag, char* buf) {
        constexpr int H = decltype(half_tag)::value;
        const uint32_t b = lds_offset(buf);
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                dma16(wbase[2 * H + j] + 128 * pair, woff[h], b + (4 * role + 2 * H + j) * 2048 + h * 1024);
    };
    auto issue_acts = [&](int step, char* buf) {
        const uint32_t b = lds_offset(buf);
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            const uint32_t dst = b + (4 * role + h) * 2048;
            dma16(xbase[h] + 2048 * step, xoff, dst);
            dma16(xbase[h] + 2048 * step + 1024, xoff, dst + 1024);
        }
    };

    // wave (wn, wm): activation tiles 4 wm .. +4; weight tiles: generic 8 wn .. +8, SwiGLU gate tiles 4 wn .. +4
    // then the up tiles 8 + 4 wn .. +4 (so slot i and i + 4 hold gate and up of the same features)
    const int wn = wave & 1, wm = wave >> 1;
    auto slot_tile = [&](int i) { return SWIGLU ? (i < 4 ? 4 * wn + i : 8 + 4 * wn + (i - 4)) : 8 * wn + i; };
    f32x4 acc[8][4];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // weight fragment of k step s' (0, 1) of the pair: row R = lane % 16, column 4 s' + lane / 16, swizzled
    const int R = lane % 16;
    uint32_t wfrag[2];
#pragma unroll
    for (int sp = 0; sp < 2; ++sp) wfrag[sp] = (R / 8) * 1024 + (R % 8) * 128 + 16 * ((4 * sp + lane / 16) ^ (R >> 1));
    // full: every weight tile of the column block exists, so the products need no per-tile check and form one
    // basic block that the scheduler interleaves with the fragment reads (the check's branches split it)
    auto compute = [&](const char* wbuf, int sp, const char* xbuf, auto full) {
        constexpr bool FULL = decltype(full)::value;
        bf16x8 bh[4], bl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const char* frag = xbuf + (4 * wm + j) * 2048 + 16 * lane;
            bh[j] = *reinterpret_cast<const bf16x8*>(frag);
            bl[j] = *reinterpret_cast<const bf16x8*>(frag + 1024);
        }
        // all eight weight fragments before the products (the LDS slots of tiles past the end hold repeats of
        // the last tile, so every read is in bounds)
        bf16x8 a[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) a[i] = *reinterpret_cast<const bf16x8*>(wbuf + slot_tile(i) * 2048 + wfrag[sp]);
        __builtin_amdgcn_sched_barrier(0); // keeps the scheduler from sinking the reads to their first use
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // weight tiles past the end (a narrow launch): no products for them
            if (!SWIGLU && !FULL && 16 * n_blk + slot_tile(i) >= tiles) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[i], bl[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    // Two rings.  Activations: three buffers of one k step; an activation wave issues step c + 2 right after
    // the barrier of step c (into the buffer of step c - 1, which every wave finished before that barrier) and
    // before the next barrier waits until only those DMAs are in flight, so step c + 1 has landed: two steps of
    // lead.  Weights: two buffers of one k pair; a weight wave issues pair p + 1 after its products of step 2p,
    // into the buffer of pair p - 1, and waits for it at the end of step 2p + 1: about one and a half steps of
    // lead.  (The other split of the 160 KB, three weight pairs two pairs ahead and two activation steps one
    // ahead, measured slower: the activation slices the work-groups of a group share wait on each other's L2
    // misses.)  Issues past the end repeat the last pair or step into a buffer nobody reads again, keeping the
    // counts uniform.  A SIMD holds waves w and w + 4, one of each kind, so one issues its DMAs before its
    // products and the other after them.  nsteps is even.
    const int npairs = nsteps / 2;
    using H0 = std::integral_constant<int, 0>;
    using H1 = std::integral_constant<int, 1>;
    if (weight_wave) {
        issue_weights(0, H0{}, wring[0]);
        issue_weights(0, H1{}, wring[0]);
        wait_vm<0>();
    } else {
        issue_acts(0, xring[0]);
        issue_acts(min(1, nsteps - 1), xring[1]);
        wait_vm<kActDma>();
    }
    ring_barrier();
    auto run = [&](auto full) {
        int wb = 0, xs = 0; // buffers of the current pair and of its first step
        for (int c = 0; c < nsteps; c += 2) {
            const int pair = c / 2;
            const int x1 = xs == 2 ? 0 : xs + 1, x2 = x1 == 2 ? 0 : x1 + 1;
            // even step c
            if (!weight_wave) issue_acts(min(c + 2, nsteps - 1), xring[x2]);
            compute(wring[wb], 0, xring[xs], full);
            if (weight_wave) {
                issue_weights(min(pair + 1, npairs - 1), H0{}, wring[1 - wb]);
                issue_weights(min(pair + 1, npairs - 1), H1{}, wring[1 - wb]);
            } else {
                wait_vm<kActDma>();
            }
            ring_barrier();
            // odd step c + 1 (step c + 3 takes the buffer of step c)
            if (!weight_wave) issue_acts(min(c + 3, nsteps - 1), xring[xs]);
            compute(wring[wb], 1, xring[x1], full);
            if (weight_wave) {
                wait_vm<0>();
            } else {
                wait_vm<kActDma>();
            }
            ring_barrier();
            wb = 1 - wb;
            xs = x2;
        }
    };
    if (SWIGLU || 16 * (n_blk + 1) <= tiles)
        run(std::true_type{});
    else
        run(std::false_type{}); // the last column block of a launch whose tiles do not fill it
    wait_vm<0>();

    const bool norm = NORM && p.apply_norm;
    float inv[4] = {1.f, 1.f, 1.f, 1.f};
    if (norm) {
#pragma unroll
        for (int j = 0; j < 4; ++j) inv[j] = stage_inv(p, min(m_first + 64 * wm + 16 * j + lane % 16, p.M - 1));
    }

    const int q = lane / 16;
    if constexpr (SWIGLU) {
        // lane holds gate (slot i) and up (slot i + 4) of features 128 n_blk + 16 (4 wn + i) + 4 q .. +4.  With
        // stage_out the four products go to the next launch's staging layout (feature f = its k): hi and lo of
        // row m, k step f / 32, lane (m % 16) + 16 ((f % 32) / 8), elements f % 8 .. +4, the split that
        // prepare_rows would make of the f32 rows.  Rows from M up to the 256-row block hold the products of the
        // staged rows past M (copies of row M - 1), as prepare_rows writes them.
        const int out_steps = p.seg_rows[0] / 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 128 * n_blk + 16 * (4 * wn + i) + 4 * q;
            if (f >= p.seg_rows[0]) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m_first + 64 * wm + 16 * j + lane % 16;
                if (m >= p.M && !p.stage_out) continue;
                const float scale = inv[j] * p.acc_scale;
                float o[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) o[r] = gemv::silu(acc[i][j][r] * scale) * (acc[i + 4][j][r] * scale);
                if (p.stage_out) {
                    const f32x4 v = {o[0], o[1], o[2], o[3]};
                    const bf16x4 h = __builtin_convertvector(v, bf16x4);
                    const bf16x4 l = __builtin_convertvector(v - __builtin_convertvector(h, f32x4), bf16x4);
                    char* at = static_cast<char*>(p.stage_out) +
                               (static_cast<int64_t>(m / 16) * out_steps + f / 32) * 2048 +
                               ((m % 16) + 16 * ((f % 32) / 8)) * 16 + (f % 8) * 2;
                    *reinterpret_cast<bf16x4*>(at) = h;
                    *reinterpret_cast<bf16x4*>(at + 1024) = l;
                } else {
                    *reinterpret_cast<float4*>(p.y + static_cast<int64_t>(m) * p.ldy + f) =
                        make_float4(o[0], o[1], o[2], o[3]);
                }
            }
        }
    } else {
        // QKV with LoRA of rank <= 32 (a multiple of 8): the rank-r products up[n, :] . hidden[m, :] of each output
        // tile are one more pair of MFMAs, with A = the tile's up rows (k padded with zeros to 32) and B = the
        // hidden rows split into hi + lo; D lands in the accumulator layout
        const bool lora_mfma = EPI == DLK_EPI_QKV && p.lora_rank > 0 && p.lora_rank <= 32 && p.lora_rank % 8 == 0;
        const bool lane_k = 8 * q < p.lora_rank; // lanes whose k slots hold rank entries
        // fully unrolled: acc is only ever indexed with constants (a runtime index puts it in scratch memory)
        const int64_t first_pos = EPI == DLK_EPI_QKV ? *p.position : 0;
#pragma clang loop unroll(full)
        for (int j = 0; j < 4; ++j) {
            const int ml = 64 * wm + 16 * j + lane % 16, m = m_first + ml;
            const float scale = inv[j] * p.acc_scale;
            gemm::RowPosition where = {0, 0, false};
            if constexpr (EPI == DLK_EPI_QKV) {
                const int64_t mg = p.m_base + m;
                where = {mg / p.length, first_pos + mg % p.length, true};
            }
            // hidden fragments of segments 0 (q) and 2 (v); the kernel-argument arrays and these are only indexed
            // with constants or selects (a runtime index would copy them to scratch memory)
            bf16x8 hh[2] = {}, hl[2] = {};
            if constexpr (EPI == DLK_EPI_QKV) {
                if (lora_mfma) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float* hidden = h == 0 ? p.lora_hidden[0] : p.lora_hidden[2];
                        if (!hidden) continue;
                        const float* row = hidden + (p.m_base + min(m, p.M - 1)) * gemv::lora_stride(p) + 8 * (lane_k ? q : 0);
                        const float4 a = *reinterpret_cast<const float4*>(row);
                        const float4 c = *reinterpret_cast<const float4*>(row + 4);
                        f32x8 x = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
                        if (!lane_k) x = f32x8{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                        hh[h] = __builtin_convertvector(x, bf16x8);
                        hl[h] = __builtin_convertvector(x - __builtin_convertvector(hh[h], f32x8), bf16x8);
                    }
                }
            }
            // the operands of four tiles at a time (up rows, rotation, residual) are loaded before their first
            // store: a load issued after a store waits for it (the outputs may alias the operands as far as the
            // compiler knows), so loads between the stores would cost a memory round trip per tile, with the
            // CU's matrix cores idle until the work-group ends (four, not eight: the QKV variant's registers)
#pragma clang loop unroll(full)
            for (int half = 0; half < 2; ++half) {
            u32x4 up_rows[4];
            float4 residual[4];
            float2 rot_c[4], rot_s[4];
#pragma clang loop unroll(full)
            for (int h = 0; h < 4; ++h) {
                const int i = 4 * half + h;
                up_rows[h] = u32x4{0u, 0u, 0u, 0u};
                residual[h] = make_float4(0.f, 0.f, 0.f, 0.f);
                rot_c[h] = rot_s[h] = make_float2(0.f, 0.f);
                const int tile = 16 * n_blk + 8 * wn + i;
                if (tile >= tiles) continue;
                const gemm::TileMap tm = gemm::locate<false>(p, tile);
                if constexpr (EPI == DLK_EPI_QKV) {
                    const bool vseg = tm.seg == 2;
                    // lanes whose k slots are past the rank keep zeros (the padding of the up operand)
                    if (lora_mfma && lane_k && tm.seg != 1 && (vseg ? p.lora_hidden[2] : p.lora_hidden[0]))
                        up_rows[h] = *reinterpret_cast<const u32x4*>(
                            static_cast<const uint16_t*>(vseg ? p.lora_up[2] : p.lora_up[0]) +
                            static_cast<int64_t>(tm.n0 + lane % 16) * p.lora_rank + 8 * q);
                    if (tm.seg < 2 && m < p.M) {
                        const int64_t table = where.position * (p.head_dim / 2) + ((tm.n0 + 4 * q) % p.head_dim) / 2;
                        rot_c[h] = *reinterpret_cast<const float2*>(p.cosine + table);
                        rot_s[h] = *reinterpret_cast<const float2*>(p.sine + table);
                    }
                }
                if constexpr (EPI == DLK_EPI_RESIDUAL) {
                    if (m < p.M)
                        residual[h] = *reinterpret_cast<const float4*>(p.residual + static_cast<int64_t>(m) * p.ldres +
                                                                       tm.n0 + 4 * q);
                }
            }
#pragma clang loop unroll(full)
            for (int h = 0; h < 4; ++h) {
                const int i = 4 * half + h;
                const int tile = 16 * n_blk + 8 * wn + i;
                if (tile >= tiles) continue; // wave-uniform: the MFMA below takes operands from every lane
                const gemm::TileMap tm = gemm::locate<false>(p, tile);
                const float v[4] = {acc[i][j][0] * scale, acc[i][j][1] * scale, acc[i][j][2] * scale,
                                    acc[i][j][3] * scale};
                double bs = 0.0;
                int64_t bi = -1;
                gemm::LoraProducts lora = {{0.f, 0.f, 0.f, 0.f}, false};
                if constexpr (EPI == DLK_EPI_QKV) {
                    const bool vseg = tm.seg == 2;
                    if (lora_mfma && tm.seg != 1 && (vseg ? p.lora_hidden[2] : p.lora_hidden[0])) {
                        const bf16x8 a = __builtin_bit_cast(bf16x8, up_rows[h]);
                        f32x4 d = {0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, vseg ? hh[1] : hh[0], d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, vseg ? hl[1] : hl[0], d, 0, 0, 0);
                        lora = {{d[0], d[1], d[2], d[3]}, true};
                    }
                }
                if (m >= p.M) continue;
                if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
                    if (EPI == DLK_EPI_RESIDUAL || !p.bias) {
                        // four consecutive outputs of row m: one 16-byte store (and residual load)
                        const int n = (EPI == DLK_EPI_STORE ? gemv::seg_column(p, tm.seg) : 0) + tm.n0 + 4 * q;
                        float4 out = make_float4(v[0], v[1], v[2], v[3]);
                        if constexpr (EPI == DLK_EPI_RESIDUAL) {
                            const float4 r = residual[h];
                            out.x += r.x; out.y += r.y; out.z += r.z; out.w += r.w;
                        }
                        *reinterpret_cast<float4*>(p.y + static_cast<int64_t>(m) * p.ldy + n) = out;
                        continue;
                    }
                }
                if constexpr (EPI == DLK_EPI_QKV) {
                    // four consecutive head-dim entries d .. d+3 of one head: LoRA, RoPE on the pairs (d, d+1),
                    // (d+2, d+3) (interleaved, src/ops/contraction.cpp:44-49), then one 16-byte q store or one
                    // 8-byte (bf16) / 16-byte (f32) K or V cache store
                    const int n = tm.n0 + 4 * q, hd = p.head_dim, d = n % hd, head = n / hd;
                    float o[4] = {v[0], v[1], v[2], v[3]};
                    if (lora.set) {
#pragma unroll
                        for (int r = 0; r < 4; ++r) o[r] += lora.v[r] * p.lora_scale;
                    } else if (tm.seg != 1 && (tm.seg == 0 ? p.lora_hidden[0] : p.lora_hidden[2])) {
                        gemm::lane_epilogue<EPI>(p, tm, q, m, v, bs, bi, p.key_seed, p.key_stream, lora, where);
                        continue; // ranks the MFMA pair does not take: the scalar path
                    }
                    if (tm.seg < 2) {
                        const float2 c = rot_c[h], sn = rot_s[h];
                        const float e0 = o[0] * c.x - o[1] * sn.x, o0 = o[0] * sn.x + o[1] * c.x;
                        const float e1 = o[2] * c.y - o[3] * sn.y, o1 = o[2] * sn.y + o[3] * c.y;
                        o[0] = e0; o[1] = o0; o[2] = e1; o[3] = o1;
                    }
                    if (tm.seg == 0) {
                        *reinterpret_cast<float4*>(p.y + (p.m_base + m) * p.ldy + n) = make_float4(o[0], o[1], o[2], o[3]);
                    } else {
                        const int64_t index = ((where.batch * p.kv_heads + head) * p.cache_capacity + where.position) * hd + d;
                        void* cache = tm.seg == 1 ? p.k_cache : p.v_cache;
                        if (p.cache_bf16)
                            *reinterpret_cast<uint2*>(static_cast<uint16_t*>(cache) + index) =
                                make_uint2(f32_to_bf16(o[0]) | (static_cast<uint32_t>(f32_to_bf16(o[1])) << 16),
                                           f32_to_bf16(o[2]) | (static_cast<uint32_t>(f32_to_bf16(o[3])) << 16));
                        else
                            *reinterpret_cast<float4*>(static_cast<float*>(cache) + index) = make_float4(o[0], o[1], o[2], o[3]);
                    }
                    continue;
                }
                gemm::lane_epilogue<EPI>(p, tm, q, m, v, bs, bi, p.key_seed, p.key_stream, lora, where);
            }
            }
        }
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (p.bump_position && blockIdx.x == 0 && t == 0) *p.bump_position += p.bump_count;
    }
}

// Narrow projections over staged rows (STORE, at most two 16-row weight tiles: the LoRA down projections of q and v,
// 2 x 16 rows): gemm_tiles would give each 256-row block one work-group of mostly idle waves (64 work-groups for
// 16384 rows, streaming the rows at ~2 TB/s).  Here each wave takes one 16-row tile of the staged rows and reads
// its hi and lo fragments straight from the staging workspace (1 KB contiguous per fragment, no LDS), with the
// weight fragments (a few KB per k step, hot in the L2) from the weights as stored; the norm factor scales the
// finished dots as in gemm_tiles.
constexpr int kNarrowWaves = 4; // waves (16-row tiles) per work-group
constexpr int kNarrowBatch = 4; // k steps per batch of loads (two batches in flight)

/// Whether a tiled-eligible launch takes gemm_narrow (host side).
inline bool narrow_eligible(const dlk_gemv_params& p) {
    return p.epilogue == DLK_EPI_STORE && !p.bias && gemm::tiles_of(p) <= 2;
}

template <bool NORM>
__global__ __launch_bounds__(kNarrowWaves * kWave) void gemm_narrow(const dlk_gemv_params p) {
    const int lane = threadIdx.x % kWave, q = lane / 16, r = lane % 16;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int mt = blockIdx.x * kNarrowWaves + wave; // this wave's 16-row tile
    if (mt * 16 >= p.M) return;                       // wave-uniform; no barrier follows
    const int K = p.K, nsteps = K / 32, tiles = gemm::tiles_of(p);
    // weight fragment of tile t, k step s: row r of the tile, columns 32 s + 8 q .. +8 (the second tile repeats
    // the first when there is one tile; its products are then not stored)
    const gemm::TileMap t0 = gemm::locate<false>(p, 0), t1 = gemm::locate<false>(p, min(1, tiles - 1));
    const uint16_t* w0 = gemm::tile_row<false>(t0, r, K) + 8 * q;
    const uint16_t* w1 = gemm::tile_row<false>(t1, r, K) + 8 * q;
    const char* xs = static_cast<const char*>(p.stage) + static_cast<int64_t>(mt) * nsteps * 2048 + 16 * lane;
    struct Frag {
        bf16x8 bh, bl, a0, a1;
    };
    auto load = [&](int step, Frag& f) {
        f.bh = *reinterpret_cast<const bf16x8*>(xs + static_cast<int64_t>(step) * 2048);
        f.bl = *reinterpret_cast<const bf16x8*>(xs + static_cast<int64_t>(step) * 2048 + 1024);
        f.a0 = *reinterpret_cast<const bf16x8*>(w0 + 32 * step);
        f.a1 = *reinterpret_cast<const bf16x8*>(w1 + 32 * step);
    };
    f32x4 acc0 = {0.f, 0.f, 0.f, 0.f}, acc1 = {0.f, 0.f, 0.f, 0.f};
    auto products = [&](const Frag& f) {
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a0, f.bh, acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a0, f.bl, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a1, f.bh, acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(f.a1, f.bl, acc1, 0, 0, 0);
    };
    // batches of kNarrowBatch k steps, two in flight: batch b + 1's loads go out before batch b's products (loads
    // past the end repeat the last step and are not used)
    constexpr int NB = kNarrowBatch;
    const int batches = nsteps / NB;
    Frag fa[NB], fb[NB];
#pragma unroll
    for (int u = 0; u < NB; ++u) load(min(u, nsteps - 1), fa[u]);
    int b = 0;
    for (; b + 2 <= batches; b += 2) {
#pragma unroll
        for (int u = 0; u < NB; ++u) load(min((b + 1) * NB + u, nsteps - 1), fb[u]);
#pragma unroll
        for (int u = 0; u < NB; ++u) products(fa[u]);
#pragma unroll
        for (int u = 0; u < NB; ++u) load(min((b + 2) * NB + u, nsteps - 1), fa[u]);
#pragma unroll
        for (int u = 0; u < NB; ++u) products(fb[u]);
    }
    if (b < batches) {
#pragma unroll
        for (int u = 0; u < NB; ++u) products(fa[u]);
    }
    for (int step = batches * NB; step < nsteps; ++step) {
        Frag f;
        load(step, f);
        products(f);
    }
    // lane holds D[weight rows 4 q .. +4][activation row r] of each tile
    const int m = 16 * mt + r;
    if (m >= p.M) return;
    const float scale = (NORM && p.apply_norm ? stage_inv(p, m) : 1.0f) * p.acc_scale;
    const int n0 = gemv::seg_column(p, t0.seg) + t0.n0 + 4 * q;
    *reinterpret_cast<float4*>(p.y + static_cast<int64_t>(m) * p.ldy + n0) =
        make_float4(acc0[0] * scale, acc0[1] * scale, acc0[2] * scale, acc0[3] * scale);
    if (tiles > 1) {
        const int n1 = gemv::seg_column(p, t1.seg) + t1.n0 + 4 * q;
        *reinterpret_cast<float4*>(p.y + static_cast<int64_t>(m) * p.ldy + n1) =
            make_float4(acc1[0] * scale, acc1[1] * scale, acc1[2] * scale, acc1[3] * scale);
    }
}

/// The narrow kernel for a STORE launch that takes it; {} otherwise.
inline gemv::Kernel resolve_narrow(const dlk_gemv_params& p) {
    if (!narrow_eligible(p)) return {};
    if (gemv::norm_variant(DLK_EPI_STORE, p.apply_norm != 0))
        return {reinterpret_cast<const void*>(&gemm_narrow<true>), 0};
    return {reinterpret_cast<const void*>(&gemm_narrow<false>), 0};
}

/// The tiled kernel for these parameters; {} if none.
template <int EPI>
gemv::Kernel resolve(const dlk_gemv_params& p) {
    if constexpr (EPI == DLK_EPI_LOGITS) {
        return {};
    } else {
        if (gemv::norm_variant(EPI, p.apply_norm != 0)) {
            if constexpr (EPI != DLK_EPI_RESIDUAL)
                return {reinterpret_cast<const void*>(&gemm_tiles<EPI, true>), kLdsBytes};
            return {};
        }
        if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL)
            return {reinterpret_cast<const void*>(&gemm_tiles<EPI, false>), kLdsBytes};
        return {};
    }
}

} // namespace dlk::tiles

dlk::gemv::Kernel dlk_tiles_kernel_store(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_narrow(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_residual(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_qkv(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_swiglu(const dlk_gemv_params& p);
