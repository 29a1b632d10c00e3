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
// fragment reads are linear and conflict-free and no register staging is needed.  A ring of kStages k steps is
// in flight.  The global->LDS traffic (48 KB per k step per work-group) is what bounds the kernel, hence the
// largest tile the LDS ring and the registers hold.
//
// Blocks are placed XCD-aware: the hardware hands consecutive work-group ids to the 8 XCDs in turn, so block b
// takes logical tile (b % 8) * per_xcd + b / 8 and the work-groups of one XCD walk adjacent tiles, which share
// activation rows and weight rows in that XCD's L2.
#pragma once

#include "kernels/gemm_rows.h"

namespace dlk::tiles {

using gemm::bf16x8;
using gemm::f32x4;
using gemv::u32x4;
typedef float f32x8 __attribute__((ext_vector_type(8)));
constexpr int kThreads = 512;                      // 8 waves
constexpr int kWaves = kThreads / kWave;
constexpr int kPrepThreads = 256;                  // prepare_rows: one work-group per activation row
constexpr int kBN = 256;                           // weight rows per work-group (16 tiles of 16)
constexpr int kBM = 256;                           // activation rows per work-group (16 tiles of 16)
constexpr int kStages = 3;                         // k steps of 32 in the LDS ring
constexpr int kWeightBytes = (kBN / 16) * 1024;    // one k step of weight fragments
constexpr int kActBytes = (kBM / 16) * 2048;       // one k step of activation fragments (hi, lo)
constexpr int kStageBytes = kWeightBytes + kActBytes;
constexpr size_t kLdsBytes = 0;                    // the ring is static LDS
constexpr int kDmaPerStep = (kBN / 16 + 2 * (kBM / 16)) / kWaves; // DMA instructions per wave per k step
constexpr int kMinBlocks = 64;                     // one row block of 256 takes the tiled path only this wide
constexpr int kXcds = 8;
static_assert(kDmaPerStep == 6, "two weight tiles and two activation tiles (hi, lo) per wave");

/// Staging workspace of a launch: hi rows, lo rows (bf16 [M][K] each), then the per-row norm factors (f32 [M]).
__host__ __device__ inline int64_t stage_bytes(const dlk_gemv_params& p) {
    return static_cast<int64_t>(p.M) * p.K * 4 + static_cast<int64_t>(p.M) * 4;
}

/// Weight-row blocks of a launch: 16 tiles of 16 rows; SwiGLU: 128 features (8 gate tiles + 8 up tiles).
__host__ __device__ inline int col_blocks(const dlk_gemv_params& p) {
    if (p.epilogue == DLK_EPI_SWIGLU) return (p.seg_rows[0] + 127) / 128;
    return (gemm::tiles_of(p) + 15) / 16;
}
__host__ __device__ inline int row_blocks(const dlk_gemv_params& p) { return (p.M + kBM - 1) / kBM; }

/// Whether the shape suits the tiled path (host side): bf16 weights, whole k steps, tile-shaped segments, rows
/// that prepare_rows reads as float4, and two or more row blocks (or one with a wide weight): narrower launches of
/// that many rows would take gemm_rows 64 rows at a time, re-streaming the weights and under-filling the device.
inline bool shape_eligible(const dlk_gemv_params& p) {
    if (!p.w_bf16 || p.epilogue == DLK_EPI_LOGITS || p.K % 32 != 0 || p.M < kBM) return false;
    if (p.ldx % 4 != 0 || reinterpret_cast<uintptr_t>(p.x) % 16 != 0) return false;
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

// wait until at most n vector-memory operations of this wave are outstanding (lgkm and exp counts untouched)
template <int N>
__device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// 16-byte global->LDS DMA: this lane's 16 bytes at base + offset land at LDS offset lds_base + 16 * lane (base
// and lds_base wave-uniform).  Issued as inline asm so that the compiler's own wait insertion does not see it
// (it would drain every DMA in flight before each LDS read); the ring's waits are explicit (wait_vm) and no
// other vector-memory operation is issued inside the ring loop.
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

// Preparation launch: one work-group per activation row m writes hi[m][k] + lo[m][k] = x[m][k] * g[k] (bf16
// pair, the remainder rounded once more) and, with the norm, inv[m] = 1/sqrt(mean x^2 + eps) (sum of squares of
// x in f32).
template <bool NORM>
__global__ __launch_bounds__(kPrepThreads) void prepare_rows(const dlk_gemv_params p) {
    __shared__ float wave_sums[kPrepThreads / kWave];
    const int m = blockIdx.x, t = threadIdx.x, K = p.K;
    const float* x = p.x + static_cast<int64_t>(m) * p.ldx;
    uint16_t* hi = static_cast<uint16_t*>(p.stage) + static_cast<int64_t>(m) * K;
    uint16_t* lo = hi + static_cast<int64_t>(p.M) * K;
    const bool affine = NORM && p.apply_norm && p.norm_weight;
    float squares = 0.0f;
    for (int k = 8 * t; k < K; k += 8 * kPrepThreads) {
        const float4 a = *reinterpret_cast<const float4*>(x + k);
        const float4 b = *reinterpret_cast<const float4*>(x + k + 4);
        f32x8 v = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        if constexpr (NORM) {
            const f32x8 v2 = v * v;
            squares += ((v2[0] + v2[1]) + (v2[2] + v2[3])) + ((v2[4] + v2[5]) + (v2[6] + v2[7]));
            if (affine) {
                f32x8 g;
                if (p.norm_bf16) {
                    const u32x4 r = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(p.norm_weight) + k);
                    g = f32x8{bf16_lo(r.x), bf16_hi(r.x), bf16_lo(r.y), bf16_hi(r.y),
                              bf16_lo(r.z), bf16_hi(r.z), bf16_lo(r.w), bf16_hi(r.w)};
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
        *reinterpret_cast<bf16x8*>(hi + k) = h;
        *reinterpret_cast<bf16x8*>(lo + k) = l;
    }
    if constexpr (NORM) {
        if (p.apply_norm) {
            squares = wave_sum(squares);
            if (t % kWave == 0) wave_sums[t / kWave] = squares;
            gemv::lds_barrier();
            if (t == 0) {
                float total = 0.0f;
#pragma unroll
                for (int w = 0; w < kPrepThreads / kWave; ++w) total += wave_sums[w];
                float* inv =
                    reinterpret_cast<float*>(static_cast<uint16_t*>(p.stage) + 2 * static_cast<int64_t>(p.M) * K);
                inv[m] = rsqrtf(total / static_cast<float>(K) + p.epsilon);
            }
        }
    }
}

template <int EPI, bool NORM>
__global__ __launch_bounds__(kThreads, 1) void gemm_tiles(const dlk_gemv_params p) {
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    __shared__ __attribute__((aligned(1024))) char ring[kStages][kStageBytes];

    const int t = threadIdx.x, lane = t % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(t / kWave);
    const int K = p.K, nsteps = K / 32;
    const int tiles = gemm::tiles_of(p);
    const int nb = col_blocks(p), total = nb * row_blocks(p);

    // XCD-aware placement: XCD x runs logical tiles [start_x, start_x + count_x)
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = blockIdx.x % kXcds, idx = blockIdx.x / kXcds;
    const int logical = (xcd < rem ? xcd * (per + 1) : rem * (per + 1) + (xcd - rem) * per) + idx;
    const int n_blk = logical % nb, m_blk = logical / nb;
    const int m_first = m_blk * kBM;

    // DMA sources: a wave-uniform base per instruction and a 32-bit lane offset; lane i loads row i%16 at k
    // 8 (i/16).  Wave w fills weight tiles 2w, 2w+1 and activation tiles 2w, 2w+1 (hi and lo); activation
    // rows past M re-read row M-1 (their results are never stored).
    const char* wbase[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) wbase[j] = tile_base<SWIGLU>(p, n_blk, 2 * wave + j, tiles);
    const uint32_t woff = static_cast<uint32_t>(lane % 16) * K * 2 + 16 * (lane / 16);
    const uint16_t* const shi = static_cast<const uint16_t*>(p.stage);
    const int64_t lo_delta = static_cast<int64_t>(p.M) * K * 2; // bytes from the hi rows to the lo rows
    const char* xbase[2];
    uint32_t xoff[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int first = min(m_first + 16 * (2 * wave + h), p.M - 1);
        const int row = min(m_first + 16 * (2 * wave + h) + lane % 16, p.M - 1);
        xbase[h] = reinterpret_cast<const char*>(shi + static_cast<int64_t>(first) * K);
        xoff[h] = static_cast<uint32_t>(row - first) * K * 2 + 16 * (lane / 16);
    }
    auto issue = [&](int step, char* buf) {
        const uint32_t b = lds_offset(buf);
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16(wbase[j] + 64 * step, woff, b + (2 * wave + j) * 1024);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t dst = b + kWeightBytes + (2 * wave + h) * 2048;
            dma16(xbase[h] + 64 * step, xoff[h], dst);
            dma16(xbase[h] + lo_delta + 64 * step, xoff[h], dst + 1024);
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

    auto compute = [&](const char* base) {
        bf16x8 bh[4], bl[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const char* frag = base + kWeightBytes + (4 * wm + j) * 2048 + 16 * lane;
            bh[j] = *reinterpret_cast<const bf16x8*>(frag);
            bl[j] = *reinterpret_cast<const bf16x8*>(frag + 1024);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            // weight tiles past the end (a narrow launch) hold repeats of the last tile: no products for them
            if (!SWIGLU && 16 * n_blk + slot_tile(i) >= tiles) continue;
            const bf16x8 a = *reinterpret_cast<const bf16x8*>(base + slot_tile(i) * 1024 + 16 * lane);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bh[j], acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bl[j], acc[i][j], 0, 0, 0);
            }
        }
    };

    // Ring of kStages buffers.  Before step c's barrier every wave waits for its own DMA of step c (steps c+1 ..
    // c+kStages-2 stay in flight); the barrier then makes every wave's step-c data visible and tells that step
    // c-1's buffer is no longer read, so step c+kStages-1 is issued into it.  Past the last step the issue
    // repeats the last step into that unread buffer, keeping the in-flight count uniform.
#pragma unroll
    for (int s = 0; s < kStages - 1; ++s) issue(min(s, nsteps - 1), ring[s]);
    int buf = 0;
    for (int c = 0; c < nsteps; ++c) {
        wait_vm<(kStages - 2) * kDmaPerStep>();
        ring_barrier();
        issue(min(c + kStages - 1, nsteps - 1), ring[buf == 0 ? kStages - 1 : buf - 1]);
        compute(ring[buf]);
        buf = buf + 1 == kStages ? 0 : buf + 1;
    }
    wait_vm<0>();

    const bool norm = NORM && p.apply_norm;
    float inv[4] = {1.f, 1.f, 1.f, 1.f};
    if (norm) {
        const float* row_inv = reinterpret_cast<const float*>(shi + 2 * static_cast<int64_t>(p.M) * K);
#pragma unroll
        for (int j = 0; j < 4; ++j) inv[j] = row_inv[min(m_first + 64 * wm + 16 * j + lane % 16, p.M - 1)];
    }

    const int q = lane / 16;
    if constexpr (SWIGLU) {
        // lane holds gate (slot i) and up (slot i + 4) of features 128 n_blk + 16 (4 wn + i) + 4 q .. +4
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int f = 128 * n_blk + 16 * (4 * wn + i) + 4 * q;
            if (f >= p.seg_rows[0]) continue;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int m = m_first + 64 * wm + 16 * j + lane % 16;
                if (m >= p.M) continue;
                const float scale = inv[j] * p.acc_scale;
                float* dst = p.y + static_cast<int64_t>(m) * p.ldy + f;
#pragma unroll
                for (int r = 0; r < 4; ++r) dst[r] = gemv::silu(acc[i][j][r] * scale) * (acc[i + 4][j][r] * scale);
            }
        }
    } else {
        // QKV with LoRA of rank <= 32 (a multiple of 8): the rank-r products up[n, :] . hidden[m, :] of each output
        // tile are one more pair of MFMAs, with A = the tile's up rows (k padded with zeros to 32) and B = the
        // hidden rows split into hi + lo; D lands in the accumulator layout
        const bool lora_mfma = EPI == DLK_EPI_QKV && p.lora_rank > 0 && p.lora_rank <= 32 && p.lora_rank % 8 == 0;
        const bool lane_k = 8 * q < p.lora_rank; // lanes whose k slots hold rank entries
        // fully unrolled: acc is only ever indexed with constants (a runtime index puts it in scratch memory)
#pragma clang loop unroll(full)
        for (int j = 0; j < 4; ++j) {
            const int ml = 64 * wm + 16 * j + lane % 16, m = m_first + ml;
            const float scale = inv[j] * p.acc_scale;
            // hidden fragments of segments 0 (q) and 2 (v); the kernel-argument arrays and these are only indexed
            // with constants or selects (a runtime index would copy them to scratch memory)
            bf16x8 hh[2] = {}, hl[2] = {};
            if constexpr (EPI == DLK_EPI_QKV) {
                if (lora_mfma) {
#pragma unroll
                    for (int h = 0; h < 2; ++h) {
                        const float* hidden = h == 0 ? p.lora_hidden[0] : p.lora_hidden[2];
                        if (!hidden) continue;
                        const float* row = hidden + (p.m_base + min(m, p.M - 1)) * p.lora_rank + 8 * (lane_k ? q : 0);
                        const float4 a = *reinterpret_cast<const float4*>(row);
                        const float4 c = *reinterpret_cast<const float4*>(row + 4);
                        f32x8 x = {a.x, a.y, a.z, a.w, c.x, c.y, c.z, c.w};
                        if (!lane_k) x = f32x8{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
                        hh[h] = __builtin_convertvector(x, bf16x8);
                        hl[h] = __builtin_convertvector(x - __builtin_convertvector(hh[h], f32x8), bf16x8);
                    }
                }
            }
#pragma clang loop unroll(full)
            for (int i = 0; i < 8; ++i) {
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
                        const uint16_t* up = static_cast<const uint16_t*>(vseg ? p.lora_up[2] : p.lora_up[0]) +
                                             static_cast<int64_t>(tm.n0 + lane % 16) * p.lora_rank + 8 * (lane_k ? q : 0);
                        u32x4 raw = *reinterpret_cast<const u32x4*>(up);
                        if (!lane_k) raw = u32x4{0u, 0u, 0u, 0u};
                        const bf16x8 a = __builtin_bit_cast(bf16x8, raw);
                        f32x4 d = {0.f, 0.f, 0.f, 0.f};
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, vseg ? hh[1] : hh[0], d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, vseg ? hl[1] : hl[0], d, 0, 0, 0);
                        lora = {{d[0], d[1], d[2], d[3]}, true};
                    }
                }
                if (m < p.M) gemm::lane_epilogue<EPI>(p, tm, q, m, v, bs, bi, p.key_seed, p.key_stream, lora);
            }
        }
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (p.bump_position && blockIdx.x == 0 && t == 0) *p.bump_position += p.bump_count;
    }
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
dlk::gemv::Kernel dlk_tiles_kernel_residual(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_qkv(const dlk_gemv_params& p);
dlk::gemv::Kernel dlk_tiles_kernel_swiglu(const dlk_gemv_params& p);
