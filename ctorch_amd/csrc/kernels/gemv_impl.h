// Projection GEMV for the decode step (see dlk_gemv_params in kernels.h): kernel templates shared by the
// per-epilogue translation units (gemv_<epilogue>.hip) and the host-side plan used by the dispatcher (gemv.hip).
//
// Two kernels share one fused epilogue:
//  * gemv_reg (rows of up to 12 * 64 16-byte chunks): every wave64 keeps its share of the activation rows in
//    registers (lane l holds chunks l, l + 64, ...), applies the preceding RMSNorm itself (sum of squares by
//    lane butterflies; no LDS, no barrier), then streams weight groups of R rows, one whole row per step,
//    persistent over groups g = wave, wave + waves, ...; the next group's chunks are loaded while the current
//    group is reduced.  On MI355X this keeps a projection within a few percent of a plain read of its bytes.
//  * gemv_lds (longer rows): the activation row is staged once per work-group in LDS (LDS-only barriers) and
//    rows are streamed in steps of 4 chunks per lane, two steps in flight.
// A group's dots are reduced by lane butterflies and the epilogue (bias, residual, RoPE + KV append,
// SiLU(gate) * up, logits + per-wave sampling candidate) runs on the reduced values.  Every weight byte is
// read once per launch.
//
// Two compiler facts shape the code.  Vector loads complete in issue order and a wait names a count of
// younger loads, so (a) loads are issued in the order their data is needed (activations, then weights) and
// (b) loads are never conditional inside the streaming loop (the last step is peeled instead): a load on
// only one path of a branch forces a full drain of the stream at the join.  Kernel-argument arrays are only
// indexed with constants: a runtime index turns them into vector loads with a full wait on every use.
#pragma once

#include "kernels/device_common.h"

#include <algorithm>

namespace dlk::gemv {

constexpr int kThreads = 256;
constexpr int kWavesPerBlock = kThreads / kWave;
constexpr int kMaxWaves = 4096;       // persistent grid cap: 1024 work-groups, 4 per CU
constexpr int kLdsBytes = 60 * 1024;  // staged activation row of the fallback kernel
constexpr int kLdsSteps = 4;          // chunks per lane per step in the fallback kernel
constexpr int kLdsXL = 15;            // float4 activation loads per thread in the fallback (K <= 15360)
constexpr int kRegBudget = 192;       // VGPRs for activations + two weight buffers in the register kernel
constexpr int kRegBudgetRows = 128;   // the same, for launches of more than one activation row (the compiler's
                                      // own temporaries roughly double it; past 256 it spills to AGPR moves)
constexpr int kOutOfRange = 0x7fffff00; // buffer offset past any range: the load returns zeros, touches nothing
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr bool pair_epilogue(int epi) { return epi == DLK_EPI_QKV || epi == DLK_EPI_SWIGLU; }
/// rows per group: RoPE pairs and gate/up pairs need two; otherwise two while rows are short
constexpr int group_rows(int epi, int cpi) { return pair_epilogue(epi) || cpi <= 4 ? 2 : 1; }
constexpr bool reg_fits(int mt, int cpi, int chunk, int epi) {
    return mt * cpi * chunk + 2 * group_rows(epi, cpi) * cpi * 4 <= (mt == 1 ? kRegBudget : kRegBudgetRows);
}

/// How one launch is shaped (host side): kernel kind, chunks per lane, rows per group, activation rows.
struct Plan {
    bool reg = false;
    int cpi = 0, rows = 2, mt_max = 1;
};

inline Plan plan_of(int K, bool bf16_weights, int epi) {
    const int chunk = bf16_weights ? 8 : 4;
    const int need = (K / chunk + kWave - 1) / kWave;
    Plan plan;
    for (int c : {1, 2, 4, 8, 12})
        if (need <= c) { plan.cpi = c; break; }
    if (plan.cpi != 0 && reg_fits(1, plan.cpi, chunk, epi)) {
        plan.reg = true;
        plan.rows = group_rows(epi, plan.cpi);
        plan.mt_max = 1;
        while (plan.mt_max < 4 && reg_fits(plan.mt_max * 2, plan.cpi, chunk, epi)) plan.mt_max *= 2;
    } else {
        plan.reg = false;
        plan.cpi = kLdsSteps;
        plan.rows = 2;
        plan.mt_max = 1;
    }
    return plan;
}

// groups of R rows never straddle a weight segment; SwiGLU groups pair gate rows with the same up rows
__host__ __device__ inline int groups_of(const dlk_gemv_params& p, int R, bool swiglu) {
    if (swiglu) return (p.seg_rows[0] + R / 2 - 1) / (R / 2);
    int g = (p.seg_rows[0] + R - 1) / R;
    if (p.nseg > 1) g += (p.seg_rows[1] + R - 1) / R;
    if (p.nseg > 2) g += (p.seg_rows[2] + R - 1) / R;
    return g;
}

template <typename WT> struct WeightTraits;
template <> struct WeightTraits<uint16_t> {
    static constexpr int chunk = 8;
    __device__ static __forceinline__ float dot(const u32x4 w, const float* x) {
        float s = bf16_lo(w.x) * x[0];
        s += bf16_hi(w.x) * x[1];
        s += bf16_lo(w.y) * x[2];
        s += bf16_hi(w.y) * x[3];
        s += bf16_lo(w.z) * x[4];
        s += bf16_hi(w.z) * x[5];
        s += bf16_lo(w.w) * x[6];
        s += bf16_hi(w.w) * x[7];
        return s;
    }
    __device__ static __forceinline__ float scalar(const void* w, int64_t i) {
        return bf16_to_f32(static_cast<const uint16_t*>(w)[i]);
    }
};
template <> struct WeightTraits<float> {
    static constexpr int chunk = 4;
    __device__ static __forceinline__ float dot(const u32x4 w, const float* x) {
        float s = __uint_as_float(w.x) * x[0];
        s += __uint_as_float(w.y) * x[1];
        s += __uint_as_float(w.z) * x[2];
        s += __uint_as_float(w.w) * x[3];
        return s;
    }
    __device__ static __forceinline__ float scalar(const void* w, int64_t i) {
        return static_cast<const float*>(w)[i];
    }
};

__device__ __forceinline__ float silu(float v) {
    // stable sigmoid of the reference CPU path (src/kernels/cpu/pointwise.cpp:31-34)
    const float e = expf(-fabsf(v));
    const float sigma = v >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return v * sigma;
}

// work-group barrier that orders LDS traffic only; outstanding global loads stay in flight
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A row group: its segment, first output row, rows in the segment and the matrices its rows come from.
template <typename WT> struct Group {
    int seg, n0, rows;
    const WT *base0, *base1;
};

// The weight segments held in scalars.  Every field of a Group is set inside the branch that picks the
// segment: selecting among adjacent members by a runtime index lets the compiler turn the selection into a
// private-memory table (scratch loads with a full wait).
template <typename WT, int R, bool SWIGLU> struct Segments {
    static constexpr int OUTS = SWIGLU ? R / 2 : R;
    const WT *w0, *w1, *w2;
    int rows0, rows1, rows2, groups0, groups1, nseg;
    __device__ explicit Segments(const dlk_gemv_params& p)
        : w0(static_cast<const WT*>(p.w[0])), w1(static_cast<const WT*>(p.w[1])),
          w2(static_cast<const WT*>(p.w[2])), rows0(p.seg_rows[0]), rows1(p.seg_rows[1]), rows2(p.seg_rows[2]),
          groups0((p.seg_rows[0] + R - 1) / R), groups1(p.nseg > 1 ? (p.seg_rows[1] + R - 1) / R : 0),
          nseg(p.nseg) {}
    __device__ __forceinline__ Group<WT> locate(int g) const {
        if constexpr (SWIGLU) return {0, g * OUTS, rows0, w0, w1};
        if (g < groups0 || nseg == 1) return {0, g * R, rows0, w0, w0};
        if (g < groups0 + groups1 || nseg == 2) return {1, (g - groups0) * R, rows1, w1, w1};
        return {2, (g - groups0 - groups1) * R, rows2, w2, w2};
    }
    // row r of a group as 16-byte chunks; rows past the segment end are clamped (loaded, never stored)
    __device__ __forceinline__ static const u32x4* row(const Group<WT>& grp, int r, int K) {
        const WT* base = SWIGLU && r >= OUTS ? grp.base1 : grp.base0;
        const int n = min(grp.n0 + (SWIGLU ? r % OUTS : r), grp.rows - 1);
        return reinterpret_cast<const u32x4*>(base + static_cast<int64_t>(n) * K);
    }
};

// Per-wave state of the LOGITS epilogue: the best (score, index) seen for each activation row.
template <int MT> struct Candidates {
    double score[MT];
    int64_t index[MT];
    uint64_t seed, stream;
};

template <int MT, int EPI>
__device__ __forceinline__ void init_candidates(const dlk_gemv_params& p, Candidates<MT>& cand) {
    cand.seed = p.key_seed;
    cand.stream = p.key_stream;
    if constexpr (EPI == DLK_EPI_LOGITS) {
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            cand.score[m] = 0.0;
            cand.index[m] = -1;
        }
        if (p.sample_mode == 2 && p.key_label)
            fold_in(p.key_seed, p.key_stream, static_cast<uint64_t>(*p.key_label), cand.seed, cand.stream);
    }
}

// One step's operands in flight: the weight chunks and the epilogue's per-output operands (residual value,
// RoPE cos/sin) of output lane m * R + r, loaded with the weights so the epilogue never waits on a
// dependent load.
template <int R, int CPI> struct Step {
    u32x4 w[R][CPI];
    float aux0, aux1;
};

// Per activation row of the launch (QKV): its sequence and absolute position, computed once per kernel in
// scalars (integer division stays out of the per-group path).
template <int MT> struct Rows {
    int batch[MT];
    int64_t pos[MT];
    __device__ Rows(const dlk_gemv_params& p, bool used) {
        const int64_t first = used ? *p.position : 0;
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int mg = static_cast<int>(p.m_base) + m;
            batch[m] = used ? mg / p.length : 0;
            pos[m] = used ? first + mg % p.length : 0;
        }
    }
    // the position of row m for a lane-dependent m (selects, no indexed access)
    __device__ __forceinline__ int64_t pos_of(int m) const {
        int64_t v = pos[0];
#pragma unroll
        for (int i = 1; i < MT; ++i)
            if (m == i) v = pos[i];
        return v;
    }
};

template <int MT, int R, int EPI, typename WT>
__device__ __forceinline__ void load_aux(const dlk_gemv_params& p, const Group<WT>& grp, int lane, const Rows<MT>& rows,
                                         float& aux0, float& aux1) {
    if constexpr (EPI == DLK_EPI_RESIDUAL || EPI == DLK_EPI_QKV) {
        // lanes past the outputs load a clamped, valid address; their values are never used
        const int m = min(min(lane / R, MT - 1), p.M - 1);
        if constexpr (EPI == DLK_EPI_RESIDUAL) {
            const int n = min(grp.n0 + lane % R, grp.rows - 1);
            aux0 = p.residual[static_cast<int64_t>(m) * p.ldres + n];
        } else {
            // rows come in even pairs and n0 is even, so the column of n0 + r in its head is (n0 % hd) + r
            const int hd = p.head_dim;
            const int d = grp.n0 % hd + lane % R;
            const int64_t table = rows.pos_of(m) * (hd / 2) + d / 2;
            aux0 = p.cosine[table];
            aux1 = p.sine[table];
        }
    }
}

// First output column of segment seg in a STORE launch (the segments' outputs sit side by side in y).
__device__ __forceinline__ int seg_column(const dlk_gemv_params& p, int seg) {
    return seg == 0 ? 0 : seg == 1 ? p.seg_rows[0] : p.seg_rows[0] + p.seg_rows[1];
}

// Row stride of the LoRA hidden rows.
__device__ __forceinline__ int64_t lora_stride(const dlk_gemv_params& p) { return p.lora_ld ? p.lora_ld : p.lora_rank; }

// The epilogue of one finished group; v[m][r] holds the full dot products (every lane has them).
template <typename WT, int MT, int R, int EPI, typename Seg>
__device__ __forceinline__ void finish_group(const dlk_gemv_params& p, const Seg& sg, const float (&v)[MT][R], int g,
                                             int lane, const Rows<MT>& rows, float aux0, float aux1,
                                             Candidates<MT>& cand) {
    using Traits = WeightTraits<WT>;
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    constexpr int OUTS = SWIGLU ? R / 2 : R;
    const auto grp = sg.locate(g);
    const int seg = grp.seg, n0 = grp.n0, seg_rows = grp.rows;
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = n0 + r;
                if (lane == m * R + r && m < p.M && n < seg_rows) {
                    float out = v[m][r];
                    int col = n;
                    if constexpr (EPI == DLK_EPI_STORE) {
                        col += seg_column(p, seg);
                        if (p.bias)
                            out += p.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p.bias)[col])
                                               : static_cast<const float*>(p.bias)[col];
                    } else {
                        out += aux0;
                    }
                    p.y[static_cast<int64_t>(m) * p.ldy + col] = out;
                }
            }
    } else if constexpr (SWIGLU) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < OUTS; ++j) {
                const int n = n0 + j;
                if (lane == m * OUTS + j && m < p.M && n < seg_rows)
                    p.y[static_cast<int64_t>(m) * p.ldy + n] = silu(v[m][j]) * v[m][OUTS + j];
            }
    } else if constexpr (EPI == DLK_EPI_QKV) {
        static_assert(R % 2 == 0, "RoPE pairs need an even group");
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = n0 + r;
                if (lane != m * R + r || m >= p.M || n >= seg_rows) continue;
                const int64_t mg = p.m_base + m;
                float value = v[m][r];
                float partner = v[m][r ^ 1];
                const float* hidden = seg == 0 ? p.lora_hidden[0] : seg == 2 ? p.lora_hidden[2] : nullptr;
                const void* lora_up = seg == 0 ? p.lora_up[0] : p.lora_up[2];
                if (hidden) {
                    // unmerged LoRA: + scale * up[n, :] . hidden[m, :] on both members of the pair
                    const int np = n ^ 1;
                    const float* hrow = hidden + mg * lora_stride(p);
                    float dv = 0.0f, dp = 0.0f;
                    for (int j = 0; j < p.lora_rank; ++j) {
                        dv += Traits::scalar(lora_up, static_cast<int64_t>(n) * p.lora_rank + j) * hrow[j];
                        dp += Traits::scalar(lora_up, static_cast<int64_t>(np) * p.lora_rank + j) * hrow[j];
                    }
                    value += dv * p.lora_scale;
                    partner += dp * p.lora_scale;
                }
                const int64_t b = rows.batch[m], pos = rows.pos[m];
                const int hd = p.head_dim;
                const int head = n0 / hd, d = n0 % hd + r;
                if (seg < 2) {
                    const float c = aux0, s = aux1;
                    // even: x_e c - x_o s ; odd: x_e s + x_o c (interleaved pairs, src/ops/contraction.cpp:44-49)
                    value = (d & 1) == 0 ? value * c - partner * s : partner * s + value * c;
                }
                if (seg == 0) {
                    p.y[mg * p.ldy + n] = value;
                } else {
                    const int64_t index = ((b * p.kv_heads + head) * p.cache_capacity + pos) * hd + d;
                    void* cache = seg == 1 ? p.k_cache : p.v_cache;
                    if (p.cache_bf16) static_cast<uint16_t*>(cache)[index] = f32_to_bf16(value);
                    else static_cast<float*>(cache)[index] = value;
                }
            }
    } else if constexpr (EPI == DLK_EPI_LOGITS) {
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int n = n0 + r;
                if (m >= p.M || n >= seg_rows) continue;
                if (p.y && lane == m * R + r) p.y[static_cast<int64_t>(m) * p.ldy + n] = v[m][r];
                if (p.sample_mode != 0 && lane == m) {
                    const int64_t mg = p.m_base + m;
                    const double s = sample_score(v[m][r], p.sample_mode, p.temperature, cand.seed, cand.stream,
                                                  static_cast<uint64_t>(mg * seg_rows + n));
                    if (cand.index[m] < 0 || prefer(s, n, cand.score[m], cand.index[m])) {
                        cand.score[m] = s;
                        cand.index[m] = n;
                    }
                }
            }
    }
}

// End of a launch.  LOGITS: the work-group's waves pool their sampling candidates in LDS and wave 0 writes the
// best one per activation row as the work-group's partial (every wave of the work-group must get here).
template <int MT, int EPI>
__device__ __forceinline__ void finish_kernel(const dlk_gemv_params& p, const Candidates<MT>& cand, int lane,
                                              int wave_in_block) {
    if constexpr (EPI == DLK_EPI_LOGITS) {
        __shared__ double pool_score[kWavesPerBlock][MT];
        __shared__ int64_t pool_index[kWavesPerBlock][MT];
        if (p.sample_mode == 0) return;
#pragma unroll
        for (int m = 0; m < MT; ++m)
            if (lane == m) {
                pool_score[wave_in_block][m] = cand.score[m];
                pool_index[wave_in_block][m] = cand.index[m];
            }
        lds_barrier();
        if (wave_in_block == 0 && lane < MT && lane < p.M) {
            double best = 0.0;
            int64_t index = -1;
#pragma unroll
            for (int w = 0; w < kWavesPerBlock; ++w) {
                const int64_t j = pool_index[w][lane];
                if (j >= 0 && (index < 0 || prefer(pool_score[w][lane], j, best, index))) {
                    best = pool_score[w][lane];
                    index = j;
                }
            }
            dlk_sample_partial out;
            out.score = best;
            out.index = index;
            p.partial[(p.m_base + lane) * p.partial_blocks + blockIdx.x] = out;
        }
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        // the device cache length advances after the attention launch that read it (stream order)
        if (p.bump_position && blockIdx.x == 0 && threadIdx.x == 0) *p.bump_position += p.bump_count;
    }
}

// Runs the streaming loop over `count` >= 1 steps with one step in flight beyond the one being used; step 0 is
// already loaded into `a` by the caller.  Loads in the loop body are unconditional, the last step is peeled.
template <typename Buf, typename Load, typename Use>
__device__ __forceinline__ void stream_steps(int count, Buf& a, Buf& b, Load&& load, Use&& use) {
    int k = 0;
    for (;;) {
        if (k + 1 >= count) {
            use(k, a);
            return;
        }
        load(k + 1, b);
        use(k, a);
        ++k;
        if (k + 1 >= count) {
            use(k, b);
            return;
        }
        load(k + 1, a);
        use(k, b);
        ++k;
    }
}

// ------------------------------------------------------------------------------------------ register kernel
// CPI = 16-byte chunks per lane per row: the whole row in one step (K <= 64 * CPI * chunk).  Each wave loads
// its own copy of the activation chunks it needs (lane l: chunks l, l + 64, ...) and applies the RMSNorm
// in-wave; on MI355X this beat staging the rows once per work-group in LDS at every decode shape.
template <typename WT, int MT, int R, int CPI, int EPI, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_reg(const dlk_gemv_params p) {
    // measured on MI355X (A/B against byte-identical builds): the C2 step 547 -> 542 us; the same touch in the
    // batched projections, the reduce and the decode attention made C2 and C4 slower (C4 9.32 -> 9.56 ms)
    touch_kernargs<sizeof(dlk_gemv_params)>();
    using Traits = WeightTraits<WT>;
    constexpr int CH = Traits::chunk;
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    const int K = p.K;
    const int nch = K / CH;
    const int lane = threadIdx.x % kWave;
    // wave-uniform in a scalar register: group and segment selection stay scalar (no per-lane branches)
    const int wave_in_block = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int my_wave = blockIdx.x * kWavesPerBlock + wave_in_block;
    const int waves = gridDim.x * kWavesPerBlock;
    const Segments<WT, R, SWIGLU> sg(p);
    const int groups = groups_of(p, R, SWIGLU);
    // idle waves (only in the last work-group) exit, except in LOGITS, whose end pools the work-group's waves
    if constexpr (EPI != DLK_EPI_LOGITS) {
        if (my_wave >= groups) return;
    }
    const int my_groups = my_wave < groups ? (groups - my_wave + waves - 1) / waves : 0;
    const bool norm = NORM && p.apply_norm;
    const bool affine = norm && p.norm_weight;

    // 1. activations and norm weights first (their wait never covers the weight loads issued after them).  No
    // load sits in a branch: a load on one path only would make the first wait drain every load.  The norm
    // weights come through a bounds-checked buffer load (16 bytes at the element offset for either dtype;
    // bytes past the vector read as zero).
    float x[MT][CPI][CH];
#pragma unroll
    for (int i = 0; i < CPI; ++i) {
        const int c = min(lane + kWave * i, nch - 1);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const float* row = p.x + static_cast<int64_t>(min(m, p.M - 1)) * p.ldx + c * CH;
#pragma unroll
            for (int j = 0; j < CH; j += 4) {
                const float4 v = *reinterpret_cast<const float4*>(row + j);
                x[m][i][j] = v.x;
                x[m][i][j + 1] = v.y;
                x[m][i][j + 2] = v.z;
                x[m][i][j + 3] = v.w;
            }
        }
    }
    u32x4 graw[NORM ? CPI : 1][CH / 4];
    if constexpr (NORM) {
        const int esize = p.norm_bf16 ? 2 : 4;
        const __amdgpu_buffer_rsrc_t gres = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<void*>(affine ? p.norm_weight : static_cast<const void*>(p.x)), 0, affine ? K * esize : 0,
            kBufferFlags);
#pragma unroll
        for (int i = 0; i < CPI; ++i) {
            const int c = min(lane + kWave * i, nch - 1);
#pragma unroll
            for (int j = 0; j < CH / 4; ++j) {
                // bf16 weights: the first 16 bytes already hold the chunk; later parts read past the range
                // (no memory access, zeros) instead of branching around the load
                const int offset = j > 0 && esize == 2 ? kOutOfRange : (c * CH + 4 * j) * esize;
                graw[i][j] = __builtin_amdgcn_raw_buffer_load_b128(gres, offset, 0, 0);
            }
        }
    }

    Candidates<MT> cand;
    init_candidates<MT, EPI>(p, cand);
    const Rows<MT> rows(p, EPI == DLK_EPI_QKV);
    auto load = [&](int k, Step<R, CPI>& buf) {
        const auto grp = sg.locate(min(my_wave + k * waves, groups - 1));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32x4* row = sg.row(grp, r, K);
#pragma unroll
            for (int i = 0; i < CPI; ++i) buf.w[r][i] = __builtin_nontemporal_load(row + min(lane + kWave * i, nch - 1));
        }
        load_aux<MT, R, EPI>(p, grp, lane, rows, buf.aux0, buf.aux1);
    };
    // 2. the first weight group (idle LOGITS waves load a valid group and ignore it)
    Step<R, CPI> a, b;
    load(0, a);

    // 3. while it is in flight: zero the tail chunks and rows, then the fused RMSNorm of this wave's copy
#pragma unroll
    for (int i = 0; i < CPI; ++i) {
        const bool in = lane + kWave * i < nch;
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int j = 0; j < CH; ++j)
                if (!in || m >= p.M) x[m][i][j] = 0.0f;
    }
    if constexpr (NORM) {
        if (norm) {
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float squares = 0.0f;
#pragma unroll
                for (int i = 0; i < CPI; ++i)
#pragma unroll
                    for (int j = 0; j < CH; ++j) squares += x[m][i][j] * x[m][i][j];
                const float inv = rsqrtf(wave_sum(squares) / static_cast<float>(K) + p.epsilon);
#pragma unroll
                for (int i = 0; i < CPI; ++i)
#pragma unroll
                    for (int j = 0; j < CH; j += 4) {
                        const u32x4 w = graw[i][j / 4];
                        float g[4] = {1.0f, 1.0f, 1.0f, 1.0f};
                        if (affine) {
                            if (p.norm_bf16) {
                                // elements j..j+3 of the chunk sit in the first load (words j/2, j/2 + 1)
                                const u32x4 c0 = graw[i][0];
                                const uint32_t lo = j == 0 ? c0.x : c0.z, hi = j == 0 ? c0.y : c0.w;
                                g[0] = bf16_lo(lo); g[1] = bf16_hi(lo); g[2] = bf16_lo(hi); g[3] = bf16_hi(hi);
                            } else {
                                g[0] = __uint_as_float(w.x); g[1] = __uint_as_float(w.y);
                                g[2] = __uint_as_float(w.z); g[3] = __uint_as_float(w.w);
                            }
                        }
#pragma unroll
                        for (int e = 0; e < 4; ++e) x[m][i][j + e] = x[m][i][j + e] * inv * g[e];
                    }
            }
        }
    }

    // 4. stream the row groups
    auto use = [&](int k, const Step<R, CPI>& buf) {
        float acc[MT][R];
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float s = 0.0f;
#pragma unroll
                for (int i = 0; i < CPI; ++i) s += Traits::dot(buf.w[r][i], x[m][i]);
                acc[m][r] = wave_sum(s) * p.acc_scale;
            }
        finish_group<WT, MT, R, EPI>(p, sg, acc, my_wave + k * waves, lane, rows, buf.aux0, buf.aux1, cand);
    };
    if (my_groups > 0) stream_steps(my_groups, a, b, load, use);
    finish_kernel<MT, EPI>(p, cand, lane, wave_in_block);
}

// ------------------------------------------------------------------------------------------ LDS kernel
// Long rows (one activation row per launch): the row is staged in LDS, weights streamed in steps of
// kLdsSteps chunks per lane.
template <typename WT, int R, int EPI, bool NORM>
__global__ __launch_bounds__(kThreads) void gemv_lds(const dlk_gemv_params p) {
    using Traits = WeightTraits<WT>;
    constexpr int CH = Traits::chunk;
    constexpr int CPI = kLdsSteps;
    constexpr int MT = 1;
    constexpr bool SWIGLU = EPI == DLK_EPI_SWIGLU;
    extern __shared__ float xs[]; // [K]
    __shared__ float block_sums[kWavesPerBlock];
    const int K = p.K;
    const int nch = K / CH;
    const int t = threadIdx.x, lane = t % kWave, wave_in_block = t / kWave;
    const int waves = gridDim.x * kWavesPerBlock;
    const int my_wave = __builtin_amdgcn_readfirstlane(blockIdx.x * kWavesPerBlock + wave_in_block);
    const Segments<WT, R, SWIGLU> sg(p);
    const int groups = groups_of(p, R, SWIGLU);
    constexpr int STEP_CHUNKS = kWave * CPI;
    const int steps_per_group = (nch + STEP_CHUNKS - 1) / STEP_CHUNKS;
    // idle waves of the last work-group take part in the staging barriers, then leave
    const int my_groups = my_wave < groups ? (groups - my_wave + waves - 1) / waves : 0;
    const int jobs = my_groups * steps_per_group;

    // the activation row (and norm weights) in registers first, so their wait never covers weight loads
    float4 xr[kLdsXL], gr[kLdsXL];
    const bool norm = NORM && p.apply_norm;
    const bool affine = norm && p.norm_weight;
#pragma unroll
    for (int i = 0; i < kLdsXL; ++i) {
        const int k = min((t + i * kThreads) * 4, K - 4);
        xr[i] = *reinterpret_cast<const float4*>(p.x + k);
        if (affine) {
            if (p.norm_bf16) {
                const uint2 w = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.norm_weight) + k);
                gr[i] = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
            } else {
                gr[i] = *reinterpret_cast<const float4*>(static_cast<const float*>(p.norm_weight) + k);
            }
        } else {
            gr[i] = make_float4(1.f, 1.f, 1.f, 1.f);
        }
    }
    float squares = 0.0f;
#pragma unroll
    for (int i = 0; i < kLdsXL; ++i) {
        if ((t + i * kThreads) * 4 >= K) xr[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        squares += xr[i].x * xr[i].x + xr[i].y * xr[i].y + xr[i].z * xr[i].z + xr[i].w * xr[i].w;
    }
    float inv = 1.0f;
    if (norm) {
        squares = wave_sum(squares);
        if (lane == 0) block_sums[wave_in_block] = squares;
        lds_barrier();
        float total = 0.0f;
#pragma unroll
        for (int w = 0; w < kWavesPerBlock; ++w) total += block_sums[w];
        inv = rsqrtf(total / static_cast<float>(K) + p.epsilon);
    }
#pragma unroll
    for (int i = 0; i < kLdsXL; ++i) {
        const int k = (t + i * kThreads) * 4;
        if (k < K)
            *reinterpret_cast<float4*>(xs + k) = make_float4(xr[i].x * inv * gr[i].x, xr[i].y * inv * gr[i].y,
                                                             xr[i].z * inv * gr[i].z, xr[i].w * inv * gr[i].w);
    }
    lds_barrier();
    if (jobs == 0) {
        if constexpr (EPI != DLK_EPI_LOGITS) return;
    }

    Candidates<MT> cand;
    init_candidates<MT, EPI>(p, cand);
    const Rows<MT> rows(p, EPI == DLK_EPI_QKV);
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;

    auto load = [&](int job, Step<R, CPI>& buf) {
        const int g = my_wave + (job / steps_per_group) * waves;
        const int c0 = (job % steps_per_group) * STEP_CHUNKS;
        const auto grp = sg.locate(g);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32x4* row = sg.row(grp, r, K);
#pragma unroll
            for (int i = 0; i < CPI; ++i) buf.w[r][i] = __builtin_nontemporal_load(row + min(c0 + lane + kWave * i, nch - 1));
        }
        load_aux<MT, R, EPI>(p, grp, lane, rows, buf.aux0, buf.aux1);
    };
    auto use = [&](int job, const Step<R, CPI>& buf) {
        const int c0 = (job % steps_per_group) * STEP_CHUNKS;
#pragma unroll
        for (int i = 0; i < CPI; ++i) {
            const int c = c0 + lane + kWave * i;
            if (c < nch) {
                float xv[CH];
#pragma unroll
                for (int j = 0; j < CH; j += 4) {
                    const float4 v = *reinterpret_cast<const float4*>(xs + c * CH + j);
                    xv[j] = v.x;
                    xv[j + 1] = v.y;
                    xv[j + 2] = v.z;
                    xv[j + 3] = v.w;
                }
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r] += Traits::dot(buf.w[r][i], xv);
            }
        }
        if (job % steps_per_group != steps_per_group - 1) return;
        float v[MT][R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            v[0][r] = wave_sum(acc[r]) * p.acc_scale;
            acc[r] = 0.0f;
        }
        finish_group<WT, MT, R, EPI>(p, sg, v, my_wave + (job / steps_per_group) * waves, lane, rows, buf.aux0,
                                     buf.aux1, cand);
    };
    Step<R, CPI> a, b;
    if (jobs > 0) {
        load(0, a);
        stream_steps(jobs, a, b, load, use);
    }
    finish_kernel<MT, EPI>(p, cand, lane, wave_in_block);
}

// ------------------------------------------------------------------------------------------ resolution
/// A resolved kernel: its function and dynamic LDS bytes (launched with kThreads threads and one argument,
/// the parameter block).
struct Kernel {
    const void* fn = nullptr;
    size_t lds = 0;
};

/// Whether an epilogue's kernels carry the RMSNorm prologue (RESIDUAL never does; STORE both ways).
constexpr bool norm_variant(int epi, bool apply_norm) { return epi != DLK_EPI_RESIDUAL && (epi != DLK_EPI_STORE || apply_norm); }

template <typename WT, int MT, int CPI, int EPI, bool NORM>
Kernel reg_kernel() {
    constexpr int R = group_rows(EPI, CPI);
    if constexpr (reg_fits(MT, CPI, WeightTraits<WT>::chunk, EPI))
        return {reinterpret_cast<const void*>(&gemv_reg<WT, MT, R, CPI, EPI, NORM>), 0};
    return {};
}

template <typename WT, int MT, int EPI, bool NORM>
Kernel reg_cpi(int cpi) {
    switch (cpi) {
    case 1: return reg_kernel<WT, MT, 1, EPI, NORM>();
    case 2: return reg_kernel<WT, MT, 2, EPI, NORM>();
    case 4: return reg_kernel<WT, MT, 4, EPI, NORM>();
    case 8: return reg_kernel<WT, MT, 8, EPI, NORM>();
    case 12: return reg_kernel<WT, MT, 12, EPI, NORM>();
    default: return {};
    }
}

template <typename WT, int EPI, bool NORM>
Kernel resolve_typed(const dlk_gemv_params& p, int mt) {
    const Plan plan = plan_of(p.K, sizeof(WT) == 2, EPI);
    if (plan.reg) {
        Kernel kernel;
        switch (mt) {
        case 1: kernel = reg_cpi<WT, 1, EPI, NORM>(plan.cpi); break;
        case 2: kernel = reg_cpi<WT, 2, EPI, NORM>(plan.cpi); break;
        case 4: kernel = reg_cpi<WT, 4, EPI, NORM>(plan.cpi); break;
        default: return {};
        }
        return kernel;
    }
    if (mt != 1) return {};
    return {reinterpret_cast<const void*>(&gemv_lds<WT, 2, EPI, NORM>), static_cast<size_t>(p.K) * sizeof(float)};
}

/// The kernel for a launch of mt (1, 2 or 4) activation rows with this parameter block; {} if none fits.
template <int EPI>
Kernel resolve(const dlk_gemv_params& p, int mt) {
    if (norm_variant(EPI, p.apply_norm != 0)) {
        if constexpr (EPI != DLK_EPI_RESIDUAL)
            return p.w_bf16 ? resolve_typed<uint16_t, EPI, true>(p, mt) : resolve_typed<float, EPI, true>(p, mt);
        return {};
    }
    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL)
        return p.w_bf16 ? resolve_typed<uint16_t, EPI, false>(p, mt) : resolve_typed<float, EPI, false>(p, mt);
    return {};
}

} // namespace dlk::gemv

// One translation unit per epilogue instantiates its kernels (parallel builds).
dlk::gemv::Kernel dlk_gemv_kernel_store(const dlk_gemv_params& p, int mt);
dlk::gemv::Kernel dlk_gemv_kernel_residual(const dlk_gemv_params& p, int mt);
dlk::gemv::Kernel dlk_gemv_kernel_qkv(const dlk_gemv_params& p, int mt);
dlk::gemv::Kernel dlk_gemv_kernel_swiglu(const dlk_gemv_params& p, int mt);
dlk::gemv::Kernel dlk_gemv_kernel_logits(const dlk_gemv_params& p, int mt);
