// Projection GEMV for the decode step (see dlk_gemv_params in kernels.h).
//
// Work split: one 256-thread work-group (4 wave64) owns ROWS consecutive weight rows.  Each thread streams
// 16-byte chunks c = t, t+256, ... of all ROWS rows (coalesced: the 256 threads of a WG read 4 KB of one
// row per instruction), multiplies them with the matching f32 chunk of every activation row (L1/L2
// resident), and accumulates f32.  Partial sums are reduced across the wave with cross-lane shuffles and
// across the 4 waves through LDS; the fused epilogue (RMSNorm scale, residual, RoPE + KV append, SiLU*up,
// logits + sampling candidates) runs on the reduced values, so no intermediate ever round-trips to HBM.
// The bytes that matter are the weights: each weight byte is read exactly once per launch.
#include "kernels/device_common.h"

#include <algorithm>

namespace dlk {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;
constexpr int kUnroll = 2;
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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

template <typename WT, int MT, int ROWS, int EPI>
__global__ __launch_bounds__(kThreads) void gemv_kernel(const dlk_gemv_params p) {
    using Traits = WeightTraits<WT>;
    constexpr int CH = Traits::chunk;
    constexpr int OUTS = EPI == DLK_EPI_SWIGLU ? ROWS / 2 : ROWS;
    constexpr int NV = MT * ROWS + MT; // reduced values: accumulators then sums of squares
    __shared__ float partial[kWaves][NV];
    __shared__ float reduced[NV];
    __shared__ float staged[MT * ROWS];

    const int K = p.K;
    const int nch = K / CH;
    const int t = threadIdx.x;

    // locate this block's segment and first output row
    int block = blockIdx.x;
    int seg = 0;
    if constexpr (EPI != DLK_EPI_SWIGLU) {
        while (seg + 1 < p.nseg) {
            const int blocks = (p.seg_rows[seg] + OUTS - 1) / OUTS;
            if (block < blocks) break;
            block -= blocks;
            ++seg;
        }
    }
    const int n0 = block * OUTS;
    const int seg_rows = p.seg_rows[seg];

    const u32x4* wrow[ROWS];
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
        const void* base = p.w[seg];
        int n = n0 + r;
        if constexpr (EPI == DLK_EPI_SWIGLU) {
            base = r < OUTS ? p.w[0] : p.w[1];
            n = n0 + (r % OUTS);
        }
        n = n < seg_rows ? n : seg_rows - 1;
        wrow[r] = reinterpret_cast<const u32x4*>(static_cast<const WT*>(base) + static_cast<int64_t>(n) * K);
    }
    const float* xrow[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) xrow[m] = p.x + static_cast<int64_t>(m < p.M ? m : p.M - 1) * p.ldx;

    float acc[MT][ROWS];
    float squares[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        squares[m] = 0.0f;
#pragma unroll
        for (int r = 0; r < ROWS; ++r) acc[m][r] = 0.0f;
    }
    const bool norm = p.apply_norm != 0;
    const bool norm_affine = p.norm_weight != nullptr;

    for (int c0 = 0; c0 < nch; c0 += kThreads * kUnroll) {
        u32x4 wv[kUnroll][ROWS];
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * kThreads + t;
#pragma unroll
            for (int r = 0; r < ROWS; ++r)
                wv[u][r] = c < nch ? __builtin_nontemporal_load(wrow[r] + c) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int c = c0 + u * kThreads + t;
            if (c >= nch) break;
            float g[CH];
            if (norm) {
                if (!norm_affine) {
#pragma unroll
                    for (int i = 0; i < CH; ++i) g[i] = 1.0f;
                } else if (p.norm_bf16) {
                    const uint16_t* gw = static_cast<const uint16_t*>(p.norm_weight) + c * CH;
#pragma unroll
                    for (int i = 0; i < CH; i += 4) {
                        const uint2 gv = *reinterpret_cast<const uint2*>(gw + i);
                        g[i] = bf16_lo(gv.x); g[i + 1] = bf16_hi(gv.x); g[i + 2] = bf16_lo(gv.y); g[i + 3] = bf16_hi(gv.y);
                    }
                } else {
                    const float* gw = static_cast<const float*>(p.norm_weight) + c * CH;
#pragma unroll
                    for (int i = 0; i < CH; i += 4) {
                        const float4 gv = *reinterpret_cast<const float4*>(gw + i);
                        g[i] = gv.x; g[i + 1] = gv.y; g[i + 2] = gv.z; g[i + 3] = gv.w;
                    }
                }
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                float xs[CH];
#pragma unroll
                for (int i = 0; i < CH; i += 4) {
                    const float4 xv = *reinterpret_cast<const float4*>(xrow[m] + c * CH + i);
                    xs[i] = xv.x; xs[i + 1] = xv.y; xs[i + 2] = xv.z; xs[i + 3] = xv.w;
                }
                if (norm) {
#pragma unroll
                    for (int i = 0; i < CH; ++i) {
                        squares[m] += xs[i] * xs[i];
                        xs[i] *= g[i];
                    }
                }
#pragma unroll
                for (int r = 0; r < ROWS; ++r) acc[m][r] += Traits::dot(wv[u][r], xs);
            }
        }
    }

    // reduction: wave butterflies, then the 4 waves through LDS
    const int lane = t % kWave, wave = t / kWave;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
            const float v = wave_sum(acc[m][r]);
            if (lane == 0) partial[wave][m * ROWS + r] = v;
        }
        if (norm) {
            const float v = wave_sum(squares[m]);
            if (lane == 0) partial[wave][MT * ROWS + m] = v;
        }
    }
    __syncthreads();
    if (t < NV) {
        float s = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) s += partial[w][t];
        reduced[t] = s;
    }
    __syncthreads();

    auto scale_of = [&](int m) -> float {
        return (norm ? rsqrtf(reduced[MT * ROWS + m] / static_cast<float>(K) + p.epsilon) : 1.0f) * p.acc_scale;
    };

    if constexpr (EPI == DLK_EPI_STORE || EPI == DLK_EPI_RESIDUAL) {
        if (t < MT * ROWS) {
            const int m = t / ROWS, r = t % ROWS, n = n0 + r;
            if (m < p.M && n < seg_rows) {
                float v = reduced[t] * scale_of(m);
                if constexpr (EPI == DLK_EPI_STORE) {
                    if (p.bias) v += p.bias_bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p.bias)[n])
                                                 : static_cast<const float*>(p.bias)[n];
                    p.y[static_cast<int64_t>(m) * p.ldy + n] = v;
                } else {
                    p.y[static_cast<int64_t>(m) * p.ldy + n] = p.residual[static_cast<int64_t>(m) * p.ldres + n] + v;
                }
            }
        }
        // the device cache length advances once the attention launch that read it has completed
        if (p.bump_position && blockIdx.x == 0 && t == 0) *p.bump_position += p.bump_count;
    } else if constexpr (EPI == DLK_EPI_SWIGLU) {
        if (t < MT * OUTS) {
            const int m = t / OUTS, j = t % OUTS, n = n0 + j;
            if (m < p.M && n < seg_rows) {
                const float s = scale_of(m);
                const float gate = reduced[m * ROWS + j] * s;
                const float up = reduced[m * ROWS + OUTS + j] * s;
                p.y[static_cast<int64_t>(m) * p.ldy + n] = silu(gate) * up;
            }
        }
    } else if constexpr (EPI == DLK_EPI_QKV) {
        const int64_t first = *p.position;
        if (t < MT * ROWS) {
            const int m = t / ROWS, r = t % ROWS, n = n0 + r;
            float v = reduced[t] * scale_of(m);
            const float* hidden = p.lora_hidden[seg];
            if (hidden && m < p.M && n < seg_rows) {
                const int64_t mg = p.m_base + m;
                const float* hrow = hidden + mg * p.lora_rank;
                float delta = 0.0f;
                for (int j = 0; j < p.lora_rank; ++j)
                    delta += Traits::scalar(p.lora_up[seg], static_cast<int64_t>(n) * p.lora_rank + j) * hrow[j];
                v += delta * p.lora_scale;
            }
            staged[t] = v;
        }
        __syncthreads();
        if (t < MT * ROWS) {
            const int m = t / ROWS, r = t % ROWS, n = n0 + r;
            if (m < p.M && n < seg_rows) {
                const int64_t mg = p.m_base + m;
                const int64_t b = mg / p.length, l = mg % p.length;
                const int64_t pos = first + l;
                const int hd = p.head_dim;
                const int d = n % hd;
                float v = staged[t];
                if (seg < 2) {
                    const float partner = staged[t ^ 1];
                    const int64_t table = pos * (hd / 2) + d / 2;
                    const float c = p.cosine[table], s = p.sine[table];
                    // even: x_e c - x_o s ; odd: x_e s + x_o c (interleaved pairs, src/ops/contraction.cpp:44-49)
                    v = (d & 1) == 0 ? v * c - partner * s : partner * s + v * c;
                }
                if (seg == 0) {
                    p.y[mg * p.ldy + n] = v;
                } else {
                    const int head = n / hd;
                    const int64_t index = ((b * p.kv_heads + head) * p.cache_capacity + pos) * hd + d;
                    void* cache = seg == 1 ? p.k_cache : p.v_cache;
                    if (p.cache_bf16) static_cast<uint16_t*>(cache)[index] = f32_to_bf16(v);
                    else static_cast<float*>(cache)[index] = v;
                }
            }
        }
    } else if constexpr (EPI == DLK_EPI_LOGITS) {
        __shared__ double cand_score[MT * ROWS];
        __shared__ int64_t cand_index[MT * ROWS];
        uint64_t seed = p.key_seed, stream = p.key_stream;
        if (p.key_label) fold_in(p.key_seed, p.key_stream, static_cast<uint64_t>(*p.key_label), seed, stream);
        if (t < MT * ROWS) {
            const int m = t / ROWS, r = t % ROWS, n = n0 + r;
            int64_t index = -1;
            double score = 0.0;
            if (m < p.M && n < seg_rows) {
                const float v = reduced[t] * scale_of(m);
                if (p.y) p.y[static_cast<int64_t>(m) * p.ldy + n] = v;
                const int64_t mg = p.m_base + m;
                index = n;
                score = sample_score(v, p.sample_mode, p.temperature, seed, stream,
                                     static_cast<uint64_t>(mg * seg_rows + n));
            }
            cand_score[t] = score;
            cand_index[t] = index;
        }
        __syncthreads();
        if (p.sample_mode != 0 && t < MT && t < p.M) {
            double best = 0.0;
            int64_t best_index = -1;
            for (int r = 0; r < ROWS; ++r) {
                const int64_t i = cand_index[t * ROWS + r];
                if (i < 0) continue;
                const double s = cand_score[t * ROWS + r];
                if (best_index < 0 || prefer(s, i, best, best_index)) { best = s; best_index = i; }
            }
            dlk_sample_partial out;
            out.score = best;
            out.index = best_index;
            p.partial[(p.m_base + t) * p.partial_blocks + blockIdx.x] = out;
        }
    }
}

template <typename WT, int MT, int ROWS, int EPI>
int launch_typed(const dlk_gemv_params& p, int blocks, hipStream_t stream) {
    hipLaunchKernelGGL((gemv_kernel<WT, MT, ROWS, EPI>), dim3(blocks), dim3(kThreads), 0, stream, p);
    return static_cast<int>(hipGetLastError());
}

template <typename WT, int ROWS, int EPI>
int launch_mt(const dlk_gemv_params& p, int blocks, hipStream_t stream) {
    if (p.M <= 1) return launch_typed<WT, 1, ROWS, EPI>(p, blocks, stream);
    if (p.M <= 2) return launch_typed<WT, 2, ROWS, EPI>(p, blocks, stream);
    if (p.M <= 4) return launch_typed<WT, 4, ROWS, EPI>(p, blocks, stream);
    return launch_typed<WT, 8, ROWS, EPI>(p, blocks, stream);
}

template <int ROWS, int EPI>
int launch_w(const dlk_gemv_params& p, int blocks, hipStream_t stream) {
    return p.w_bf16 ? launch_mt<uint16_t, ROWS, EPI>(p, blocks, stream) : launch_mt<float, ROWS, EPI>(p, blocks, stream);
}

constexpr int kMaxRowsPerLaunch = 8;

int rows_per_block(const dlk_gemv_params* p) {
    // SwiGLU pairs 4 gate rows with 4 up rows; QKV needs even rows for the RoPE pairs.  Other epilogues use
    // 4 rows when that still gives >= 2 work-groups per CU-slot of the chip, else 8.
    (void)p;
    return p->epilogue == DLK_EPI_SWIGLU ? 8 : 4;
}

} // namespace
} // namespace dlk

extern "C" int dlk_gemv_blocks(const dlk_gemv_params* p) {
    const int rows = dlk::rows_per_block(p);
    const int outs = p->epilogue == DLK_EPI_SWIGLU ? rows / 2 : rows;
    if (p->epilogue == DLK_EPI_SWIGLU) return (p->seg_rows[0] + outs - 1) / outs;
    int blocks = 0;
    for (int s = 0; s < p->nseg; ++s) blocks += (p->seg_rows[s] + outs - 1) / outs;
    return blocks;
}

extern "C" int dlk_gemv(const dlk_gemv_params* params, dlh_stream stream_handle) {
    hipStream_t stream = reinterpret_cast<hipStream_t>(stream_handle);
    const int chunk = params->w_bf16 ? 8 : 4;
    if (params->K <= 0 || params->K % chunk != 0 || params->M <= 0) return static_cast<int>(hipErrorInvalidValue);
    if (params->epilogue == DLK_EPI_SWIGLU && (params->nseg != 2 || params->seg_rows[0] != params->seg_rows[1]))
        return static_cast<int>(hipErrorInvalidValue);
    const int blocks = dlk_gemv_blocks(params);
    const int rows = dlk::rows_per_block(params);
    dlk_gemv_params p = *params;
    // activation rows are processed kMaxRowsPerLaunch at a time (weights re-streamed per group)
    for (int m0 = 0; m0 < params->M; m0 += dlk::kMaxRowsPerLaunch) {
        p.M = std::min(dlk::kMaxRowsPerLaunch, params->M - m0);
        p.x = params->x + static_cast<int64_t>(m0) * params->ldx;
        p.m_base = params->m_base + m0;
        if (params->epilogue != DLK_EPI_QKV) p.y = params->y ? params->y + static_cast<int64_t>(m0) * params->ldy : nullptr;
        if (params->residual) p.residual = params->residual + static_cast<int64_t>(m0) * params->ldres;
        p.bump_position = m0 + dlk::kMaxRowsPerLaunch >= params->M ? params->bump_position : nullptr;
        int status = 0;
        switch (params->epilogue) {
        case DLK_EPI_STORE: status = rows == 4 ? dlk::launch_w<4, DLK_EPI_STORE>(p, blocks, stream)
                                               : dlk::launch_w<8, DLK_EPI_STORE>(p, blocks, stream); break;
        case DLK_EPI_RESIDUAL: status = rows == 4 ? dlk::launch_w<4, DLK_EPI_RESIDUAL>(p, blocks, stream)
                                                  : dlk::launch_w<8, DLK_EPI_RESIDUAL>(p, blocks, stream); break;
        case DLK_EPI_QKV: status = rows == 4 ? dlk::launch_w<4, DLK_EPI_QKV>(p, blocks, stream)
                                             : dlk::launch_w<8, DLK_EPI_QKV>(p, blocks, stream); break;
        case DLK_EPI_SWIGLU: status = dlk::launch_w<8, DLK_EPI_SWIGLU>(p, blocks, stream); break;
        case DLK_EPI_LOGITS: status = rows == 4 ? dlk::launch_w<4, DLK_EPI_LOGITS>(p, blocks, stream)
                                                : dlk::launch_w<8, DLK_EPI_LOGITS>(p, blocks, stream); break;
        default: return static_cast<int>(hipErrorInvalidValue);
        }
        if (status != 0) return status;
    }
    return 0;
}
