// Launch entries of the hand-written CDNA4 kernels (gfx950).  Plain C structs of device pointers, sizes and a
// stream; each entry returns 0 or a HIP error code.  The host C++ layers fill these from tensors.
#pragma once

#include "backends/hip_backend.h"

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* element codes follow dl_dtype */
enum { DLK_F32 = 0, DLK_F64 = 1, DLK_I64 = 2, DLK_BOOL = 3, DLK_BF16 = 5 };

/* ------------------------------------------------------------------------------------------------------
 * Projection GEMV over bf16 (or f32) weights, f32 activations and f32 accumulation:
 *   y[m, n] = epilogue( s_m * sum_k x[m, k] * g[k] * W[n, k] )
 * with g = the RMSNorm weight and s_m = 1/sqrt(mean_k x[m,k]^2 + eps) when apply_norm (the preceding RMSNorm
 * fused into this launch), else g = 1, s_m = 1.
 * Replaces the reference's cast_pair upcast + cuBLAS GEMM of every decoder Linear
 * (src/ops/matmul.cpp:14-67, src/kernels/cuda/matmul.cpp:9-93) and the RMSNorm/RoPE/KV-append/SiLU/residual
 * passes around them (src/kernels/cuda/normalization.cu:12-42, pointwise.cu:38-44,147-153,267-281).
 * ---------------------------------------------------------------------------------------------------- */
enum {
    DLK_EPI_STORE = 0,    /* y = acc (+ bias); optionally advances *bump_position by bump_count */
    DLK_EPI_RESIDUAL = 1, /* y = residual + acc; optionally advances *bump_position by bump_count */
    DLK_EPI_QKV = 2,      /* segments q|k|v: (+LoRA) RoPE on q,k; q -> y, k,v -> cache at position + l */
    DLK_EPI_SWIGLU = 3,   /* segments gate|up: y = silu(gate) * up */
    DLK_EPI_LOGITS = 4    /* y = acc; per-block best (value, index) for greedy / Gumbel-max sampling */
};

typedef struct dlk_sample_partial {
    double score;
    int64_t index;
} dlk_sample_partial;

typedef struct dlk_gemv_params {
    const float* x;         /* [M, ldx] f32 */
    int64_t ldx;
    int M, K;
    int nseg;               /* 1..3 weight segments stacked along n (STORE: their outputs side by side in y) */
    const void* w[3];       /* [seg_rows[i], K] row-major */
    const void* w_tiles[3]; /* optional, bf16: segment i repacked by dlk_pack_tiles, which the batched matrix-core
                               path reads instead of w (1 KB contiguous per load instruction) */
    int seg_rows[3];
    int w_bf16;
    int apply_norm;         /* fuse the preceding RMSNorm: scale row m by 1/sqrt(mean(x^2)+eps), weight g */
    const void* norm_weight; /* RMSNorm weight [K] (f32, or bf16 when norm_bf16); NULL means g = 1 */
    int norm_bf16;
    float epsilon;
    float acc_scale;        /* multiplies the accumulated dot products (1 for a plain projection) */
    int epilogue;
    float* y;               /* output rows [M, ldy] (QKV: the q rows) */
    int64_t ldy;
    const float* residual;  /* RESIDUAL: [M, ldres] f32 (may alias y) */
    int64_t ldres;
    const void* bias;       /* STORE: optional [N] */
    int bias_bf16;
    int64_t m_base;         /* global row of x row 0 (QKV position mapping, sample partial rows) */
    /* QKV */
    int head_dim, kv_heads, length; /* global row m -> batch m / length, position *position + m % length */
    const float* cosine;    /* [capacity, head_dim/2] f32 */
    const float* sine;
    const int64_t* position;
    void* k_cache;          /* [B, kv_heads, capacity, head_dim] */
    void* v_cache;
    int cache_bf16;
    int64_t cache_capacity;
    const float* lora_hidden[3]; /* per segment: [M_total, rank] f32 hidden = down(norm(x)) or NULL */
    int64_t lora_ld;             /* row stride of the lora_hidden rows (0: lora_rank) */
    const void* lora_up[3];      /* per segment: [seg_rows, rank] */
    const void* lora_down[3];    /* per segment: [rank, K] bf16 down rows that the launch applies itself (its
                                    lora_hidden NULL), when dlk_gemv_folds_lora says it can; else NULL */
    int lora_rank;
    float lora_scale;
    /* STORE / RESIDUAL: device cache length advanced by one thread after the launch's reads of it */
    int64_t* bump_position;
    int64_t bump_count;
    /* LOGITS */
    int sample_mode;        /* 0: none, 1: greedy, 2: Gumbel-max */
    double temperature;
    uint64_t key_seed, key_stream;
    const int64_t* key_label; /* if set, the key is fold_in(key, *key_label) */
    dlk_sample_partial* partial; /* [M_total, blocks] */
    int partial_blocks;
    /* Workspace for key-split launches of the matrix-core path (NULL: never split): partial dot products and
     * per-row sums of squares of each key slice, reduced in fixed order by a second launch. */
    float* split_partial;
    int64_t split_capacity; /* floats */
    /* Workspace of the tiled (prefill) path: a preparation launch writes the activation rows (times the norm
     * weight) split into bf16 hi + lo rows and the per-row norm factors.  NULL: many-row launches take the
     * batched matrix-core path (64 rows per launch) instead. */
    void* stage;
    int64_t stage_bytes;
    int stage_ready;        /* the workspace already holds this launch's split rows (same x, norm weight, M, K) */
    int row_parts;          /* set by dlk_gemv for a launch it splits over activation rows (callers leave 0) */
    int defer_reduce;       /* QKV on the key-split matrix-core path: leave the partials for the one-position
                               attention to finish (no reduce launch); see dlk_attention_params.qkv_partial */
    void* stage_out;        /* SWIGLU on the tiled path: write silu(gate) * up, split into bf16 hi + lo, in the
                               staging layout of a following tiled launch over these rows (K = seg_rows[0]) instead
                               of y; that launch then takes it as its stage with stage_ready set */
} dlk_gemv_params;

/* Repacks bf16 weights for the batched matrix-core path: for each 16-row tile and 32-wide k step a 1 KB block
   whose 16 bytes at 16 l hold tile row l % 16, columns 32 s + 8 (l / 16) .. +8 (the MFMA operand of lane l).
   swiglu = 0: rows of w0 [rows, K], tile t = rows 16 t .. +16.  swiglu = 1: w0 = gate, w1 = up, each [rows, K];
   tile t interleaves gate and up rows 8 t .. +8 (tile row 2 j: gate 8 t + j, 2 j + 1: up 8 t + j).  out holds
   rows * K (swiglu: 2 * rows * K) bf16. */
int dlk_pack_tiles(const void* w0, const void* w1, int swiglu, int64_t rows, int64_t K, void* out, dlh_stream stream);
/* 1 when dlk_gemv takes a batched matrix-core kernel (gemm_rows or gemm_wide, which read w_tiles) for this
   launch. */
int dlk_gemv_uses_rows(const dlk_gemv_params* p);
/* 1 when this QKV launch, with lora_down set for its adapted segments (and their lora_hidden NULL), computes the
   LoRA down projections itself: a launch over at most 16 rows on the few-row matrix-core kernel, bf16 weights,
   rank 4..16 in steps of 4, acc_scale 1.  dlk_gemv refuses lora_down otherwise. */
int dlk_gemv_folds_lora(const dlk_gemv_params* p);
/* Floats of workspace that lets dlk_gemv split the keys of this launch (0 when it would not split). */
int64_t dlk_gemv_split_floats(const dlk_gemv_params* p);
/* Key slices dlk_gemv will use for this launch as attached (1: no split). */
int dlk_gemv_split_count(const dlk_gemv_params* p);
/* Bytes of staging workspace that lets this launch take the tiled (prefill) path: attach it as stage /
   stage_bytes (0 when the shape does not suit that path). */
int64_t dlk_gemv_stage_bytes(const dlk_gemv_params* p);

/* Work-groups of the persistent launch (the LOGITS partial row length: one sampling candidate per work-group);
   -1 when no kernel fits the parameters.  Depends on the current device's CU count and the kernel's occupancy. */
int dlk_gemv_blocks(const dlk_gemv_params* p);
int dlk_gemv(const dlk_gemv_params* p, dlh_stream stream);

/* ------------------------------------------------------------------------------------------------------
 * Split-K GQA decode attention (flash-decoding).  Q rows m = b*L + l of [B*L, H*hd] f32 (post-RoPE);
 * K/V cache [B, KV, capacity, hd] (bf16 or f32, keys already rotated); first = *position (or first_host);
 * S = first + L keys; causal: row l sees keys <= first + l.  One work-group per (key split, query-row
 * block, b, kv head) stages 64-key K/V tiles in LDS and serves all H/KV query heads of that KV head.
 * Replaces grouped_block + attention_weights (src/ops/attention.cpp:65-95) i.e. two batched cuBLAS GEMMs
 * and attention_softmax_kernel (src/kernels/cuda/reduction.cu:149-169).
 * ---------------------------------------------------------------------------------------------------- */
typedef struct dlk_attention_params {
    const float* q;
    int64_t ldq;
    const void* k;
    const void* v;
    int kv_bf16;
    int64_t capacity;        /* rows per (b, kv head) in the K/V storage */
    const int64_t* position; /* device length before this chunk, or NULL to use first_host */
    int64_t first_host;
    int B, L, H, KV, hd;
    float scale;
    int causal;
    float* out;              /* [B*L, ldo] f32, head h at columns h*hd */
    int64_t ldo;
    int splits;              /* key splits; > 1 needs partial buffers */
    int chunk;               /* keys per split (multiple of the tile) */
    float* partial_o;        /* [B*H*L, splits, hd] */
    float* partial_ml;       /* [B*H*L, splits, 2] */
    int partials_only;       /* splits > 1: leave the merge of the partials to the caller (no combine launch) */
    /* One position on the matrix-core kernel: the QKV projection's key-split partials, left unreduced by it
       (dlk_gemv_params.defer_reduce).  The attention sums them in slice order for its sequence's q, k and v
       columns, applies the RMSNorm factor (row sums of squares after the dots) and RoPE at *position, and writes
       the new K/V row into the cache at *position (and uses the finished row for that key in place of the cache's).  Layout: [qkv_splits][B][qkv_width]
       dot products (q columns, then k, then v), then [qkv_splits][B] sums of squares. */
    const float* qkv_partial;
    int qkv_splits, qkv_width, qkv_K, qkv_norm;
    float qkv_scale, qkv_epsilon;
    const float* rope_cos;   /* [capacity, hd/2] */
    const float* rope_sin;
    void* stage_out;         /* prefill kernel only: write the output rows (row b * L + l, K = H * hd) split into
                                bf16 hi + lo in the staging layout of the tiled projection that reads them, instead
                                of out (see dlk_gemv_params.stage_out) */
    void* kv_split;          /* prefill kernel over an f32 cache: dlk_attention_split_bytes of workspace
                                (kv_split_tiles 64-key tiles per (b, kv head), covering the capacity).  A preparation
                                launch splits the live K/V tiles into bf16 hi + lo planes once, and the attention
                                copies them into LDS as they are instead of splitting each tile it reads */
    int kv_split_tiles;
    /* Explicit keep mask (reference grouped_query_attention, src/ops/attention.cpp:48-50,156-183), or NULL: bool
       bytes, key s of query row (b, h, l) kept when keep_mask[b * mask_stride[0] + h * mask_stride[1] +
       l * mask_stride[2] + s * mask_stride[3]] is nonzero (element strides, 0 on broadcast axes).  A dropped key's
       score is -inf before the softmax, and a row that keeps no key comes out NaN, as the reference's softmax of
       an all -inf row does.  Taken by the general and small-head kernels only (not causal, not the matrix-core or
       prefill kernels). */
    const unsigned char* keep_mask;
    int64_t mask_stride[4];
    /* Matrix-core decode kernel: keys the caller knows the cache holds at this launch (its host length plus the
       new position: the capture-time count for a replayed graph, whose length only grows), or 0.  A wave whose run
       of keys starts below it requests its first K/V tile before it reads the device length.  A hint for speed
       only: any value gives the same result. */
    int64_t early_keys;
} dlk_attention_params;

/* Keys per split of a short one-position decode over a bf16 cache (few keys in all): 256 or 512, one work-group. */
#define DLK_DECODE_CHUNK_MAX 512
/* One-position decodes over at least this many keys in all (B * KV * keys), or over an f32 cache, split the keys
   into runs of 64..256 keys per wave (~4096 runs in all; a work-group per (sequence, KV head) from 256 pairs). */
#define DLK_STREAM_DECODE_KEYS 32768
/* 1 when the matrix-core one-position kernel serves this head layout (head dim 64 or 128, H/KV <= 16). */
int dlk_attention_matrix_heads(int heads, int kv_heads, int head_dim);


int dlk_attention(const dlk_attention_params* p, dlh_stream stream);
/* Floats of the device-resident scratch array behind the allocation-free attention entry (8 MiB per GPU). */
#define DLK_ATTENTION_SCRATCH_FLOATS (2 << 20)
/* The address of that array on GPU `device` (looked up once per device with the device current; later calls
   return the kept address). */
int dlk_attention_scratch(int device, float** address);
/* The matrix-core causal prefill kernel (attention_prefill.hip), which dlk_attention takes for causal launches
   over bf16 or f32 K/V, head dim 64 or 128, L >= 16 new positions, one split and H/KV dividing 128. */
int dlk_attention_prefill_eligible(const dlk_attention_params* p);
/* One position on the matrix cores (attention_matrix.hip): eligibility, and the launch of the attention kernel
   alone (with several splits it writes the partials; dlk_attention adds the merge). */
int dlk_attention_matrix_eligible(const dlk_attention_params* p);
int dlk_attention_matrix_decode(const dlk_attention_params* p, dlh_stream stream);
int dlk_attention_prefill(const dlk_attention_params* p, dlh_stream stream);
/* Bytes of kv_split workspace for these parameters: the capacity's 64-key tiles of every (b, kv head) as bf16
   hi + lo planes of K and V^T (0: no such path, a bf16 cache or not the prefill kernel). */
int64_t dlk_attention_split_bytes(const dlk_attention_params* p);

/* ------------------------------------------------------------------------------------------------------
 * Small kernels of the token loop and the tensor API.
 * ---------------------------------------------------------------------------------------------------- */
/* Strided copy with dtype conversion: dst[idx(dst_strides)] = convert(src[idx(src_strides)]), rank <= 8. */
int dlk_copy(const void* src, int src_dtype, const int64_t* src_strides, void* dst, int dst_dtype,
             const int64_t* dst_strides, const int64_t* shape, int rank, dlh_stream stream);
int dlk_fill(void* dst, int dtype, int64_t count, double value, dlh_stream stream);
/* Embedding rows: out[i, :] = weight[ids[i], :] converted to out_dtype; ids outside [0, V) give a zero row
 * and set *error_flag (if given) to 1. */
int dlk_embedding(const int64_t* ids, int64_t count, const void* weight, int weight_dtype, int64_t vocabulary,
                  int64_t width, void* out, int out_dtype, int32_t* error_flag, dlh_stream stream);
/* y[r, :] = x[r, :] / sqrt(mean(x^2) + eps) * weight (weight f32 or bf16, may be NULL); f32 in and out. */
int dlk_rms_norm(const float* x, int64_t rows, int64_t width, const void* weight, int weight_bf16, float epsilon,
                 float* y, dlh_stream stream);
/* Interleaved RoPE on contiguous x [outer, L, D] f32 with tables [L, D/2]. */
int dlk_rope(const float* x, int64_t outer, int64_t length, int64_t dim, const float* cosine, const float* sine,
             float* y, dlh_stream stream);
/* First maximum of each row (NaN first); x [rows, n] f32 contiguous -> out i64 [rows]. */
int dlk_argmax(const float* x, int64_t rows, int64_t n, int64_t* out, dlh_stream stream);
/* Per-block candidates of a [rows, n] logits matrix (greedy or Gumbel-max), for dlk_sample_finalize. */
int dlk_sample_partials(const float* logits, int64_t rows, int64_t n, int mode, double temperature,
                        uint64_t key_seed, uint64_t key_stream, const int64_t* key_label,
                        dlk_sample_partial* partial, int blocks, dlh_stream stream);
int dlk_sample_blocks(int64_t n);
/* Reduces partial [rows, blocks] to ids: out[r] (may be NULL), next_ids[r] (may be NULL), and
 * tokens[r * token_stride + *step] when tokens != NULL; then advances *step by one if step != NULL.
 * With embedding != NULL it also writes the next step's input rows x[r, :] = f32(embedding[id, :]). */
int dlk_sample_finalize(const dlk_sample_partial* partial, int64_t rows, int blocks, int64_t* out,
                        int64_t* next_ids, int64_t* tokens, int64_t token_stride, int64_t* step,
                        const void* embedding, int embedding_dtype, int64_t width, float* x, dlh_stream stream);
/* Keyed Philox: mode 0 uniform [low, high), mode 1 standard normal times scale; output f32 or bf16. */
int dlk_random(uint64_t seed, uint64_t stream_bits, int64_t count, int mode, double low, double high,
               double scale, void* out, int out_dtype, dlh_stream stream);
/* Plain y = x W^T (+ bias) for shapes the GEMV cannot take (K not a multiple of the 16-byte chunk). */
int dlk_linear_generic(const float* x, int64_t rows, int64_t K, const void* w, int w_dtype, int64_t N,
                       const void* bias, int bias_dtype, float* y, dlh_stream stream);
/* Streaming copy of `bytes` (multiple of 16) for the bandwidth probe. */
int dlk_stream_copy(const void* src, void* dst, uint64_t bytes, dlh_stream stream);

#ifdef __cplusplus
}
#endif
