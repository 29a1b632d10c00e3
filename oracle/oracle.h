/*
 * CPU oracle for the Ctorch decoder token loop — TEST INFRASTRUCTURE ONLY.
 *
 * This is a plain-C17 restatement of the arithmetic of the reference CPU path
 * (Ctorch, reference tree under /root/reference).  It exists so that tests,
 * the smoke check and the bench's cpu_baseline leg can check the HIP product
 * against the reference's numerics.  Nothing in the product (ctorch_amd/,
 * include/) includes, links or loads it.
 *
 * Every function cites the reference file:line it restates.  Build with
 * -O3 -ffp-contract=off so that no multiply-add is contracted: the reference
 * is compiled for baseline x86-64 (no FMA), and its f32 dot products are
 * sequential in k (src/kernels/cpu/matmul.h:10-22).
 *
 * Parity pins (see tests/test_oracle.py):
 *   philox          Random123 philox4x32-10 known-answer vectors
 *   bf16 codec      exhaustive round trip + torch's RNE conversion
 *   rope tables     closed form in float64, pair-norm invariance
 *   rms_norm        float64 closed form
 *   linear          float64 matmul; exact on integer-valued inputs
 *   softmax         scipy softmax; trailing -inf -> exact 0; single key -> 1
 *   attention       torch float64 SDPA with GQA + causal window
 *   argmax          numpy argmax (first max, first NaN) brute force
 *   decoder         chunked decode == full forward (tests/state.cpp:55-70),
 *                   truncate/rollback, and a float64 torch restatement
 *   sample          Gumbel-max frequencies vs softmax (chi-square), T->0 ==
 *                   argmax, portable log vs math.log
 *   lora            adapter output == merged weight output (tests/state.cpp:71-75)
 */
#ifndef CTORCH_ORACLE_H
#define CTORCH_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_BF16 = 5 }; /* dtype codes follow include/dl/types.h:15 of the reference */

void orc_set_threads(int threads);
int orc_get_threads(void);

/* ---- keyed randomness: src/core/philox.h:26-52, src/core/random.cpp:14-27 ---- */
void orc_philox(uint64_t seed, uint64_t index, uint64_t stream, uint32_t out[4]);
void orc_fold_in(uint64_t seed, uint64_t stream, uint64_t label, uint64_t out[2]);
float orc_unit_f32(uint32_t first, int open_left);
double orc_unit_f64(uint32_t first, uint32_t second, int open_left);
/* src/kernels/cpu/random.cpp:52-83 (keyed uniform / normal, f32) */
void orc_uniform_f32(uint64_t seed, uint64_t stream, int64_t count, double low, double high, float* out);
void orc_randn_f32(uint64_t seed, uint64_t stream, int64_t count, float* out);
/* token ids in [0, vocab): (u32 Philox x * vocab) >> 32 (harness definition) */
void orc_random_ids(uint64_t seed, uint64_t stream, int64_t count, int64_t vocab, int64_t* out);

/* ---- bf16 codec: include/dl/half.h:43-47,60-66 ---- */
uint16_t orc_bf16_encode(float value);
float orc_bf16_decode(uint16_t bits);
void orc_bf16_encode_n(const float* input, int64_t count, uint16_t* output);
void orc_bf16_decode_n(const uint16_t* input, int64_t count, float* output);
/* weight synthesis: w = scale * randn (numeric::scale semantics, f32), optionally RNE to bf16 */
void orc_normal_weights(uint64_t seed, uint64_t stream, int64_t count, double scale, int dtype, void* out);

/* ---- building blocks ---- */
/* src/nn/decoder.cpp:38-46 + RotaryEmbedding ctor :48-52: tables [capacity, hd/2] f32 */
void orc_rope_tables(int64_t head_dim, int64_t capacity, double base, float* cosine, float* sine);
/* src/kernels/cpu/normalization.cpp:21-56 with moments.h:12-24 (centered=false); weight may be NULL */
void orc_rms_norm(const float* x, int64_t rows, int64_t width, const float* weight, double epsilon, float* y);
/* src/ops/matmul.cpp:35-67 -> numeric.cpp:199-209 -> cpu/matmul.h:10-22; W [out,in] f32 or bf16 */
void orc_linear(const float* x, int64_t rows, int64_t in, const void* weight, int wdtype, int64_t out, float* y);
/* src/ops/contraction.cpp:44-49: x [rows, heads, hd] rotated in place; row r uses table row positions[r] */
void orc_rope(float* x, int64_t rows, int64_t heads, int64_t head_dim, const float* cosine, const float* sine,
              const int64_t* positions);
/* src/kernels/cpu/reduction.cpp:155-203 (non-log softmax over one row) */
void orc_softmax_row(const float* x, int64_t n, float* y);
/* src/kernels/cpu/reduction.cpp:128-151 */
int64_t orc_argmax_row(const float* x, int64_t n);
/* src/kernels/cpu/pointwise.cpp:31-34,57 */
float orc_silu(float v);
/* src/ops/attention.cpp:65-95,161-188: q [B,H,L,hd]; k,v [B,KV,*,hd] with row stride kv_stride (>= S)
 * per (b,kvh); S visible keys; causal_first < 0 disables the causal window. out [B,H,L,hd] */
void orc_attention(const float* q, const float* k, const float* v, int64_t batch, int64_t heads, int64_t kv_heads,
                   int64_t length, int64_t source, int64_t kv_stride, int64_t head_dim, int64_t causal_first,
                   float* out);
/* the same with a keep mask (src/ops/attention.cpp:48-50,156-183): bool bytes read at b*st[0] + h*st[1] + l*st[2]
 * + s*st[3] (strides in elements, 0 on broadcast axes); a dropped key's scaled score becomes -inf before the
 * softmax, so a row that keeps no key comes out NaN (the reference softmax over an all -inf row) */
void orc_attention_masked(const float* q, const float* k, const float* v, int64_t batch, int64_t heads,
                          int64_t kv_heads, int64_t length, int64_t source, int64_t kv_stride, int64_t head_dim,
                          int64_t causal_first, const uint8_t* mask, const int64_t* mask_strides, float* out);

/* ---- sampling (the build's new op; no reference counterpart, see a13) ---- */
double orc_log(double x);                       /* portable natural log: atanh series, basic IEEE ops only */
double orc_gumbel(uint64_t seed, uint64_t stream, uint64_t index);
int64_t orc_sample_row(const float* logits, int64_t n, double temperature, uint64_t seed, uint64_t stream,
                       int64_t row);

/* ---- decoder: src/nn/decoder.cpp:61-142, src/nn/kv_cache.cpp:12-41 ---- */
typedef struct orc_config {
    int64_t vocab, layers, dimensions, heads, kv_heads, hidden, context;
    double rope_base, epsilon;
    int wdtype;      /* ORC_F32 or ORC_BF16 for every projection / embedding / head */
    int kv_bf16;     /* 0: f32 K/V as the reference stores them; 1: rounded to bf16 on append (the bf16 cache opt-in) */
    int64_t lora_rank; double lora_alpha; /* rank 0: no adapters */
} orc_config;

typedef struct orc_layer {
    const void *query, *key, *value, *output;   /* [H*hd,d], [KV*hd,d], [KV*hd,d], [d,H*hd] */
    const void *gate, *up, *down;               /* [F,d], [F,d], [d,F] */
    const float *attention_norm, *feedforward_norm; /* [d] */
    const float *cosine, *sine;                 /* [context, hd/2] */
    const void *query_down, *query_up, *value_down, *value_up; /* LoRA A [r,d], B [out,r]; NULL if absent */
} orc_layer;

typedef struct orc_model {
    orc_config config;
    const void* embedding;      /* [V,d] */
    const orc_layer* layers;    /* [layers] */
    const float* normalization; /* [d] */
    const void* head;           /* [V,d] */
} orc_model;

typedef struct orc_cache {
    float *key, *value;         /* [batch, KV, capacity, hd] f32 (bf16-rounded values when kv_bf16) */
    int64_t batch, capacity, length;
} orc_cache;

/* Returns 0 on success, nonzero (cache untouched beyond its prefix) on capacity/shape errors. */
int orc_decoder_decode(const orc_model* model, const float* input, int64_t batch, int64_t length,
                       orc_cache* caches, float* output);
/* Embedding -> decode -> head on every position; logits [B, L, V] (L*V floats per row) */
int orc_lm_logits(const orc_model* model, const int64_t* ids, int64_t batch, int64_t length, orc_cache* caches,
                  float* logits);
/* prompt [B,P] then `steps` tokens; temperature 0 = greedy; step s uses key fold_in(root, s).
 * tokens [B, steps]; last_logits [B, V] of the final step (may be NULL). */
int orc_generate(const orc_model* model, const int64_t* prompt, int64_t batch, int64_t prompt_length,
                 int64_t steps, double temperature, uint64_t seed, uint64_t stream, orc_cache* caches,
                 int64_t* tokens, float* last_logits);

#ifdef __cplusplus
}
#endif
#endif
