#ifndef CTORCH_DECODER_C_API_H
#define CTORCH_DECODER_C_API_H
/*
 * Decoder C17 surface: every entry of the reference's include/dl/decoder_c_api.h:13-41 (same names and
 * arguments; bodies in ctorch_amd/csrc/api/decoder.cpp), plus two additive extensions marked below.
 * The cache handle belongs to one inference request, holds one K/V store per layer and is released
 * independently of the model.
 */
#include "dl/c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dl_decoder_cache dl_decoder_cache;

/* decoder_c_api.h:15-20 */
DL_API dl_status dl_tensordot(const dl_tensor* a, const dl_tensor* b,
    dl_shape axes_a, dl_shape axes_b, dl_tensor** output);
DL_API dl_status dl_rotary_embedding(const dl_tensor* input, const dl_tensor* cosine,
    const dl_tensor* sine, dl_tensor** output);
DL_API dl_status dl_grouped_query_attention(const dl_tensor* query, const dl_tensor* key,
    const dl_tensor* value, const dl_tensor* keep_mask, dl_tensor** output);

/* No counterpart in the reference: dl_grouped_query_attention for callers that cannot allocate device memory
 * (code under HIP graph capture, serving loops that forbid allocation).  The caller passes device pointers:
 * query [B, L, H, D] f32 (position-major rows, head h at columns h*D), key and value [B, KV, S, D] contiguous in
 * `kv_dtype` (DL_F32 or DL_BF16), output [B, L, H, D] f32.  The result is dl_grouped_query_attention's with no
 * keep mask (every query row sees all S keys) and its kernels; key-split partials live in a fixed 8 MiB device
 * array per GPU instead of allocated memory, and a shape whose partials would not fit (B*H*L * splits * (D + 2)
 * floats) is rejected with DL_ERROR before anything runs.  Work is queued on the library's stream for `device`.
 * The first call on a device sets up its context and the array's address; later calls allocate nothing.  Calls
 * that overlap on one GPU share the array and race: issue them in order on that stream. */
DL_API dl_status dl_grouped_query_attention_noalloc(const float* query, const void* key, const void* value,
    dl_dtype kv_dtype, int64_t batch, int64_t heads, int64_t kv_heads, int64_t length, int64_t source,
    int64_t head_dim, float* output, int32_t device);

/* decoder_c_api.h:22-35 */
DL_API dl_status dl_swiglu_create(int64_t dimensions, int64_t hidden, int32_t bias,
    dl_tensor_options options, dl_module** output);
DL_API dl_status dl_lora_linear_create(const dl_module* base, int64_t rank, double alpha, dl_module** output);
DL_API dl_status dl_lora_linear_merge(const dl_module* adapter, dl_module** output);
DL_API dl_status dl_rotary_embedding_create(int64_t dimensions, int64_t capacity, double base,
    dl_tensor_options options, dl_module** output);
DL_API dl_status dl_rotary_embedding_forward(dl_module* rotary, const dl_tensor* input,
    int64_t offset, dl_tensor** output);
DL_API dl_status dl_grouped_query_attention_create(int64_t dimensions, int64_t heads, int64_t kv_heads,
    int64_t context, dl_tensor_options options, dl_module** output);
DL_API dl_status dl_transformer_decoder_create(int64_t layers, int64_t dimensions, int64_t heads,
    int64_t kv_heads, int64_t hidden, int64_t context, dl_tensor_options options, dl_module** output);

/* decoder_c_api.h:37-42 */
DL_API dl_status dl_decoder_cache_create(const dl_module* decoder, dl_decoder_cache** output);
DL_API void dl_decoder_cache_release(dl_decoder_cache* cache);
DL_API dl_status dl_decoder_cache_clear(dl_decoder_cache* cache);
DL_API dl_status dl_decoder_cache_truncate(dl_decoder_cache* cache, int64_t length);
DL_API dl_status dl_decoder_cache_length(const dl_decoder_cache* cache, int64_t* length);
DL_API dl_status dl_transformer_decoder_decode(dl_module* decoder, const dl_tensor* input,
    dl_decoder_cache* cache, dl_tensor** output);

/* Extension (no reference counterpart): the same constructor with the RoPE base the reference hard-codes
 * to 10000 (src/nn/decoder.cpp:70), needed by base-500000 models. */
DL_API dl_status dl_transformer_decoder_create_with_base(int64_t layers, int64_t dimensions, int64_t heads,
    int64_t kv_heads, int64_t hidden, int64_t context, double rope_base, dl_tensor_options options,
    dl_module** output);
/* Extension (no reference counterpart): attaches unmerged rank-`rank` LoRA adapters (scale alpha/rank,
 * `up` zero-initialised) to the query and/or value projection of every layer; they appear in the state as
 * layer{i}.attention.{query,value}_adapter.{down,up}.weight. */
DL_API dl_status dl_transformer_decoder_attach_lora(dl_module* decoder, int64_t rank, double alpha,
    int32_t query, int32_t value);
/* Extension (no reference counterpart): the dtype of the K/V storage every layer's decode reserves.  DL_F32, the
 * default, is the reference's: its KVCache takes the dtype of the appended keys (src/nn/kv_cache.cpp:16-21),
 * which is linear's f32 output (src/ops/matmul.cpp:35-67).  DL_BF16 is an opt-in that halves the cache bytes of
 * long-context decode and rounds every stored key and value to bf16.  Set it before the first decode into a
 * cache: a cache already holding storage of the other dtype is refused on the next decode. */
DL_API dl_status dl_transformer_decoder_set_cache_dtype(dl_module* decoder, dl_dtype dtype);
DL_API dl_status dl_transformer_decoder_cache_dtype(const dl_module* decoder, dl_dtype* dtype);
/* The ONNX decoder's cache wire format (reference extensions/onnx/src/decoder.cpp:64-69, docs/onnx.md:68-113):
 * per layer i, past_key_i / past_value_i as f32 [batch, kv_heads, length, head_dim].  cache_state writes the
 * cache under those names (ready to feed an ONNX Runtime session as its next past_* inputs).  cache_load_state
 * replaces the cache's contents with such a state; each layer may be named past_* or present_* (an ONNX
 * session's outputs), all layers must share batch and length, and the values are stored in the decoder's cache
 * dtype.  Nothing changes when the state does not fit (chunk-atomic). */
DL_API dl_status dl_decoder_cache_state(const dl_decoder_cache* cache, dl_state** output);
DL_API dl_status dl_decoder_cache_load_state(const dl_module* decoder, dl_decoder_cache* cache, const dl_state* state);
/* Extension: writes the K and V of one layer's cache directly (keys already rotated), the reference's
 * KVCache::append route (include/dl/decoder.h:52) for seeding a prefix.  key/value are [B, KV, n, D]. */
DL_API dl_status dl_decoder_cache_append(dl_decoder_cache* cache, int64_t layer, const dl_tensor* key,
    const dl_tensor* value);

#ifdef __cplusplus
}
#endif

#endif
