#ifndef CTORCH_GENERATE_C_API_H
#define CTORCH_GENERATE_C_API_H
/*
 * On-device token loop (extension; no reference C counterpart).
 *
 * The reference composes the language model in application code: Embedding -> TransformerDecoder ->
 * Linear head -> argmax -> .item() -> feed back (examples/decoder_model.h:10-39,
 * examples/decoder_generate.cpp:20-31), and samples with temperature on the host
 * (examples/text_generate.cpp:29-41).  A dl_decoder_lm binds those three reference modules and runs the
 * whole step on the GPU: embedding gather, the fused decoder layers, the LM head for the last position,
 * and greedy or explicit-key Gumbel-max sampling, with the sampled ids fed back in device memory.  Steps
 * after the first can be replayed from a captured HIP graph.
 */
#include "dl/decoder_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct dl_decoder_lm dl_decoder_lm;

/* embedding: Embedding [V, d]; decoder: TransformerDecoder; head: Linear [V, d] without bias.  All three
 * must already live on the same GPU.  The handles are retained. */
DL_API dl_status dl_decoder_lm_create(const dl_module* embedding, const dl_module* decoder,
    const dl_module* head, dl_decoder_lm** output);
DL_API void dl_decoder_lm_release(dl_decoder_lm* lm);

/* Feeds ids [B, L] (i64, any device) through the cache and returns the logits of the last position,
 * [B, V] f32 on the GPU.  The cache advances by L. */
DL_API dl_status dl_decoder_lm_logits(dl_decoder_lm* lm, const dl_tensor* ids, dl_decoder_cache* cache,
    dl_tensor** logits);

/* Feeds prompt [B, P], then produces `steps` tokens: token s is drawn from the last logits of step s with
 * key dl_random_fold_in(key, s) (temperature <= 0: argmax) and fed back.  tokens [B, steps] i64 and
 * last_logits [B, V] f32 (the logits token steps-1 was drawn from) stay on the GPU; either output slot may
 * be NULL.  use_graph != 0 replays steps 2.. from a captured HIP graph. */
DL_API dl_status dl_decoder_lm_generate(dl_decoder_lm* lm, const dl_tensor* prompt, dl_decoder_cache* cache,
    int64_t steps, double temperature, dl_random_key key, int32_t use_graph, dl_tensor** tokens,
    dl_tensor** last_logits);

/* Throughput measurement of the token step: feeds prompt [B, P] and draws token 0, runs two more steps
 * eagerly (sizing buffers; with use_graph the next step is captured), then `warmup` untimed steps, then
 * synchronises and brackets exactly `timed` single-token steps (embedding -> layers -> LM head -> sample ->
 * feed back) with HIP events on the compute stream.  *milliseconds receives their device time; tokens
 * [B, 3 + warmup + timed] (may be NULL) receives every drawn id. */
DL_API dl_status dl_decoder_lm_benchmark(dl_decoder_lm* lm, const dl_tensor* prompt, dl_decoder_cache* cache,
    int64_t warmup, int64_t timed, double temperature, dl_random_key key, int32_t use_graph, double* milliseconds,
    dl_tensor** tokens);

/* Per-kernel-class device time of a single-token step.  One greedy step is run eagerly from ids [B, 1]
 * (appending one position to `cache`, which needs room for two); then each kernel class is timed on its
 * own: all of its launches of that step (one per layer) are issued again, complete and unchanged except
 * that they leave the cache lengths alone, `rounds` times back to back between two HIP events on the
 * compute stream.  For each class the launch count, summed duration and algorithmic HBM bytes (weights +
 * KV read/written, counted once per launch) are written to `timings` (up to `capacity` entries; *count
 * receives the number used). */
typedef struct dl_kernel_timing {
    char name[48];
    int64_t launches;
    double total_ms;
    double bytes;
} dl_kernel_timing;
DL_API dl_status dl_decoder_lm_profile(dl_decoder_lm* lm, const dl_tensor* ids, dl_decoder_cache* cache,
    int64_t rounds, dl_kernel_timing* timings, size_t capacity, size_t* count);

/* Whether batched decode (3 to 64 rows per step) reads a second copy of every bf16 weight, repacked in the
 * matrix-core kernel's tile order (1.6 GB for a 1B model, 14 GB for an 8B one; built on the first batched step).
 * On by default.  enabled = 0 drops the copies held now (after the work already queued that reads them) and has
 * batched decode read the weights as stored: the same results bit for bit, slower (measured on MI355X at batch
 * 32, 1B: 1.17 -> 1.40 ms a step, 1.57 GB freed).  Batch-1 decode never builds the copies.  No reference counterpart: for serving processes that need the
 * memory. */
DL_API dl_status dl_decoder_lm_set_weight_repack(dl_decoder_lm* lm, int32_t enabled);

/* One index per row of logits [B, V] (f32 or bf16, GPU): temperature <= 0 is the reference argmax rule;
 * otherwise Gumbel-max argmax_i(logit_i / T + g_i), g = -log(-log u), u from Philox(key, b*V + i) on (0, 1),
 * evaluated with basic IEEE double operations so that any restatement gives the same index.  [B] i64. */
DL_API dl_status dl_sample(const dl_tensor* logits, double temperature, dl_random_key key, dl_tensor** output);

/* scale * N(0, 1) from the keyed Philox normal (dl_randn_with_key's mapping), rounded once to options.dtype
 * (f32 or bf16); for synthesising large seeded weights directly in device memory. */
DL_API dl_status dl_normal_with_key(dl_random_key key, dl_shape shape, double scale, dl_tensor_options options,
    dl_tensor** output);

/* Device timer on the library's compute stream of `device` (HIP events). */
typedef struct dl_timer dl_timer;
DL_API dl_status dl_timer_create(dl_device device, dl_timer** output);
DL_API void dl_timer_release(dl_timer* timer);
DL_API dl_status dl_timer_start(dl_timer* timer);
/* Records the stop event, waits for it and returns the elapsed milliseconds. */
DL_API dl_status dl_timer_stop(dl_timer* timer, double* milliseconds);

/* Streaming-copy bandwidth probe: copies `bytes` between two device buffers `iterations` times with this
 * library's copy kernel and returns the achieved GB/s (read + write bytes / time). */
DL_API dl_status dl_gpu_copy_bandwidth(int32_t device, uint64_t bytes, int32_t iterations, double* gigabytes_per_second);

#ifdef __cplusplus
}
#endif

#endif
