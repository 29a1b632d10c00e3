/*
 * CPU oracle for the Ctorch decoder token loop — TEST INFRASTRUCTURE ONLY.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load it,
 * and only as the checker.  See oracle.h for the parity pins.
 *
 * Restates the reference CPU arithmetic (paths relative to the reference tree):
 * f32 dot products sequential in k, RMSNorm statistics in double, the CPU
 * softmax/argmax rules, interleaved RoPE from f32 tables, Philox4x32-10.
 * Parallelism is over independent output elements only, so results do not
 * depend on the thread count.
 */
#include "oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* threading: a static split of [0, n) over worker threads                   */
/* ------------------------------------------------------------------------ */

static int g_threads = 1;

void orc_set_threads(int threads) { g_threads = threads < 1 ? 1 : (threads > 256 ? 256 : threads); }
int orc_get_threads(void) { return g_threads; }

typedef void (*range_fn)(int64_t begin, int64_t end, void* context);
typedef struct { range_fn fn; void* context; int64_t begin, end; } range_task;

static void* run_range(void* argument) {
    range_task* task = (range_task*)argument;
    task->fn(task->begin, task->end, task->context);
    return NULL;
}

static void parallel_for(int64_t count, int64_t grain, range_fn fn, void* context) {
    int threads = g_threads;
    if (count <= 0) return;
    if (threads > 1 && count / threads < grain) threads = (int)(count / (grain > 0 ? grain : 1));
    if (threads <= 1) { fn(0, count, context); return; }
    pthread_t handles[256];
    range_task tasks[256];
    int started[256];
    for (int t = 0; t < threads; ++t) {
        tasks[t].fn = fn; tasks[t].context = context;
        tasks[t].begin = count * t / threads; tasks[t].end = count * (t + 1) / threads;
        started[t] = t > 0 && pthread_create(&handles[t], NULL, run_range, &tasks[t]) == 0;
    }
    run_range(&tasks[0]);
    for (int t = 1; t < threads; ++t) {
        if (started[t]) pthread_join(handles[t], NULL);
        else run_range(&tasks[t]);
    }
}

/* ------------------------------------------------------------------------ */
/* Philox4x32-10 and keys: src/core/philox.h:26-52, src/core/random.cpp:14-18 */
/* ------------------------------------------------------------------------ */

void orc_philox(uint64_t seed, uint64_t index, uint64_t stream, uint32_t out[4]) {
    /* counter = (index lo, index hi, stream lo, stream hi); key = (seed lo, seed hi) */
    uint32_t c0 = (uint32_t)index, c1 = (uint32_t)(index >> 32);
    uint32_t c2 = (uint32_t)stream, c3 = (uint32_t)(stream >> 32);
    uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
    for (int round = 0; round < 10; ++round) {
        const uint64_t p0 = (uint64_t)c0 * 0xd2511f53u;
        const uint64_t p1 = (uint64_t)c2 * 0xcd9e8d57u;
        const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        const uint32_t n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9e3779b9u;
        k1 += 0xbb67ae85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

void orc_fold_in(uint64_t seed, uint64_t stream, uint64_t label, uint64_t out[2]) {
    uint32_t bits[4];
    orc_philox(seed, label, stream, bits);
    out[0] = (uint64_t)bits[0] | ((uint64_t)bits[1] << 32);
    out[1] = (uint64_t)bits[2] | ((uint64_t)bits[3] << 32);
}

float orc_unit_f32(uint32_t first, int open_left) {
    return ((float)(first >> 8) + (float)(open_left != 0)) * 0x1p-24f;
}

double orc_unit_f64(uint32_t first, uint32_t second, int open_left) {
    const uint64_t bits = ((uint64_t)(first >> 5) << 26) | (second >> 6);
    return ((double)bits + (double)(open_left != 0)) * 0x1p-53;
}

typedef struct { uint64_t seed, stream; float low, high, scale; int mode; int dtype; void* out; } random_job;

static void random_range(int64_t begin, int64_t end, void* context) {
    const random_job* job = (const random_job*)context;
    uint32_t b[4];
    for (int64_t i = begin; i < end; ++i) {
        orc_philox(job->seed, (uint64_t)i, job->stream, b);
        float value;
        if (job->mode == 0) {
            value = job->low + (job->high - job->low) * orc_unit_f32(b[0], 0);
        } else {
            /* src/kernels/cpu/random.cpp:74-77 with T = float */
            const float radius = sqrtf(-2.0f * logf(orc_unit_f32(b[0], 1)));
            value = radius * cosf((float)6.2831853071795864769 * orc_unit_f32(b[2], 0));
        }
        if (job->mode == 2) {
            value = value * job->scale; /* numeric::scale: value * (float)factor */
            if (job->dtype == ORC_BF16) { ((uint16_t*)job->out)[i] = orc_bf16_encode(value); continue; }
        }
        ((float*)job->out)[i] = value;
    }
}

void orc_uniform_f32(uint64_t seed, uint64_t stream, int64_t count, double low, double high, float* out) {
    random_job job = {seed, stream, (float)low, (float)high, 1.0f, 0, ORC_F32, out};
    parallel_for(count, 1 << 16, random_range, &job);
}

void orc_randn_f32(uint64_t seed, uint64_t stream, int64_t count, float* out) {
    random_job job = {seed, stream, 0.0f, 1.0f, 1.0f, 1, ORC_F32, out};
    parallel_for(count, 1 << 16, random_range, &job);
}

void orc_normal_weights(uint64_t seed, uint64_t stream, int64_t count, double scale, int dtype, void* out) {
    random_job job = {seed, stream, 0.0f, 1.0f, (float)scale, 2, dtype, out};
    parallel_for(count, 1 << 16, random_range, &job);
}

void orc_random_ids(uint64_t seed, uint64_t stream, int64_t count, int64_t vocab, int64_t* out) {
    uint32_t b[4];
    for (int64_t i = 0; i < count; ++i) {
        orc_philox(seed, (uint64_t)i, stream, b);
        out[i] = (int64_t)(((uint64_t)b[0] * (uint64_t)vocab) >> 32);
    }
}

/* ------------------------------------------------------------------------ */
/* bf16 codec: include/dl/half.h:43-47 (encode), :60-66 (decode by shift)     */
/* ------------------------------------------------------------------------ */

static uint32_t float_bits(float value) { uint32_t b; memcpy(&b, &value, 4); return b; }
static float bits_float(uint32_t b) { float value; memcpy(&value, &b, 4); return value; }

uint16_t orc_bf16_encode(float value) {
    const uint32_t bits = float_bits(value);
    if ((bits & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((bits >> 16) | 0x40u);
    return (uint16_t)((bits + 0x7fffu + ((bits >> 16) & 1u)) >> 16);
}

float orc_bf16_decode(uint16_t bits) { return bits_float((uint32_t)bits << 16); }

void orc_bf16_encode_n(const float* input, int64_t count, uint16_t* output) {
    for (int64_t i = 0; i < count; ++i) output[i] = orc_bf16_encode(input[i]);
}

void orc_bf16_decode_n(const uint16_t* input, int64_t count, float* output) {
    for (int64_t i = 0; i < count; ++i) output[i] = orc_bf16_decode(input[i]);
}

static float load_weight(const void* w, int dtype, int64_t index) {
    return dtype == ORC_BF16 ? orc_bf16_decode(((const uint16_t*)w)[index]) : ((const float*)w)[index];
}

/* ------------------------------------------------------------------------ */
/* RoPE tables: src/nn/decoder.cpp:38-46 (angles) and :48-52 (cos/sin)        */
/* ------------------------------------------------------------------------ */

void orc_rope_tables(int64_t head_dim, int64_t capacity, double base, float* cosine, float* sine) {
    const int64_t half = head_dim / 2;
    /* exp(arange(hd/2) * (-2 ln base / hd)): arange is exact, `* double` is numeric::scale (f32 multiply
     * by the factor rounded to f32), exp is the f32 libm call */
    const float factor = (float)(-2.0 * log(base) / (double)head_dim);
    float* frequencies = (float*)malloc((size_t)(half > 0 ? half : 1) * sizeof(float));
    for (int64_t i = 0; i < half; ++i) frequencies[i] = expf((float)i * factor);
    for (int64_t p = 0; p < capacity; ++p) {
        for (int64_t i = 0; i < half; ++i) {
            const float angle = (float)p * frequencies[i]; /* [cap,1] * [hd/2] broadcast multiply */
            cosine[p * half + i] = cosf(angle);
            sine[p * half + i] = sinf(angle);
        }
    }
    free(frequencies);
}

/* ------------------------------------------------------------------------ */
/* RMSNorm: src/kernels/cpu/normalization.cpp:21-56, moments.h:12-24          */
/* ------------------------------------------------------------------------ */

void orc_rms_norm(const float* x, int64_t rows, int64_t width, const float* weight, double epsilon, float* y) {
    for (int64_t r = 0; r < rows; ++r) {
        const float* row = x + r * width;
        double squares = 0;
        for (int64_t i = 0; i < width; ++i) {
            const double value = (double)row[i] - 0.0;
            squares += value * value;
        }
        const double variance = squares / (double)width;
        const double inverse_std = 1.0 / sqrt(variance + epsilon);
        for (int64_t i = 0; i < width; ++i) {
            double value = ((double)row[i] - 0.0) * inverse_std;
            if (weight) value *= (double)weight[i];
            y[r * width + i] = (float)value;
        }
    }
}

/* ------------------------------------------------------------------------ */
/* Linear: Y = X W^T, f32 accumulation sequential in k (cpu/matmul.h:10-22)   */
/* ------------------------------------------------------------------------ */

typedef struct { const float* x; int64_t rows, in, out; const void* w; int wdtype; float* y; } linear_job;

static void linear_range(int64_t begin, int64_t end, void* context) {
    const linear_job* job = (const linear_job*)context;
    const int64_t in = job->in;
    float* row_f32 = NULL;
    if (job->wdtype == ORC_BF16) row_f32 = (float*)malloc((size_t)in * 4 * sizeof(float));
    int64_t j = begin;
    /* four independent output chains at a time; each chain is sequential in k */
    for (; j < end; j += 4) {
        const int64_t n = end - j < 4 ? end - j : 4;
        const float* w[4];
        for (int64_t t = 0; t < n; ++t) {
            if (job->wdtype == ORC_BF16) {
                const uint16_t* source = (const uint16_t*)job->w + (j + t) * in;
                float* dest = row_f32 + t * in;
                for (int64_t k = 0; k < in; ++k) dest[k] = orc_bf16_decode(source[k]);
                w[t] = dest;
            } else {
                w[t] = (const float*)job->w + (j + t) * in;
            }
        }
        for (int64_t r = 0; r < job->rows; ++r) {
            const float* x = job->x + r * in;
            float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
            if (n == 4) {
                for (int64_t k = 0; k < in; ++k) {
                    const float xv = x[k];
                    a0 += xv * w[0][k]; a1 += xv * w[1][k]; a2 += xv * w[2][k]; a3 += xv * w[3][k];
                }
            } else {
                for (int64_t k = 0; k < in; ++k) {
                    const float xv = x[k];
                    a0 += xv * w[0][k];
                    if (n > 1) a1 += xv * w[1][k];
                    if (n > 2) a2 += xv * w[2][k];
                }
            }
            float* y = job->y + r * job->out + j;
            y[0] = a0;
            if (n > 1) y[1] = a1;
            if (n > 2) y[2] = a2;
            if (n > 3) y[3] = a3;
        }
    }
    free(row_f32);
}

void orc_linear(const float* x, int64_t rows, int64_t in, const void* weight, int wdtype, int64_t out, float* y) {
    linear_job job = {x, rows, in, out, weight, wdtype, y};
    /* chunk boundaries are multiples of 4 so every thread count forms the same chains */
    const int64_t groups = (out + 3) / 4;
    if (groups == 0) return;
    int threads = g_threads;
    if (threads > 1 && groups < (int64_t)threads * 4) threads = (int)(groups / 4 > 0 ? groups / 4 : 1);
    if (threads <= 1 || rows * in * out < (1 << 20)) { linear_range(0, out, &job); return; }
    pthread_t handles[256];
    linear_job jobs[256];
    range_task tasks[256];
    int started[256];
    for (int t = 0; t < threads; ++t) {
        jobs[t] = job;
        tasks[t].fn = linear_range; tasks[t].context = &jobs[t];
        tasks[t].begin = groups * t / threads * 4;
        tasks[t].end = groups * (t + 1) / threads * 4;
        if (tasks[t].end > out) tasks[t].end = out;
        started[t] = t > 0 && pthread_create(&handles[t], NULL, run_range, &tasks[t]) == 0;
    }
    run_range(&tasks[0]);
    for (int t = 1; t < threads; ++t) {
        if (started[t]) pthread_join(handles[t], NULL);
        else run_range(&tasks[t]);
    }
}

/* ------------------------------------------------------------------------ */
/* RoPE apply: src/ops/contraction.cpp:44-49 (interleaved pairs)              */
/* ------------------------------------------------------------------------ */

void orc_rope(float* x, int64_t rows, int64_t heads, int64_t head_dim, const float* cosine, const float* sine,
              const int64_t* positions) {
    const int64_t half = head_dim / 2;
    for (int64_t r = 0; r < rows; ++r) {
        const float* c = cosine + positions[r] * half;
        const float* s = sine + positions[r] * half;
        for (int64_t h = 0; h < heads; ++h) {
            float* v = x + (r * heads + h) * head_dim;
            for (int64_t i = 0; i < half; ++i) {
                const float even = v[2 * i], odd = v[2 * i + 1];
                const float a = even * c[i], b = odd * s[i];
                const float e = even * s[i], f = odd * c[i];
                v[2 * i] = a - b;
                v[2 * i + 1] = e + f;
            }
        }
    }
}

/* ------------------------------------------------------------------------ */
/* softmax / argmax / silu: src/kernels/cpu/reduction.cpp:128-203,            */
/* pointwise.cpp:31-34                                                        */
/* ------------------------------------------------------------------------ */

void orc_softmax_row(const float* x, int64_t n, float* y) {
    float maximum = -INFINITY;
    for (int64_t i = 0; i < n; ++i) {
        const float value = x[i];
        maximum = isnan(value) ? value : (maximum < value ? value : maximum);
    }
    int64_t active = n;
    if (isfinite(maximum)) {
        while (active > 0 && x[active - 1] == -INFINITY) --active;
    }
    float total = 0;
    for (int64_t i = 0; i < active; ++i) {
        const float e = expf(x[i] - maximum);
        y[i] = e;
        total += e;
    }
    for (int64_t i = 0; i < active; ++i) y[i] /= total;
    for (int64_t i = active; i < n; ++i) y[i] = 0.0f;
}

int64_t orc_argmax_row(const float* x, int64_t n) {
    float best = x[0];
    int64_t selected = 0;
    for (int64_t i = 1; i < n; ++i) {
        const float value = x[i];
        if (best == best && (value != value || value > best)) { best = value; selected = i; }
    }
    return selected;
}

float orc_silu(float v) {
    const float e = expf(-fabsf(v));
    const float sigma = v >= 0.0f ? 1.0f / (1.0f + e) : e / (1.0f + e);
    return v * sigma;
}

/* ------------------------------------------------------------------------ */
/* grouped-query attention: src/ops/attention.cpp:52-95,161-188               */
/* ------------------------------------------------------------------------ */

typedef struct {
    const float *q, *k, *v; int64_t batch, heads, kv_heads, length, source, kv_stride, head_dim, first; float* out;
    const uint8_t* mask; const int64_t* mask_strides;
} attention_job;

static void attention_range(int64_t begin, int64_t end, void* context) {
    const attention_job* job = (const attention_job*)context;
    const int64_t S = job->source, hd = job->head_dim, L = job->length, G = job->heads / job->kv_heads;
    /* 1/sqrt(hd) is applied to the f32 scores as numeric::scale: multiply by the factor rounded to f32 */
    const float scale = (float)(1.0 / sqrt((double)hd));
    float* scores = (float*)malloc((size_t)(S > 0 ? S : 1) * sizeof(float));
    float* probabilities = (float*)malloc((size_t)(S > 0 ? S : 1) * sizeof(float));
    for (int64_t item = begin; item < end; ++item) {
        const int64_t b = item / (job->heads * L), h = (item / L) % job->heads, l = item % L;
        const int64_t kvh = h / G;
        const float* q = job->q + ((b * job->heads + h) * L + l) * hd;
        const float* keys = job->k + (b * job->kv_heads + kvh) * job->kv_stride * hd;
        const float* values = job->v + (b * job->kv_heads + kvh) * job->kv_stride * hd;
        /* eight scores at a time: each sum runs over d in order, the eight chains side by side */
        int64_t s0 = 0;
        for (; s0 + 8 <= S; s0 += 8) {
            float acc[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};
            for (int64_t d = 0; d < hd; ++d) {
                const float qd = q[d];
                for (int j = 0; j < 8; ++j) acc[j] += qd * keys[(s0 + j) * hd + d];
            }
            for (int j = 0; j < 8; ++j) scores[s0 + j] = acc[j] * scale;
        }
        for (int64_t s = s0; s < S; ++s) {
            float acc = 0.0f;
            for (int64_t d = 0; d < hd; ++d) acc += q[d] * keys[s * hd + d];
            scores[s] = acc * scale;
        }
        /* keep mask (src/ops/attention.cpp:48-50,80): where(mask, scores * scale, -inf), the mask read through
           its broadcast strides over [B, H, L, S] */
        if (job->mask) {
            const int64_t* st = job->mask_strides;
            const uint8_t* row = job->mask + b * st[0] + h * st[1] + l * st[2];
            for (int64_t s = 0; s < S; ++s)
                if (!row[s * st[3]]) scores[s] = -INFINITY;
        }
        if (job->first >= 0 && job->first < S - 1) {
            for (int64_t s = job->first + l + 1; s < S; ++s) scores[s] = -INFINITY;
        }
        orc_softmax_row(scores, S, probabilities);
        /* P V: one sum per head dimension, each over s in order, all of them side by side */
        float* o = job->out + ((b * job->heads + h) * L + l) * hd;
        for (int64_t d = 0; d < hd; ++d) o[d] = 0.0f;
        for (int64_t s = 0; s < S; ++s) {
            const float p = probabilities[s];
            const float* v = values + s * hd;
            for (int64_t d = 0; d < hd; ++d) o[d] += p * v[d];
        }
    }
    free(scores);
    free(probabilities);
}

void orc_attention(const float* q, const float* k, const float* v, int64_t batch, int64_t heads, int64_t kv_heads,
                   int64_t length, int64_t source, int64_t kv_stride, int64_t head_dim, int64_t causal_first,
                   float* out) {
    orc_attention_masked(q, k, v, batch, heads, kv_heads, length, source, kv_stride, head_dim, causal_first, NULL,
                         NULL, out);
}

void orc_attention_masked(const float* q, const float* k, const float* v, int64_t batch, int64_t heads,
                          int64_t kv_heads, int64_t length, int64_t source, int64_t kv_stride, int64_t head_dim,
                          int64_t causal_first, const uint8_t* mask, const int64_t* mask_strides, float* out) {
    attention_job job = {q, k, v, batch, heads, kv_heads, length, source, kv_stride, head_dim, causal_first, out,
                         mask, mask_strides};
    parallel_for(batch * heads * length, 4, attention_range, &job);
}

/* ------------------------------------------------------------------------ */
/* sampling: Gumbel-max over keyed Philox noise (the build's new op)          */
/* ------------------------------------------------------------------------ */

/* Natural log of a positive finite double from basic IEEE operations only, so that host and
 * device evaluate it to identical bits: x = m * 2^e with m in [sqrt(1/2), sqrt(2)),
 * log m = 2 atanh(s), s = (m-1)/(m+1), |s| < 0.1716, 12-term odd series (Horner in s^2). */
double orc_log(double x) {
    uint64_t bits;
    memcpy(&bits, &x, 8);
    int64_t exponent = (int64_t)((bits >> 52) & 0x7ff);
    if (exponent == 0) { /* subnormal: scale into the normal range exactly */
        x = x * 0x1p54;
        memcpy(&bits, &x, 8);
        exponent = (int64_t)((bits >> 52) & 0x7ff) - 54;
    }
    exponent -= 1023;
    uint64_t mantissa_bits = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &mantissa_bits, 8);
    if (m > 1.4142135623730951) { m = m * 0.5; exponent += 1; }
    const double s = (m - 1.0) / (m + 1.0);
    const double t = s * s;
    double p = 1.0 / 23.0;
    p = p * t + 1.0 / 21.0;
    p = p * t + 1.0 / 19.0;
    p = p * t + 1.0 / 17.0;
    p = p * t + 1.0 / 15.0;
    p = p * t + 1.0 / 13.0;
    p = p * t + 1.0 / 11.0;
    p = p * t + 1.0 / 9.0;
    p = p * t + 1.0 / 7.0;
    p = p * t + 1.0 / 5.0;
    p = p * t + 1.0 / 3.0;
    p = p * t + 1.0;
    const double log_m = 2.0 * s * p;
    const double e = (double)exponent;
    return e * 6.93147180369123816490e-01 + (e * 1.90821492927058770002e-10 + log_m);
}

/* g = -log(-log(u)), u = ((53-bit Philox value >> 1) + 0.5) * 2^-52 in the open interval (0, 1) */
double orc_gumbel(uint64_t seed, uint64_t stream, uint64_t index) {
    uint32_t b[4];
    orc_philox(seed, index, stream, b);
    const uint64_t bits = ((uint64_t)(b[0] >> 5) << 26) | (b[1] >> 6);
    const double u = ((double)(bits >> 1) + 0.5) * 0x1p-52;
    return -orc_log(-orc_log(u));
}

int64_t orc_sample_row(const float* logits, int64_t n, double temperature, uint64_t seed, uint64_t stream,
                       int64_t row) {
    if (!(temperature > 0.0)) return orc_argmax_row(logits, n);
    double best = 0;
    int64_t selected = -1;
    for (int64_t i = 0; i < n; ++i) {
        const double score = (double)logits[i] / temperature + orc_gumbel(seed, stream, (uint64_t)(row * n + i));
        if (selected < 0) { best = score; selected = i; continue; }
        /* the argmax rules: strict > keeps the first tie; the first NaN stays selected */
        if (best == best && (score != score || score > best)) { best = score; selected = i; }
    }
    return selected;
}

/* ------------------------------------------------------------------------ */
/* decoder: src/nn/decoder.cpp:73-142, src/nn/kv_cache.cpp:12-30              */
/* ------------------------------------------------------------------------ */

static void add_lora(const float* x, int64_t rows, int64_t in, const void* down, const void* up, int64_t rank,
                     int64_t out, int wdtype, double alpha, float* y) {
    /* src/nn/decoder.cpp:30-32: linear(x, W) + up(down(x)) * (alpha / rank) */
    float* hidden = (float*)malloc((size_t)(rows * rank) * sizeof(float));
    float* delta = (float*)malloc((size_t)(rows * out) * sizeof(float));
    orc_linear(x, rows, in, down, wdtype, rank, hidden);
    orc_linear(hidden, rows, rank, up, wdtype, out, delta);
    const float scale = (float)(alpha / (double)rank);
    for (int64_t i = 0; i < rows * out; ++i) y[i] = y[i] + delta[i] * scale;
    free(hidden);
    free(delta);
}

static int layer_decode(const orc_config* c, const orc_layer* w, const float* input, int64_t B, int64_t L,
                        orc_cache* cache, float* output) {
    const int64_t d = c->dimensions, H = c->heads, KV = c->kv_heads, hd = d / H, F = c->hidden;
    const int64_t rows = B * L, offset = cache->length;
    if (L > cache->capacity - offset) return 1;       /* kv_cache.cpp:14-15 */
    if (offset + L > c->context) return 2;             /* decoder.cpp:54-56 RoPE capacity */
    float* normed = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* q = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* k = (float*)malloc((size_t)(rows * KV * hd) * sizeof(float));
    float* v = (float*)malloc((size_t)(rows * KV * hd) * sizeof(float));
    float* qt = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* attended = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* merged = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* residual = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* gate = (float*)malloc((size_t)(rows * F) * sizeof(float));
    float* up = (float*)malloc((size_t)(rows * F) * sizeof(float));
    int64_t* positions = (int64_t*)malloc((size_t)rows * sizeof(int64_t));

    orc_rms_norm(input, rows, d, w->attention_norm, c->epsilon, normed);
    orc_linear(normed, rows, d, w->query, c->wdtype, H * hd, q);
    orc_linear(normed, rows, d, w->key, c->wdtype, KV * hd, k);
    orc_linear(normed, rows, d, w->value, c->wdtype, KV * hd, v);
    if (c->lora_rank > 0 && w->query_down) add_lora(normed, rows, d, w->query_down, w->query_up, c->lora_rank,
                                                    H * hd, c->wdtype, c->lora_alpha, q);
    if (c->lora_rank > 0 && w->value_down) add_lora(normed, rows, d, w->value_down, w->value_up, c->lora_rank,
                                                    KV * hd, c->wdtype, c->lora_alpha, v);
    for (int64_t r = 0; r < rows; ++r) positions[r] = offset + r % L;
    orc_rope(q, rows, H, hd, w->cosine, w->sine, positions);
    orc_rope(k, rows, KV, hd, w->cosine, w->sine, positions);
    /* KVCache::append: copy into [length, length+L) along the sequence axis of [B,KV,cap,hd] */
    for (int64_t b = 0; b < B; ++b)
        for (int64_t l = 0; l < L; ++l)
            for (int64_t h = 0; h < KV; ++h)
                for (int64_t i = 0; i < hd; ++i) {
                    const int64_t src = ((b * L + l) * KV + h) * hd + i;
                    const int64_t dst = ((b * KV + h) * cache->capacity + offset + l) * hd + i;
                    float kv_k = k[src], kv_v = v[src];
                    if (c->kv_bf16) {
                        kv_k = orc_bf16_decode(orc_bf16_encode(kv_k));
                        kv_v = orc_bf16_decode(orc_bf16_encode(kv_v));
                    }
                    cache->key[dst] = kv_k;
                    cache->value[dst] = kv_v;
                }
    /* q [B,L,H,hd] -> [B,H,L,hd] */
    for (int64_t b = 0; b < B; ++b)
        for (int64_t l = 0; l < L; ++l)
            for (int64_t h = 0; h < H; ++h)
                memcpy(qt + ((b * H + h) * L + l) * hd, q + ((b * L + l) * H + h) * hd, (size_t)hd * sizeof(float));
    orc_attention(qt, cache->key, cache->value, B, H, KV, L, offset + L, cache->capacity, hd, offset, attended);
    /* [B,H,L,hd] -> [B,L,H*hd] */
    for (int64_t b = 0; b < B; ++b)
        for (int64_t l = 0; l < L; ++l)
            for (int64_t h = 0; h < H; ++h)
                memcpy(merged + ((b * L + l) * H + h) * hd, attended + ((b * H + h) * L + l) * hd,
                       (size_t)hd * sizeof(float));
    orc_linear(merged, rows, d, w->output, c->wdtype, d, residual);
    for (int64_t i = 0; i < rows * d; ++i) residual[i] = input[i] + residual[i];
    orc_rms_norm(residual, rows, d, w->feedforward_norm, c->epsilon, normed);
    orc_linear(normed, rows, d, w->gate, c->wdtype, F, gate);
    orc_linear(normed, rows, d, w->up, c->wdtype, F, up);
    for (int64_t i = 0; i < rows * F; ++i) gate[i] = orc_silu(gate[i]) * up[i];
    orc_linear(gate, rows, F, w->down, c->wdtype, d, output);
    for (int64_t i = 0; i < rows * d; ++i) output[i] = residual[i] + output[i];
    cache->length = offset + L;

    free(normed); free(q); free(k); free(v); free(qt); free(attended); free(merged); free(residual);
    free(gate); free(up); free(positions);
    return 0;
}

int orc_decoder_decode(const orc_model* model, const float* input, int64_t batch, int64_t length,
                       orc_cache* caches, float* output) {
    const orc_config* c = &model->config;
    const int64_t d = c->dimensions, rows = batch * length;
    const int64_t prefix = caches[0].length;
    for (int64_t i = 0; i < c->layers; ++i)
        if (caches[i].length != prefix || caches[i].batch != batch) return 3; /* decoder.cpp:128-131 */
    float* current = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* next = (float*)malloc((size_t)(rows * d) * sizeof(float));
    memcpy(current, input, (size_t)(rows * d) * sizeof(float));
    int status = 0;
    for (int64_t i = 0; i < c->layers && status == 0; ++i) {
        status = layer_decode(c, &model->layers[i], current, batch, length, &caches[i], next);
        float* swap = current; current = next; next = swap;
    }
    if (status != 0) {
        for (int64_t i = 0; i < c->layers; ++i) caches[i].length = prefix; /* decoder.cpp:137-141 rollback */
    } else {
        orc_rms_norm(current, rows, d, model->normalization, c->epsilon, output);
    }
    free(current);
    free(next);
    return status;
}

int orc_lm_logits(const orc_model* model, const int64_t* ids, int64_t batch, int64_t length, orc_cache* caches,
                  float* logits) {
    const orc_config* c = &model->config;
    const int64_t d = c->dimensions, rows = batch * length;
    float* embedded = (float*)malloc((size_t)(rows * d) * sizeof(float));
    float* features = (float*)malloc((size_t)(rows * d) * sizeof(float));
    for (int64_t r = 0; r < rows; ++r) {
        if (ids[r] < 0 || ids[r] >= c->vocab) { free(embedded); free(features); return 4; }
        for (int64_t i = 0; i < d; ++i) embedded[r * d + i] = load_weight(model->embedding, c->wdtype, ids[r] * d + i);
    }
    int status = orc_decoder_decode(model, embedded, batch, length, caches, features);
    if (status == 0) orc_linear(features, rows, d, model->head, c->wdtype, c->vocab, logits);
    free(embedded);
    free(features);
    return status;
}

int orc_generate(const orc_model* model, const int64_t* prompt, int64_t batch, int64_t prompt_length,
                 int64_t steps, double temperature, uint64_t seed, uint64_t stream, orc_cache* caches,
                 int64_t* tokens, float* last_logits) {
    const int64_t V = model->config.vocab;
    int64_t length = prompt_length;
    int64_t* input = (int64_t*)malloc((size_t)(batch * (prompt_length > 1 ? prompt_length : 1)) * sizeof(int64_t));
    float* logits = (float*)malloc((size_t)(batch * prompt_length * V) * sizeof(float));
    memcpy(input, prompt, (size_t)(batch * prompt_length) * sizeof(int64_t));
    int status = 0;
    for (int64_t s = 0; s < steps; ++s) {
        status = orc_lm_logits(model, input, batch, length, caches, logits);
        if (status != 0) break;
        uint64_t key[2];
        orc_fold_in(seed, stream, (uint64_t)s, key);
        for (int64_t b = 0; b < batch; ++b) {
            const float* row = logits + (b * length + (length - 1)) * V;
            const int64_t next = orc_sample_row(row, V, temperature, key[0], key[1], b);
            tokens[b * steps + s] = next;
            input[b] = next;
            if (last_logits && s == steps - 1) memcpy(last_logits + b * V, row, (size_t)V * sizeof(float));
        }
        length = 1;
    }
    free(input);
    free(logits);
    return status;
}
