/*
 * CPU oracle for the int8 weight-only decode path of qwen3-tts-native.
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker.  The shipped HIP library never
 * links or calls it.
 *
 * Each function restates the reference arithmetic in the reference's own
 * operation order.  K/ = /root/reference/native/qwen3-tts-native/native/src/.
 * Build flags (oracle/Makefile) forbid floating-point contraction, so every
 * fused multiply-add below is an explicit fmaf(), exactly where the CUDA
 * source has one (or where nvcc's default -fmad=true contracts `a*b + c`).
 *
 * Parity pinning (what each function is checked against, tests/test_oracle.py):
 *   - int8 GEMV family: fp64 formula, brute force on tiny shapes, zero weights,
 *     one-hot activations, integer-exact cases.
 *   - quantizer: closed-form invariants (|q|<=127, row max -> +-127,
 *     zero row -> scale 1, dequant error <= scale/2).
 *   - RMSNorm / RoPE / attention / SiLU-gate: the reference's own host-float
 *     known-answer formulas from K/primitive_parity.cu:115-368 with its 0.016
 *     tolerance, plus closed forms.
 *   - argmax: the known-answer test of K/runtime.cu:153-159 (token 1729) and
 *     benchmarks/results/bf16-argmax-vocab{2048,3072}.json.
 *   - sampler: closed forms (greedy == argmax, top_k=1 == argmax, empirical
 *     frequencies of top-k draws match softmax weights); the exact sampled
 *     stream of the CUDA sampler is "parity unpinned" (the reference must run
 *     on its own GPU for that).
 *
 * exp: the reference calls CUDA's expf (SiLU, softmax).  This restatement and
 * the HIP kernels both call q3_expf (q3_math.h: Cody-Waite reduction + degree-7
 * polynomial, <= 1 ulp from the correctly rounded result, pinned against
 * libm's exp in tests/test_oracle.py), so GPU and oracle agree bit-for-bit;
 * against the reference a 1-ulp difference in an exp result is possible.
 * Likewise rsqrtf (RMSNorm, attention scale) is restated as the correctly
 * rounded 1/sqrtf, and RoPE's powf/cosf/sinf come from the host libm.
 */
#include "oracle.h"
#include "../qwen3-tts-native_amd/csrc/q3_math.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------------ */
/* bf16 helpers                                                              */
/* ------------------------------------------------------------------------ */

float orc_bf16_to_f32(uint16_t v) {
    uint32_t u = (uint32_t)v << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* Round-to-nearest-even, as __float2bfloat16 (NaN -> canonical quiet NaN). */
uint16_t orc_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return 0x7fff;
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_f32_to_bf16(in[i]);
}

void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = orc_bf16_to_f32(in[i]);
}

void orc_expf_array(const float* in, float* out, size_t n) {
    for (size_t i = 0; i < n; ++i) out[i] = q3_expf(in[i]);
}

static inline float bf(uint16_t v) { return orc_bf16_to_f32(v); }
static inline uint16_t tobf(float f) { return orc_f32_to_bf16(f); }
static inline float rbf(float f) { return bf(tobf(f)); }

/* xorshift64* as next_random, K/sampling_kernels.cu:53-63 (zero state is
 * replaced by the golden-ratio constant). */
uint64_t orc_xorshift64star(uint64_t* state) {
    uint64_t value = *state;
    if (value == 0) value = 0x9e3779b97f4a7c15ULL;
    value ^= value >> 12;
    value ^= value << 25;
    value ^= value >> 27;
    *state = value;
    return value * 0x2545f4914f6cdd1dULL;
}

/* uniform_random, K/sampling_kernels.cu:65-69. */
float orc_uniform_random(uint64_t* state) {
    const double scale = 1.0 / 9007199254740992.0;
    const uint64_t value = orc_xorshift64star(state);
    return (float)((double)(value >> 11) * scale);
}

/* ------------------------------------------------------------------------ */
/* int8 GEMV family                                                          */
/* ------------------------------------------------------------------------ */

/* Channel-range parallelism for the model-level restatement: every output
 * channel is computed independently in the exact order, so splitting the
 * channels over threads changes no bit.  orc_set_threads(n) sets the count
 * (1 by default); small matrices always run on the calling thread. */
static int g_threads = 1;

void orc_set_threads(int threads) {
    g_threads = threads < 1 ? 1 : (threads > 256 ? 256 : threads);
}

typedef OrcRangeFn ChannelRangeFn;
typedef struct RangeJob {
    ChannelRangeFn fn;
    void* ctx;
    int c0, c1;
} RangeJob;

static void* range_worker(void* arg) {
    RangeJob* j = (RangeJob*)arg;
    j->fn(j->ctx, j->c0, j->c1);
    return NULL;
}

void orc_for_channels(int channels, size_t work, OrcRangeFn fn, void* ctx) {
    int threads = g_threads;
    if (work < ((size_t)1 << 20) || threads <= 1) {
        fn(ctx, 0, channels);
        return;
    }
    if (threads > channels) threads = channels;
    pthread_t tid[256];
    RangeJob jobs[256];
    const int per = (channels + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        const int c0 = t * per;
        const int c1 = c0 + per < channels ? c0 + per : channels;
        if (c0 >= c1) break;
        jobs[t] = (RangeJob){fn, ctx, c0, c1};
        if (pthread_create(&tid[t], NULL, range_worker, &jobs[t]) != 0) {
            range_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t) {
        if (tid[t]) pthread_join(tid[t], NULL);
    }
}

typedef struct QuantCtx {
    const uint16_t* weight;
    int8_t* quantized;
    float* scales;
    int in_features;
} QuantCtx;

static void quantize_range(void* p, int r0, int r1) {
    const QuantCtx* q = (const QuantCtx*)p;
    const int in_features = q->in_features;
    for (int r = r0; r < r1; ++r) {
        const uint16_t* row = q->weight + (size_t)r * in_features;
        float maximum = 0.0f;
        for (int i = 0; i < in_features; ++i) {
            maximum = fmaxf(maximum, fabsf(bf(row[i])));
        }
        const float scale = maximum > 0.0f ? maximum / 127.0f : 1.0f;
        const float inverse = 1.0f / scale;
        q->scales[r] = scale;
        for (int i = 0; i < in_features; ++i) {
            const float value = bf(row[i]) * inverse;
            const float clamped = fminf(fmaxf(value, -127.0f), 127.0f);
            q->quantized[(size_t)r * in_features + i] = (int8_t)lrintf(clamped);
        }
    }
}

/* quantize_weight_rows_kernel, K/int8_gemv.cu:20-52: per row absmax
 * (max is order independent), scale = amax/127 or 1, value = w * (1/scale),
 * clamp to +-127, lrintf (round half to even). */
void orc_quantize_weight_rows(const uint16_t* weight, int8_t* quantized,
                              float* scales, int in_features, int out_features) {
    QuantCtx q = {weight, quantized, scales, in_features};
    orc_for_channels(out_features, (size_t)out_features * in_features, quantize_range, &q);
}

/* One output channel, one activation row, in the reference's exact order
 * (K/int8_gemv.cu:67-125): 32 lanes; lane l owns 16-element vectors
 * l, l+32, ...; each vector is a fresh 16-term fmaf chain from 0 that is then
 * added to the lane accumulator; lanes are folded by shuffle-down with
 * offsets 16, 8, 4, 2, 1; lane 0 holds the dot product. */
/* Test switch (not a reference semantics): every int8 GEMV sums in double
 * and rounds once -- a second valid summation order, used to measure how far
 * two valid orders drift apart through a whole model. */
static int g_double_sum = 0;
void orc_set_gemv_double_sum(int on) { g_double_sum = on; }

__attribute__((target_clones("fma", "default")))
static float dot_channel_exact(const int8_t* w, const float* x, int in_features) {
    if (g_double_sum) {
        double sum = 0.0;
        for (int k = 0; k < in_features; ++k) sum += (double)w[k] * (double)x[k];
        return (float)sum;
    }
    float acc[32];
    for (int l = 0; l < 32; ++l) acc[l] = 0.0f;
    const int vectors = in_features / 16;
    for (int v = 0; v < vectors; ++v) {
        const int l = v & 31;
        const int8_t* wv = w + (size_t)v * 16;
        const float* xv = x + (size_t)v * 16;
        float sum = 0.0f;
        for (int j = 0; j < 16; ++j) sum = fmaf((float)wv[j], xv[j], sum);
        acc[l] += sum;
    }
    for (int offset = 16; offset > 0; offset >>= 1) {
        for (int l = 0; l < offset; ++l) acc[l] += acc[l + offset];
    }
    return acc[0];
}

static float* widen_rows(const uint16_t* input, int rows, int in_features) {
    float* x = (float*)malloc((size_t)rows * in_features * sizeof(float));
    orc_bf16_to_f32_array(input, x, (size_t)rows * in_features);
    return x;
}

typedef struct GemmCtx {
    const int8_t* weight;
    const float* scales;
    const float* x;
    int in_features, out_features, rows;
    float* y32;
    uint16_t* y16;
    uint16_t* inout;
} GemmCtx;

static void gemm_range(void* p, int c0, int c1) {
    const GemmCtx* g = (const GemmCtx*)p;
    for (int r = 0; r < g->rows; ++r) {
        for (int c = c0; c < c1; ++c) {
            const float value = dot_channel_exact(g->weight + (size_t)c * g->in_features,
                                                  g->x + (size_t)r * g->in_features, g->in_features);
            const float y = value * g->scales[c];
            if (g->y32) g->y32[(size_t)r * g->out_features + c] = y;
            if (g->y16) g->y16[(size_t)r * g->out_features + c] = tobf(y);
        }
    }
}

/* int8_dequant_gemm_kernel<kRows>, K/int8_gemv.cu:58-128: output =
 * bf16(value * scale[c]).  Requires in_features % 16 == 0. */
void orc_int8_gemm_rows(const int8_t* weight, const float* scales,
                        const uint16_t* input, int in_features,
                        int out_features, int rows, float* y32, uint16_t* y16) {
    float* x = widen_rows(input, rows, in_features);
    GemmCtx g = {weight, scales, x, in_features, out_features, rows, y32, y16, NULL};
    orc_for_channels(out_features, (size_t)out_features * in_features * rows, gemm_range, &g);
    free(x);
}

void orc_int8_gemm_rows_f64(const int8_t* weight, const float* scales,
                            const uint16_t* input, int in_features,
                            int out_features, int rows, double* y) {
    for (int r = 0; r < rows; ++r) {
        for (int c = 0; c < out_features; ++c) {
            double sum = 0.0;
            for (int k = 0; k < in_features; ++k) {
                sum += (double)weight[(size_t)c * in_features + k]
                     * (double)bf(input[(size_t)r * in_features + k]);
            }
            y[(size_t)r * out_features + c] = sum * (double)scales[c];
        }
    }
}

static void gemm_add_range(void* p, int c0, int c1) {
    const GemmCtx* g = (const GemmCtx*)p;
    for (int r = 0; r < g->rows; ++r) {
        for (int c = c0; c < c1; ++c) {
            const float value = dot_channel_exact(g->weight + (size_t)c * g->in_features,
                                                  g->x + (size_t)r * g->in_features, g->in_features);
            const size_t i = (size_t)r * g->out_features + c;
            g->inout[i] = tobf(fmaf(value, g->scales[c], bf(g->inout[i])));
        }
    }
}

/* int8_dequant_gemm_add_kernel, K/int8_gemv.cu:132-199.  The epilogue
 * `float(out) + value * scale` is contracted to one fma by nvcc's default
 * -fmad=true, so it is restated as fmaf(value, scale, out). */
void orc_int8_gemm_rows_add(const int8_t* weight, const float* scales,
                            const uint16_t* input, uint16_t* inout,
                            int in_features, int out_features, int rows) {
    float* x = widen_rows(input, rows, in_features);
    GemmCtx g = {weight, scales, x, in_features, out_features, rows, NULL, NULL, inout};
    orc_for_channels(out_features, (size_t)out_features * in_features * rows, gemm_add_range, &g);
    free(x);
}

static void gate_up_range(void* p, int c0, int c1) {
    const GemmCtx* g = (const GemmCtx*)p;
    const int in_features = g->in_features, out_features = g->out_features;
    for (int r = 0; r < g->rows; ++r) {
        const float* xr = g->x + (size_t)r * in_features;
        for (int c = c0; c < c1; ++c) {
            const float gv = dot_channel_exact(g->weight + (size_t)c * in_features, xr, in_features);
            const float uv = dot_channel_exact(
                g->weight + ((size_t)out_features + c) * in_features, xr, in_features);
            const float gate = gv * g->scales[c];
            const float up = uv * g->scales[out_features + c];
            const float activated = gate / (1.0f + q3_expf(-gate));
            g->inout[(size_t)r * out_features + c] = tobf(activated * up);
        }
    }
}

/* int8_dequant_gate_up_silu_kernel, K/int8_gemv.cu:206-293: weight is
 * [2*out][in] (gate rows first), out = bf16(silu(g*sg) * (u*su)). */
void orc_int8_gate_up_silu_rows(const int8_t* weight, const float* scales,
                                const uint16_t* input, uint16_t* output,
                                int in_features, int out_features, int rows) {
    float* x = widen_rows(input, rows, in_features);
    GemmCtx g = {weight, scales, x, in_features, out_features, rows, NULL, NULL, output};
    orc_for_channels(out_features, (size_t)2 * out_features * in_features * rows, gate_up_range, &g);
    free(x);
}

typedef struct MtJob {
    const int8_t* weight;
    const float* scales;
    const float* x;
    int in_features, out_features, rows, c0, c1;
    float* y32;
    uint16_t* y16;
} MtJob;

static void* mt_worker(void* arg) {
    MtJob* j = (MtJob*)arg;
    for (int r = 0; r < j->rows; ++r) {
        for (int c = j->c0; c < j->c1; ++c) {
            const float value = dot_channel_exact(j->weight + (size_t)c * j->in_features,
                                                  j->x + (size_t)r * j->in_features,
                                                  j->in_features);
            const float y = value * j->scales[c];
            if (j->y32) j->y32[(size_t)r * j->out_features + c] = y;
            if (j->y16) j->y16[(size_t)r * j->out_features + c] = tobf(y);
        }
    }
    return NULL;
}

void orc_int8_gemm_rows_mt(const int8_t* weight, const float* scales,
                           const uint16_t* input, int in_features,
                           int out_features, int rows, float* y32,
                           uint16_t* y16, int threads) {
    if (threads < 1) threads = 1;
    if (threads > 256) threads = 256;
    float* x = widen_rows(input, rows, in_features);
    pthread_t tid[256];
    MtJob jobs[256];
    const int per = (out_features + threads - 1) / threads;
    int started = 0;
    for (int t = 0; t < threads; ++t) {
        const int c0 = t * per;
        const int c1 = c0 + per < out_features ? c0 + per : out_features;
        if (c0 >= c1) break;
        jobs[t] = (MtJob){weight, scales, x, in_features, out_features, rows, c0, c1, y32, y16};
        if (pthread_create(&tid[t], NULL, mt_worker, &jobs[t]) != 0) {
            mt_worker(&jobs[t]);
            tid[t] = 0;
        }
        started = t + 1;
    }
    for (int t = 0; t < started; ++t) {
        if (tid[t]) pthread_join(tid[t], NULL);
    }
    free(x);
}

/* ------------------------------------------------------------------------ */
/* Transformer primitives                                                    */
/* ------------------------------------------------------------------------ */

/* block_sum over 256 threads, K/talker_kernels.cu:14-25: partial[t] +=
 * partial[t + stride] for stride 128, 64, ..., 1. */
static float block_sum_256(float* partial) {
    for (int stride = 128; stride > 0; stride >>= 1) {
        for (int t = 0; t < stride; ++t) partial[t] += partial[t + stride];
    }
    return partial[0];
}

/* rms_norm_kernel, K/talker_kernels.cu:27-48, 256 threads per row: thread t
 * sums fmaf(x,x) over t, t+256, ...; inv = 1/sqrt(sum/width + eps);
 * y = bf16(bf16(x*inv) * g).  The reference uses rsqrtf; the restatement uses
 * the correctly rounded 1/sqrtf, which the HIP build also uses. */
void orc_rms_norm_rows(const uint16_t* input, const uint16_t* weight,
                       uint16_t* output, int rows, int width, float epsilon) {
    float partial[256];
    for (int r = 0; r < rows; ++r) {
        const uint16_t* in = input + (size_t)r * width;
        uint16_t* out = output + (size_t)r * width;
        for (int t = 0; t < 256; ++t) {
            float s = 0.0f;
            for (int i = t; i < width; i += 256) {
                const float v = bf(in[i]);
                s = fmaf(v, v, s);
            }
            partial[t] = s;
        }
        const float inv = 1.0f / sqrtf(block_sum_256(partial) / (float)width + epsilon);
        for (int i = 0; i < width; ++i) {
            const float normalized = rbf(bf(in[i]) * inv);
            out[i] = tobf(normalized * bf(weight[i]));
        }
    }
}

/* head_rms_norm_kernel, K/talker_kernels.cu:50-70: same per head of
 * head_dimension values, in place. */
void orc_head_rms_norm_rows(uint16_t* values, const uint16_t* weight, int rows,
                            int heads, int head_dimension, float epsilon) {
    for (int h = 0; h < rows * heads; ++h) {
        uint16_t* head = values + (size_t)h * head_dimension;
        orc_rms_norm_rows(head, weight, head, 1, head_dimension, epsilon);
    }
}

/* rope_kernel / rope_rows_at_kernel, K/talker_kernels.cu:72-114: rotate-half
 * RoPE with bf16 rounding of cos, sin, every product and every sum. */
void orc_rope_rows(uint16_t* values, int rows, int heads, int head_dimension,
                   const int* positions, float theta) {
    const int half = head_dimension / 2;
    for (int r = 0; r < rows; ++r) {
        for (int h = 0; h < heads; ++h) {
            uint16_t* base = values + ((size_t)r * heads + h) * head_dimension;
            for (int d = 0; d < half; ++d) {
                const float exponent = (float)(2 * d) / (float)head_dimension;
                const float angle = (float)positions[r] * powf(theta, -exponent);
                const float c = rbf(cosf(angle));
                const float s = rbf(sinf(angle));
                const float first = bf(base[d]);
                const float second = bf(base[d + half]);
                const float fc = rbf(first * c);
                const float ss = rbf(second * s);
                const float sc = rbf(second * c);
                const float fs = rbf(first * s);
                base[d] = tobf(fc - ss);
                base[d + half] = tobf(sc + fs);
            }
        }
    }
}

/* causal_gqa_attention_kernel, K/talker_kernels.cu:287-357 (256 threads):
 * per position, thread t < head_dim computes one exact product, block_sum,
 * dot rounded to bf16, score = bf16(dot * rsqrt(d)); thread 0 runs the
 * softmax sequentially in fp32 with bf16-rounded probabilities; each output
 * dimension is a sequential fmaf over positions, then bf16. */
void orc_causal_gqa_attention(const uint16_t* query, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* output,
                              int query_heads, int key_value_heads,
                              int head_dimension, int sequence_length) {
    const int groups = query_heads / key_value_heads;
    const float scale = 1.0f / sqrtf((float)head_dimension);
    float* scores = (float*)malloc((size_t)sequence_length * sizeof(float));
    float partial[256];
    for (int qh = 0; qh < query_heads; ++qh) {
        const int kvh = qh / groups;
        const uint16_t* q = query + (size_t)qh * head_dimension;
        for (int p = 0; p < sequence_length; ++p) {
            const uint16_t* k = key_cache + ((size_t)p * key_value_heads + kvh) * head_dimension;
            for (int t = 0; t < 256; ++t) {
                float dot = 0.0f;
                for (int d = t; d < head_dimension; d += 256) dot = fmaf(bf(q[d]), bf(k[d]), dot);
                partial[t] = dot;
            }
            const float dot = rbf(block_sum_256(partial));
            scores[p] = rbf(dot * scale);
        }
        float maximum = -INFINITY;
        for (int p = 0; p < sequence_length; ++p) maximum = fmaxf(maximum, scores[p]);
        float denominator = 0.0f;
        for (int p = 0; p < sequence_length; ++p) {
            scores[p] = q3_expf(scores[p] - maximum);
            denominator += scores[p];
        }
        const float inverse = 1.0f / denominator;
        for (int p = 0; p < sequence_length; ++p) scores[p] = rbf(scores[p] * inverse);
        uint16_t* out = output + (size_t)qh * head_dimension;
        for (int d = 0; d < head_dimension; ++d) {
            float acc = 0.0f;
            for (int p = 0; p < sequence_length; ++p) {
                const uint16_t* v = value_cache + ((size_t)p * key_value_heads + kvh) * head_dimension;
                acc = fmaf(scores[p], bf(v[d]), acc);
            }
            out[d] = tobf(acc);
        }
    }
    free(scores);
}

/* batch_causal_gqa_attention_fast_kernel, K/talker_kernels.cu:506-595 (one
 * row, 256 threads): fp32 scores from a sequential fmaf over d; max; per-thread
 * strided exp sums folded by the block_sum tree; normalization folded into the
 * output (acc * (1/sum)). */
void orc_causal_gqa_attention_fast(const uint16_t* query,
                                   const uint16_t* key_cache,
                                   const uint16_t* value_cache,
                                   uint16_t* output, int query_heads,
                                   int key_value_heads, int head_dimension,
                                   int sequence_length) {
    const int groups = query_heads / key_value_heads;
    const float scale = 1.0f / sqrtf((float)head_dimension);
    float* scores = (float*)malloc((size_t)sequence_length * sizeof(float));
    float partial[256];
    for (int qh = 0; qh < query_heads; ++qh) {
        const int kvh = qh / groups;
        const uint16_t* q = query + (size_t)qh * head_dimension;
        float maximum = -INFINITY;
        for (int p = 0; p < sequence_length; ++p) {
            const uint16_t* k = key_cache + ((size_t)p * key_value_heads + kvh) * head_dimension;
            float dot = 0.0f;
            for (int d = 0; d < head_dimension; ++d) dot = fmaf(bf(q[d]), bf(k[d]), dot);
            scores[p] = dot * scale;
            maximum = fmaxf(maximum, scores[p]);
        }
        /* thread t sums positions t, t+256, ... in order; then the tree */
        for (int t = 0; t < 256; ++t) {
            float local = 0.0f;
            for (int p = t; p < sequence_length; p += 256) {
                scores[p] = q3_expf(scores[p] - maximum);
                local += scores[p];
            }
            partial[t] = local;
        }
        const float inverse = 1.0f / block_sum_256(partial);
        uint16_t* out = output + (size_t)qh * head_dimension;
        for (int d = 0; d < head_dimension; ++d) {
            float acc = 0.0f;
            for (int p = 0; p < sequence_length; ++p) {
                const uint16_t* v = value_cache + ((size_t)p * key_value_heads + kvh) * head_dimension;
                acc = fmaf(scores[p], bf(v[d]), acc);
            }
            out[d] = tobf(acc * inverse);
        }
    }
    free(scores);
}

/* add_in_place_kernel, K/talker_kernels.cu:359-370. */
void orc_add_in_place(uint16_t* destination, const uint16_t* source, int width) {
    for (int i = 0; i < width; ++i) destination[i] = tobf(bf(destination[i]) + bf(source[i]));
}

/* bias_activation(_rows)_kernel, K/talker_kernels.cu:386-402,660-678:
 * v = x + b; silu: v *= 1/(1+q3_expf(-v)). */
void orc_bias_activation(uint16_t* values, const uint16_t* bias, int rows,
                         int width, int silu) {
    for (int i = 0; i < rows * width; ++i) {
        float value = bf(values[i]) + bf(bias[i % width]);
        if (silu) value *= 1.0f / (1.0f + q3_expf(-value));
        values[i] = tobf(value);
    }
}

/* silu_gate_kernel, K/talker_kernels.cu:404-420:
 * gate = bf16(bf16(g/(1+q3_expf(-g))) * up). */
void orc_silu_gate(uint16_t* gate, const uint16_t* up, int width) {
    for (int i = 0; i < width; ++i) {
        const float g = bf(gate[i]);
        const float activated = rbf(g / (1.0f + q3_expf(-g)));
        gate[i] = tobf(activated * bf(up[i]));
    }
}

/* ------------------------------------------------------------------------ */
/* Sampler                                                                   */
/* ------------------------------------------------------------------------ */

/* adjusted_logit, K/sampling_kernels.cu:30-51. */
static float adjusted_logit(const uint16_t* logits, int token, int suppress,
                            int eos, const int* history, int history_count,
                            float penalty) {
    if (suppress && token >= 2048 && token != eos) return -INFINITY;
    float value = bf(logits[token]);
    if (suppress && penalty != 1.0f) {
        for (int i = 0; i < history_count; ++i) {
            if (history[i] == token) {
                value = value < 0.0f ? value * penalty : value / penalty;
                break;
            }
        }
    }
    return value;
}

typedef struct Cand { float v; int i; } Cand;

/* Total order of the reference selection: value descending, ties (IEEE ==,
 * so -0 == +0) by lower index (sort_before, K/sampling_kernels.cu:71-75). */
static int cand_cmp(const void* a, const void* b) {
    const Cand* x = (const Cand*)a;
    const Cand* y = (const Cand*)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->i > y->i) - (x->i < y->i);
}

int orc_argmax_bf16(const uint16_t* logits, int vocabulary) {
    int best = -1;
    float bv = -INFINITY;
    for (int t = 0; t < vocabulary; ++t) {
        const float v = bf(logits[t]);
        if (best < 0 || v > bv) { bv = v; best = t; }
    }
    return best;
}

/* sample_logits_kernel, K/sampling_kernels.cu:143-389.  The reference's
 * radix-select + bitonic sort produce the top-`selections` tokens in the
 * total order above; the restatement sorts all tokens in that order, which is
 * the same sequence. */
int orc_sample_logits(const uint16_t* logits, int vocabulary,
                      int suppress_talker_reserved, int codec_eos_token,
                      const int* semantic_history, int semantic_history_count,
                      int do_sample, int top_k, float top_p, float temperature,
                      float repetition_penalty, uint64_t* random_state) {
    Cand* c = (Cand*)malloc((size_t)vocabulary * sizeof(Cand));
    double* weights = (double*)malloc((size_t)vocabulary * sizeof(double));
    for (int t = 0; t < vocabulary; ++t) {
        c[t].v = adjusted_logit(logits, t, suppress_talker_reserved, codec_eos_token,
                                semantic_history, semantic_history_count, repetition_penalty);
        c[t].i = t;
    }
    const int direct_categorical = do_sample != 0 && top_k == 0 && top_p >= 1.0f;
    const int selections = do_sample == 0 ? 1 : (top_k == 0 ? vocabulary
                                              : (top_k < vocabulary ? top_k : vocabulary));
    int selected;
    if (do_sample == 0 || direct_categorical) {
        /* argmax, lower index on ties (:208-236) */
        float lv = -INFINITY;
        int li = -1;
        for (int t = 0; t < vocabulary; ++t) {
            if (c[t].v > lv || (c[t].v == lv && li < 0)) { lv = c[t].v; li = t; }
        }
        if (do_sample == 0) {
            selected = li;
        } else {
            /* direct categorical (:242-265) */
            const float maximum = lv / temperature;
            for (int t = 0; t < vocabulary; ++t) {
                weights[t] = exp((double)(c[t].v / temperature - maximum));
            }
            double total = 0.0;
            for (int t = 0; t < vocabulary; ++t) total += weights[t];
            const double target = (double)orc_uniform_random(random_state) * total;
            double cumulative = 0.0;
            selected = li;
            for (int t = 0; t < vocabulary; ++t) {
                cumulative += weights[t];
                if (cumulative >= target) { selected = t; break; }
            }
        }
    } else {
        qsort(c, (size_t)vocabulary, sizeof(Cand), cand_cmp);
        /* softmax / top-p / single draw tail (:350-387) */
        const float maximum = c[0].v / temperature;
        for (int r = 0; r < selections; ++r) {
            weights[r] = exp((double)(c[r].v / temperature - maximum));
        }
        double denominator = 0.0;
        for (int r = 0; r < selections; ++r) denominator += weights[r];
        double cumulative = 0.0;
        int retained = selections;
        for (int r = 0; r < selections; ++r) {
            cumulative += weights[r] / denominator;
            if (cumulative >= (double)top_p) { retained = r + 1; break; }
        }
        double retained_total = 0.0;
        for (int r = 0; r < retained; ++r) retained_total += weights[r];
        const double target = (double)orc_uniform_random(random_state) * retained_total;
        cumulative = 0.0;
        selected = c[retained - 1].i;
        for (int r = 0; r < retained; ++r) {
            cumulative += weights[r];
            if (cumulative >= target) { selected = c[r].i; break; }
        }
    }
    free(c);
    free(weights);
    return selected;
}

/* ------------------------------------------------------------------------ */
/* Model-level restatement                                                   */
/* ------------------------------------------------------------------------ */

static void gemv_bf16(const int8_t* w, const float* s, const uint16_t* x,
                      uint16_t* y, int in, int out) {
    orc_int8_gemm_rows(w, s, x, in, out, 1, NULL, y);
}

/* run_decoder, K/talker.cu:3251-3456 (single-session, int8 weights): unfused
 * q/k/v GEMVs, head norms, RoPE, KV append, exact attention, o + residual,
 * post norm, separate gate and up GEMVs, silu_gate, down + residual. */
void orc_run_decoder(const OrcLayer* layers, const OrcDims* dims,
                     uint16_t* hidden, uint16_t* k_cache, uint16_t* v_cache,
                     int cache_rows, int position, float eps, float theta,
                     int batch_semantics) {
    const int H = dims->hidden;
    const int I = dims->intermediate;
    const int qw = dims->query_heads * dims->head_dimension;
    const int kvw = dims->key_value_heads * dims->head_dimension;
    uint16_t* normalized = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* q = (uint16_t*)malloc((size_t)qw * 2);
    uint16_t* k = (uint16_t*)malloc((size_t)kvw * 2);
    uint16_t* v = (uint16_t*)malloc((size_t)kvw * 2);
    uint16_t* attn = (uint16_t*)malloc((size_t)qw * 2);
    uint16_t* proj = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* gate = (uint16_t*)malloc((size_t)I * 2);
    uint16_t* up = (uint16_t*)malloc((size_t)I * 2);
    for (int li = 0; li < dims->layers; ++li) {
        const OrcLayer* L = &layers[li];
        uint16_t* kc = k_cache + (size_t)li * cache_rows * kvw;
        uint16_t* vc = v_cache + (size_t)li * cache_rows * kvw;
        orc_rms_norm_rows(hidden, L->input_norm, normalized, 1, H, eps);
        gemv_bf16(L->q, L->q_s, normalized, q, H, qw);
        gemv_bf16(L->k, L->k_s, normalized, k, H, kvw);
        gemv_bf16(L->v, L->v_s, normalized, v, H, kvw);
        orc_head_rms_norm_rows(q, L->q_norm, 1, dims->query_heads, dims->head_dimension, eps);
        orc_head_rms_norm_rows(k, L->k_norm, 1, dims->key_value_heads, dims->head_dimension, eps);
        orc_rope_rows(q, 1, dims->query_heads, dims->head_dimension, &position, theta);
        orc_rope_rows(k, 1, dims->key_value_heads, dims->head_dimension, &position, theta);
        memcpy(kc + (size_t)position * kvw, k, (size_t)kvw * 2);
        memcpy(vc + (size_t)position * kvw, v, (size_t)kvw * 2);
        if (batch_semantics) {
            /* batch_run_decoder, int8 branch (K/talker.cu:2178-2285) */
            orc_causal_gqa_attention_fast(q, kc, vc, attn, dims->query_heads, dims->key_value_heads,
                                          dims->head_dimension, position + 1);
            orc_int8_gemm_rows_add(L->o, L->o_s, attn, hidden, qw, H, 1);
            orc_rms_norm_rows(hidden, L->post_norm, normalized, 1, H, eps);
            orc_int8_gate_up_silu_rows(L->gate_up, L->gate_up_s, normalized, gate, H, I, 1);
            orc_int8_gemm_rows_add(L->down, L->down_s, gate, hidden, I, H, 1);
            continue;
        }
        orc_causal_gqa_attention(q, kc, vc, attn, dims->query_heads, dims->key_value_heads,
                                 dims->head_dimension, position + 1);
        gemv_bf16(L->o, L->o_s, attn, proj, qw, H);
        orc_add_in_place(hidden, proj, H);
        orc_rms_norm_rows(hidden, L->post_norm, normalized, 1, H, eps);
        gemv_bf16(L->gate_up, L->gate_up_s, normalized, gate, H, I);
        gemv_bf16(L->gate_up + (size_t)I * H, L->gate_up_s + I, normalized, up, H, I);
        orc_silu_gate(gate, up, I);
        gemv_bf16(L->down, L->down_s, gate, proj, I, H);
        orc_add_in_place(hidden, proj, H);
    }
    free(normalized); free(q); free(k); free(v); free(attn); free(proj); free(gate); free(up);
}

/* project_text, K/talker.cu:2676-2719. */
void orc_project_text(const OrcModel* m, int token, uint16_t* output) {
    const int H = m->talker.hidden;
    uint16_t* projection = (uint16_t*)malloc((size_t)H * 2);
    const uint16_t* embedding = m->text_embedding + (size_t)token * H;
    gemv_bf16(m->text_fc1, m->text_fc1_s, embedding, projection, H, H);
    orc_bias_activation(projection, m->text_fc1_bias, 1, H, 1);
    gemv_bf16(m->text_fc2, m->text_fc2_s, projection, output, H, H);
    orc_bias_activation(output, m->text_fc2_bias, 1, H, 0);
    free(projection);
}

/* run_talker_step(emit_logits=true), K/talker.cu:3458-3495. */
void orc_talker_step(const OrcModel* m, OrcSession* s, const uint16_t* input) {
    const int H = m->talker.hidden;
    uint16_t* hidden = (uint16_t*)malloc((size_t)H * 2);
    memcpy(hidden, input, (size_t)H * 2);
    orc_run_decoder(m->talker_layers, &m->talker, hidden, s->talker_k, s->talker_v,
                    s->max_seq, s->position, m->rms_eps, m->rope_theta, m->batch_semantics);
    orc_rms_norm_rows(hidden, m->talker_norm, s->last_hidden, 1, H, m->rms_eps);
    gemv_bf16(m->codec_head, m->codec_head_s, s->last_hidden, s->logits, H, m->talker_vocab);
    free(hidden);
}

/* sample_logits_device for the talker (K/talker.cu:3583-3627): sample, then
 * append to the semantic history. */
static int sample_talker(const OrcModel* m, OrcSession* s, const OrcSampling* cfg) {
    const int token = orc_sample_logits(s->logits, m->talker_vocab, 1, m->codec_eos,
                                        s->history, s->history_count, cfg->do_sample,
                                        cfg->top_k, cfg->top_p, cfg->temperature,
                                        cfg->repetition_penalty, &s->random_state);
    s->history[s->history_count++] = token;
    return token;
}

/* run_predictor_position, K/talker.cu:3497-3544. */
static void predictor_position(const OrcModel* m, OrcSession* s, const uint16_t* input,
                               int position, int head) {
    const int PH = m->predictor.hidden;
    const int H = m->talker.hidden;
    uint16_t* hidden = (uint16_t*)malloc((size_t)PH * 2);
    gemv_bf16(m->small_to_mtp, m->small_to_mtp_s, input, hidden, H, PH);
    orc_bias_activation(hidden, m->small_to_mtp_bias, 1, PH, 0);
    orc_run_decoder(m->predictor_layers, &m->predictor, hidden, s->pred_k, s->pred_v,
                    m->codebooks, position, m->rms_eps, m->rope_theta, m->batch_semantics);
    if (head >= 0) {
        uint16_t* normalized = (uint16_t*)malloc((size_t)PH * 2);
        orc_rms_norm_rows(hidden, m->predictor_norm, normalized, 1, PH, m->rms_eps);
        gemv_bf16(m->predictor_heads[head], m->predictor_heads_s[head], normalized,
                  s->logits, PH, m->predictor_vocab);
        free(normalized);
    }
    free(hidden);
}

static void trace(const OrcModel* m, const OrcSession* s, int row) {
    if (s->trace_logits == NULL) return;
    const int width = m->talker_vocab > m->predictor_vocab ? m->talker_vocab : m->predictor_vocab;
    const int vocab = row == 0 ? m->talker_vocab : m->predictor_vocab;
    memcpy(s->trace_logits + (size_t)row * width, s->logits, (size_t)vocab * 2);
}

/* begin_frame, K/talker.cu:1095-1244 (single session); with
 * m->batch_semantics one session's row of batch_begin_frames,
 * K/talker.cu:1495-1881 (each row of the lockstep batch is independent). */
int orc_frame_step(const OrcModel* m, OrcSession* s, int semantic_token,
                   int trailing_text_token, const OrcSampling* ts,
                   const OrcSampling* ps, uint16_t* codes) {
    const int H = m->talker.hidden;
    int tokens[64];
    uint16_t* input = (uint16_t*)malloc((size_t)H * 2);
    uint16_t* text = (uint16_t*)malloc((size_t)H * 2);
    tokens[0] = semantic_token;
    predictor_position(m, s, s->last_hidden, 0, -1);
    memcpy(input, m->codec_embedding + (size_t)semantic_token * H, (size_t)H * 2);
    predictor_position(m, s, input, 1, 0);
    trace(m, s, 1);
    tokens[1] = orc_sample_logits(s->logits, m->predictor_vocab, 0, m->codec_eos, s->history,
                                  s->history_count, ps->do_sample, ps->top_k, ps->top_p,
                                  ps->temperature, ps->repetition_penalty, &s->random_state);
    for (int residual = 1; residual < m->codebooks - 1; ++residual) {
        const int tok = tokens[residual];
        if (tok >= 0 && tok < m->predictor_vocab) {
            memcpy(input, m->predictor_embeddings[residual - 1] + (size_t)tok * H, (size_t)H * 2);
        }
        predictor_position(m, s, input, residual + 1, residual);
        trace(m, s, residual + 1);
        tokens[residual + 1] = orc_sample_logits(
            s->logits, m->predictor_vocab, 0, m->codec_eos, s->history, s->history_count,
            ps->do_sample, ps->top_k, ps->top_p, ps->temperature, ps->repetition_penalty,
            &s->random_state);
    }
    for (int i = 0; i < m->codebooks; ++i) codes[i] = (uint16_t)tokens[i];
    /* prepare_generated_embedding, K/talker.cu:3546-3581 */
    memcpy(input, m->codec_embedding + (size_t)tokens[0] * H, (size_t)H * 2);
    for (int residual = 0; residual < m->codebooks - 1; ++residual) {
        const int tok = tokens[residual + 1];
        if (tok >= 0 && tok < m->predictor_vocab) {
            orc_add_in_place(input, m->predictor_embeddings[residual] + (size_t)tok * H, H);
        }
    }
    orc_project_text(m, trailing_text_token, text);
    orc_add_in_place(input, text, H);
    orc_talker_step(m, s, input);
    trace(m, s, 0);
    s->position += 1;
    const int next = sample_talker(m, s, ts);
    free(input);
    free(text);
    return next;
}

/* Prefill as consecutive decode steps.  Each prompt embedding follows
 * prepare_prompt_embedding, K/talker.cu:2721-2748. */
int orc_prefill(const OrcModel* m, OrcSession* s, const int* text_ids,
                const int* codec_ids, int count, const OrcSampling* sampling) {
    const int H = m->talker.hidden;
    uint16_t* input = (uint16_t*)malloc((size_t)H * 2);
    s->position = 0;
    s->history_count = 0;
    for (int i = 0; i < count; ++i) {
        if (text_ids[i] >= 0) {
            orc_project_text(m, text_ids[i], input);
        } else {
            memset(input, 0, (size_t)H * 2);
        }
        if (codec_ids[i] >= 0) {
            orc_add_in_place(input, m->codec_embedding + (size_t)codec_ids[i] * H, H);
        }
        orc_talker_step(m, s, input);
        s->position += 1;
    }
    free(input);
    return sample_talker(m, s, sampling);
}

/* ------------------------------------------------------------------------ */
/* bf16 prefill                                                              */
/* ------------------------------------------------------------------------ */

typedef struct Bf16GemmCtx {
    const float *a, *b;
    uint16_t* c;
    int m, n, k, ldc;
} Bf16GemmCtx;

/* 0: fp32 fmaf chain in k order; 1: the sum accumulated in double (the
 * product of two bf16 is exact in double) and rounded once to fp32. */
static int g_gemm_order = 0;

void orc_set_gemm_order(int order) { g_gemm_order = order; }
int orc_get_gemm_order(void) { return g_gemm_order; }

static void bf16_gemm_range(void* p, int j0, int j1) {
    const Bf16GemmCtx* g = (const Bf16GemmCtx*)p;
    for (int i = 0; i < g->m; ++i) {
        const float* ai = g->a + (size_t)i * g->k;
        for (int j = j0; j < j1; ++j) {
            const float* bj = g->b + (size_t)j * g->k;
            float acc = 0.0f;
            if (g_gemm_order == 1) {
                double sum = 0.0;
                for (int t = 0; t < g->k; ++t) sum += (double)ai[t] * (double)bj[t];
                acc = (float)sum;
            } else {
                for (int t = 0; t < g->k; ++t) acc = fmaf(ai[t], bj[t], acc);
            }
            g->c[(size_t)i * g->ldc + j] = tobf(acc);
        }
    }
}

void orc_bf16_gemm(const uint16_t* a, const uint16_t* b, uint16_t* c, int m, int n, int k,
                   int lda, int ldb, int ldc) {
    float* af = (float*)malloc((size_t)m * k * sizeof(float));
    float* bf_ = (float*)malloc((size_t)n * k * sizeof(float));
    for (int i = 0; i < m; ++i) orc_bf16_to_f32_array(a + (size_t)i * lda, af + (size_t)i * k, (size_t)k);
    for (int j = 0; j < n; ++j) orc_bf16_to_f32_array(b + (size_t)j * ldb, bf_ + (size_t)j * k, (size_t)k);
    Bf16GemmCtx g = {af, bf_, c, m, n, k, ldc};
    orc_for_channels(n, (size_t)m * n * k, bf16_gemm_range, &g);
    free(af);
    free(bf_);
}

void orc_causal_softmax(uint16_t* scores, int heads, int rows, int stride, int head_dimension) {
    const float scale = 1.0f / sqrtf((float)head_dimension);
    float* e = (float*)malloc((size_t)rows * sizeof(float));
    for (int h = 0; h < heads; ++h) {
        for (int q = 0; q < rows; ++q) {
            uint16_t* row = scores + ((size_t)h * rows + q) * stride;
            float maximum = -INFINITY;
            for (int key = 0; key <= q; ++key) {
                e[key] = rbf(bf(row[key]) * scale);
                maximum = fmaxf(maximum, e[key]);
            }
            float denominator = 0.0f;
            for (int key = 0; key <= q; ++key) denominator += q3_expf(e[key] - maximum);
            const float inverse = 1.0f / denominator;
            for (int key = 0; key < stride; ++key) {
                row[key] = key <= q ? tobf(q3_expf(e[key] - maximum) * inverse) : tobf(0.0f);
            }
        }
    }
    free(e);
}

/* run_decoder_prefill, K/talker.cu:2854-3202: per layer RMSNorm rows, q/k/v
 * GEMMs, head norms, RoPE from position 0, cache writes, attention (GEMM path
 * or exact kernel), O GEMM + residual, RMSNorm, gate and up GEMMs, SiLU gate,
 * down GEMM + residual. */
static void prefill_decoder(const OrcModel* m, OrcSession* s, uint16_t* hidden, int rows, int gemm_capacity) {
    const OrcDims* d = &m->talker;
    const int H = d->hidden, I = d->intermediate, hd = d->head_dimension;
    const int qw = d->query_heads * hd, kvw = d->key_value_heads * hd;
    const int group = d->query_heads / d->key_value_heads;
    uint16_t* normalized = (uint16_t*)malloc((size_t)rows * H * 2);
    uint16_t* q = (uint16_t*)malloc((size_t)rows * qw * 2);
    uint16_t* k = (uint16_t*)malloc((size_t)rows * kvw * 2);
    uint16_t* v = (uint16_t*)malloc((size_t)rows * kvw * 2);
    uint16_t* attn = (uint16_t*)malloc((size_t)rows * qw * 2);
    uint16_t* proj = (uint16_t*)malloc((size_t)rows * H * 2);
    uint16_t* gate = (uint16_t*)malloc((size_t)rows * I * 2);
    uint16_t* up = (uint16_t*)malloc((size_t)rows * I * 2);
    int* positions = (int*)malloc((size_t)rows * sizeof(int));
    for (int r = 0; r < rows; ++r) positions[r] = r;
    const int gemm_path = rows <= gemm_capacity;
    uint16_t* scores = gemm_path ? (uint16_t*)malloc((size_t)rows * rows * 2) : NULL;
    uint16_t* qh = gemm_path ? (uint16_t*)malloc((size_t)rows * hd * 2) : NULL;
    uint16_t* kh = gemm_path ? (uint16_t*)malloc((size_t)rows * hd * 2) : NULL;
    uint16_t* vt = gemm_path ? (uint16_t*)malloc((size_t)rows * hd * 2) : NULL;
    uint16_t* oh = gemm_path ? (uint16_t*)malloc((size_t)rows * hd * 2) : NULL;
    for (int li = 0; li < d->layers; ++li) {
        const OrcLayer* L = &m->talker_layers[li];
        uint16_t* kc = s->talker_k + (size_t)li * s->max_seq * kvw;
        uint16_t* vc = s->talker_v + (size_t)li * s->max_seq * kvw;
        orc_rms_norm_rows(hidden, L->input_norm, normalized, rows, H, m->rms_eps);
        orc_bf16_gemm(normalized, L->q16, q, rows, qw, H, H, H, qw);
        orc_bf16_gemm(normalized, L->k16, k, rows, kvw, H, H, H, kvw);
        orc_bf16_gemm(normalized, L->v16, v, rows, kvw, H, H, H, kvw);
        orc_head_rms_norm_rows(q, L->q_norm, rows, d->query_heads, hd, m->rms_eps);
        orc_head_rms_norm_rows(k, L->k_norm, rows, d->key_value_heads, hd, m->rms_eps);
        orc_rope_rows(q, rows, d->query_heads, hd, positions, m->rope_theta);
        orc_rope_rows(k, rows, d->key_value_heads, hd, positions, m->rope_theta);
        memcpy(kc, k, (size_t)rows * kvw * 2);
        memcpy(vc, v, (size_t)rows * kvw * 2);
        if (gemm_path) {
            /* run_prefill_gqa_gemm, K/talker.cu:2750-2852: per query head,
             * scores = bf16(q k^T), causal softmax, out = bf16(p v). */
            for (int h = 0; h < d->query_heads; ++h) {
                const int kvh = h / group;
                for (int r = 0; r < rows; ++r) {
                    memcpy(qh + (size_t)r * hd, q + (size_t)r * qw + (size_t)h * hd, (size_t)hd * 2);
                    memcpy(kh + (size_t)r * hd, k + (size_t)r * kvw + (size_t)kvh * hd, (size_t)hd * 2);
                    for (int t = 0; t < hd; ++t) vt[(size_t)t * rows + r] = v[(size_t)r * kvw + (size_t)kvh * hd + t];
                }
                orc_bf16_gemm(qh, kh, scores, rows, rows, hd, hd, hd, rows);
                orc_causal_softmax(scores, 1, rows, rows, hd);
                orc_bf16_gemm(scores, vt, oh, rows, hd, rows, rows, rows, hd);
                for (int r = 0; r < rows; ++r) {
                    memcpy(attn + (size_t)r * qw + (size_t)h * hd, oh + (size_t)r * hd, (size_t)hd * 2);
                }
            }
        } else {
            /* prefill_causal_gqa_attention_kernel, K/talker_kernels.cu:115-191:
             * row r attends positions 0..r with the exact kernel's order. */
            for (int r = 0; r < rows; ++r) {
                orc_causal_gqa_attention(q + (size_t)r * qw, kc, vc, attn + (size_t)r * qw, d->query_heads,
                                         d->key_value_heads, hd, r + 1);
            }
        }
        orc_bf16_gemm(attn, L->o16, proj, rows, H, qw, qw, qw, H);
        orc_add_in_place(hidden, proj, rows * H);
        orc_rms_norm_rows(hidden, L->post_norm, normalized, rows, H, m->rms_eps);
        orc_bf16_gemm(normalized, L->gate16, gate, rows, I, H, H, H, I);
        orc_bf16_gemm(normalized, L->up16, up, rows, I, H, H, H, I);
        orc_silu_gate(gate, up, rows * I);
        orc_bf16_gemm(gate, L->down16, proj, rows, H, I, I, I, H);
        orc_add_in_place(hidden, proj, rows * H);
    }
    free(normalized); free(q); free(k); free(v); free(attn); free(proj); free(gate); free(up); free(positions);
    free(scores); free(qh); free(kh); free(vt); free(oh);
}

int orc_prefill_bf16(const OrcModel* m, OrcSession* s, const int* text_ids, const int* codec_ids,
                     int count, const OrcSampling* sampling, int gemm_capacity) {
    const int H = m->talker.hidden;
    uint16_t* hidden = (uint16_t*)malloc((size_t)count * H * 2);
    for (int i = 0; i < count; ++i) {
        /* prepare_prompt_embedding, K/talker.cu:2721-2748 (int8 text projection) */
        uint16_t* row = hidden + (size_t)i * H;
        if (text_ids[i] >= 0) {
            orc_project_text(m, text_ids[i], row);
        } else {
            memset(row, 0, (size_t)H * 2);
        }
        if (codec_ids[i] >= 0) orc_add_in_place(row, m->codec_embedding + (size_t)codec_ids[i] * H, H);
    }
    prefill_decoder(m, s, hidden, count, gemm_capacity);
    /* run_talker_prefill, K/talker.cu:3204-3249: final norm of the last row,
     * bf16 codec head GEMM (rows = 1). */
    orc_rms_norm_rows(hidden + (size_t)(count - 1) * H, m->talker_norm, s->last_hidden, 1, H, m->rms_eps);
    orc_bf16_gemm(s->last_hidden, m->codec_head16, s->logits, 1, m->talker_vocab, H, H, H, m->talker_vocab);
    free(hidden);
    s->position = count;
    s->history_count = 0;
    return sample_talker(m, s, sampling);
}
