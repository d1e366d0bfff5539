/*
 * CPU oracle for the int8 weight-only decode path of qwen3-tts-native.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library links, loads or
 * calls this code; only tests/, __graft_entry__.smoke() and the cpu_baseline
 * leg of bench.py use it, and only as the checker (or as the timed CPU
 * baseline), never as the thing measured on the GPU.
 *
 * Every function restates the arithmetic of the reference implementation at
 * /root/reference (path abbreviations: K/ = native/qwen3-tts-native/native/src/)
 * in plain C, in the same operation order, so that a GPU result can be
 * compared bit-for-bit wherever the reference's own order is reproducible.
 * Citations are given per function in oracle.c.
 *
 * bf16 values are carried as uint16_t bit patterns.
 */
#ifndef QWEN3_TTS_ORACLE_H
#define QWEN3_TTS_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------- */
float orc_bf16_to_f32(uint16_t v);
uint16_t orc_f32_to_bf16(float f);
void orc_f32_to_bf16_array(const float* in, uint16_t* out, size_t n);
void orc_bf16_to_f32_array(const uint16_t* in, float* out, size_t n);
uint64_t orc_xorshift64star(uint64_t* state);
/* q3_expf (the exp shared with the HIP kernels) over an array. */
void orc_expf_array(const float* in, float* out, size_t n);
float orc_uniform_random(uint64_t* state);

/* ---- int8 GEMV family (K/int8_gemv.cu) --------------------------------- */
void orc_quantize_weight_rows(const uint16_t* weight, int8_t* quantized,
                              float* scales, int in_features, int out_features);

/* Threads used by the GEMV restatements for large matrices (default 1);
 * results do not depend on it. */
void orc_set_threads(int threads);
/* Test switch: int8 GEMVs sum in double, rounded once (a second valid order). */
void orc_set_gemv_double_sum(int on);
/* Runs fn(ctx, c0, c1) over [0, channels) split across the oracle's threads
 * (one call on the calling thread when work is small). */
typedef void (*OrcRangeFn)(void* ctx, int c0, int c1);
void orc_for_channels(int channels, size_t work, OrcRangeFn fn, void* ctx);

/* y32 (optional) receives value*scale before the bf16 store; y16 (optional)
 * receives the bf16 store.  Both are [rows][out]. */
void orc_int8_gemm_rows(const int8_t* weight, const float* scales,
                        const uint16_t* input, int in_features,
                        int out_features, int rows, float* y32, uint16_t* y16);
/* fp64 restatement of the same formula (order independent). */
void orc_int8_gemm_rows_f64(const int8_t* weight, const float* scales,
                            const uint16_t* input, int in_features,
                            int out_features, int rows, double* y);
void orc_int8_gemm_rows_add(const int8_t* weight, const float* scales,
                            const uint16_t* input, uint16_t* inout,
                            int in_features, int out_features, int rows);
void orc_int8_gate_up_silu_rows(const int8_t* weight, const float* scales,
                                const uint16_t* input, uint16_t* output,
                                int in_features, int out_features, int rows);
/* Multithreaded exact-order GEMV used as the CPU baseline. */
void orc_int8_gemm_rows_mt(const int8_t* weight, const float* scales,
                           const uint16_t* input, int in_features,
                           int out_features, int rows, float* y32,
                           uint16_t* y16, int threads);

/* ---- transformer primitives (K/talker_kernels.cu) ---------------------- */
void orc_rms_norm_rows(const uint16_t* input, const uint16_t* weight,
                       uint16_t* output, int rows, int width, float epsilon);
void orc_head_rms_norm_rows(uint16_t* values, const uint16_t* weight, int rows,
                            int heads, int head_dimension, float epsilon);
void orc_rope_rows(uint16_t* values, int rows, int heads, int head_dimension,
                   const int* positions, float theta);
void orc_causal_gqa_attention(const uint16_t* query, const uint16_t* key_cache,
                              const uint16_t* value_cache, uint16_t* output,
                              int query_heads, int key_value_heads,
                              int head_dimension, int sequence_length);
void orc_causal_gqa_attention_fast(const uint16_t* query,
                                   const uint16_t* key_cache,
                                   const uint16_t* value_cache,
                                   uint16_t* output, int query_heads,
                                   int key_value_heads, int head_dimension,
                                   int sequence_length);
void orc_add_in_place(uint16_t* destination, const uint16_t* source, int width);
void orc_bias_activation(uint16_t* values, const uint16_t* bias, int rows,
                         int width, int silu);
void orc_silu_gate(uint16_t* gate, const uint16_t* up, int width);

/* ---- sampler (K/sampling_kernels.cu) ----------------------------------- */
int orc_sample_logits(const uint16_t* logits, int vocabulary,
                      int suppress_talker_reserved, int codec_eos_token,
                      const int* semantic_history, int semantic_history_count,
                      int do_sample, int top_k, float top_p, float temperature,
                      float repetition_penalty, uint64_t* random_state);
int orc_argmax_bf16(const uint16_t* logits, int vocabulary);

/* ---- model-level restatement (K/talker.cu) ----------------------------- */
typedef struct OrcDims {
    int hidden, intermediate, query_heads, key_value_heads, head_dimension;
    int layers;
} OrcDims;

typedef struct OrcLayer {
    const uint16_t *input_norm, *q_norm, *k_norm, *post_norm;
    const int8_t *q, *k, *v, *o, *gate_up, *down; /* gate_up: gate rows first */
    const float *q_s, *k_s, *v_s, *o_s, *gate_up_s, *down_s;
    /* bf16 weights (the prefill's, K/talker.cu:2750-3202) */
    const uint16_t *q16, *k16, *v16, *o16, *gate16, *up16, *down16;
} OrcLayer;

typedef struct OrcModel {
    OrcDims talker, predictor;
    int talker_vocab, predictor_vocab, text_vocab, codebooks; /* 16 */
    int codec_eos;
    float rms_eps, rope_theta;
    const OrcLayer* talker_layers;    /* [talker.layers] */
    const OrcLayer* predictor_layers; /* [predictor.layers] */
    const uint16_t* codec_embedding;  /* [talker_vocab][talker.hidden] */
    const uint16_t* text_embedding;   /* [text_vocab][talker.hidden] */
    const int8_t *text_fc1, *text_fc2; const float *text_fc1_s, *text_fc2_s;
    const uint16_t *text_fc1_bias, *text_fc2_bias, *talker_norm;
    const int8_t* codec_head; const float* codec_head_s;
    const int8_t* small_to_mtp; const float* small_to_mtp_s;
    const uint16_t *small_to_mtp_bias, *predictor_norm;
    const uint16_t* const* predictor_embeddings; /* [codebooks-1] x [pvocab][talker.hidden] */
    const int8_t* const* predictor_heads;        /* [codebooks-1] x [pvocab][predictor.hidden] */
    const float* const* predictor_heads_s;
    /* 0: single-session decoder (K/talker.cu:3251-3456); 1: the lockstep
     * batched int8 decoder (K/talker.cu:2038-2334): fast attention, fma
     * residual epilogue, fused gate/up SiLU. */
    int batch_semantics;
    const uint16_t* codec_head16; /* bf16 codec head (prefill logits) */
} OrcModel;

typedef struct OrcSession {
    int max_seq;
    int position;
    int history_count;
    int* history;        /* [max_seq] */
    uint64_t random_state;
    uint16_t* talker_k;  /* [layers][max_seq][kv_width] */
    uint16_t* talker_v;
    uint16_t* pred_k;    /* [players][16][kv_width] */
    uint16_t* pred_v;
    uint16_t* last_hidden; /* [talker.hidden] (final-normed) */
    uint16_t* logits;      /* [max(talker_vocab, predictor_vocab)] */
    /* Optional (NULL: off): the logits each sample of orc_frame_step reads,
     * [16][max(talker_vocab, predictor_vocab)]: row 0 the talker's (raw,
     * before mask and penalty), rows 1..15 the predictor codebooks'. */
    uint16_t* trace_logits;
} OrcSession;

typedef struct OrcSampling {
    int do_sample, top_k;
    float top_p, temperature, repetition_penalty;
} OrcSampling;

/* One single-session decoder stack step at `position` on hidden[dims.hidden]
 * (K/talker.cu:3251-3456).  k_cache/v_cache: [layers][cache_rows][kv_width]. */
void orc_run_decoder(const OrcLayer* layers, const OrcDims* dims,
                     uint16_t* hidden, uint16_t* k_cache, uint16_t* v_cache,
                     int cache_rows, int position, float eps, float theta,
                     int batch_semantics);
/* Talker step on a prepared input embedding; writes logits + last_hidden. */
void orc_talker_step(const OrcModel* m, OrcSession* s, const uint16_t* input);
/* Text projection fc1+SiLU, fc2+bias (K/talker.cu:2676-2719). */
void orc_project_text(const OrcModel* m, int token, uint16_t* output);
/* One full codec frame (K/talker.cu:1095-1244): predictor 16 positions from
 * last_hidden + semantic token, then the talker step.  Writes codes[16] and
 * returns the next semantic token. */
int orc_frame_step(const OrcModel* m, OrcSession* s, int semantic_token,
                   int trailing_text_token, const OrcSampling* talker_sampling,
                   const OrcSampling* predictor_sampling, uint16_t* codes);
/* Prefill restated as consecutive single-token decode steps (the build's
 * prefill design; the reference prefill runs bf16 GEMMs, see talker.cu:2721+).
 * Returns the first semantic token. */
int orc_prefill(const OrcModel* m, OrcSession* s, const int* text_ids,
                const int* codec_ids, int count, const OrcSampling* sampling);

/* ---- bf16 prefill (K/talker.cu:2750-3249) ------------------------------ */
/* c[i][j] = bf16(sum_k a[i][k] * b[j][k]): fp32 fmaf chain in k order (the
 * reference's cuBLAS order is unspecified; this is the oracle's own). */
void orc_bf16_gemm(const uint16_t* a, const uint16_t* b, uint16_t* c, int m, int n, int k,
                   int lda, int ldb, int ldc);
/* Accumulation of orc_bf16_gemm: 0 (default) the fp32 chain above; 1 the sum
 * in double rounded once -- a second valid order, used to measure how far
 * two fp32 GEMM orders drift apart through a deep prefill. */
void orc_set_gemm_order(int order);
int orc_get_gemm_order(void);
/* causal_softmax_kernel (K/talker_kernels.cu:232-260) on [heads][rows][stride]. */
void orc_causal_softmax(uint16_t* scores, int heads, int rows, int stride, int head_dimension);
/* run_talker_prefill with the prompt embeddings of prepare_prompt_embedding:
 * fills the session's talker caches 0..count-1, last_hidden and logits, then
 * samples the first semantic token.  Attention uses the GEMM path when count
 * <= gemm_capacity (min(max_seq, 512) in the reference), else the exact
 * per-row kernel. */
int orc_prefill_bf16(const OrcModel* m, OrcSession* s, const int* text_ids, const int* codec_ids,
                     int count, const OrcSampling* sampling, int gemm_capacity);

#ifdef __cplusplus
}
#endif
#endif
