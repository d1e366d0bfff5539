/*
 * qwen3-tts talker C ABI, version 3 -- MI355X (gfx950 / HIP) implementation.
 *
 * The first part of this header is the drop-in boundary: every type, constant
 * and function keeps the name, argument order, struct layout and status-code
 * meaning of the reference library's public header
 * native/qwen3-tts-native/native/include/qwen3_tts_native.h (cited as H:line),
 * so a caller that dlopens the reference library by symbol name (the Rust
 * NativeTalkerModel, native/qwen3-tts-native/src/native_talker.rs:765-840)
 * can load this library instead.  The "CUDA" spellings are ABI names; on this
 * build an event handle carries a hipEvent_t and status -2 reports a HIP error.
 *
 * The second part lists additive exports of this build (no counterpart in the
 * reference): the int8 GEMV entry point and its benchmark, the primitive ops
 * the parity tests drive, a reduced-size model configuration for tests, and
 * small device-memory helpers.  They follow the reference's additive-ABI
 * convention (int32 status, caller-owned error buffer).
 */
#ifndef QWEN3_TTS_NATIVE_H
#define QWEN3_TTS_NATIVE_H

#include <stddef.h>
#include <stdint.h>

#define QWEN3_TTS_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* H:16-18 */
#define QWEN3_TTS_TALKER_ABI_VERSION 3U
#define QWEN3_TTS_MAX_BATCH_SESSIONS 8
#define QWEN3_TTS_CODEC_CODEBOOKS 16U

/* H:20-27 status codes */
enum {
    QWEN3_TTS_TALKER_STATUS_OK = 0,
    QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT = -1,
    QWEN3_TTS_TALKER_STATUS_CUDA = -2, /* device (HIP) runtime error */
    QWEN3_TTS_TALKER_STATUS_STATE = -3,
    QWEN3_TTS_TALKER_STATUS_ALLOCATION = -4,
    QWEN3_TTS_TALKER_STATUS_MODEL = -5,
};

/* H:29-37 */
typedef struct Qwen3TtsDeviceInfo {
    int32_t device_index;
    int32_t compute_major;
    int32_t compute_minor;
    uint64_t total_global_memory_bytes;
    uint64_t runtime_free_memory_bytes;
    uint64_t runtime_total_memory_bytes;
    char device_name[256];
} Qwen3TtsDeviceInfo;

/* H:39-46 */
typedef struct Qwen3TtsArgmaxBenchmark {
    int32_t vocabulary_size;
    int32_t iterations;
    int32_t selected_token;
    int32_t expected_token;
    float cold_launch_microseconds;
    float mean_launch_microseconds;
} Qwen3TtsArgmaxBenchmark;

/* H:48-57 */
typedef struct Qwen3TtsGemvBenchmark {
    int32_t input_features;
    int32_t output_features;
    int32_t iterations;
    int32_t reserved;
    uint64_t weight_bytes;
    float cold_launch_microseconds;
    float mean_launch_microseconds;
    float tera_operations_per_second;
} Qwen3TtsGemvBenchmark;

/* H:59 */
typedef struct Qwen3TtsDeviceBuffer Qwen3TtsDeviceBuffer;

/* H:61-72 */
typedef struct Qwen3TtsWeightUploadMetrics {
    int32_t device_index;
    int32_t reserved;
    uint64_t allocation_bytes;
    uint64_t pinned_staging_bytes;
    uint64_t uploaded_bytes;
    uint64_t upload_calls;
    uint64_t free_before_bytes;
    uint64_t free_after_allocation_bytes;
    float allocation_microseconds;
    float upload_microseconds;
} Qwen3TtsWeightUploadMetrics;

/* H:74-79 */
typedef struct Qwen3TtsPrimitiveParity {
    float rms_norm_max_absolute_error;
    float rope_max_absolute_error;
    float attention_max_absolute_error;
    float silu_gate_max_absolute_error;
} Qwen3TtsPrimitiveParity;

/* H:81-87 (20 bytes) */
typedef struct Qwen3TtsSamplingConfig {
    int32_t do_sample;
    int32_t top_k;
    float top_p;
    float temperature;
    float repetition_penalty;
} Qwen3TtsSamplingConfig;

/* H:89-94 (12 bytes) */
typedef struct Qwen3TtsTalkerPrefillResult {
    uint16_t first_semantic_token;
    uint16_t reserved;
    uint32_t prompt_tokens;
    float talker_gpu_milliseconds;
} Qwen3TtsTalkerPrefillResult;

/* H:96-103 */
typedef struct Qwen3TtsCodecFrameResult {
    uint16_t codes[QWEN3_TTS_CODEC_CODEBOOKS];
    uint16_t next_semantic_token;
    uint16_t ended_by_eos;
    uint32_t talker_position;
    float predictor_gpu_milliseconds;
    float talker_gpu_milliseconds;
} Qwen3TtsCodecFrameResult;

/* H:105-110 (16 bytes) */
typedef struct Qwen3TtsCodecFrameInfo {
    uint32_t talker_position;
    uint32_t ended_by_eos;
    float predictor_gpu_milliseconds;
    float talker_gpu_milliseconds;
} Qwen3TtsCodecFrameInfo;

/* H:112-114: borrowed device event (a hipEvent_t on this build). */
typedef void* Qwen3TtsCudaEventHandle;

/* H:116-128 (40 bytes, 8-byte aligned) */
typedef struct Qwen3TtsDeviceFrameViewV2 {
    uint32_t struct_size;
    uint32_t code_count;
    const uint16_t* device_codes;
    Qwen3TtsCudaEventHandle ready_event;
    uint64_t lease_id;
    int32_t device_index;
    uint32_t reserved;
} Qwen3TtsDeviceFrameViewV2;

/* H:130-135 */
typedef enum Qwen3TtsTalkerPhase {
    QWEN3_TTS_TALKER_CREATED = 0,
    QWEN3_TTS_TALKER_READY = 1,
    QWEN3_TTS_TALKER_PREFILLED = 2,
    QWEN3_TTS_TALKER_ENDED = 3,
} Qwen3TtsTalkerPhase;

/* H:137-145 (40 bytes) */
typedef struct Qwen3TtsTalkerStateInfo {
    uint32_t abi_version;
    uint32_t phase;
    uint32_t talker_position;
    uint32_t semantic_history_count;
    uint64_t frames_generated;
    uint64_t device_sample_count;
    uint64_t host_sync_count;
} Qwen3TtsTalkerStateInfo;

/* H:147-151 (16 bytes) */
typedef struct Qwen3TtsModelMemory {
    uint64_t shared_weight_bytes;
    uint32_t tensor_count;
    int32_t device_index;
} Qwen3TtsModelMemory;

/* H:153-159 (32 bytes) */
typedef struct Qwen3TtsSessionMemory {
    uint64_t talker_kv_bytes;
    uint64_t predictor_kv_bytes;
    uint64_t workspace_bytes;
    uint32_t max_sequence_length;
    uint32_t reserved;
} Qwen3TtsSessionMemory;

typedef void* Qwen3TtsModelHandle;   /* H:161 */
typedef void* Qwen3TtsSessionHandle; /* H:162 */

/* ---- drop-in boundary: reference ABI v3 entry points (H:164-371) ---- */

QWEN3_TTS_API uint32_t qwen3_tts_talker_abi_version(void); /* H:164 */

QWEN3_TTS_API int32_t qwen3_tts_probe_device( /* H:166-171, runtime.cu:86 */
    int32_t device_index, Qwen3TtsDeviceInfo* output, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_benchmark_bf16_argmax( /* H:173-180, runtime.cu:124 */
    int32_t device_index, int32_t vocabulary_size, int32_t iterations,
    Qwen3TtsArgmaxBenchmark* output, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_benchmark_bf16_gemv( /* H:182-190, gemv.cu:88 */
    int32_t device_index, int32_t input_features, int32_t output_features, int32_t iterations,
    Qwen3TtsGemvBenchmark* output, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_create( /* H:192-200, weights.cu */
    int32_t device_index, uint64_t capacity_bytes, uint64_t staging_bytes,
    Qwen3TtsDeviceBuffer** output, Qwen3TtsWeightUploadMetrics* metrics, char* error,
    size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_validate_transformer_primitives( /* H:202-207, primitive_parity.cu:328 */
    int32_t device_index, Qwen3TtsPrimitiveParity* output, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_upload( /* H:209-216 */
    Qwen3TtsDeviceBuffer* buffer, uint64_t offset_bytes, const void* source, uint64_t bytes,
    char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_finish( /* H:218-223 */
    Qwen3TtsDeviceBuffer* buffer, Qwen3TtsWeightUploadMetrics* metrics, char* error,
    size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_read( /* H:225-232 */
    Qwen3TtsDeviceBuffer* buffer, uint64_t offset_bytes, void* destination, uint64_t bytes,
    char* error, size_t error_capacity);

QWEN3_TTS_API const void* qwen3_tts_device_buffer_data( /* H:234-236 */
    const Qwen3TtsDeviceBuffer* buffer);

QWEN3_TTS_API void qwen3_tts_device_buffer_destroy(Qwen3TtsDeviceBuffer* buffer); /* H:238-240 */

QWEN3_TTS_API int32_t qwen3_tts_model_create( /* H:242-247, talker.cu:3819 */
    int32_t device_index, Qwen3TtsModelHandle* output, char* error, size_t error_capacity);

QWEN3_TTS_API void qwen3_tts_model_destroy(Qwen3TtsModelHandle handle); /* H:249 */

QWEN3_TTS_API int32_t qwen3_tts_model_upload_tensor( /* H:251-260, talker.cu:3838 */
    Qwen3TtsModelHandle handle, const char* name, const void* bf16_data, uint64_t byte_size,
    int32_t rank, const uint64_t* shape, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_model_finalize( /* H:262-267, talker.cu:3853 */
    Qwen3TtsModelHandle handle, Qwen3TtsModelMemory* memory, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_session_create( /* H:269-277, talker.cu:3868 */
    Qwen3TtsModelHandle model, int32_t max_sequence_length, uint64_t random_seed,
    Qwen3TtsSessionHandle* output, Qwen3TtsSessionMemory* memory, char* error,
    size_t error_capacity);

QWEN3_TTS_API void qwen3_tts_session_destroy(Qwen3TtsSessionHandle handle); /* H:279 */

QWEN3_TTS_API int32_t qwen3_tts_session_reset( /* H:281-286 */
    Qwen3TtsSessionHandle handle, uint64_t random_seed, char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_session_prefill( /* H:288-297, talker.cu:3905 */
    Qwen3TtsSessionHandle handle, const int32_t* text_token_ids, const int32_t* codec_token_ids,
    int32_t token_count, Qwen3TtsSamplingConfig sampling, Qwen3TtsTalkerPrefillResult* output,
    char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_session_next_frame( /* H:299-311, talker.cu:3931 */
    Qwen3TtsSessionHandle handle, uint16_t semantic_token, int32_t trailing_text_token_id,
    Qwen3TtsSamplingConfig talker_sampling, Qwen3TtsSamplingConfig predictor_sampling,
    uint16_t* output_codes, size_t output_code_capacity, uint16_t* next_semantic_token,
    Qwen3TtsCodecFrameInfo* frame_info, char* error, size_t error_capacity);

/* H:313-328: enqueue one frame without a host synchronization; the view and
 * its event stay valid until the matching finish. */
QWEN3_TTS_API int32_t qwen3_tts_session_next_frame_begin_v2(
    Qwen3TtsSessionHandle handle, int32_t trailing_text_token_id,
    Qwen3TtsSamplingConfig talker_sampling, Qwen3TtsSamplingConfig predictor_sampling,
    Qwen3TtsDeviceFrameViewV2* output, char* error, size_t error_capacity);

/* H:330-343 */
QWEN3_TTS_API int32_t qwen3_tts_session_next_frame_finish_v2(
    Qwen3TtsSessionHandle handle, uint64_t lease_id, Qwen3TtsCudaEventHandle consumer_done_event,
    uint16_t* next_semantic_token, Qwen3TtsCodecFrameInfo* frame_info, char* error,
    size_t error_capacity);

/* H:345-364: lockstep batch of up to 8 sessions sharing one weight read. */
QWEN3_TTS_API int32_t qwen3_tts_model_batch_next_frame_begin_v2(
    Qwen3TtsModelHandle model_handle, Qwen3TtsSessionHandle* sessions, int32_t session_count,
    const int32_t* trailing_text_token_ids, const Qwen3TtsSamplingConfig* talker_sampling,
    const Qwen3TtsSamplingConfig* predictor_sampling, Qwen3TtsDeviceFrameViewV2* outputs,
    char* error, size_t error_capacity);

QWEN3_TTS_API int32_t qwen3_tts_session_state_info( /* H:366-371 */
    Qwen3TtsSessionHandle handle, Qwen3TtsTalkerStateInfo* output, char* error,
    size_t error_capacity);

/* ====================================================================== */
/* Additive exports of this build (no counterpart in the reference ABI).  */
/* ====================================================================== */

/* Reduced model geometry for tests (the reference fixes the VoiceDesign
 * dimensions at compile time, talker.cu:29-52).  head_dimension must be 128.
 * Tensor names and the shape contract follow talker.cu:488-562,693-747 with
 * these dimensions substituted. */
typedef struct Qwen3TtsModelConfigV1 {
    uint32_t struct_size;
    int32_t talker_layers, talker_hidden, talker_intermediate;
    int32_t talker_query_heads, talker_key_value_heads;
    int32_t predictor_layers, predictor_hidden, predictor_intermediate;
    int32_t predictor_query_heads, predictor_key_value_heads;
    int32_t head_dimension;
    int32_t talker_vocabulary, predictor_vocabulary, text_vocabulary;
    int32_t codec_eos_token;
    float rms_epsilon, rope_theta;
} Qwen3TtsModelConfigV1;

/* Diagnostics (what the reference traces as "final_norm", talker.cu:3484 and
 * :3230): copies the session's final-normalized talker
 * hidden state (talker_hidden bf16 values, `bytes` must equal 2 *
 * talker_hidden) after the last completed prefill or frame to host memory.
 * Fails with QWEN3_TTS_TALKER_STATUS_STATE while a frame lease is in flight. */
QWEN3_TTS_API int32_t qwen3_tts_session_read_last_hidden_v1(
    Qwen3TtsSessionHandle handle, void* destination, uint64_t bytes, char* error,
    size_t error_capacity);

/* Diagnostics: positions 0..count-1 of talker layer `layer`'s key cache
 * (which = 0) or value cache (which = 1) as [position][kv_width] bf16 in host
 * memory; `bytes` must equal 2 * count * kv_width.  Fails with
 * QWEN3_TTS_TALKER_STATUS_STATE while a frame lease is in flight. */
QWEN3_TTS_API int32_t qwen3_tts_session_read_talker_cache_v1(
    Qwen3TtsSessionHandle handle, int32_t layer, int32_t which, int32_t count, void* destination,
    uint64_t bytes, char* error, size_t error_capacity);

/* Fills `output` with the VoiceDesign geometry of the reference. */
QWEN3_TTS_API void qwen3_tts_model_config_default(Qwen3TtsModelConfigV1* output);

QWEN3_TTS_API int32_t qwen3_tts_model_create_with_config(
    int32_t device_index, const Qwen3TtsModelConfigV1* config, Qwen3TtsModelHandle* output,
    char* error, size_t error_capacity);

/* int8 GEMV epilogues (y = scale[c] * dot(W[c], x)):
 * 0 STORE          out16 = bf16(y), out32 = y          (int8_gemv.cu:123)
 * 1 ADD_FMA        out16 = bf16(fma(dot, scale, out16))   (int8_gemv.cu:192-196)
 * 2 ADD_ROUNDED    out16 = bf16(out16 + bf16(y))        (GEMV + add_in_place)
 * 3 SILU_FUSED     out16 = bf16(silu(yg) * yu), W = [gate;up] (int8_gemv.cu:283-289)
 * 4 SILU_ROUNDED   bf16 gate/up, then silu_gate (talker_kernels.cu:404-420)
 * 5 BIAS           out16 = bf16(bf16(y) + bias)         (GEMV + bias_activation)
 * 6 BIAS_SILU      v = bf16(y) + bias; out16 = bf16(v * (1/(1+exp(-v))))
 * 7 BIAS_ADD       out16 = bf16(out16 + bf16(bf16(y) + bias))
 * Modes: 0 auto (exact for rows == 1, MFMA for rows >= 2), 1 exact (the
 * reference's lane order, bit-exact), 2 MFMA. */
typedef struct Qwen3TtsInt8GemvV1 {
    uint32_t struct_size;
    int32_t in_features;
    int32_t out_features;
    int32_t rows;
    int32_t epilogue;
    int32_t mode;
    float norm_epsilon;
    int32_t reserved;
    const int8_t* weight;      /* device, [out_rows][in], 16-byte aligned */
    const float* scales;       /* device, [out_rows] */
    const uint16_t* input;     /* device bf16 [rows][in], 16-byte aligned */
    const uint16_t* norm_weight; /* optional device bf16 [in]: fused RMSNorm prologue */
    const uint16_t* bias;      /* device bf16 [out] for BIAS epilogues */
    const int32_t* input_row_index; /* optional device int: input += index * in */
    uint16_t* out16;           /* device bf16 [rows][out] */
    float* out32;              /* device fp32 [rows][out] (STORE only) */
} Qwen3TtsInt8GemvV1;

/* Replaces the internal launch_int8_gemm_rows / _add / gate_up_silu_rows
 * launchers (int8_gemv.cu:319-422, talker_internal.cuh:326-356), which the
 * reference does not export.  `stream` is a hipStream_t (null = default). */
QWEN3_TTS_API int32_t qwen3_tts_int8_gemv_v1(
    const Qwen3TtsInt8GemvV1* args, void* stream, char* error, size_t error_capacity);

/* launch_quantize_weight_rows (int8_gemv.cu:302-317). */
QWEN3_TTS_API int32_t qwen3_tts_quantize_weight_rows_v1(
    const uint16_t* weight, int8_t* quantized, float* scales, int32_t in_features,
    int32_t out_features, void* stream, char* error, size_t error_capacity);

/* int8 GEMV benchmark on synthetic data with rotating weight copies (enough
 * to exceed the 256 MB last-level cache); fills the reference's
 * Qwen3TtsGemvBenchmark (tera_operations_per_second = 2*in*out/t). */
QWEN3_TTS_API int32_t qwen3_tts_benchmark_int8_gemv(
    int32_t device_index, int32_t input_features, int32_t output_features, int32_t iterations,
    Qwen3TtsGemvBenchmark* output, char* error, size_t error_capacity);

/* Primitive ops driven by the parity tests (device pointers, hipStream_t). */
QWEN3_TTS_API int32_t qwen3_tts_op_rms_norm_rows(
    const uint16_t* input, const uint16_t* weight, uint16_t* output, int32_t rows,
    int32_t width, float epsilon, void* stream, char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_head_rms_norm_rows(
    uint16_t* values, const uint16_t* weight, int32_t rows, int32_t heads,
    int32_t head_dimension, float epsilon, void* stream, char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_rope_rows(
    uint16_t* values, int32_t rows, int32_t heads, int32_t head_dimension,
    const int32_t* positions, float theta, void* stream, char* error, size_t error_capacity);
/* Host-side RoPE table as used by the decode path: [positions][d/2][2] bf16. */
QWEN3_TTS_API int32_t qwen3_tts_rope_table_v1(
    int32_t positions, int32_t head_dimension, float theta, uint16_t* host_output,
    char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_qk_norm_rope_kv_append(
    uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm, uint16_t* const* key_bases,
    uint16_t* const* value_bases, const int32_t* positions, const uint16_t* rope_table,
    int32_t rows, int32_t query_heads, int32_t key_value_heads, int32_t head_dimension,
    float epsilon, void* stream, char* error, size_t error_capacity);
/* exact != 0: causal_gqa_attention semantics; 0: the batched "fast" kernel. */
QWEN3_TTS_API int32_t qwen3_tts_op_attention(
    int32_t exact, const uint16_t* query, int32_t query_stride, uint16_t* const* key_bases,
    uint16_t* const* value_bases, const int32_t* positions, uint16_t* output, int32_t rows,
    int32_t query_heads, int32_t key_value_heads, int32_t head_dimension,
    int32_t max_sequence_length, void* stream, char* error, size_t error_capacity);
/* The prefill's exact attention for prompts beyond the GEMM path
 * (talker.cu:3035-3054): query rows r = 0..rows-1 against one shared, complete
 * cache (key_cache and value_cache [capacity][key_value_heads*head_dimension]),
 * row r attending to positions 0..positions[r]; causal_gqa_attention
 * semantics when exact != 0. */
QWEN3_TTS_API int32_t qwen3_tts_op_prompt_attention_v1(
    int32_t exact, const uint16_t* query, int32_t query_stride, const uint16_t* key_cache,
    const uint16_t* value_cache, const int32_t* positions, uint16_t* output, int32_t rows,
    int32_t query_heads, int32_t key_value_heads, int32_t head_dimension, int32_t capacity,
    void* stream, char* error, size_t error_capacity);
/* qk_norm_rope_kv_append followed by attention, as one fused decode step:
 * qkv holds the raw fused q|k|v rows (row stride qkv_stride); query heads are
 * head-normalized and rotated, the key of position positions[row] is
 * normalized, rotated and appended to the caches with its value, then
 * attention runs over positions 0..positions[row].  Results and cache
 * contents are identical to the two separate ops; the query part of qkv is
 * left unrotated.  Replaces the head norm / RoPE / cache append / attention
 * sequence at talker.cu:3298-3380 (single session) and talker.cu:2100-2195
 * (batched). */
QWEN3_TTS_API int32_t qwen3_tts_op_decode_attention(
    int32_t exact, const uint16_t* qkv, int32_t qkv_stride, const uint16_t* q_norm,
    const uint16_t* k_norm, const uint16_t* rope_table, float epsilon, uint16_t* const* key_bases,
    uint16_t* const* value_bases, const int32_t* positions, uint16_t* output, int32_t rows,
    int32_t query_heads, int32_t key_value_heads, int32_t head_dimension,
    int32_t max_sequence_length, void* stream, char* error, size_t error_capacity);
/* The same fused decode step without any device allocation (no counterpart
 * in the reference: for callers that cannot call hipMalloc -- code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation).  The
 * score workspace and the value temporary live in a static per-device
 * scratch of 32 MiB held until the process ends; calls needing more (roughly
 * rows * (4 * query_heads + 2 * key_value_heads * 128) * max_sequence_length
 * bytes) fail with QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT.  Every call on a
 * device shares that device's scratch, which keeps the last call's contents.
 * Eager calls are serialized in stream order: a call on another stream (or
 * thread) than the previous call on the device first makes its stream wait
 * for that call's kernels.  A call made while its stream is being captured
 * is ordered by the graph instead: replays of such graphs must not overlap
 * each other, or eager calls, on one device.  Results are identical to
 * qwen3_tts_op_decode_attention. */
QWEN3_TTS_API int32_t qwen3_tts_op_decode_attention_noalloc_v1(
    int32_t exact, const uint16_t* qkv, int32_t qkv_stride, const uint16_t* q_norm,
    const uint16_t* k_norm, const uint16_t* rope_table, float epsilon, uint16_t* const* key_bases,
    uint16_t* const* value_bases, const int32_t* positions, uint16_t* output, int32_t rows,
    int32_t query_heads, int32_t key_value_heads, int32_t head_dimension,
    int32_t max_sequence_length, void* stream, char* error, size_t error_capacity);
/* The prefill's bf16 GEMM (the reference's cublasGemmEx / StridedBatchedEx
 * calls with CUBLAS_COMPUTE_32F, talker.cu:2637-2674,2772-2842):
 * C[m][n] = bf16(sum_k A[m][k] * B[n][k]) with fp32 accumulation, all
 * row-major; batch z uses A + z*a_batch, B + (z / b_group)*b_batch and
 * C + z*c_batch (elements).  k, lda, ldb, a_batch, b_batch multiples of 8;
 * A and B 16-byte aligned. */
QWEN3_TTS_API int32_t qwen3_tts_op_bf16_gemm_v1(
    const uint16_t* a, const uint16_t* b, uint16_t* c, int32_t m, int32_t n, int32_t k, int32_t lda,
    int32_t ldb, int32_t ldc, int32_t batch, int32_t b_group, int64_t a_batch, int64_t b_batch,
    int64_t c_batch, void* stream, char* error, size_t error_capacity);
/* The same product with a split-K workspace (no counterpart in the reference,
 * whose cuBLAS calls choose their own split): partial holds partial_floats
 * fp32; tile 0 (planned) or 32/64/128, k_step (K per pipeline step) 0
 * (planned) or 64/128/256 (32 tile), 64/128 (64 tile), 64 (128 tile), and
 * splits 0 (planned) or a K slice count,
 * bounded by the workspace (splits * batch * m * n floats).  The slices' sums
 * are added in slice order.  epilogue 0 stores bf16(sum); 1 adds it into C
 * as add_in_place does after a GEMM (C = bf16(C + bf16(sum))); 2 applies
 * silu_gate with C holding the gate product (C = bf16(bf16(silu(C)) *
 * bf16(sum))).  The prefill uses the planned form. */
QWEN3_TTS_API int32_t qwen3_tts_op_bf16_gemm_split_v1(
    const uint16_t* a, const uint16_t* b, uint16_t* c, int32_t m, int32_t n, int32_t k, int32_t lda,
    int32_t ldb, int32_t ldc, int32_t batch, int32_t b_group, int64_t a_batch, int64_t b_batch,
    int64_t c_batch, float* partial, uint64_t partial_floats, int32_t tile, int32_t k_step, int32_t splits,
    int32_t epilogue, void* stream, char* error, size_t error_capacity);
/* causal_softmax_kernel (talker_kernels.cu:232-260) on bf16 scores
 * [heads][rows][stride], in place; keys past the query (up to stride) are set
 * to 0.  rows <= 512. */
QWEN3_TTS_API int32_t qwen3_tts_op_causal_softmax_v1(
    uint16_t* scores, int32_t heads, int32_t rows, int32_t stride, int32_t head_dimension, void* stream,
    char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_kv_scatter_rows(
    const uint16_t* rows_data, uint16_t* const* cache_bases, const int32_t* positions,
    int32_t rows, int32_t width, int32_t row_stride, void* stream, char* error,
    size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_elementwise(
    int32_t op, uint16_t* values, const uint16_t* other, int32_t rows, int32_t width,
    void* stream, char* error, size_t error_capacity); /* 0 add, 1 bias, 2 bias+silu, 3 silu_gate */
QWEN3_TTS_API int32_t qwen3_tts_op_sample_logits(
    const uint16_t* logits, int32_t vocabulary, int32_t suppress_talker_reserved,
    int32_t codec_eos_token, const int32_t* semantic_history, const int32_t* history_count,
    Qwen3TtsSamplingConfig sampling, uint64_t* random_state, int32_t* selected_token,
    void* stream, char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_op_sum_embeddings(
    const uint16_t* const* tables, int32_t count, int32_t vocabulary0, int32_t vocabulary,
    int32_t width, const int32_t* tokens, uint16_t* output, void* stream, char* error,
    size_t error_capacity);

/* Device memory / stream helpers for harnesses. */
QWEN3_TTS_API int32_t qwen3_tts_device_malloc(int32_t device_index, uint64_t bytes, void** output,
                                              char* error, size_t error_capacity);
QWEN3_TTS_API void qwen3_tts_device_free(void* pointer);
QWEN3_TTS_API int32_t qwen3_tts_device_memcpy(void* destination, const void* source,
                                              uint64_t bytes, char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_device_fill_bf16_normal(
    uint16_t* destination, uint64_t count, uint64_t seed, float mean, float stddev, void* stream,
    char* error, size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_device_synchronize(int32_t device_index, char* error,
                                                   size_t error_capacity);
QWEN3_TTS_API int32_t qwen3_tts_stream_create(int32_t device_index, void** output, char* error,
                                              size_t error_capacity);
QWEN3_TTS_API void qwen3_tts_stream_destroy(void* stream);
QWEN3_TTS_API int32_t qwen3_tts_stream_synchronize(void* stream, char* error,
                                                   size_t error_capacity);
/* Device time of `steps` back-to-back talker-step GEMV chains (per layer:
 * fused QKV with the input RMSNorm prologue, O + residual, gate/up with the
 * post-attention RMSNorm prologue + SiLU-gate, down + residual) on synthetic
 * int8 weights (uniform [-127,127], scales uniform [1e-3,2e-2]) distinct per
 * layer, x ~ N(0,1).  Timed with hipEvents on the library's own stream,
 * optionally as one hipGraph per step.  algorithmic_bytes_per_step counts
 * int8 weights + fp32 scales + bf16 activations read + bf16 outputs written
 * (+ RMSNorm gains). */
typedef struct Qwen3TtsStepBenchmarkV1 {
    uint32_t struct_size;
    int32_t layers;
    int32_t hidden;
    int32_t intermediate;
    int32_t query_width;
    int32_t key_value_width;
    int32_t rows;
    int32_t mode;
    int32_t warmup;
    int32_t steps;
    int32_t use_graph;     /* 0 eager launches, 1 hipGraph per step, 2 the same launches as plain
                              16-byte reads of the weights in one hipGraph (the launch-shape
                              ceiling; no GEMV arithmetic, rows must be 1), 3 the whole step as
                              one persistent launch (rows 1, exact mode, whole chain, hidden
                              2048 / intermediate 6144 / query 2048 / key-value 1024 only) */
    int32_t kernel_filter; /* 0 whole chain; 1 QKV, 2 O, 3 gate/up, 4 down GEMVs only */
    uint64_t weight_bytes;
    uint64_t algorithmic_bytes_per_step;
    double total_milliseconds;
    double milliseconds_per_step;
    double gemv_kernel_milliseconds_per_step;
    uint64_t output_checksum; /* FNV-1a of the final hidden, qkv and activation rows */
} Qwen3TtsStepBenchmarkV1;
QWEN3_TTS_API int32_t qwen3_tts_benchmark_talker_step_gemvs(
    int32_t device_index, Qwen3TtsStepBenchmarkV1* inout, char* error, size_t error_capacity);

#ifdef __cplusplus
}
#endif
#endif
