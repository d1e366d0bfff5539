/*
 * qwen3-tts speech-tokenizer decoder C ABI (versions 1 and 2) -- MI355X
 * (gfx950 / HIP) implementation.
 *
 * Every type, constant and function keeps the name, argument order, struct
 * layout and status-code meaning of the reference decoder's public header
 * native/qwen3-tts-native-codec/native/include/qwen3_tts_codec.h (cited as
 * C:line), so the reference's Rust NativeCodecLibrary
 * (native/qwen3-tts-native-codec/src/ffi.rs) can load this library by symbol
 * name.  The "Cuda" spellings are ABI names; here an event handle carries a
 * hipEvent_t and status -2 reports a HIP error.
 *
 * As in the reference, this header and qwen3_tts_native.h both name
 * QWEN3_TTS_CODEC_CODEBOOKS (a macro there, an enumerator here): a translation
 * unit includes one of them.
 */
#ifndef QWEN3_TTS_CODEC_H
#define QWEN3_TTS_CODEC_H

#include <stddef.h>
#include <stdint.h>

#define QWEN3_TTS_CODEC_API __attribute__((visibility("default")))

#ifdef __cplusplus
extern "C" {
#endif

/* C:16-31 */
enum {
    QWEN3_TTS_CODEC_ABI_VERSION_V1 = 1,
    QWEN3_TTS_CODEC_ABI_VERSION_V2 = 2,
    QWEN3_TTS_CODEC_CODEBOOKS = 16,
    QWEN3_TTS_CODEC_MAX_PACKET_FRAMES = 4,
    QWEN3_TTS_CODEC_SAMPLES_PER_FRAME = 1920,
    QWEN3_TTS_CODEC_MAX_PACKET_SAMPLES = 7680,
    QWEN3_TTS_CODEC_RING_SLOTS = 3,
    QWEN3_TTS_CODEC_MAX_BATCH_STREAMS = 6,
    QWEN3_TTS_CODEC_TRANSFORMER_LAYERS = 8,
    QWEN3_TTS_CODEC_KV_HEADS = 16,
    QWEN3_TTS_CODEC_HEAD_DIM = 64,
    QWEN3_TTS_CODEC_KV_WINDOW = 72,
};

/* C:33-42: waveform-decoder checkpoints of the debug hook */
enum {
    QWEN3_TTS_CODEC_CHECKPOINT_DECODER_PRECONV = 6,
    QWEN3_TTS_CODEC_CHECKPOINT_DECODER_BLOCK_1 = 7,
    QWEN3_TTS_CODEC_CHECKPOINT_DECODER_BLOCK_2 = 8,
    QWEN3_TTS_CODEC_CHECKPOINT_DECODER_BLOCK_3 = 9,
    QWEN3_TTS_CODEC_CHECKPOINT_DECODER_BLOCK_4 = 10,
    QWEN3_TTS_CODEC_CHECKPOINT_FINAL_SNAKE = 11,
    QWEN3_TTS_CODEC_CHECKPOINT_FINAL_PRECLAMP = 12,
    QWEN3_TTS_CODEC_CHECKPOINT_FINAL_CLAMP = 13,
};

/* C:44-51 */
enum {
    QWEN3_TTS_CODEC_STATUS_OK = 0,
    QWEN3_TTS_CODEC_STATUS_INVALID_ARGUMENT = -1,
    QWEN3_TTS_CODEC_STATUS_CUDA = -2, /* device (HIP) runtime error */
    QWEN3_TTS_CODEC_STATUS_STATE = -3,
    QWEN3_TTS_CODEC_STATUS_ALLOCATION = -4,
    QWEN3_TTS_CODEC_STATUS_MODEL = -5,
};

/* C:53-57 */
enum {
    QWEN3_TTS_CODEC_TENSOR_F32 = 1,
    QWEN3_TTS_CODEC_TENSOR_BF16 = 2,
    QWEN3_TTS_CODEC_MAX_TENSOR_RANK = 4,
};

typedef struct Qwen3TtsCodecContextV1 Qwen3TtsCodecContextV1;
typedef struct Qwen3TtsCodecModelV1 Qwen3TtsCodecModelV1;
typedef Qwen3TtsCodecContextV1 Qwen3TtsCodecSessionV1;

/* C:63-68 */
typedef struct Qwen3TtsCodecConfigV1 {
    int32_t device_index;
    int32_t ring_slots;
    int32_t max_packet_frames;
    int32_t reserved;
} Qwen3TtsCodecConfigV1;

/* C:70-83 */
typedef struct Qwen3TtsCodecStateInfoV1 {
    uint64_t frame_position;
    uint64_t emitted_samples;
    uint64_t device_bytes;
    uint64_t host_pinned_bytes;
    uint64_t transformer_kv_bytes;
    uint64_t convolution_history_bytes;
    uint64_t codec_ring_bytes;
    uint64_t pcm_ring_bytes;
    uint32_t kv_ring_head;
    uint32_t next_ring_slot;
    uint32_t ring_slots;
    uint32_t max_packet_frames;
} Qwen3TtsCodecStateInfoV1;

/* C:85-94 */
typedef struct Qwen3TtsCodecPacketResultV1 {
    uint64_t first_frame_position;
    uint64_t first_sample_position;
    uint32_t frame_count;
    uint32_t sample_count;
    uint32_t ring_slot;
    uint32_t is_final;
    float gpu_microseconds;
    float end_to_end_microseconds;
} Qwen3TtsCodecPacketResultV1;

/* C:96-104 */
typedef struct Qwen3TtsCodecBatchItemV1 {
    Qwen3TtsCodecContextV1* context;
    const uint16_t* codec_frames;
    uint32_t frame_count;
    int32_t is_final;
    int16_t* pcm_output;
    size_t pcm_capacity_samples;
    Qwen3TtsCodecPacketResultV1* result;
} Qwen3TtsCodecBatchItemV1;

/* C:106-113 */
typedef struct Qwen3TtsCodecTensorViewV1 {
    const void* data;
    uint64_t byte_length;
    uint64_t shape[QWEN3_TTS_CODEC_MAX_TENSOR_RANK];
    uint32_t rank;
    uint32_t dtype;
} Qwen3TtsCodecTensorViewV1;

/* C:115-122 */
typedef int32_t (*Qwen3TtsCodecTensorAtV1)(void* user_data, uint64_t index, const char** name,
                                           Qwen3TtsCodecTensorViewV1* tensor, char* error,
                                           size_t error_capacity);

/* C:124-130 */
typedef struct Qwen3TtsCodecWeightProviderV1 {
    uint32_t abi_version;
    uint32_t reserved;
    uint64_t tensor_count;
    void* user_data;
    Qwen3TtsCodecTensorAtV1 tensor_at;
} Qwen3TtsCodecWeightProviderV1;

/* C:132-140 */
typedef struct Qwen3TtsCodecModelInfoV1 {
    uint64_t source_bytes;
    uint64_t device_bytes;
    uint64_t parameter_count;
    uint32_t tensor_count;
    uint32_t source_dtype_f32_count;
    uint32_t source_dtype_bf16_count;
    uint32_t loaded;
} Qwen3TtsCodecModelInfoV1;

/* C:144-153 */
typedef struct Qwen3TtsCodecModelMemoryInfoV1 {
    uint64_t source_bytes;
    uint64_t shared_weight_device_bytes;
    uint64_t parameter_count;
    uint64_t transient_upload_device_bytes;
    uint32_t tensor_count;
    uint32_t warmup_completed;
    uint32_t active_session_count;
    uint32_t reserved;
} Qwen3TtsCodecModelMemoryInfoV1;

/* C:156-165 */
typedef struct Qwen3TtsCodecSessionMemoryInfoV1 {
    uint64_t device_bytes;
    uint64_t host_pinned_bytes;
    uint64_t transformer_kv_bytes;
    uint64_t convolution_history_bytes;
    uint64_t codec_ring_bytes;
    uint64_t pcm_ring_bytes;
    uint64_t workspace_device_bytes;
    uint64_t reserved;
} Qwen3TtsCodecSessionMemoryInfoV1;

/* C:167-175 */
typedef struct Qwen3TtsCodecSessionBatchItemV1 {
    Qwen3TtsCodecSessionV1* session;
    const uint16_t* codec_frames;
    uint32_t frame_count;
    int32_t is_final;
    int16_t* pcm_output;
    size_t pcm_capacity_samples;
    Qwen3TtsCodecPacketResultV1* result;
} Qwen3TtsCodecSessionBatchItemV1;

/* C:177-206: device-code handoff (ABI v2); the event handle is a hipEvent_t */
typedef void* Qwen3TtsCodecCudaEventV2;

typedef struct Qwen3TtsCodecDevicePacketBeginV2 {
    uint32_t struct_size;
    uint32_t reserved;
    const uint16_t* device_codec_frames;
    uint32_t frame_count;
    uint32_t reserved_2;
    Qwen3TtsCodecCudaEventV2 producer_ready_event;
    uint64_t reserved_3;
} Qwen3TtsCodecDevicePacketBeginV2;

typedef struct Qwen3TtsCodecDevicePacketBeginResultV2 {
    uint32_t struct_size;
    uint32_t reserved;
    uint64_t ticket_id;
    Qwen3TtsCodecCudaEventV2 codes_consumed_event;
    uint64_t reserved_2;
} Qwen3TtsCodecDevicePacketBeginResultV2;

typedef struct Qwen3TtsCodecDevicePacketFinishV2 {
    uint32_t struct_size;
    uint32_t reserved;
    uint64_t ticket_id;
    int32_t is_final;
    uint32_t reserved_2;
    int16_t* pcm_output;
    size_t pcm_capacity_samples;
    Qwen3TtsCodecPacketResultV1* result;
    uint64_t reserved_3;
} Qwen3TtsCodecDevicePacketFinishV2;

/* C:208-210 */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_abi_version_v1(void);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_abi_version_v2(void);

/* Legacy single-context API (C:212-262): a context owns a private model. */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_create_v1(const Qwen3TtsCodecConfigV1* config,
                                                      Qwen3TtsCodecContextV1** output, char* error,
                                                      size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_destroy_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                       size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_reset_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                     size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_state_info_v1(const Qwen3TtsCodecContextV1* context,
                                                          Qwen3TtsCodecStateInfoV1* output, char* error,
                                                          size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_load_model_v1(Qwen3TtsCodecContextV1* context,
                                                          const Qwen3TtsCodecWeightProviderV1* provider,
                                                          Qwen3TtsCodecModelInfoV1* output, char* error,
                                                          size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_model_info_v1(const Qwen3TtsCodecContextV1* context,
                                                          Qwen3TtsCodecModelInfoV1* output, char* error,
                                                          size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_warmup_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                      size_t error_capacity);

/* Debug hooks (C:263-314).  Layouts: RVQ [512][frames] channel-major,
 * pre-convolution [frames][1024]; transformer [frames][1024]; latent stages
 * channel-major [1024][frames*2] and [1024][frames*4]; decoder checkpoints
 * channel-major [channels][positions].  Each runs the packet through the
 * context's state (it advances it like a real packet). */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_frontend_packet_v1(
    Qwen3TtsCodecContextV1* context, const uint16_t* codec_frames, uint32_t frame_count, float* rvq_output,
    size_t rvq_capacity, float* preconv_output, size_t preconv_capacity, char* error, size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_transformer_packet_v1(
    Qwen3TtsCodecContextV1* context, const uint16_t* codec_frames, uint32_t frame_count, float* transformer_output,
    size_t transformer_capacity, char* error, size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_latent_packet_v1(
    Qwen3TtsCodecContextV1* context, const uint16_t* codec_frames, uint32_t frame_count, float* stage_one_output,
    size_t stage_one_capacity, float* stage_two_output, size_t stage_two_capacity, char* error,
    size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_decoder_checkpoint_v1(
    Qwen3TtsCodecContextV1* context, const uint16_t* codec_frames, uint32_t frame_count, uint32_t checkpoint,
    float* checkpoint_output, size_t checkpoint_capacity, char* error, size_t error_capacity);

/* C:316-336 */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_packet_v1(Qwen3TtsCodecContextV1* context,
                                                              const uint16_t* codec_frames, uint32_t frame_count,
                                                              int32_t is_final, int16_t* pcm_output,
                                                              size_t pcm_capacity_samples,
                                                              Qwen3TtsCodecPacketResultV1* result, char* error,
                                                              size_t error_capacity);
/* Items are validated and queued in array order; the first failure ends the
 * batch and is returned, and the items before it still complete.  Every
 * item's result is cleared on entry, so after an error the items whose packet
 * completed (and advanced their stream) are exactly those with a nonzero
 * result->frame_count. */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_batch_v1(Qwen3TtsCodecBatchItemV1* items, uint32_t item_count,
                                                             char* error, size_t error_capacity);

/* C:337-351: the deterministic state-machine fixture.  It executes no neural
 * weights (integer stand-ins for each stage, carried across packets) and is no
 * model-quality or latency measurement; the reference's Rust loader requires
 * the symbol. */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_fixture_packet_v1(Qwen3TtsCodecContextV1* context,
                                                                      const uint16_t* codec_frames,
                                                                      uint32_t frame_count, int32_t is_final,
                                                                      int16_t* pcm_output,
                                                                      size_t pcm_capacity_samples,
                                                                      Qwen3TtsCodecPacketResultV1* result,
                                                                      char* error, size_t error_capacity);

/* Shared-model API (C:353-392). */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_create_v1(int32_t device_index,
                                                                   Qwen3TtsCodecModelV1** output, char* error,
                                                                   size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_destroy_v1(Qwen3TtsCodecModelV1* model, char* error,
                                                                    size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_load_v1(Qwen3TtsCodecModelV1* model,
                                                                 const Qwen3TtsCodecWeightProviderV1* provider,
                                                                 Qwen3TtsCodecModelInfoV1* output, char* error,
                                                                 size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_warmup_v1(Qwen3TtsCodecModelV1* model, char* error,
                                                                   size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_info_v1(const Qwen3TtsCodecModelV1* model,
                                                                 Qwen3TtsCodecModelInfoV1* output, char* error,
                                                                 size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_memory_info_v1(const Qwen3TtsCodecModelV1* model,
                                                                        Qwen3TtsCodecModelMemoryInfoV1* output,
                                                                        char* error, size_t error_capacity);

/* Sessions (C:394-431, 433-487). */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_create_v1(Qwen3TtsCodecModelV1* model,
                                                              Qwen3TtsCodecSessionV1** output, char* error,
                                                              size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_destroy_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                               size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_reset_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                             size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_cancel_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                              size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_state_info_v1(const Qwen3TtsCodecSessionV1* session,
                                                                  Qwen3TtsCodecStateInfoV1* output, char* error,
                                                                  size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_memory_info_v1(const Qwen3TtsCodecSessionV1* session,
                                                                   Qwen3TtsCodecSessionMemoryInfoV1* output,
                                                                   char* error, size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_packet_v1(
    Qwen3TtsCodecSessionV1* session, const uint16_t* codec_frames, uint32_t frame_count, int32_t is_final,
    int16_t* pcm_output, size_t pcm_capacity_samples, Qwen3TtsCodecPacketResultV1* result, char* error,
    size_t error_capacity);
/* C:433-470: device codes in, producer_ready_event waited on the session's
 * stream, codes snapshotted into the session's ring, codes_consumed_event
 * recorded, the decoder and the pinned PCM copy queued; finish completes the
 * ticket and copies the PCM out. */
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_device_packet_begin_v2(
    Qwen3TtsCodecSessionV1* session, const Qwen3TtsCodecDevicePacketBeginV2* request,
    Qwen3TtsCodecDevicePacketBeginResultV2* output, char* error, size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_device_packet_finish_v2(
    Qwen3TtsCodecSessionV1* session, const Qwen3TtsCodecDevicePacketFinishV2* request, char* error,
    size_t error_capacity);
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_batch_v1(Qwen3TtsCodecSessionBatchItemV1* items,
                                                                     uint32_t item_count, char* error,
                                                                     size_t error_capacity);

#ifdef __cplusplus
}
#endif
#endif
