/*
 * CPU oracle of the qwen3-tts speech-tokenizer decoder (the codec that turns
 * 16-codebook frames into 24 kHz PCM).
 *
 * TEST INFRASTRUCTURE ONLY: used by tests/ and bench.py's CPU leg as the
 * checker, never by the shipped library.  It restates, in plain C and fp32,
 * the reference decoder native/qwen3-tts-native-codec/native/src/
 * codec_state.cu (cited as CS:line per function in codec_oracle.c).  Where the
 * reference runs its own kernels the operation order is theirs; where it
 * calls cuBLAS (linear layers, im2col convolutions) the order is this
 * oracle's: one fp32 fmaf chain in k order, bias added afterwards.
 */
#ifndef QWEN3_TTS_CODEC_ORACLE_H
#define QWEN3_TTS_CODEC_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Decoder tensors in a fixed order (see orc_codec_tensor_name). */
enum { ORC_CODEC_TENSORS = 269 };
const char* orc_codec_tensor_name(int index);
/* float elements of tensor `index` */
uint64_t orc_codec_tensor_elements(int index);

typedef struct OrcCodecState OrcCodecState;
OrcCodecState* orc_codec_state_create(void);
void orc_codec_state_destroy(OrcCodecState* state);
void orc_codec_state_reset(OrcCodecState* state);

/* Optional stage outputs of one packet (NULL: not wanted), row-major
 * [positions][channels]: rvq [F][512], preconv [F][1024], transformer
 * [F][1024], latent1 [2F][1024], latent2 [4F][1024], and decoder
 * checkpoint c in checkpoints[c] for c = 6..13 (CS:2066-2274).
 *
 * stop_after mirrors the reference's debug hooks, which run a prefix of the
 * pipeline and advance only that prefix's state: 1 after the frontend
 * (CS:3506-3756), 2 after the transformer (CS:3759-3821), 3 after the latent
 * upsampler (CS:3824-3904), 6..13 at that decoder checkpoint (CS:2029-2274,
 * 3907-3957); 0 runs the whole packet.  A stopped packet writes no PCM. */
typedef struct OrcCodecTrace {
    float *rvq, *preconv, *transformer, *latent1, *latent2;
    float* checkpoints[14];
    int stop_after;
} OrcCodecTrace;

/* Decodes one packet of `frames` (1..4) frame-major [frames][16] codes into
 * frames * 1920 samples of PCM, advancing the state; returns the sample count
 * (0 for a stopped packet, -1 for a bad frame count).  `weights` holds
 * ORC_CODEC_TENSORS float pointers in orc_codec_tensor_name order.  GEMM
 * accumulation order as orc_set_gemm_order (0: fp32 chain, 1: double). */
int orc_codec_packet(const float* const* weights, OrcCodecState* state, const uint16_t* codes, int frames,
                     int16_t* pcm, OrcCodecTrace* trace);

#ifdef __cplusplus
}
#endif
#endif
