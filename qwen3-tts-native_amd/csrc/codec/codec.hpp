// Speech-tokenizer decoder (codes -> 24 kHz PCM) for MI355X: shared
// definitions of the kernels (codec_kernels.hip) and the runtime behind the
// C ABI (codec_runtime.hip).
//
// Every tensor is fp32, row-major [positions][channels].  A causal
// convolution reads an "extended" buffer: H history rows (the convolution's
// input from earlier packets) followed by the packet's P rows, so tap t of
// output row p is extended row p + t * dilation.  Transposed convolutions
// (kernel 2 * stride) are the same GEMM over two taps of an extended buffer
// with one history row, with the output columns ordered (phase, channel) so
// that the GEMM's [P][stride * C] output is the [P * stride][C] sequence.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace q3c {

constexpr int kCodebooks = 16;
constexpr int kMaxFrames = 4;
constexpr int kSamplesPerFrame = 1920;
constexpr int kLayers = 8;
constexpr int kHeads = 16;
constexpr int kHeadDim = 64;
constexpr int kHidden = 512;
constexpr int kWindow = 72;
// KV ring slots: a packet of up to 4 frames appends its keys before its first
// frame attends, so the ring holds the 72-position window of the packet's
// first frame plus the 3 newer positions (75) without overwriting.
constexpr int kKvSlots = 80;
constexpr int kStageIn[4] = {1536, 768, 384, 192};
constexpr int kStageOut[4] = {768, 384, 192, 96};
constexpr int kStride[4] = {8, 5, 4, 3};
constexpr int kDilation[3] = {1, 3, 9};

// ---- fp32 MFMA convolution GEMM -------------------------------------------
// out[p][col] = epilogue( sum_k A[p][k] * W[col][k] ),  k = t * C + c,
// A[p][t * C + c] = a[(p + t * dilation) * C + c].
enum GemmEpilogue : int {
    kEpStore = 0,          // v = acc + bias
    kEpGelu = 1,           // v = gelu(acc + bias)          (erf form)
    kEpGammaResidual = 2,  // v = residual + (acc + bias) * gamma
    kEpResidual = 3,       // v = (acc + bias) + residual
};

struct ConvGemmArgs {
    const float* a;
    int channels_in;  // C: floats per extended row
    int taps;
    int dilation;
    const float* w;  // [n][k]
    const float* bias;
    int m, n, k;
    int channels_out;  // parameter index of column col is col % channels_out
    int epilogue;
    const float* residual;  // same [m][n] indexing as out
    const float* gamma;
    float* out;  // [m][n] (may be null)
    // SnakeBeta of v into a second [m][n] destination (may be null):
    // snake = v + sin(v * alpha)^2 / beta_den, alpha = exp(a), beta_den = exp(b) + 1e-9
    float* snake_out;
    const float* snake_alpha;
    const float* snake_beta_den;
    // split-K over `splits` slices: partial sums in `partial`, reduced by a
    // second launch
    int splits;
    float* partial;
};

// block tiles (rows x columns): 16x64 for 1..16 rows (weight streaming),
// 32x32, 32x64 and 64x64 for longer sequences
enum class GemmShape : int { k16x64 = 0, k32x32 = 1, k32x64 = 2, k64x64 = 3 };

struct GemmPlan {
    GemmShape shape;
    int tiles_m, tiles_n, splits;
    int k_step;  // 32 or 64 floats of K per pipeline step
    size_t partial_floats() const;
    size_t tiles() const { return (size_t)tiles_m * tiles_n; }
};
GemmPlan plan_conv_gemm(int m, int n, int k, int channels_in, int cus);
hipError_t launch_conv_gemm(const ConvGemmArgs& args, const GemmPlan& plan, hipStream_t stream);

// ---- rows GEMV (1..4 rows) -------------------------------------------------
enum RowsEpilogue : int {
    kRowsStore = 0,           // v = acc (+ bias)
    kRowsScaledResidual = 1,  // v = residual + acc * scale
    kRowsSiluPair = 2,        // v = silu(acc_gate) * acc_up, W holds [gate n][up n]
};

struct RowsGemvArgs {
    const float* x;  // rows r at x + r * ldx, k floats each (rows may overlap)
    int ldx;
    int rows, k, n;
    const float* w;  // [n][k] ([2n][k] for kRowsSiluPair)
    const float* norm;  // RMSNorm (eps 1e-5) of each input row first, or null
    const float* bias;
    int epilogue;
    const float* residual;  // [rows][n]
    const float* scale;
    float* out;  // [rows][ldo]
    int ldo;
    unsigned long long* advance_position;  // if set: *p += advance_by after the launch's reads
    int advance_by;
};
hipError_t launch_rows_gemv(const RowsGemvArgs& args, hipStream_t stream);

// ---- transformer attention --------------------------------------------------
// RoPE (base 10000, rotate-half pairs d, d + 32) on q and k of `frames` rows of
// qkv [frames][3072] at positions *position + f, appends k and v to the layer's
// ring ([16][kKvSlots][64] each), and writes the 72-window causal attention of
// each frame to out [frames][1024].
hipError_t launch_codec_attention(const float* qkv, int frames, const unsigned long long* position, float* kv_k,
                                  float* kv_v, float* out, hipStream_t stream);

// ---- frontend -----------------------------------------------------------------
// Codebook gather: x[f][0:256] = first codebook entry, x[f][256:512] = sum of
// the 15 acoustic entries (each entry embedding_sum / max(usage, 1e-5)).  The
// same launch copies every history segment in `seg` into its extended buffer.
struct CopySegment {
    const float* src;
    float* dst;
    unsigned floats;
};
hipError_t launch_codec_frontend(const uint16_t* codes, int frames, const float* const* embeddings,
                                 const float* const* usages, float* x, const CopySegment* seg, int segments,
                                 hipStream_t stream);
hipError_t launch_copy_segments(const CopySegment* seg, int segments, hipStream_t stream);

// ---- ConvNeXt depthwise convolution (k = 7) + LayerNorm (eps 1e-6) -----------
hipError_t launch_dwconv_layernorm(const float* ext, int positions, const float* w, const float* b,
                                   const float* ln_w, const float* ln_b, float* out, hipStream_t stream);

// ---- final convolution 96 -> 1 (k = 7), clamp, 16-bit PCM --------------------
hipError_t launch_final_conv_pcm(const float* ext, int positions, const float* w, const float* b, int16_t* pcm,
                                 float* preclamp, float* clamped, hipStream_t stream);

// ---- the reference's weight-free state-machine fixture (22 ints of state) -----
hipError_t launch_fixture_packet(const uint16_t* codes, int frames, int* state, int16_t* pcm, hipStream_t stream);

// ---- load-time helpers ----------------------------------------------------------
hipError_t launch_bf16_to_f32(const uint16_t* src, size_t count, float* dst, hipStream_t stream);
// [o][c][taps] -> [o][taps][c]
hipError_t launch_repack_conv(const float* src, int out_ch, int in_ch, int taps, float* dst, hipStream_t stream);
// transposed conv [in][out][span] -> [(phase, o)][(tap, c)]; overlap: span = 2 * stride,
// tap 0 = kernel index stride + phase (previous input), tap 1 = phase; otherwise
// span = stride and one tap.
hipError_t launch_repack_transpose(const float* src, int in_ch, int out_ch, int stride, bool overlap, float* dst,
                                   hipStream_t stream);
// alpha -> exp(alpha), beta -> exp(beta) + 1e-9 (in place)
hipError_t launch_snake_params(float* alpha, float* beta, int channels, hipStream_t stream);
hipError_t launch_fill_f32(float* dst, size_t count, float value, hipStream_t stream);

}  // namespace q3c
