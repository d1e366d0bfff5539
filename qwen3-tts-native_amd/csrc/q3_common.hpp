// Shared definitions of the MI355X (gfx950) int8 decode-path library.
//
// bf16 values are carried as raw uint16_t bit patterns everywhere (device and
// host) so that no vendor bf16 type with its own rounding rules sits on the
// hot path.  All conversions round to nearest even, like the reference's
// __float2bfloat16.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>

namespace q3 {

// Raises a kernel's dynamic LDS limit once per device (the attribute is held
// per device): `done` is the call site's bit set of devices already set up.
inline hipError_t set_dynamic_lds_once(std::atomic<unsigned long long>& done, const void* kernel, int bytes) {
    int device = 0;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) return st;
    const unsigned long long bit = 1ull << (device & 63);
    if (done.load(std::memory_order_acquire) & bit) return hipSuccess;
    st = hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    if (st == hipSuccess) done.fetch_or(bit, std::memory_order_acq_rel);
    return st;
}

using bf16_t = uint16_t;

// ---------------------------------------------------------------------------
// bf16 conversions
// ---------------------------------------------------------------------------
__host__ __device__ inline float bf2f(bf16_t v) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __uint_as_float(static_cast<uint32_t>(v) << 16);
#else
    uint32_t u = static_cast<uint32_t>(v) << 16;
    float f;
    __builtin_memcpy(&f, &u, 4);
    return f;
#endif
}

__host__ __device__ inline bf16_t f2bf(float f) {
#if defined(__HIP_DEVICE_COMPILE__)
    uint32_t u = __float_as_uint(f);
#else
    uint32_t u;
    __builtin_memcpy(&u, &f, 4);
#endif
    if ((u & 0x7fffffffu) > 0x7f800000u) {
        return 0x7fff;
    }
    u += 0x7fffu + ((u >> 16) & 1u);
    return static_cast<bf16_t>(u >> 16);
}

__host__ __device__ inline float round_bf(float f) { return bf2f(f2bf(f)); }

// ---------------------------------------------------------------------------
// Shuffle-down sum tree over groups of kWidth lanes (64 or 32) without the LDS
// crossbar.  Lane 0 of each group ends with exactly what
//   for (d = kWidth / 2; d > 0; d /= 2) v += __shfl_down(v, d, kWidth);
// leaves there: the same additions in the same order (lane i < d adds lane
// i + d at level d).  Other lanes hold partial values and must not be used.
// Level 32 uses v_permlane32_swap, level 16 v_permlane16_swap (gfx950), levels
// 8..1 a DPP row shift; each is a VALU operation instead of a ds_bpermute
// round trip.
// ---------------------------------------------------------------------------
#if defined(__HIP_DEVICE_COMPILE__)
template <int kShift>
__device__ __forceinline__ float row_from_higher(float v) {
    // row_shl:kShift -- lane i reads lane i + kShift of its 16-lane row (0 past the row's end)
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x100 + kShift, 0xf, 0xf, true));
}
#endif

template <int kWidth>
__device__ __forceinline__ float wave_sum_down(float v) {
    static_assert(kWidth == 64 || kWidth == 32, "wave_sum_down width");
#if defined(__HIP_DEVICE_COMPILE__)
    const unsigned bits = __float_as_uint(v);
    if constexpr (kWidth == 64) {
        // second result: lanes 0-31 hold the old lanes 32-63
        v += __uint_as_float(__builtin_amdgcn_permlane32_swap(bits, bits, false, false)[1]);
    }
    {
        // second result: rows 0 and 2 hold the old rows 1 and 3
        const unsigned b = __float_as_uint(v);
        v += __uint_as_float(__builtin_amdgcn_permlane16_swap(b, b, false, false)[1]);
    }
    v += row_from_higher<8>(v);
    v += row_from_higher<4>(v);
    v += row_from_higher<2>(v);
    v += row_from_higher<1>(v);
#endif
    return v;
}

// Maximum over the wave (order independent), valid in lane 0; the same
// cross-lane steps as wave_sum_down.
__device__ __forceinline__ float wave_max_down(float v) {
#if defined(__HIP_DEVICE_COMPILE__)
    const unsigned bits = __float_as_uint(v);
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_permlane32_swap(bits, bits, false, false)[1]));
    const unsigned b = __float_as_uint(v);
    v = fmaxf(v, __uint_as_float(__builtin_amdgcn_permlane16_swap(b, b, false, false)[1]));
    v = fmaxf(v, row_from_higher<8>(v));
    v = fmaxf(v, row_from_higher<4>(v));
    v = fmaxf(v, row_from_higher<2>(v));
    v = fmaxf(v, row_from_higher<1>(v));
#endif
    return v;
}

// ---------------------------------------------------------------------------
// Errors: internal code throws; the C ABI maps exceptions to status codes.
// ---------------------------------------------------------------------------
class DeviceFailure final : public std::runtime_error {
public:
    using std::runtime_error::runtime_error;
};

inline void check_hip(hipError_t status, const char* operation) {
    if (status != hipSuccess) {
        throw DeviceFailure(std::string(operation) + " failed: " + hipGetErrorString(status));
    }
}

// ---------------------------------------------------------------------------
// Kernel launch layer.  Names, argument meaning and the hipErrorInvalidValue
// rule mirror the reference's internal launch API
// (native/qwen3-tts-native/native/src/talker_internal.cuh:11-356).
// ---------------------------------------------------------------------------

// Epilogue applied by the int8 GEMV family to y = scale[c] * dot(W[c], x).
enum GemvEpilogue : int {
    kEpiStore = 0,        // out16 = bf16(y); out32 = y                (int8_gemv.cu:123)
    kEpiAddFma = 1,       // out16 = bf16(fma(dot, scale, out16))      (int8_gemv.cu:192-196)
    kEpiAddRounded = 2,   // out16 = bf16(out16 + bf16(y))   GEMV + add_in_place (talker.cu:3391-3405)
    kEpiSiluFused = 3,    // out16 = bf16(silu(yg) * yu)               (int8_gemv.cu:283-289)
    kEpiSiluRounded = 4,  // gate/up bf16, silu_gate kernel            (talker.cu:3416-3442)
    kEpiBias = 5,         // out16 = bf16(bf16(y) + bias)   GEMV + bias_activation (talker.cu:3498-3515)
    kEpiBiasSilu = 6,     // v = bf16(y) + bias; out16 = bf16(v * (1/(1+exp(-v))))  (talker.cu:2683-2696)
    kEpiBiasAdd = 7,      // out16 = bf16(out16 + bf16(bf16(y) + bias))  fc2 + bias + add (talker.cu:2697-2719,3572-3580)
};

// Weight-streaming implementation used for a GEMV launch.
enum GemvMode : int {
    kModeAuto = 0,   // exact order for rows == 1, MFMA for rows >= 2
    kModeExact = 1,  // reference lane order on VALU (bit-exact to the reference)
    kModeMfma = 2,   // int8 -> bf16 dequant in registers + v_mfma_f32_16x16x32_bf16
};

struct GemvArgs {
    const int8_t* weight = nullptr;   // [out_rows][in] row-major (gate/up: [2*out][in])
    const float* scales = nullptr;    // [out_rows]
    const bf16_t* input = nullptr;    // [rows][in]
    const bf16_t* norm_weight = nullptr;  // optional fused RMSNorm gain [in]
    const bf16_t* bias = nullptr;         // [out] for the bias epilogues
    const int* input_row_index = nullptr; // optional: input += (*index) * in (rows == 1)
    float norm_epsilon = 1.0e-6f;
    bf16_t* out16 = nullptr;          // [rows][out] (nullable for kEpiStore)
    float* out32 = nullptr;           // [rows][out] (kEpiStore only, nullable)
    int in_features = 0;
    int out_features = 0;             // channels written (gate/up: intermediate)
    int rows = 1;
    int epilogue = kEpiStore;
    int mode = kModeAuto;
};

hipError_t launch_int8_gemv(const GemvArgs& args, hipStream_t stream);

// Persistent batch-1 talker-step GEMV chain (step_chain.hip): every layer's
// QKV (+RMSNorm), O (+residual), gate/up (+RMSNorm, SiLU) and down
// (+residual) GEMV in one launch, bit-identical to the per-GEMV exact
// kernels.  Fixed geometry: hidden 2048, intermediate 6144, 4096 fused QKV
// rows, O input 2048; one launch must finish before the next starts on the
// same workspace (words / epoch / status).
struct StepChainArgs {
    const int8_t* weights = nullptr;   // per layer: qkv, o, gate/up, down (row-major int8)
    const float* scales = nullptr;     // per layer: 4096 + 2048 + 12288 + 2048
    size_t weight_layer_stride = 0;    // bytes between layers
    size_t scale_layer_stride = 0;     // floats between layers
    const bf16_t* gain_qkv = nullptr;  // [2048] RMSNorm gain before QKV
    const bf16_t* gain_gu = nullptr;   // [2048] before gate/up
    size_t gain_layer_stride = 0;      // elements between layers (0: shared)
    bf16_t* hidden = nullptr;          // [2048] in / out
    bf16_t* qkv = nullptr;             // [4096] out (last layer)
    bf16_t* act = nullptr;             // [6144] out (last layer)
    unsigned long long* words = nullptr;  // talker_step_chain_words() zeroed words
    unsigned* epoch = nullptr;         // one word, initialized to 1
    int* status = nullptr;             // one word, 0; set to 1 if a wait timed out
    int hidden_size = 0, intermediate = 0, qkv_rows = 0, query_width = 0, layers = 0;
    float epsilon = 1.0e-6f;
};
size_t talker_step_chain_words();
hipError_t launch_talker_step_chain(const StepChainArgs& args, hipStream_t stream);
// True when every workgroup of the chain can be resident at once on `device`.
hipError_t talker_step_chain_supported(int device, bool* supported);
// One code-predictor pass in one persistent launch (pred_chain.hip):
// small_to_mtp + bias, 5 decoder layers with the exact 16-position
// attention, and (head_w non-null) the final RMSNorm + codebook head.
struct PredLayerArgs {
    const int8_t *qkv_w = nullptr, *o_w = nullptr, *gu_w = nullptr, *d_w = nullptr;
    const float *qkv_s = nullptr, *o_s = nullptr, *gu_s = nullptr, *d_s = nullptr;
    const bf16_t *input_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
    bf16_t* key_cache = nullptr;    // [16][kv heads * 128]
    bf16_t* value_cache = nullptr;  // blocked dimension-major, stride 16
};
struct PredictorPassArgs {
    const int8_t* s2m_w = nullptr;
    const float* s2m_s = nullptr;
    const bf16_t* s2m_bias = nullptr;
    const bf16_t* input = nullptr;  // [rows][input_width]
    const int* input_row = nullptr;  // device row index (nullable: row 0)
    PredLayerArgs layer[5];
    const int8_t* head_w = nullptr;  // null: no head
    const float* head_s = nullptr;
    const bf16_t* final_norm = nullptr;
    bf16_t* logits = nullptr;
    const bf16_t* rope_table = nullptr;
    const int* position = nullptr;  // device
    unsigned long long* words = nullptr;  // predictor_pass_words() zeroed words
    unsigned* epoch = nullptr;            // one word, initialized to 1
    int* status = nullptr;                // one word, 0; set to 1 if a wait timed out
    int hidden = 0, intermediate = 0, query_heads = 0, key_value_heads = 0, input_width = 0, vocabulary = 0;
    int layers = 0, capacity = 0;
    float epsilon = 1.0e-6f;
};
size_t predictor_pass_words();
hipError_t launch_predictor_pass(const PredictorPassArgs& args, hipStream_t stream);
hipError_t predictor_pass_supported(int device, bool* supported);
// Orders the persistent predictor launches of every session on a device
// (two of them side by side could each hold part of the CUs and wait for
// workgroups that cannot start): constructed before a stream's predictor
// launches, it makes the stream wait for the device's previous ones when
// they were another stream's; done() after them records their end.  Holds
// the device's lock from construction to destruction.
class PredictorPassOrder {
public:
    PredictorPassOrder(int device, hipStream_t stream);
    ~PredictorPassOrder();
    PredictorPassOrder(const PredictorPassOrder&) = delete;
    PredictorPassOrder& operator=(const PredictorPassOrder&) = delete;
    hipError_t status() const { return status_; }
    hipError_t done();
private:
    struct PassOrderSlot* slot_ = nullptr;
    hipStream_t stream_ = nullptr;
    hipError_t status_ = hipSuccess;
};
// Exact-order rows of a prompt (any count, no RMSNorm) in one launch.
hipError_t launch_int8_gemv_prompt_rows(const GemvArgs& a, hipStream_t stream);

hipError_t launch_quantize_weight_rows(const bf16_t* weight, int8_t* quantized, float* scales,
                                       int in_features, int out_features, hipStream_t stream);
hipError_t launch_int8_gemm_rows(const int8_t* weight, const float* scales, const bf16_t* input,
                                 bf16_t* output, int in_features, int out_features, int rows,
                                 hipStream_t stream);
hipError_t launch_int8_gemm_rows_add(const int8_t* weight, const float* scales,
                                     const bf16_t* input, bf16_t* output, int in_features,
                                     int out_features, int rows, hipStream_t stream);
hipError_t launch_int8_gate_up_silu_rows(const int8_t* weight, const float* scales,
                                         const bf16_t* input, bf16_t* output, int in_features,
                                         int out_features, int rows, hipStream_t stream);

// Transformer primitives (talker_kernels.cu equivalents).
hipError_t launch_rms_norm_rows(const bf16_t* input, const bf16_t* weight, bf16_t* output,
                                int rows, int width, float epsilon, hipStream_t stream);
hipError_t launch_head_rms_norm_rows(bf16_t* values, const bf16_t* weight, int rows, int heads,
                                     int head_dimension, float epsilon, hipStream_t stream);
hipError_t launch_rope_rows(bf16_t* values, int rows, int heads, int head_dimension,
                            int first_position, float theta, hipStream_t stream);
hipError_t launch_rope_rows_at(bf16_t* values, int rows, int heads, int head_dimension,
                               const int* positions, float theta, hipStream_t stream);
// Fused per-head epilogue of the QKV projection: head RMSNorm on q and k,
// RoPE at `position`, and the KV-cache append of k and v.  qkv is
// [rows][q_width + 2*kv_width]; q is rewritten in place; k/v rows go to
// key_bases[r] / value_bases[r] + positions[r] * kv_width.
hipError_t launch_qk_norm_rope_kv_append(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm,
                                         bf16_t* const* key_bases, bf16_t* const* value_bases,
                                         const int* positions, const bf16_t* rope_table, int rows,
                                         int query_heads, int key_value_heads, int head_dimension,
                                         float epsilon, hipStream_t stream);
// Decode attention.  exact: causal_gqa_attention semantics (talker_kernels.cu:287-357);
// otherwise batch_causal_gqa_attention_fast semantics (:506-595).  Keys/values come
// from key_bases[row] (or key_cache when key_bases is null); the length is
// positions[row] + 1 (or fixed_sequence_length when positions is null).
// Decode attention (head dimension 128).  workspace: attention_workspace_bytes
// of device memory owned by the caller's stream.
size_t attention_workspace_bytes(int rows, int query_heads, int capacity);
// Value caches of launch_attention / launch_decode_attention are blocked
// dimension-major: element (position p, kv head h, dimension d) at
// [((h * stride / 8 + p / 8) * 128 + d) * 8 + p % 8].  The stride of a cache of `capacity`
// positions is value_cache_stride(capacity) unless value_strides (device,
// one per row) gives it per row (each a multiple of 8, at least the row's
// own capacity).  Key caches stay [position][kv_width].
int value_cache_stride(int capacity);
hipError_t launch_attention(bool exact, const bf16_t* query, int query_stride,
                            bf16_t* const* key_bases, bf16_t* const* value_bases,
                            const bf16_t* key_cache, const bf16_t* value_cache,
                            const int* positions, int fixed_sequence_length, bf16_t* output,
                            int rows, int query_heads, int key_value_heads, int head_dimension,
                            int max_sequence_length, float* workspace, const int* value_strides,
                            hipStream_t stream);
// Decode attention with the QKV epilogue fused in: qkv holds the raw fused
// q|k|v rows; query heads are normalized and rotated, the key of position
// positions[row] is normalized, rotated and appended with its value, then
// attention runs over positions 0..positions[row].
hipError_t launch_decode_attention(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                   const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                   bf16_t* const* key_bases, bf16_t* const* value_bases, const bf16_t* key_cache,
                                   const bf16_t* value_cache, const int* positions, bf16_t* output, int rows,
                                   int query_heads, int key_value_heads, int head_dimension, int capacity,
                                   float* workspace, const int* value_strides, hipStream_t stream,
                                   int position_splits = 1);
// Workspace of launch_decode_attention with position_splits > 1 (the
// batched, non-exact semantics only: the value chains of each row and head
// run as `splits` segments whose sums are added afterwards -- tolerance, not
// the reference's single chain).
size_t attention_split_workspace_bytes(int rows, int query_heads, int capacity, int splits);
hipError_t launch_decode_attention_op(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                      const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                      bf16_t* const* key_bases, bf16_t* const* value_bases, const int* positions,
                                      bf16_t* output, int rows, int query_heads, int key_value_heads,
                                      int head_dimension, int max_sequence_length, hipStream_t stream);
// The same on the library's per-device static scratch (no allocation); fails
// with hipErrorInvalidValue when decode_attention_scratch_bytes exceeds
// decode_attention_scratch_limit().
hipError_t launch_decode_attention_op_noalloc(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                              const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                              bf16_t* const* key_bases, bf16_t* const* value_bases,
                                              const int* positions, bf16_t* output, int rows, int query_heads,
                                              int key_value_heads, int head_dimension, int max_sequence_length,
                                              hipStream_t stream);
size_t decode_attention_scratch_bytes(int rows, int query_heads, int key_value_heads, int head_dimension,
                                      int max_sequence_length);
size_t decode_attention_scratch_limit();
hipError_t launch_attention_op(bool exact, const bf16_t* query, int query_stride, bf16_t* const* key_bases,
                               bf16_t* const* value_bases, const int* positions, bf16_t* output, int rows,
                               int query_heads, int key_value_heads, int head_dimension, int max_sequence_length,
                               hipStream_t stream);
// Prompt rows against one shared key/value cache ([capacity][kv_width] each,
// complete): row r attends to positions 0..positions[r].
hipError_t launch_prompt_attention_op(bool exact, const bf16_t* query, int query_stride, const bf16_t* key_cache,
                                      const bf16_t* value_cache, const int* positions, bf16_t* output, int rows,
                                      int query_heads, int key_value_heads, int head_dimension, int capacity,
                                      hipStream_t stream);
hipError_t launch_causal_gqa_attention(const bf16_t* query, const bf16_t* key_cache,
                                       const bf16_t* value_cache, bf16_t* output, int query_heads,
                                       int key_value_heads, int head_dimension,
                                       int sequence_length, int query_stride, hipStream_t stream);
hipError_t launch_batch_causal_gqa_attention_fast(const bf16_t* query,
                                                  bf16_t* const* key_bases,
                                                  bf16_t* const* value_bases,
                                                  const int* positions, bf16_t* output, int rows,
                                                  int query_heads, int key_value_heads,
                                                  int head_dimension, int max_sequence_length,
                                                  int query_stride, hipStream_t stream);
hipError_t launch_kv_scatter_rows(const bf16_t* rows_data, bf16_t* const* cache_bases,
                                  const int* positions, int rows, int width, int row_stride,
                                  hipStream_t stream);
hipError_t launch_add_in_place(bf16_t* destination, const bf16_t* source, int width,
                               hipStream_t stream);
hipError_t launch_bias_activation_rows(bf16_t* values, const bf16_t* bias, int rows, int width,
                                       bool silu, hipStream_t stream);
hipError_t launch_silu_gate(bf16_t* gate, const bf16_t* up, int width, hipStream_t stream);
hipError_t launch_fill_zero(bf16_t* values, int width, hipStream_t stream);
hipError_t launch_increment(int* counter, hipStream_t stream);
hipError_t launch_fill_bf16_normal(bf16_t* destination, uint64_t count, uint64_t seed, float mean,
                                   float stddev, hipStream_t stream);

// Sampling / frame glue (sampling_kernels.cu equivalents).
// Arguments of one sampler invocation (sampling.hip documents the fields'
// semantics; every pointer is a device pointer).
struct SampleArgs {
    const bf16_t* logits;
    int vocabulary;
    bool suppress;
    int eos;
    const int* history;
    const int* history_count;
    int history_count_fallback;
    int do_sample;
    int top_k;
    float top_p;
    float temperature;
    float penalty;
    uint64_t* random_state;
    int* selected;
    int* store_tokens;
    const int* store_index;
    int store_index_fallback;
    int* append_history;   // history array to append to (talker), nullable
    int* append_count;     // device history counter to increment, nullable
};
// Host check of one row's arguments (the launchers' validation).
bool sample_args_valid(const SampleArgs& a);
// One sampler block per row, rows in [1, 64], arguments read from device
// memory (a table the caller uploads; each row validated with
// sample_args_valid on the host).
hipError_t launch_sample_rows(const SampleArgs* device_rows, int rows, hipStream_t stream);
hipError_t launch_sample_logits(const bf16_t* logits, int vocabulary,
                                bool suppress_talker_reserved, int codec_eos_token,
                                const int* semantic_history, const int* semantic_history_count,
                                int semantic_history_count_fallback, int do_sample, int top_k,
                                float top_p, float temperature, float repetition_penalty,
                                uint64_t* random_state, int* selected_token,
                                int* store_tokens, const int* store_index,
                                int store_index_fallback, hipStream_t stream);
hipError_t launch_sample_logits_ex(const bf16_t* logits, int vocabulary, bool suppress, int eos,
                                   const int* history, const int* history_count,
                                   int history_count_fallback, int do_sample, int top_k,
                                   float top_p, float temperature, float penalty,
                                   uint64_t* random_state, int* selected, int* store_tokens,
                                   const int* store_index, int store_index_fallback,
                                   int* append_history, int* append_count, hipStream_t stream);
hipError_t launch_argmax_bf16(const bf16_t* logits, int vocabulary, int* selected_token,
                              hipStream_t stream);
hipError_t launch_store_token(int* tokens, int index, int value, hipStream_t stream);
hipError_t launch_pack_frame_codes(const int* tokens, uint16_t* codes, int count,
                                   hipStream_t stream);
// Batch form: row r packs tokens[r][0..count) into codes[r].
hipError_t launch_pack_frame_codes_rows(const int* const* tokens, uint16_t* const* codes, int count, int rows,
                                        hipStream_t stream);
hipError_t launch_gather_embedding(const bf16_t* table, int vocabulary, int width,
                                   const int* token, bf16_t* output, bool add,
                                   hipStream_t stream);
// output = bf16( table0[tok[0]] + table1[tok[1]] + ... ) summed in order with
// bf16 rounding after every addition (the reference's chained add_embedding).
hipError_t launch_sum_embeddings(const bf16_t* const* tables, int count, int vocabulary0,
                                 int vocabulary, int width, const int* tokens, bf16_t* output,
                                 hipStream_t stream);

// ---------------------------------------------------------------------------
// bf16 prefill (prefill.hip)
// ---------------------------------------------------------------------------
// C[m][n] = bf16(sum_k A[m][k] * B[n][k]) with fp32 accumulation; A, B, C
// row-major with leading dimensions lda, ldb, ldc (elements).  Batch z uses
// A + z * a_batch, B + (z / b_group) * b_batch, C + z * c_batch.  K, lda,
// ldb, a_batch and b_batch must be multiples of 8 and A, B 16-byte aligned.
// Epilogues of the bf16 GEMM: C = bf16(sum); C = bf16(C + bf16(sum)) (the
// residual add_in_place); C = bf16(bf16(silu(C)) * bf16(sum)) (silu_gate with
// C holding the gate product).
enum Bf16GemmEpilogue : int { kGemmStore = 0, kGemmAddInto = 1, kGemmSiluGateInto = 2 };

struct Bf16GemmArgs {
    const bf16_t* a = nullptr;
    const bf16_t* b = nullptr;
    bf16_t* c = nullptr;
    int m = 0, n = 0, k = 0;
    int lda = 0, ldb = 0, ldc = 0;
    int batch = 1;
    int b_group = 1;
    long long a_batch = 0, b_batch = 0, c_batch = 0;
    // Split-K workspace (may be null: no split).  With `splits` > 1 each K
    // slice writes fp32 partial sums here and a second launch adds the slices
    // in slice order and rounds to bf16.
    float* partial = nullptr;
    size_t partial_floats = 0;
    int force_tile = 0;    // 0: planned; else 32, 64 or 128
    int force_k_step = 0;  // 0: planned; else K per pipeline step (32 tile: 64/128/256; 64: 64/128; 128: 64)
    int force_splits = 0;  // 0: planned; else the K slices (bounded by the workspace)
    int epilogue = kGemmStore;
    // B in row segments (batch 1): rows from b2_row on come from b2, rows
    // from b3_row on from b3 (each segment row-major with stride ldb).
    const bf16_t* b2 = nullptr;
    const bf16_t* b3 = nullptr;
    int b2_row = 0, b3_row = 0;
};
hipError_t launch_bf16_gemm(const Bf16GemmArgs& args, hipStream_t stream);
// Prompts of at most this many positions run the reference's GEMM attention
// (scores materialized, causal softmax); longer ones the exact per-row kernel
// (talker.cu:3035-3054 with kPrefillGemmCapacity = 512).
constexpr int kPrefillAttentionRows = 512;
hipError_t launch_causal_softmax(bf16_t* scores, int heads, int rows, int stride, int head_dimension,
                                 hipStream_t stream);
hipError_t launch_prefill_qkv_epilogue(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const bf16_t* rope_table,
                                       bf16_t* key_cache, bf16_t* value_cache, int value_stride, int first, int rows,
                                       int query_heads, int key_value_heads, float epsilon, hipStream_t stream);
hipError_t launch_transpose_values(const bf16_t* qkv, int qkv_width, int v_offset, int rows, int stride,
                                   int key_value_heads, bf16_t* vt, hipStream_t stream);
hipError_t launch_prompt_rows(bf16_t* rows_data, const int* text, const int* codec, const bf16_t* codec_embedding,
                              int codec_vocabulary, int rows, int width, hipStream_t stream);
hipError_t launch_gather_text_rows(const bf16_t* table, const int* text, int vocabulary, int rows, int width,
                                   bf16_t* out, hipStream_t stream);

// Lockstep-batch glue: rows of a batch from / to per-session buffers.
hipError_t launch_gather_rows(const bf16_t* const* sources, int rows, int width, bf16_t* output,
                              hipStream_t stream);
hipError_t launch_scatter_rows(const bf16_t* input, bf16_t* const* destinations, int rows, int width,
                               hipStream_t stream);
hipError_t launch_gather_embedding_rows(const bf16_t* table, int vocabulary, int width,
                                        const int* const* token_bases, int offset, bf16_t* output,
                                        int rows, hipStream_t stream);
hipError_t launch_sum_embeddings_rows(const bf16_t* const* tables, int count, int vocabulary0,
                                      int vocabulary, int width, const int* const* token_bases,
                                      bf16_t* output, int rows, hipStream_t stream);
hipError_t launch_increment_each(int* const* counters, int count, hipStream_t stream);

}  // namespace q3
