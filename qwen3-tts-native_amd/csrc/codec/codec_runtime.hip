// C ABI of the speech-tokenizer decoder for MI355X (include/qwen3_tts_codec.h).
//
// Model: the 271 decoder tensors are uploaded as fp32 (bf16 sources widened
// on the device, CS:3107-3302); convolution and projection weights are then
// regrouped once into the layouts the GEMM kernels stream ([out][tap][in],
// transposed convolutions [(phase, out)][(tap, in)], Q/K/V and gate/up
// concatenated) and the SnakeBeta parameters exponentiated.  A model is
// immutable after load and shared by any number of sessions.
//
// Session: one HIP stream, one device arena (KV ring, convolution histories,
// packet buffers, split-K workspace) and a pinned PCM ring.  A full packet is
// captured once per frame count into a hipGraph and replayed; the neural
// position lives in device memory so replays need no re-capture.  Debug hooks
// run the same launch sequence eagerly, stopping where the reference stops.
#include "codec.hpp"

#include "../../../include/qwen3_tts_codec.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <type_traits>
#include <unordered_map>
#include <vector>

using namespace q3c;

// The ABI's layouts, as the reference's Rust binding and its contract test
// pin them (native/qwen3-tts-native-codec/src/ffi.rs:169-201,
// native/qwen3-tts-native-codec/native/tests/abi_v2_contract.cpp).
static_assert(sizeof(Qwen3TtsCodecPacketResultV1) == 40 && alignof(Qwen3TtsCodecPacketResultV1) == 8, "ABI");
static_assert(sizeof(Qwen3TtsCodecDevicePacketBeginV2) == 40 && alignof(Qwen3TtsCodecDevicePacketBeginV2) == 8, "ABI");
static_assert(sizeof(Qwen3TtsCodecDevicePacketBeginResultV2) == 32, "ABI");
static_assert(sizeof(Qwen3TtsCodecDevicePacketFinishV2) == 56, "ABI");
static_assert(std::is_standard_layout<Qwen3TtsCodecDevicePacketBeginV2>::value &&
                  std::is_standard_layout<Qwen3TtsCodecDevicePacketBeginResultV2>::value &&
                  std::is_standard_layout<Qwen3TtsCodecDevicePacketFinishV2>::value,
              "ABI");
static_assert(offsetof(Qwen3TtsCodecDevicePacketBeginV2, struct_size) == 0 &&
                  offsetof(Qwen3TtsCodecDevicePacketBeginResultV2, struct_size) == 0 &&
                  offsetof(Qwen3TtsCodecDevicePacketFinishV2, struct_size) == 0,
              "ABI");
static_assert(sizeof(Qwen3TtsCodecStateInfoV1) == 80 && sizeof(Qwen3TtsCodecBatchItemV1) == 48 &&
                  sizeof(Qwen3TtsCodecTensorViewV1) == 56 && sizeof(Qwen3TtsCodecWeightProviderV1) == 32 &&
                  sizeof(Qwen3TtsCodecModelInfoV1) == 40,
              "ABI");

namespace {

constexpr int32_t kOk = QWEN3_TTS_CODEC_STATUS_OK;
constexpr int32_t kInvalid = QWEN3_TTS_CODEC_STATUS_INVALID_ARGUMENT;
constexpr int32_t kDevice = QWEN3_TTS_CODEC_STATUS_CUDA;
constexpr int32_t kState = QWEN3_TTS_CODEC_STATUS_STATE;
constexpr int32_t kAlloc = QWEN3_TTS_CODEC_STATUS_ALLOCATION;
constexpr int32_t kModel = QWEN3_TTS_CODEC_STATUS_MODEL;
constexpr uint32_t kExpectedTensors = 271;  // CS:137
constexpr uint64_t kStagingBytes = 8ull << 20;
constexpr int kRingSlots = QWEN3_TTS_CODEC_RING_SLOTS;
constexpr int kMaxSamples = QWEN3_TTS_CODEC_MAX_PACKET_SAMPLES;

void clear_error(char* error, size_t capacity) {
    if (error && capacity) error[0] = '\0';
}

void write_error(char* error, size_t capacity, const char* fmt, ...) {
    if (!error || !capacity) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(error, capacity, fmt, ap);
    va_end(ap);
}

int32_t hip_error(char* error, size_t capacity, const char* what, hipError_t st) {
    write_error(error, capacity, "%s: %s", what, hipGetErrorString(st));
    return kDevice;
}

// ---- tensor table: name -> float elements ----------------------------------
struct TensorSpec {
    std::string name;
    uint64_t elements;
};

const std::vector<TensorSpec>& tensor_table() {
    static const std::vector<TensorSpec> table = [] {
        std::vector<TensorSpec> t;
        auto add = [&](std::string n, uint64_t e) { t.push_back({std::move(n), e}); };
        const std::string q = "decoder.quantizer.";
        add(q + "rvq_first.vq.layers.0._codebook.embedding_sum", 2048ull * 256);
        add(q + "rvq_first.vq.layers.0._codebook.cluster_usage", 2048);
        for (int c = 0; c < 15; ++c) {
            add(q + "rvq_rest.vq.layers." + std::to_string(c) + "._codebook.embedding_sum", 2048ull * 256);
            add(q + "rvq_rest.vq.layers." + std::to_string(c) + "._codebook.cluster_usage", 2048);
        }
        add(q + "rvq_first.output_proj.weight", 512ull * 256);
        add(q + "rvq_rest.output_proj.weight", 512ull * 256);
        add("decoder.pre_conv.conv.weight", 1024ull * 512 * 3);
        add("decoder.pre_conv.conv.bias", 1024);
        const std::string t0 = "decoder.pre_transformer.";
        add(t0 + "input_proj.weight", 512ull * 1024);
        add(t0 + "input_proj.bias", 512);
        for (int l = 0; l < kLayers; ++l) {
            const std::string p = t0 + "layers." + std::to_string(l) + ".";
            add(p + "input_layernorm.weight", 512);
            add(p + "self_attn.q_proj.weight", 1024ull * 512);
            add(p + "self_attn.k_proj.weight", 1024ull * 512);
            add(p + "self_attn.v_proj.weight", 1024ull * 512);
            add(p + "self_attn.o_proj.weight", 512ull * 1024);
            add(p + "self_attn_layer_scale.scale", 512);
            add(p + "post_attention_layernorm.weight", 512);
            add(p + "mlp.gate_proj.weight", 1024ull * 512);
            add(p + "mlp.up_proj.weight", 1024ull * 512);
            add(p + "mlp.down_proj.weight", 512ull * 1024);
            add(p + "mlp_layer_scale.scale", 512);
        }
        add(t0 + "norm.weight", 512);
        add(t0 + "output_proj.weight", 1024ull * 512);
        add(t0 + "output_proj.bias", 1024);
        for (int u = 0; u < 2; ++u) {
            const std::string p = "decoder.upsample." + std::to_string(u) + ".";
            add(p + "0.conv.weight", 1024ull * 1024 * 2);
            add(p + "0.conv.bias", 1024);
            add(p + "1.dwconv.conv.weight", 1024ull * 7);
            add(p + "1.dwconv.conv.bias", 1024);
            add(p + "1.norm.weight", 1024);
            add(p + "1.norm.bias", 1024);
            add(p + "1.pwconv1.weight", 4096ull * 1024);
            add(p + "1.pwconv1.bias", 4096);
            add(p + "1.pwconv2.weight", 1024ull * 4096);
            add(p + "1.pwconv2.bias", 1024);
            add(p + "1.gamma", 1024);
        }
        add("decoder.decoder.0.conv.weight", 1536ull * 1024 * 7);
        add("decoder.decoder.0.conv.bias", 1536);
        for (int s = 0; s < 4; ++s) {
            const uint64_t ci = kStageIn[s], co = kStageOut[s];
            const std::string p = "decoder.decoder." + std::to_string(s + 1) + ".block.";
            add(p + "0.alpha", ci);
            add(p + "0.beta", ci);
            add(p + "1.conv.weight", ci * co * 2 * kStride[s]);
            add(p + "1.conv.bias", co);
            for (int u = 0; u < 3; ++u) {
                const std::string r = p + std::to_string(u + 2) + ".";
                add(r + "act1.alpha", co);
                add(r + "act1.beta", co);
                add(r + "conv1.conv.weight", co * co * 7);
                add(r + "conv1.conv.bias", co);
                add(r + "act2.alpha", co);
                add(r + "act2.beta", co);
                add(r + "conv2.conv.weight", co * co);
                add(r + "conv2.conv.bias", co);
            }
        }
        add("decoder.decoder.5.alpha", 96);
        add("decoder.decoder.5.beta", 96);
        add("decoder.decoder.6.conv.weight", 96ull * 7);
        add("decoder.decoder.6.conv.bias", 1);
        return t;
    }();
    return table;
}

// ---- executable weights -------------------------------------------------------
struct LayerW {
    const float *in_norm, *qkv, *o, *attn_scale, *post_norm, *gate_up, *down, *mlp_scale;
};
struct UpW {
    const float *tconv, *tconv_b, *dw, *dw_b, *ln_w, *ln_b, *pw1, *pw1_b, *pw2, *pw2_b, *gamma;
};
struct UnitW {
    const float *alpha1, *beta1, *conv1, *conv1_b, *alpha2, *beta2, *conv2, *conv2_b;
};
struct StageW {
    const float *alpha, *beta, *tconv, *tconv_b;
    UnitW unit[3];
};
struct Weights {
    const float* emb[kCodebooks];
    const float* usage[kCodebooks];
    const float *rvq_proj, *preconv, *preconv_b, *in_proj, *in_proj_b;
    LayerW layer[kLayers];
    const float *norm, *out_proj, *out_proj_b;
    UpW up[2];
    const float *conv0, *conv0_b;
    StageW stage[4];
    const float *final_alpha, *final_beta, *final_w, *final_b;
};

}  // namespace

// ---------------------------------------------------------------------------
// model
// ---------------------------------------------------------------------------
struct Qwen3TtsCodecModelV1 {
    int device = 0;
    std::atomic<int> refs{1};
    std::mutex lifecycle;
    std::atomic<uint32_t> active_sessions{0};
    std::atomic<bool> warmed{false};
    Qwen3TtsCodecModelInfoV1 info{};
    std::vector<void*> allocations;
    Weights w{};

    ~Qwen3TtsCodecModelV1() { release_weights(); }
    void release_weights() {
        if (!allocations.empty()) {
            int previous = 0;
            (void)hipGetDevice(&previous);
            (void)hipSetDevice(device);
            for (void* p : allocations) (void)hipFree(p);
            (void)hipSetDevice(previous);
        }
        allocations.clear();
        w = Weights{};
        info = Qwen3TtsCodecModelInfoV1{};
    }
};

namespace {

void retain(Qwen3TtsCodecModelV1* m) { m->refs.fetch_add(1, std::memory_order_relaxed); }
void release(Qwen3TtsCodecModelV1* m) {
    if (m && m->refs.fetch_sub(1, std::memory_order_acq_rel) == 1) delete m;
}

// ---------------------------------------------------------------------------
// session buffers
// ---------------------------------------------------------------------------
struct Ext {  // an extended buffer and its history
    float* ext = nullptr;
    float* hist = nullptr;
    int channels = 0, history = 0;
};

struct Plans {
    GemmPlan up_tconv[2], pw1[2], pw2[2], conv0, tconv[4], conv7[4], conv1[4];
};

struct Arena {
    char* base = nullptr;
    size_t used = 0;
    template <class T>
    T* take(size_t count) {
        used = (used + 255) & ~size_t(255);
        T* p = reinterpret_cast<T*>(base ? base + used : nullptr);
        used += count * sizeof(T);
        return p;
    }
};

size_t stage_input_positions(int stage, int frames) {
    size_t p = 4ull * frames;
    for (int s = 0; s < stage; ++s) p *= kStride[s];
    return p;
}

}  // namespace

struct Qwen3TtsCodecContextV1 {
    int device = 0;
    Qwen3TtsCodecModelV1* model = nullptr;
    bool counts_as_shared_session = false;
    hipStream_t stream = nullptr;
    hipEvent_t start_event = nullptr, stop_event = nullptr, consumed_event = nullptr;
    int cus = 256;

    // host-side stream state (CS:1240-1290)
    uint64_t frame_position = 0, emitted_samples = 0, neural_frame_position = 0;
    uint32_t next_ring_slot = 0, kv_ring_head = 0;
    bool finalized = false, cancelled = false, device_packet_pending = false;
    uint64_t next_ticket = 1, pending_ticket = 0;
    uint32_t pending_frames = 0, pending_slot = 0;
    std::chrono::steady_clock::time_point pending_start{};

    // device arena
    void* arena = nullptr;
    size_t arena_bytes = 0, kv_bytes = 0, history_bytes = 0;
    int16_t* host_pcm = nullptr;  // pinned [ring][7680]
    uint16_t* code_ring = nullptr;
    uint16_t* codes_in = nullptr;
    int16_t* pcm_ring = nullptr;
    int16_t* pcm_dev = nullptr;
    unsigned long long* position = nullptr;
    int* fixture_state = nullptr;
    float *x_rvq = nullptr, *t_in = nullptr, *h = nullptr, *h2 = nullptr, *qkv = nullptr, *attn = nullptr,
          *act = nullptr, *t_out = nullptr;
    float *kv_k = nullptr, *kv_v = nullptr;
    Ext pre, up_dw[2], conv0, tconv[4], unit[4][3], final_conv;
    float *ln = nullptr, *pw = nullptr, *up1_out = nullptr, *conv0_raw = nullptr;
    float *cur[4] = {}, *ext2[4] = {};
    float *preclamp = nullptr, *clamped = nullptr;
    float* partial = nullptr;
    CopySegment* seg_in[kMaxFrames + 1] = {};
    CopySegment* seg_out[kMaxFrames + 1] = {};
    Plans plans[kMaxFrames + 1];

    hipGraphExec_t graphs[kMaxFrames + 1] = {};
    bool use_graphs = true;
};

namespace {

constexpr int kSegments = 21;  // histories in pipeline order

// segments advanced by a packet that stops after `stop` (0: whole packet)
int segments_for_stop(int stop) {
    switch (stop) {
        case 1:
        case 2: return 1;
        case 3: return 3;
        case 6: return 4;
        case 7: case 8: case 9: case 10: return 4 + 4 * (stop - 6);
        case 11: return 20;
        default: return kSegments;
    }
}

void layout_session(Qwen3TtsCodecContextV1* s, Arena& a) {
    s->code_ring = a.take<uint16_t>(kRingSlots * kMaxFrames * kCodebooks);
    s->codes_in = a.take<uint16_t>(kMaxFrames * kCodebooks);
    s->pcm_ring = a.take<int16_t>((size_t)kRingSlots * kMaxSamples);
    s->pcm_dev = a.take<int16_t>(kMaxSamples);
    s->position = a.take<unsigned long long>(1);
    s->fixture_state = a.take<int>(22);
    const size_t kv_start = a.used;
    s->kv_k = a.take<float>((size_t)kLayers * kHeads * kKvSlots * kHeadDim);
    s->kv_v = a.take<float>((size_t)kLayers * kHeads * kKvSlots * kHeadDim);
    s->kv_bytes = a.used - kv_start;
    size_t hist = 0;
    auto ext = [&](Ext& e, int channels, int history, size_t positions) {
        e.channels = channels;
        e.history = history;
        e.ext = a.take<float>((size_t)(history + positions) * channels);
        e.hist = a.take<float>((size_t)history * channels);
        hist += (size_t)history * channels * sizeof(float);
    };
    const int F = kMaxFrames;
    s->x_rvq = a.take<float>(F * 512);
    ext(s->pre, 512, 2, F);
    s->t_in = a.take<float>(F * 1024);
    s->h = a.take<float>(F * 512);
    s->h2 = a.take<float>(F * 512);
    s->qkv = a.take<float>(F * 3072);
    s->attn = a.take<float>(F * 1024);
    s->act = a.take<float>(F * 1024);
    s->t_out = a.take<float>(F * 1024);
    ext(s->up_dw[0], 1024, 6, 2 * F);
    ext(s->up_dw[1], 1024, 6, 4 * F);
    s->ln = a.take<float>(4 * F * 1024);
    s->pw = a.take<float>(4 * F * 4096);
    s->up1_out = a.take<float>(2 * F * 1024);
    ext(s->conv0, 1024, 6, 4 * F);
    s->conv0_raw = a.take<float>(4 * F * 1536);
    for (int t = 0; t < 4; ++t) {
        const size_t p_in = stage_input_positions(t, F), p_out = p_in * kStride[t];
        ext(s->tconv[t], kStageIn[t], 1, p_in);
        s->cur[t] = a.take<float>(p_out * kStageOut[t]);
        s->ext2[t] = a.take<float>(p_out * kStageOut[t]);
        for (int u = 0; u < 3; ++u) ext(s->unit[t][u], kStageOut[t], 6 * kDilation[u], p_out);
    }
    ext(s->final_conv, 96, 6, (size_t)F * kSamplesPerFrame);
    s->preclamp = a.take<float>((size_t)F * kSamplesPerFrame);
    s->clamped = a.take<float>((size_t)F * kSamplesPerFrame);
    s->history_bytes = hist;
    // split-K workspace: the largest plan over every frame count
    size_t partial = 0;
    for (int f = 1; f <= kMaxFrames; ++f) {
        Plans& p = s->plans[f];
        for (int u = 0; u < 2; ++u) {
            const int m = f << u;  // 1x / 2x frames in, then 2x / 4x after the transposed conv
            p.up_tconv[u] = plan_conv_gemm(m, 2048, 1024, 1024, s->cus);
            p.pw1[u] = plan_conv_gemm(2 * m, 4096, 1024, 1024, s->cus);
            p.pw2[u] = plan_conv_gemm(2 * m, 1024, 4096, 4096, s->cus);
        }
        p.conv0 = plan_conv_gemm(4 * f, 1536, 7 * 1024, 1024, s->cus);
        for (int t = 0; t < 4; ++t) {
            const int p_in = (int)stage_input_positions(t, f), p_out = p_in * kStride[t];
            p.tconv[t] = plan_conv_gemm(p_in, kStride[t] * kStageOut[t], 2 * kStageIn[t], kStageIn[t], s->cus);
            p.conv7[t] = plan_conv_gemm(p_out, kStageOut[t], 7 * kStageOut[t], kStageOut[t], s->cus);
            p.conv1[t] = plan_conv_gemm(p_out, kStageOut[t], kStageOut[t], kStageOut[t], s->cus);
        }
        const GemmPlan* all[] = {&p.up_tconv[0], &p.up_tconv[1], &p.pw1[0], &p.pw1[1], &p.pw2[0], &p.pw2[1],
                                 &p.conv0, &p.tconv[0], &p.tconv[1], &p.tconv[2], &p.tconv[3], &p.conv7[0],
                                 &p.conv7[1], &p.conv7[2], &p.conv7[3], &p.conv1[0], &p.conv1[1], &p.conv1[2],
                                 &p.conv1[3]};
        for (const GemmPlan* g : all) {
            partial = std::max(partial, g->partial_floats());
        }
    }
    s->partial = a.take<float>(std::max<size_t>(partial, 1));
    for (int f = 0; f <= kMaxFrames; ++f) {
        s->seg_in[f] = a.take<CopySegment>(kSegments);
        s->seg_out[f] = a.take<CopySegment>(kSegments);
    }
}

// Histories in pipeline order: pre-conv, two ConvNeXt depthwise, decoder
// conv 0, per stage (transposed conv, three residual units), final conv.
std::vector<Ext*> history_order(Qwen3TtsCodecContextV1* s) {
    std::vector<Ext*> v = {&s->pre, &s->up_dw[0], &s->up_dw[1], &s->conv0};
    for (int t = 0; t < 4; ++t) {
        v.push_back(&s->tconv[t]);
        for (int u = 0; u < 3; ++u) v.push_back(&s->unit[t][u]);
    }
    v.push_back(&s->final_conv);
    return v;
}

// packet positions of each history's layer for `frames`
std::vector<size_t> history_positions(int frames) {
    std::vector<size_t> v = {(size_t)frames, 2ull * frames, 4ull * frames, 4ull * frames};
    for (int t = 0; t < 4; ++t) {
        const size_t p_in = stage_input_positions(t, frames);
        v.push_back(p_in);
        for (int u = 0; u < 3; ++u) v.push_back(p_in * kStride[t]);
    }
    v.push_back((size_t)frames * kSamplesPerFrame);
    return v;
}

hipError_t upload_segments(Qwen3TtsCodecContextV1* s) {
    const auto order = history_order(s);
    for (int f = 1; f <= kMaxFrames; ++f) {
        const auto pos = history_positions(f);
        CopySegment in[kSegments], out[kSegments];
        for (int i = 0; i < kSegments; ++i) {
            const Ext& e = *order[i];
            const unsigned floats = (unsigned)(e.history * e.channels);
            in[i] = {e.hist, e.ext, floats};
            out[i] = {e.ext + pos[i] * e.channels, e.hist, floats};
        }
        hipError_t st = hipMemcpyAsync(s->seg_in[f], in, sizeof(in), hipMemcpyHostToDevice, s->stream);
        if (st == hipSuccess) st = hipMemcpyAsync(s->seg_out[f], out, sizeof(out), hipMemcpyHostToDevice, s->stream);
        if (st != hipSuccess) return st;
    }
    return hipStreamSynchronize(s->stream);
}

hipError_t reset_device_state(Qwen3TtsCodecContextV1* s) {
    hipError_t st = hipSuccess;
    for (Ext* e : history_order(s)) {
        if (st == hipSuccess) st = launch_fill_f32(e->hist, (size_t)e->history * e->channels, 0.f, s->stream);
    }
    if (st == hipSuccess)
        st = hipMemsetAsync(s->position, 0, sizeof(unsigned long long), s->stream);
    if (st == hipSuccess) st = hipMemsetAsync(s->fixture_state, 0, 22 * sizeof(int), s->stream);
    if (st == hipSuccess) st = hipStreamSynchronize(s->stream);
    return st;
}

// ---------------------------------------------------------------------------
// packet launch sequence (CS:3989-4089 and the stages it calls)
// ---------------------------------------------------------------------------
struct Launcher {
    Qwen3TtsCodecContextV1* s;
    const Weights& w;
    hipError_t st = hipSuccess;

    void ok(hipError_t e) {
        if (st == hipSuccess) st = e;
    }

    void rows(const float* x, int ldx, int rows, int k, int n, const float* wt, const float* norm, const float* bias,
              int epilogue, const float* residual, const float* scale, float* out, int ldo,
              unsigned long long* advance = nullptr, int by = 0) {
        RowsGemvArgs g{x, ldx, rows, k, n, wt, norm, bias, epilogue, residual, scale, out, ldo, advance, by};
        ok(launch_rows_gemv(g, s->stream));
    }

    void gemm(const GemmPlan& plan, const float* a, int cin, int taps, int dilation, const float* wt,
              const float* bias, int m, int n, int k, int cout, int epilogue, const float* residual,
              const float* gamma, float* out, float* snake_out, const float* alpha, const float* beta) {
        ConvGemmArgs g{a,   cin,    taps,     dilation, wt,    bias,      m,     n,     k,
                       cout, epilogue, residual, gamma,    out,   snake_out, alpha, beta, plan.splits,
                       s->partial};
        ok(launch_conv_gemm(g, plan, s->stream));
    }

    void history_out(int frames, int stop) { ok(launch_copy_segments(s->seg_out[frames], segments_for_stop(stop), s->stream)); }

    // stop: 0 whole packet; 1 frontend; 2 transformer; 3 latent; 6..13 decoder checkpoint
    void packet(int F, int stop) {
        const Plans& pl = s->plans[F];
        ok(launch_codec_frontend(s->codes_in, F, w.emb, w.usage, s->x_rvq, s->seg_in[F], kSegments, s->stream));
        float* rvq = s->pre.ext + 2 * 512;
        rows(s->x_rvq, 512, F, 512, 512, w.rvq_proj, nullptr, nullptr, kRowsStore, nullptr, nullptr, rvq, 512);
        rows(s->pre.ext, 512, F, 3 * 512, 1024, w.preconv, nullptr, w.preconv_b, kRowsStore, nullptr, nullptr,
             s->t_in, 1024);
        if (stop == 1) return history_out(F, stop);

        rows(s->t_in, 1024, F, 1024, 512, w.in_proj, nullptr, w.in_proj_b, kRowsStore, nullptr, nullptr, s->h, 512);
        const size_t kv_layer = (size_t)kHeads * kKvSlots * kHeadDim;
        for (int l = 0; l < kLayers; ++l) {
            const LayerW& L = w.layer[l];
            rows(s->h, 512, F, 512, 3072, L.qkv, L.in_norm, nullptr, kRowsStore, nullptr, nullptr, s->qkv, 3072);
            ok(launch_codec_attention(s->qkv, F, s->position, s->kv_k + l * kv_layer, s->kv_v + l * kv_layer,
                                      s->attn, s->stream));
            rows(s->attn, 1024, F, 1024, 512, L.o, nullptr, nullptr, kRowsScaledResidual, s->h, L.attn_scale, s->h2,
                 512);
            rows(s->h2, 512, F, 512, 1024, L.gate_up, L.post_norm, nullptr, kRowsSiluPair, nullptr, nullptr, s->act,
                 1024);
            rows(s->act, 1024, F, 1024, 512, L.down, nullptr, nullptr, kRowsScaledResidual, s->h2, L.mlp_scale, s->h,
                 512);
        }
        rows(s->h, 512, F, 512, 1024, w.out_proj, w.norm, w.out_proj_b, kRowsStore, nullptr, nullptr, s->t_out, 1024,
             s->position, F);
        if (stop == 2) return history_out(F, stop);

        // latent upsampling: 2 x (transposed conv k2 s2, ConvNeXt)
        const float* in = s->t_out;
        for (int u = 0; u < 2; ++u) {
            const UpW& U = w.up[u];
            const int m = F << u, p = 2 * m;
            float* dw_in = s->up_dw[u].ext + 6 * 1024;
            gemm(pl.up_tconv[u], in, 1024, 1, 1, U.tconv, U.tconv_b, m, 2048, 1024, 1024, kEpStore, nullptr, nullptr,
                 dw_in, nullptr, nullptr, nullptr);
            ok(launch_dwconv_layernorm(s->up_dw[u].ext, p, U.dw, U.dw_b, U.ln_w, U.ln_b, s->ln, s->stream));
            gemm(pl.pw1[u], s->ln, 1024, 1, 1, U.pw1, U.pw1_b, p, 4096, 1024, 4096, kEpGelu, nullptr, nullptr, s->pw,
                 nullptr, nullptr, nullptr);
            float* out = u == 0 ? s->up1_out : s->conv0.ext + 6 * 1024;
            gemm(pl.pw2[u], s->pw, 4096, 1, 1, U.pw2, U.pw2_b, p, 1024, 4096, 1024, kEpGammaResidual, dw_in, U.gamma,
                 out, nullptr, nullptr, nullptr);
            in = out;
        }
        if (stop == 3) return history_out(F, stop);

        // waveform decoder
        const StageW& S0 = w.stage[0];
        gemm(pl.conv0, s->conv0.ext, 1024, 7, 1, w.conv0, w.conv0_b, 4 * F, 1536, 7 * 1024, 1536, kEpStore, nullptr,
             nullptr, s->conv0_raw, s->tconv[0].ext + 1536, S0.alpha, S0.beta);
        if (stop == 6) return history_out(F, stop);
        for (int t = 0; t < 4; ++t) {
            const StageW& S = w.stage[t];
            const int ci = kStageIn[t], co = kStageOut[t];
            const int p_in = (int)stage_input_positions(t, F), p = p_in * kStride[t];
            gemm(pl.tconv[t], s->tconv[t].ext, ci, 2, 1, S.tconv, S.tconv_b, p_in, kStride[t] * co, 2 * ci, co,
                 kEpStore, nullptr, nullptr, s->cur[t], s->unit[t][0].ext + (size_t)6 * kDilation[0] * co,
                 S.unit[0].alpha1, S.unit[0].beta1);
            for (int u = 0; u < 3; ++u) {
                const UnitW& R = S.unit[u];
                gemm(pl.conv7[t], s->unit[t][u].ext, co, 7, kDilation[u], R.conv1, R.conv1_b, p, co, 7 * co, co,
                     kEpStore, nullptr, nullptr, nullptr, s->ext2[t], R.alpha2, R.beta2);
                float* next;
                const float *alpha, *beta;
                if (u < 2) {
                    next = s->unit[t][u + 1].ext + (size_t)6 * kDilation[u + 1] * co;
                    alpha = S.unit[u + 1].alpha1;
                    beta = S.unit[u + 1].beta1;
                } else if (t < 3) {
                    next = s->tconv[t + 1].ext + co;
                    alpha = w.stage[t + 1].alpha;
                    beta = w.stage[t + 1].beta;
                } else {
                    next = s->final_conv.ext + 6 * 96;
                    alpha = w.final_alpha;
                    beta = w.final_beta;
                }
                gemm(pl.conv1[t], s->ext2[t], co, 1, 1, R.conv2, R.conv2_b, p, co, co, co, kEpResidual, s->cur[t],
                     nullptr, s->cur[t], next, alpha, beta);
            }
            if (stop == 7 + t) return history_out(F, stop);
        }
        if (stop == 11) return history_out(F, stop);
        ok(launch_final_conv_pcm(s->final_conv.ext, F * kSamplesPerFrame, w.final_w, w.final_b, s->pcm_dev,
                                 s->preclamp, s->clamped, s->stream));
        history_out(F, 0);
    }
};

hipError_t enqueue_full_packet(Qwen3TtsCodecContextV1* s, int frames) {
    Launcher l{s, s->model->w};
    if (!s->use_graphs) {
        l.packet(frames, 0);
        return l.st;
    }
    if (!s->graphs[frames]) {
        hipError_t st = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
        if (st != hipSuccess) return st;
        l.packet(frames, 0);
        hipGraph_t graph = nullptr;
        st = hipStreamEndCapture(s->stream, &graph);
        if (l.st != hipSuccess || st != hipSuccess) {
            if (graph) (void)hipGraphDestroy(graph);
            return l.st != hipSuccess ? l.st : st;
        }
        st = hipGraphInstantiate(&s->graphs[frames], graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        if (st != hipSuccess) {
            s->graphs[frames] = nullptr;
            return st;
        }
    }
    return hipGraphLaunch(s->graphs[frames], s->stream);
}

// ---------------------------------------------------------------------------
// model load (CS:3107-3302) + regrouping into the executable layouts
// ---------------------------------------------------------------------------
struct Loader {
    Qwen3TtsCodecModelV1* m;
    hipStream_t stream;
    std::unordered_map<std::string, float*> raw;
    std::unordered_map<std::string, uint64_t> elements;
    std::vector<float*> transient;

    float* alloc(size_t floats) {
        void* p = nullptr;
        if (hipMalloc(&p, floats * sizeof(float)) != hipSuccess) return nullptr;
        m->allocations.push_back(p);
        return static_cast<float*>(p);
    }
    float* get(const std::string& name) const { return raw.at(name); }
    // a raw tensor that only feeds a regrouped copy: freed after load
    float* consume(const std::string& name) {
        float* p = raw.at(name);
        transient.push_back(p);
        return p;
    }
};

int32_t build_weights(Loader& L, char* error, size_t capacity) {
    Weights& w = L.m->w;
    hipStream_t st = L.stream;
    hipError_t e = hipSuccess;
    auto ok = [&](hipError_t x) {
        if (e == hipSuccess) e = x;
    };
    const std::string q = "decoder.quantizer.";
    for (int cb = 0; cb < kCodebooks; ++cb) {
        const std::string p = cb == 0 ? q + "rvq_first.vq.layers.0._codebook."
                                      : q + "rvq_rest.vq.layers." + std::to_string(cb - 1) + "._codebook.";
        w.emb[cb] = L.get(p + "embedding_sum");
        w.usage[cb] = L.get(p + "cluster_usage");
    }
    // RVQ projections [512][256] x 2 -> [512][first 256 | rest 256]
    float* rvq = L.alloc(512 * 512);
    if (!rvq) return kAlloc;
    ok(hipMemcpy2DAsync(rvq, 512 * sizeof(float), L.consume(q + "rvq_first.output_proj.weight"), 256 * sizeof(float),
                        256 * sizeof(float), 512, hipMemcpyDeviceToDevice, st));
    ok(hipMemcpy2DAsync(rvq + 256, 512 * sizeof(float), L.consume(q + "rvq_rest.output_proj.weight"),
                        256 * sizeof(float), 256 * sizeof(float), 512, hipMemcpyDeviceToDevice, st));
    w.rvq_proj = rvq;
    auto conv = [&](const std::string& name, int out_ch, int in_ch, int taps) -> const float* {
        float* d = L.alloc((size_t)out_ch * in_ch * taps);
        if (!d) return nullptr;
        ok(launch_repack_conv(L.consume(name), out_ch, in_ch, taps, d, st));
        return d;
    };
    auto transpose = [&](const std::string& name, int in_ch, int out_ch, int stride, bool overlap) -> const float* {
        float* d = L.alloc((size_t)in_ch * out_ch * stride * (overlap ? 2 : 1));
        if (!d) return nullptr;
        ok(launch_repack_transpose(L.consume(name), in_ch, out_ch, stride, overlap, d, st));
        return d;
    };
    w.preconv = conv("decoder.pre_conv.conv.weight", 1024, 512, 3);
    w.preconv_b = L.get("decoder.pre_conv.conv.bias");
    const std::string t0 = "decoder.pre_transformer.";
    w.in_proj = L.get(t0 + "input_proj.weight");
    w.in_proj_b = L.get(t0 + "input_proj.bias");
    for (int l = 0; l < kLayers; ++l) {
        const std::string p = t0 + "layers." + std::to_string(l) + ".";
        LayerW& Lw = w.layer[l];
        float* qkv = L.alloc(3ull * 1024 * 512);
        float* gu = L.alloc(2ull * 1024 * 512);
        if (!qkv || !gu) return kAlloc;
        const size_t mat = 1024ull * 512 * sizeof(float);
        ok(hipMemcpyAsync(qkv, L.consume(p + "self_attn.q_proj.weight"), mat, hipMemcpyDeviceToDevice, st));
        ok(hipMemcpyAsync(qkv + 1024 * 512, L.consume(p + "self_attn.k_proj.weight"), mat, hipMemcpyDeviceToDevice, st));
        ok(hipMemcpyAsync(qkv + 2048 * 512, L.consume(p + "self_attn.v_proj.weight"), mat, hipMemcpyDeviceToDevice, st));
        ok(hipMemcpyAsync(gu, L.consume(p + "mlp.gate_proj.weight"), mat, hipMemcpyDeviceToDevice, st));
        ok(hipMemcpyAsync(gu + 1024 * 512, L.consume(p + "mlp.up_proj.weight"), mat, hipMemcpyDeviceToDevice, st));
        Lw.qkv = qkv;
        Lw.gate_up = gu;
        Lw.in_norm = L.get(p + "input_layernorm.weight");
        Lw.o = L.get(p + "self_attn.o_proj.weight");
        Lw.attn_scale = L.get(p + "self_attn_layer_scale.scale");
        Lw.post_norm = L.get(p + "post_attention_layernorm.weight");
        Lw.down = L.get(p + "mlp.down_proj.weight");
        Lw.mlp_scale = L.get(p + "mlp_layer_scale.scale");
    }
    w.norm = L.get(t0 + "norm.weight");
    w.out_proj = L.get(t0 + "output_proj.weight");
    w.out_proj_b = L.get(t0 + "output_proj.bias");
    for (int u = 0; u < 2; ++u) {
        const std::string p = "decoder.upsample." + std::to_string(u) + ".";
        UpW& U = w.up[u];
        U.tconv = transpose(p + "0.conv.weight", 1024, 1024, 2, false);
        U.tconv_b = L.get(p + "0.conv.bias");
        U.dw = L.get(p + "1.dwconv.conv.weight");
        U.dw_b = L.get(p + "1.dwconv.conv.bias");
        U.ln_w = L.get(p + "1.norm.weight");
        U.ln_b = L.get(p + "1.norm.bias");
        U.pw1 = L.get(p + "1.pwconv1.weight");
        U.pw1_b = L.get(p + "1.pwconv1.bias");
        U.pw2 = L.get(p + "1.pwconv2.weight");
        U.pw2_b = L.get(p + "1.pwconv2.bias");
        U.gamma = L.get(p + "1.gamma");
    }
    w.conv0 = conv("decoder.decoder.0.conv.weight", 1536, 1024, 7);
    w.conv0_b = L.get("decoder.decoder.0.conv.bias");
    auto snake_params = [&](const std::string& prefix, int channels, const float*& alpha, const float*& beta) {
        float* a = L.get(prefix + "alpha");
        float* b = L.get(prefix + "beta");
        ok(launch_snake_params(a, b, channels, st));
        alpha = a;
        beta = b;
    };
    for (int t = 0; t < 4; ++t) {
        const int ci = kStageIn[t], co = kStageOut[t];
        const std::string p = "decoder.decoder." + std::to_string(t + 1) + ".block.";
        StageW& S = w.stage[t];
        snake_params(p + "0.", ci, S.alpha, S.beta);
        S.tconv = transpose(p + "1.conv.weight", ci, co, kStride[t], true);
        S.tconv_b = L.get(p + "1.conv.bias");
        for (int u = 0; u < 3; ++u) {
            const std::string r = p + std::to_string(u + 2) + ".";
            UnitW& R = S.unit[u];
            snake_params(r + "act1.", co, R.alpha1, R.beta1);
            snake_params(r + "act2.", co, R.alpha2, R.beta2);
            R.conv1 = conv(r + "conv1.conv.weight", co, co, 7);
            R.conv1_b = L.get(r + "conv1.conv.bias");
            R.conv2 = L.get(r + "conv2.conv.weight");
            R.conv2_b = L.get(r + "conv2.conv.bias");
            if (!R.conv1) return kAlloc;
        }
        if (!S.tconv) return kAlloc;
    }
    snake_params("decoder.decoder.5.", 96, w.final_alpha, w.final_beta);
    w.final_w = L.get("decoder.decoder.6.conv.weight");
    w.final_b = L.get("decoder.decoder.6.conv.bias");
    if (!w.preconv || !w.conv0 || !w.up[0].tconv || !w.up[1].tconv) return kAlloc;
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_error(error, capacity, "regroup decoder weights", e);
    // free the raw tensors that only fed regrouped copies
    for (float* p : L.transient) {
        auto it = std::find(L.m->allocations.begin(), L.m->allocations.end(), static_cast<void*>(p));
        if (it != L.m->allocations.end()) {
            (void)hipFree(p);
            L.m->allocations.erase(it);
        }
    }
    return kOk;
}

// ---------------------------------------------------------------------------
// packet helpers
// ---------------------------------------------------------------------------
int32_t validate_packet_state(const Qwen3TtsCodecContextV1* s, uint32_t frames, char* error, size_t capacity) {
    if (frames == 0 || frames > QWEN3_TTS_CODEC_MAX_PACKET_FRAMES) {
        write_error(error, capacity, "packet must contain 1-4 frames");
        return kInvalid;
    }
    if (s->model->info.loaded == 0) {
        write_error(error, capacity, "decoder model is not loaded");
        return kState;
    }
    if (s->finalized || s->cancelled) {
        write_error(error, capacity, "stream is finalized; reset is required");
        return kState;
    }
    if (s->device_packet_pending) {
        write_error(error, capacity, "a device packet ticket is already pending");
        return kState;
    }
    return kOk;
}

bool host_codes_valid(const uint16_t* codes, uint32_t frames) {
    for (uint32_t i = 0; i < frames * kCodebooks; ++i)
        if (codes[i] >= 2048) return false;
    return true;
}

// stages codes already in the ring slot into the graph input, runs the
// packet, queues the PCM copy and the stop event
int32_t enqueue_staged_packet(Qwen3TtsCodecContextV1* s, uint32_t frames, uint32_t slot, char* error,
                              size_t capacity) {
    const uint16_t* staged = s->code_ring + (size_t)slot * kMaxFrames * kCodebooks;
    hipError_t st = hipMemcpyAsync(s->codes_in, staged, (size_t)frames * kCodebooks * sizeof(uint16_t),
                                   hipMemcpyDeviceToDevice, s->stream);
    if (st == hipSuccess) st = enqueue_full_packet(s, (int)frames);
    if (st != hipSuccess) return hip_error(error, capacity, "launch decoder packet", st);
    const size_t samples = (size_t)frames * kSamplesPerFrame;
    int16_t* dev_slot = s->pcm_ring + (size_t)slot * kMaxSamples;
    st = hipMemcpyAsync(dev_slot, s->pcm_dev, samples * sizeof(int16_t), hipMemcpyDeviceToDevice, s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "stage packet PCM", st);
    st = hipMemcpyAsync(s->host_pcm + (size_t)slot * kMaxSamples, dev_slot, samples * sizeof(int16_t),
                        hipMemcpyDeviceToHost, s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "queue packet PCM copy", st);
    st = hipEventRecord(s->stop_event, s->stream);
    return st == hipSuccess ? kOk : hip_error(error, capacity, "record packet completion", st);
}

int32_t finish_staged_packet(Qwen3TtsCodecContextV1* s, uint32_t slot, uint32_t frames, int32_t is_final,
                             int16_t* pcm, Qwen3TtsCodecPacketResultV1* result,
                             std::chrono::steady_clock::time_point start, char* error, size_t capacity) {
    hipError_t st = hipEventSynchronize(s->stop_event);
    if (st != hipSuccess) return hip_error(error, capacity, "complete neural decoder packet", st);
    float ms = 0.f;
    st = hipEventElapsedTime(&ms, s->start_event, s->stop_event);
    if (st != hipSuccess) return hip_error(error, capacity, "measure packet GPU time", st);
    const size_t samples = (size_t)frames * kSamplesPerFrame;
    std::memcpy(pcm, s->host_pcm + (size_t)slot * kMaxSamples, samples * sizeof(int16_t));
    const uint64_t first_frame = s->frame_position, first_sample = s->emitted_samples;
    s->frame_position += frames;
    s->emitted_samples += samples;
    s->neural_frame_position += frames;
    s->kv_ring_head = (uint32_t)(s->neural_frame_position % kWindow);
    s->next_ring_slot = (s->next_ring_slot + 1) % kRingSlots;
    s->finalized = is_final != 0;
    const float e2e = std::chrono::duration<float, std::micro>(std::chrono::steady_clock::now() - start).count();
    *result = Qwen3TtsCodecPacketResultV1{first_frame,  first_sample, frames,    (uint32_t)samples,
                                          slot,         (uint32_t)is_final,     ms * 1000.f, e2e};
    return kOk;
}

int32_t begin_host_packet(Qwen3TtsCodecContextV1* s, const uint16_t* codes, uint32_t frames, uint32_t* slot_out,
                          char* error, size_t capacity) {
    const uint32_t slot = s->next_ring_slot;
    hipError_t st = hipSetDevice(s->device);
    if (st != hipSuccess) return hip_error(error, capacity, "select HIP device", st);
    st = hipEventRecord(s->start_event, s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "start packet timing", st);
    st = hipMemcpyAsync(s->code_ring + (size_t)slot * kMaxFrames * kCodebooks, codes,
                        (size_t)frames * kCodebooks * sizeof(uint16_t), hipMemcpyHostToDevice, s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "upload frontend codes", st);
    *slot_out = slot;
    return enqueue_staged_packet(s, frames, slot, error, capacity);
}

int32_t check_packet_args(Qwen3TtsCodecContextV1* s, const uint16_t* codes, uint32_t frames, int32_t is_final,
                          int16_t* pcm, size_t capacity_samples, Qwen3TtsCodecPacketResultV1* result, char* error,
                          size_t capacity) {
    if (!s || !codes || !pcm || !result) {
        write_error(error, capacity, "context, codec frames, PCM output, and result are required");
        return kInvalid;
    }
    if (frames == 0 || frames > QWEN3_TTS_CODEC_MAX_PACKET_FRAMES || (is_final != 0 && is_final != 1)) {
        write_error(error, capacity, "packet must contain 1-4 frames");
        return kInvalid;
    }
    const int32_t v = validate_packet_state(s, frames, error, capacity);
    if (v != kOk) return v;
    if (capacity_samples < (size_t)frames * kSamplesPerFrame) {
        write_error(error, capacity, "PCM output capacity is too small");
        return kInvalid;
    }
    if (!host_codes_valid(codes, frames)) {
        write_error(error, capacity, "codec codes must be below 2048");
        return kInvalid;
    }
    return kOk;
}

// ---------------------------------------------------------------------------
// context lifecycle
// ---------------------------------------------------------------------------
void release_context(Qwen3TtsCodecContextV1* s) {
    if (!s) return;
    int previous = 0;
    (void)hipGetDevice(&previous);
    (void)hipSetDevice(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    for (auto& g : s->graphs)
        if (g) (void)hipGraphExecDestroy(g);
    if (s->arena) (void)hipFree(s->arena);
    if (s->host_pcm) (void)hipHostFree(s->host_pcm);
    if (s->start_event) (void)hipEventDestroy(s->start_event);
    if (s->stop_event) (void)hipEventDestroy(s->stop_event);
    if (s->consumed_event) (void)hipEventDestroy(s->consumed_event);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    (void)hipSetDevice(previous);
    if (s->model) {
        if (s->counts_as_shared_session) s->model->active_sessions.fetch_sub(1, std::memory_order_acq_rel);
        release(s->model);
    }
    delete s;
}

int32_t create_context(int32_t device, Qwen3TtsCodecModelV1* model, bool shared_session,
                       Qwen3TtsCodecContextV1** output, char* error, size_t capacity) {
    int count = 0;
    hipError_t st = hipGetDeviceCount(&count);
    if (st != hipSuccess) return hip_error(error, capacity, "query HIP devices", st);
    if (device >= count) {
        write_error(error, capacity, "HIP device index is out of range");
        return kInvalid;
    }
    st = hipSetDevice(device);
    if (st != hipSuccess) return hip_error(error, capacity, "select HIP device", st);
    auto* s = new (std::nothrow) Qwen3TtsCodecContextV1{};
    if (!s) {
        write_error(error, capacity, "allocate codec context");
        return kAlloc;
    }
    s->device = device;
    if (model) {
        retain(model);
        s->model = model;
    } else {
        s->model = new (std::nothrow) Qwen3TtsCodecModelV1{};
        if (!s->model) {
            delete s;
            write_error(error, capacity, "allocate codec model");
            return kAlloc;
        }
        s->model->device = device;
    }
    s->counts_as_shared_session = shared_session;
    if (shared_session) model->active_sessions.fetch_add(1, std::memory_order_acq_rel);
    const char* graphs = std::getenv("QWEN3_TTS_CODEC_GRAPH");
    s->use_graphs = !(graphs && graphs[0] == '0');
    hipDeviceProp_t prop{};
    if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
        s->cus = prop.multiProcessorCount;
    st = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (st == hipSuccess) st = hipEventCreate(&s->start_event);
    if (st == hipSuccess) st = hipEventCreate(&s->stop_event);
    if (st == hipSuccess) st = hipEventCreateWithFlags(&s->consumed_event, hipEventDisableTiming);
    if (st != hipSuccess) {
        release_context(s);
        return hip_error(error, capacity, "create decoder stream and events", st);
    }
    Arena sizing;
    layout_session(s, sizing);
    s->arena_bytes = sizing.used;
    if (hipMalloc(&s->arena, s->arena_bytes) != hipSuccess ||
        hipHostMalloc(reinterpret_cast<void**>(&s->host_pcm), (size_t)kRingSlots * kMaxSamples * sizeof(int16_t),
                      hipHostMallocDefault) != hipSuccess) {
        release_context(s);
        write_error(error, capacity, "allocate decoder session memory");
        return kAlloc;
    }
    Arena real{static_cast<char*>(s->arena), 0};
    layout_session(s, real);
    st = hipMemsetAsync(s->arena, 0, s->arena_bytes, s->stream);
    if (st == hipSuccess) st = upload_segments(s);
    if (st == hipSuccess) st = reset_device_state(s);
    if (st != hipSuccess) {
        release_context(s);
        return hip_error(error, capacity, "initialise decoder session", st);
    }
    *output = s;
    return kOk;
}

int32_t reset_context(Qwen3TtsCodecContextV1* s, char* error, size_t capacity) {
    hipError_t st = hipSetDevice(s->device);
    if (st == hipSuccess) st = hipStreamSynchronize(s->stream);
    if (st == hipSuccess) st = reset_device_state(s);
    if (st != hipSuccess) return hip_error(error, capacity, "reset decoder state", st);
    s->frame_position = s->emitted_samples = s->neural_frame_position = 0;
    s->next_ring_slot = s->kv_ring_head = 0;
    s->finalized = s->cancelled = s->device_packet_pending = false;
    s->pending_ticket = 0;
    s->pending_frames = s->pending_slot = 0;
    return kOk;
}

uint64_t session_device_bytes(const Qwen3TtsCodecContextV1* s) { return s->arena_bytes; }

// runs a debug prefix of the pipeline eagerly and waits for it
int32_t run_debug_prefix(Qwen3TtsCodecContextV1* s, const uint16_t* codes, uint32_t frames, int stop, char* error,
                         size_t capacity) {
    if (s->model->info.loaded == 0) {
        write_error(error, capacity, "decoder model is not loaded");
        return kState;
    }
    if (s->device_packet_pending) {
        write_error(error, capacity, "a device packet ticket is already pending");
        return kState;
    }
    if (!host_codes_valid(codes, frames)) {
        write_error(error, capacity, "codec codes must be below 2048");
        return kInvalid;
    }
    hipError_t st = hipSetDevice(s->device);
    if (st == hipSuccess)
        st = hipMemcpyAsync(s->codes_in, codes, (size_t)frames * kCodebooks * sizeof(uint16_t),
                            hipMemcpyHostToDevice, s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "upload frontend codes", st);
    Launcher l{s, s->model->w};
    l.packet((int)frames, stop);
    st = l.st;
    if (st == hipSuccess) st = hipStreamSynchronize(s->stream);
    if (st != hipSuccess) return hip_error(error, capacity, "run decoder stages", st);
    if (stop >= 2) {
        s->neural_frame_position += frames;
        s->kv_ring_head = (uint32_t)(s->neural_frame_position % kWindow);
    }
    return kOk;
}

int32_t copy_channel_major(Qwen3TtsCodecContextV1* s, const float* src, size_t positions, size_t channels,
                           float* out, char* error, size_t capacity) {
    std::vector<float> rows(positions * channels);
    hipError_t st = hipMemcpy(rows.data(), src, rows.size() * sizeof(float), hipMemcpyDeviceToHost);
    if (st != hipSuccess) return hip_error(error, capacity, "copy decoder checkpoint", st);
    for (size_t c = 0; c < channels; ++c)
        for (size_t p = 0; p < positions; ++p) out[c * positions + p] = rows[p * channels + c];
    return kOk;
}

}  // namespace

// ===========================================================================
// exported ABI
// ===========================================================================
extern "C" {

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_abi_version_v1(void) { return QWEN3_TTS_CODEC_ABI_VERSION_V1; }
QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_abi_version_v2(void) { return QWEN3_TTS_CODEC_ABI_VERSION_V2; }

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_create_v1(const Qwen3TtsCodecConfigV1* config,
                                                      Qwen3TtsCodecContextV1** output, char* error,
                                                      size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!config || !output) {
        write_error(error, error_capacity, "config and output are required");
        return kInvalid;
    }
    *output = nullptr;
    if (config->ring_slots != kRingSlots || config->max_packet_frames != kMaxFrames || config->reserved != 0 ||
        config->device_index < 0) {
        write_error(error, error_capacity,
                    "config must request device >= 0, three ring slots, four frames, and reserved=0");
        return kInvalid;
    }
    return create_context(config->device_index, nullptr, false, output, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_destroy_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                       size_t error_capacity) {
    clear_error(error, error_capacity);
    release_context(context);
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_reset_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                     size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context) {
        write_error(error, error_capacity, "context is required");
        return kInvalid;
    }
    return reset_context(context, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_state_info_v1(const Qwen3TtsCodecContextV1* context,
                                                          Qwen3TtsCodecStateInfoV1* output, char* error,
                                                          size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !output) {
        write_error(error, error_capacity, "context and output are required");
        return kInvalid;
    }
    const uint64_t pcm_ring = (uint64_t)kRingSlots * kMaxSamples * sizeof(int16_t);
    *output = Qwen3TtsCodecStateInfoV1{
        context->frame_position,
        context->emitted_samples,
        session_device_bytes(context) + context->model->info.device_bytes,
        pcm_ring,
        context->kv_bytes,
        context->history_bytes,
        (uint64_t)kRingSlots * kMaxFrames * kCodebooks * sizeof(uint16_t),
        pcm_ring,
        context->kv_ring_head,
        context->next_ring_slot,
        (uint32_t)kRingSlots,
        (uint32_t)kMaxFrames,
    };
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_load_model_v1(Qwen3TtsCodecContextV1* context,
                                                          const Qwen3TtsCodecWeightProviderV1* provider,
                                                          Qwen3TtsCodecModelInfoV1* output, char* error,
                                                          size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !provider || !output || !provider->tensor_at) {
        write_error(error, error_capacity, "context, weight provider, and output are required");
        return kInvalid;
    }
    if (provider->abi_version != QWEN3_TTS_CODEC_ABI_VERSION_V1) {
        write_error(error, error_capacity, "unsupported weight provider ABI version");
        return kInvalid;
    }
    Qwen3TtsCodecModelV1* m = context->model;
    if (m->info.loaded != 0 || !m->allocations.empty()) {
        write_error(error, error_capacity, "model is already loaded");
        return kState;
    }
    hipError_t st = hipSetDevice(context->device);
    if (st != hipSuccess) return hip_error(error, error_capacity, "select HIP device", st);
    Loader L{m, context->stream, {}, {}, {}};
    uint16_t* staging = nullptr;
    auto fail = [&](int32_t status) {
        if (staging) (void)hipFree(staging);
        (void)hipStreamSynchronize(context->stream);
        m->release_weights();
        return status;
    };
    Qwen3TtsCodecModelInfoV1 info{};
    for (uint64_t index = 0; index < provider->tensor_count; ++index) {
        const char* name = nullptr;
        Qwen3TtsCodecTensorViewV1 src{};
        if (provider->tensor_at(provider->user_data, index, &name, &src, error, error_capacity) != kOk) {
            if (!error || !error_capacity || error[0] == '\0')
                write_error(error, error_capacity, "weight provider rejected tensor index");
            return fail(kModel);
        }
        if (!name || std::strncmp(name, "decoder.", 8) != 0) continue;
        if (!src.data || src.byte_length == 0 || src.rank == 0 || src.rank > QWEN3_TTS_CODEC_MAX_TENSOR_RANK ||
            (src.dtype != QWEN3_TTS_CODEC_TENSOR_F32 && src.dtype != QWEN3_TTS_CODEC_TENSOR_BF16)) {
            write_error(error, error_capacity, "decoder tensor metadata is invalid");
            return fail(kModel);
        }
        uint64_t elements = 1;
        for (uint32_t d = 0; d < src.rank; ++d) {
            if (src.shape[d] == 0 || elements > UINT64_MAX / src.shape[d]) {
                write_error(error, error_capacity, "decoder tensor shape is invalid");
                return fail(kModel);
            }
            elements *= src.shape[d];
        }
        const uint64_t scalar = src.dtype == QWEN3_TTS_CODEC_TENSOR_F32 ? 4 : 2;
        if (elements > UINT64_MAX / scalar || elements * scalar != src.byte_length) {
            write_error(error, error_capacity, "decoder tensor byte length is invalid");
            return fail(kModel);
        }
        if (L.raw.count(name)) {
            write_error(error, error_capacity, "duplicate decoder tensor name");
            return fail(kModel);
        }
        float* dst = L.alloc(elements);
        if (!dst) {
            write_error(error, error_capacity, "allocate decoder tensor");
            return fail(kAlloc);
        }
        if (src.dtype == QWEN3_TTS_CODEC_TENSOR_F32) {
            st = hipMemcpyAsync(dst, src.data, src.byte_length, hipMemcpyHostToDevice, context->stream);
        } else {
            if (!staging && hipMalloc(reinterpret_cast<void**>(&staging), kStagingBytes) != hipSuccess) {
                write_error(error, error_capacity, "allocate bf16 upload staging");
                return fail(kAlloc);
            }
            const size_t chunk = kStagingBytes / sizeof(uint16_t);
            const auto* bytes = static_cast<const uint8_t*>(src.data);
            st = hipSuccess;
            for (uint64_t off = 0; st == hipSuccess && off < elements; off += chunk) {
                const size_t n = (size_t)std::min<uint64_t>(chunk, elements - off);
                // the staging buffer is reused: the previous chunk's widening must be done
                st = hipStreamSynchronize(context->stream);
                if (st == hipSuccess)
                    st = hipMemcpyAsync(staging, bytes + off * 2, n * 2, hipMemcpyHostToDevice, context->stream);
                if (st == hipSuccess) st = launch_bf16_to_f32(staging, n, dst + off, context->stream);
            }
        }
        if (st != hipSuccess) {
            hip_error(error, error_capacity, "upload decoder tensor", st);
            return fail(kDevice);
        }
        L.raw.emplace(name, dst);
        L.elements.emplace(name, elements);
        info.source_bytes += src.byte_length;
        info.device_bytes += elements * sizeof(float);
        info.parameter_count += elements;
        info.tensor_count += 1;
        if (src.dtype == QWEN3_TTS_CODEC_TENSOR_F32)
            info.source_dtype_f32_count += 1;
        else
            info.source_dtype_bf16_count += 1;
    }
    st = hipStreamSynchronize(context->stream);
    if (st != hipSuccess) {
        hip_error(error, error_capacity, "finish decoder upload", st);
        return fail(kDevice);
    }
    if (staging) {
        (void)hipFree(staging);
        staging = nullptr;
    }
    if (info.tensor_count != kExpectedTensors) {
        write_error(error, error_capacity, "model does not contain exactly 271 decoder tensors");
        return fail(kModel);
    }
    const char* anchors[] = {"decoder.quantizer.rvq_first.vq.layers.0._codebook.embedding_sum",
                             "decoder.pre_transformer.layers.0.self_attn.q_proj.weight",
                             "decoder.decoder.6.conv.weight"};
    for (const char* a : anchors) {
        if (!L.raw.count(a)) {
            write_error(error, error_capacity, "model is missing a required decoder tensor");
            return fail(kModel);
        }
    }
    // every executed tensor present with its element count (the kernels index by it)
    for (const TensorSpec& t : tensor_table()) {
        auto it = L.elements.find(t.name);
        if (it == L.elements.end()) {
            write_error(error, error_capacity, "model is missing decoder tensor %s", t.name.c_str());
            return fail(kModel);
        }
        if (it->second != t.elements) {
            write_error(error, error_capacity, "decoder tensor %s has %llu elements, expected %llu", t.name.c_str(),
                        (unsigned long long)it->second, (unsigned long long)t.elements);
            return fail(kModel);
        }
    }
    const int32_t built = build_weights(L, error, error_capacity);
    if (built != kOk) {
        if (built == kAlloc && error && error[0] == '\0') write_error(error, error_capacity, "allocate decoder weights");
        return fail(built);
    }
    info.loaded = 1;
    m->info = info;
    *output = info;
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_model_info_v1(const Qwen3TtsCodecContextV1* context,
                                                          Qwen3TtsCodecModelInfoV1* output, char* error,
                                                          size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !output) {
        write_error(error, error_capacity, "context and output are required");
        return kInvalid;
    }
    *output = context->model->info;
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_frontend_packet_v1(Qwen3TtsCodecContextV1* context,
                                                                     const uint16_t* codec_frames,
                                                                     uint32_t frame_count, float* rvq_output,
                                                                     size_t rvq_capacity, float* preconv_output,
                                                                     size_t preconv_capacity, char* error,
                                                                     size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !codec_frames || !rvq_output || !preconv_output) {
        write_error(error, error_capacity, "context, codes, and checkpoint outputs are required");
        return kInvalid;
    }
    if (frame_count == 0 || frame_count > kMaxFrames || rvq_capacity < (size_t)frame_count * 512 ||
        preconv_capacity < (size_t)frame_count * 1024) {
        write_error(error, error_capacity, "invalid frontend packet or output capacity");
        return kInvalid;
    }
    int32_t r = run_debug_prefix(context, codec_frames, frame_count, 1, error, error_capacity);
    if (r != kOk) return r;
    r = copy_channel_major(context, context->pre.ext + 2 * 512, frame_count, 512, rvq_output, error, error_capacity);
    if (r != kOk) return r;
    const hipError_t st = hipMemcpy(preconv_output, context->t_in, (size_t)frame_count * 1024 * sizeof(float),
                                    hipMemcpyDeviceToHost);
    return st == hipSuccess ? kOk : hip_error(error, error_capacity, "copy neural frontend checkpoints", st);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_transformer_packet_v1(Qwen3TtsCodecContextV1* context,
                                                                        const uint16_t* codec_frames,
                                                                        uint32_t frame_count,
                                                                        float* transformer_output,
                                                                        size_t transformer_capacity, char* error,
                                                                        size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !codec_frames || !transformer_output || frame_count == 0 || frame_count > kMaxFrames ||
        transformer_capacity < (size_t)frame_count * 1024) {
        write_error(error, error_capacity, "invalid transformer checkpoint packet");
        return kInvalid;
    }
    const int32_t r = run_debug_prefix(context, codec_frames, frame_count, 2, error, error_capacity);
    if (r != kOk) return r;
    const hipError_t st = hipMemcpy(transformer_output, context->t_out, (size_t)frame_count * 1024 * sizeof(float),
                                    hipMemcpyDeviceToHost);
    return st == hipSuccess ? kOk : hip_error(error, error_capacity, "copy transformer checkpoint", st);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_latent_packet_v1(Qwen3TtsCodecContextV1* context,
                                                                   const uint16_t* codec_frames,
                                                                   uint32_t frame_count, float* stage_one_output,
                                                                   size_t stage_one_capacity,
                                                                   float* stage_two_output,
                                                                   size_t stage_two_capacity, char* error,
                                                                   size_t error_capacity) {
    clear_error(error, error_capacity);
    const size_t one = (size_t)frame_count * 2, two = (size_t)frame_count * 4;
    if (!context || !codec_frames || !stage_one_output || !stage_two_output || frame_count == 0 ||
        frame_count > kMaxFrames || stage_one_capacity < one * 1024 || stage_two_capacity < two * 1024) {
        write_error(error, error_capacity, "invalid latent checkpoint packet");
        return kInvalid;
    }
    int32_t r = run_debug_prefix(context, codec_frames, frame_count, 3, error, error_capacity);
    if (r != kOk) return r;
    r = copy_channel_major(context, context->up1_out, one, 1024, stage_one_output, error, error_capacity);
    if (r != kOk) return r;
    return copy_channel_major(context, context->conv0.ext + 6 * 1024, two, 1024, stage_two_output, error,
                              error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_debug_decoder_checkpoint_v1(Qwen3TtsCodecContextV1* context,
                                                                        const uint16_t* codec_frames,
                                                                        uint32_t frame_count, uint32_t checkpoint,
                                                                        float* checkpoint_output,
                                                                        size_t checkpoint_capacity, char* error,
                                                                        size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !codec_frames || !checkpoint_output || frame_count == 0 || frame_count > kMaxFrames ||
        checkpoint < 6 || checkpoint > 13) {
        write_error(error, error_capacity, "invalid waveform decoder checkpoint request");
        return kInvalid;
    }
    const size_t latent = (size_t)frame_count * 4;
    const float* src;
    size_t positions, channels;
    if (checkpoint == 6) {
        src = context->conv0_raw, positions = latent, channels = 1536;
    } else if (checkpoint <= 10) {
        const int t = (int)checkpoint - 7;
        src = context->cur[t], positions = stage_input_positions(t, frame_count) * kStride[t],
        channels = kStageOut[t];
    } else if (checkpoint == 11) {
        src = context->final_conv.ext + 6 * 96, positions = (size_t)frame_count * kSamplesPerFrame, channels = 96;
    } else {
        src = checkpoint == 12 ? context->preclamp : context->clamped;
        positions = (size_t)frame_count * kSamplesPerFrame, channels = 1;
    }
    if (checkpoint_capacity < positions * channels) {
        // the reference reports this after running the packet (CS:2039-2042)
        const int32_t r = run_debug_prefix(context, codec_frames, frame_count, (int)checkpoint, error, error_capacity);
        if (r != kOk) return r;
        write_error(error, error_capacity, "decoder checkpoint capacity is too small");
        return kInvalid;
    }
    const int32_t r = run_debug_prefix(context, codec_frames, frame_count, (int)checkpoint, error, error_capacity);
    if (r != kOk) return r;
    return copy_channel_major(context, src, positions, channels, checkpoint_output, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_packet_v1(Qwen3TtsCodecContextV1* context,
                                                              const uint16_t* codec_frames, uint32_t frame_count,
                                                              int32_t is_final, int16_t* pcm_output,
                                                              size_t pcm_capacity_samples,
                                                              Qwen3TtsCodecPacketResultV1* result, char* error,
                                                              size_t error_capacity) {
    clear_error(error, error_capacity);
    int32_t r = check_packet_args(context, codec_frames, frame_count, is_final, pcm_output, pcm_capacity_samples,
                                  result, error, error_capacity);
    if (r != kOk) return r;
    const auto start = std::chrono::steady_clock::now();
    uint32_t slot = 0;
    r = begin_host_packet(context, codec_frames, frame_count, &slot, error, error_capacity);
    if (r != kOk) return r;
    return finish_staged_packet(context, slot, frame_count, is_final, pcm_output, result, start, error,
                                error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_warmup_v1(Qwen3TtsCodecContextV1* context, char* error,
                                                      size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context) {
        write_error(error, error_capacity, "context is required");
        return kInvalid;
    }
    if (context->model->info.loaded == 0) {
        write_error(error, error_capacity, "decoder model is not loaded");
        return kState;
    }
    if (context->frame_position != 0 || context->neural_frame_position != 0 || context->emitted_samples != 0 ||
        context->next_ring_slot != 0 || context->finalized || context->device_packet_pending) {
        write_error(error, error_capacity, "warmup requires a fresh decoder state");
        return kState;
    }
    uint16_t codes[kMaxFrames * kCodebooks] = {};
    std::vector<int16_t> pcm(kMaxSamples);
    Qwen3TtsCodecPacketResultV1 result{};
    const int32_t r = qwen3_tts_codec_process_packet_v1(context, codes, kMaxFrames, 0, pcm.data(), kMaxSamples,
                                                        &result, error, error_capacity);
    const int32_t reset = reset_context(context, r == kOk ? error : nullptr, r == kOk ? error_capacity : 0);
    return r == kOk ? reset : r;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_batch_v1(Qwen3TtsCodecBatchItemV1* items, uint32_t item_count,
                                                             char* error, size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!items || item_count == 0 || item_count > QWEN3_TTS_CODEC_MAX_BATCH_STREAMS) {
        write_error(error, error_capacity, "batch must contain 1-6 stream items");
        return kInvalid;
    }
    for (uint32_t i = 0; i < item_count; ++i) {
        if (!items[i].context) {
            write_error(error, error_capacity, "batch item context is required");
            return kInvalid;
        }
        for (uint32_t j = 0; j < i; ++j) {
            if (items[i].context == items[j].context) {
                write_error(error, error_capacity, "batch state handles must be independent");
                return kInvalid;
            }
        }
    }
    // Every stream's packet is queued on its own HIP stream before any is
    // waited for, so the streams decode concurrently; items complete in
    // order and the first failure ends the batch (earlier items are done).
    // Results are cleared first: after a failed batch, an item whose packet
    // completed (and advanced its stream) is the one whose result has a
    // nonzero frame_count.
    for (uint32_t i = 0; i < item_count; ++i)
        if (items[i].result) *items[i].result = Qwen3TtsCodecPacketResultV1{};
    const auto start = std::chrono::steady_clock::now();
    uint32_t slots[QWEN3_TTS_CODEC_MAX_BATCH_STREAMS] = {};
    uint32_t queued = 0;
    int32_t status = kOk;
    for (; queued < item_count; ++queued) {
        Qwen3TtsCodecBatchItemV1& it = items[queued];
        status = check_packet_args(it.context, it.codec_frames, it.frame_count, it.is_final, it.pcm_output,
                                   it.pcm_capacity_samples, it.result, error, error_capacity);
        if (status == kOk)
            status = begin_host_packet(it.context, it.codec_frames, it.frame_count, &slots[queued], error,
                                       error_capacity);
        if (status != kOk) break;
    }
    for (uint32_t i = 0; i < queued; ++i) {
        Qwen3TtsCodecBatchItemV1& it = items[i];
        char* e = status == kOk ? error : nullptr;
        const int32_t r = finish_staged_packet(it.context, slots[i], it.frame_count, it.is_final, it.pcm_output,
                                               it.result, start, e, e ? error_capacity : 0);
        if (status == kOk && r != kOk) status = r;
    }
    return status;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_process_fixture_packet_v1(Qwen3TtsCodecContextV1* context,
                                                                      const uint16_t* codec_frames,
                                                                      uint32_t frame_count, int32_t is_final,
                                                                      int16_t* pcm_output,
                                                                      size_t pcm_capacity_samples,
                                                                      Qwen3TtsCodecPacketResultV1* result,
                                                                      char* error, size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!context || !codec_frames || !pcm_output || !result) {
        write_error(error, error_capacity, "context, codec frames, PCM output, and result are required");
        return kInvalid;
    }
    if (frame_count == 0 || frame_count > QWEN3_TTS_CODEC_MAX_PACKET_FRAMES || (is_final != 0 && is_final != 1)) {
        write_error(error, error_capacity, "packet must contain 1-4 frames");
        return kInvalid;
    }
    const size_t samples = (size_t)frame_count * kSamplesPerFrame;
    if (pcm_capacity_samples < samples) {
        write_error(error, error_capacity, "PCM output capacity is too small");
        return kInvalid;
    }
    if (context->finalized || context->device_packet_pending) {
        write_error(error, error_capacity, "stream is finalized; reset is required");
        return kState;
    }
    hipError_t st = hipSetDevice(context->device);
    if (st != hipSuccess) return hip_error(error, error_capacity, "select HIP device", st);
    const auto start = std::chrono::steady_clock::now();
    const uint32_t slot = context->next_ring_slot;
    uint16_t* codes = context->code_ring + (size_t)slot * kMaxFrames * kCodebooks;
    int16_t* dev_pcm = context->pcm_ring + (size_t)slot * kMaxSamples;
    int16_t* host_pcm = context->host_pcm + (size_t)slot * kMaxSamples;
    st = hipEventRecord(context->start_event, context->stream);
    if (st == hipSuccess)
        st = hipMemcpyAsync(codes, codec_frames, (size_t)frame_count * kCodebooks * sizeof(uint16_t),
                            hipMemcpyHostToDevice, context->stream);
    if (st != hipSuccess) return hip_error(error, error_capacity, "queue codec copy", st);
    st = launch_fixture_packet(codes, (int)frame_count, context->fixture_state, dev_pcm, context->stream);
    if (st != hipSuccess) return hip_error(error, error_capacity, "launch fixture packet", st);
    st = hipMemcpyAsync(host_pcm, dev_pcm, samples * sizeof(int16_t), hipMemcpyDeviceToHost, context->stream);
    if (st == hipSuccess) st = hipEventRecord(context->stop_event, context->stream);
    if (st == hipSuccess) st = hipEventSynchronize(context->stop_event);
    if (st != hipSuccess) return hip_error(error, error_capacity, "complete fixture packet", st);
    float ms = 0.f;
    st = hipEventElapsedTime(&ms, context->start_event, context->stop_event);
    if (st != hipSuccess) return hip_error(error, error_capacity, "measure packet GPU time", st);
    std::memcpy(pcm_output, host_pcm, samples * sizeof(int16_t));
    const uint64_t first_frame = context->frame_position, first_sample = context->emitted_samples;
    context->frame_position += frame_count;
    context->emitted_samples += samples;
    context->kv_ring_head = (uint32_t)(context->frame_position % kWindow);
    context->next_ring_slot = (context->next_ring_slot + 1) % kRingSlots;
    context->finalized = is_final != 0;
    const float e2e = std::chrono::duration<float, std::micro>(std::chrono::steady_clock::now() - start).count();
    *result = Qwen3TtsCodecPacketResultV1{first_frame, first_sample, frame_count, (uint32_t)samples,
                                          slot,        (uint32_t)is_final, ms * 1000.f, e2e};
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_create_v1(int32_t device_index,
                                                                   Qwen3TtsCodecModelV1** output, char* error,
                                                                   size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!output || device_index < 0) {
        write_error(error, error_capacity, "non-negative device index and output are required");
        return kInvalid;
    }
    *output = nullptr;
    int count = 0;
    hipError_t st = hipGetDeviceCount(&count);
    if (st != hipSuccess) return hip_error(error, error_capacity, "query HIP devices", st);
    if (device_index >= count) {
        write_error(error, error_capacity, "HIP device index is out of range");
        return kInvalid;
    }
    auto* m = new (std::nothrow) Qwen3TtsCodecModelV1{};
    if (!m) {
        write_error(error, error_capacity, "allocate shared codec model");
        return kAlloc;
    }
    m->device = device_index;
    *output = m;
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_destroy_v1(Qwen3TtsCodecModelV1* model, char* error,
                                                                    size_t error_capacity) {
    clear_error(error, error_capacity);
    release(model);
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_load_v1(Qwen3TtsCodecModelV1* model,
                                                                 const Qwen3TtsCodecWeightProviderV1* provider,
                                                                 Qwen3TtsCodecModelInfoV1* output, char* error,
                                                                 size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!model || !provider || !output) {
        write_error(error, error_capacity, "model, weight provider, and output are required");
        return kInvalid;
    }
    std::lock_guard<std::mutex> guard(model->lifecycle);
    if (model->active_sessions.load(std::memory_order_acquire) != 0) {
        write_error(error, error_capacity, "cannot load a model with active sessions");
        return kState;
    }
    if (model->info.loaded != 0 || !model->allocations.empty()) {
        write_error(error, error_capacity, "model is already loaded");
        return kState;
    }
    Qwen3TtsCodecContextV1* loader = nullptr;
    int32_t r = create_context(model->device, model, false, &loader, error, error_capacity);
    if (r == kOk) r = qwen3_tts_codec_load_model_v1(loader, provider, output, error, error_capacity);
    release_context(loader);
    return r;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_warmup_v1(Qwen3TtsCodecModelV1* model, char* error,
                                                                   size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!model) {
        write_error(error, error_capacity, "model is required");
        return kInvalid;
    }
    std::lock_guard<std::mutex> guard(model->lifecycle);
    if (model->info.loaded == 0) {
        write_error(error, error_capacity, "decoder model is not loaded");
        return kState;
    }
    if (model->warmed.load(std::memory_order_acquire)) return kOk;
    if (model->active_sessions.load(std::memory_order_acquire) != 0) {
        write_error(error, error_capacity, "warmup must finish before sessions are created");
        return kState;
    }
    Qwen3TtsCodecContextV1* warm = nullptr;
    int32_t r = create_context(model->device, model, false, &warm, error, error_capacity);
    if (r == kOk) r = qwen3_tts_codec_warmup_v1(warm, error, error_capacity);
    release_context(warm);
    if (r == kOk) model->warmed.store(true, std::memory_order_release);
    return r;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_info_v1(const Qwen3TtsCodecModelV1* model,
                                                                 Qwen3TtsCodecModelInfoV1* output, char* error,
                                                                 size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!model || !output) {
        write_error(error, error_capacity, "model and output are required");
        return kInvalid;
    }
    *output = model->info;
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_shared_model_memory_info_v1(const Qwen3TtsCodecModelV1* model,
                                                                        Qwen3TtsCodecModelMemoryInfoV1* output,
                                                                        char* error, size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!model || !output) {
        write_error(error, error_capacity, "model and memory output are required");
        return kInvalid;
    }
    *output = Qwen3TtsCodecModelMemoryInfoV1{
        model->info.source_bytes,
        model->info.device_bytes,
        model->info.parameter_count,
        kStagingBytes,
        model->info.tensor_count,
        (uint32_t)model->warmed.load(std::memory_order_acquire),
        model->active_sessions.load(std::memory_order_acquire),
        0,
    };
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_create_v1(Qwen3TtsCodecModelV1* model,
                                                              Qwen3TtsCodecSessionV1** output, char* error,
                                                              size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!model || !output) {
        write_error(error, error_capacity, "model and session output are required");
        return kInvalid;
    }
    std::lock_guard<std::mutex> guard(model->lifecycle);
    if (model->info.loaded == 0 || !model->warmed.load(std::memory_order_acquire)) {
        write_error(error, error_capacity, "model must be loaded and warmed before session start");
        return kState;
    }
    return create_context(model->device, model, true, output, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_destroy_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                               size_t error_capacity) {
    return qwen3_tts_codec_destroy_v1(session, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_reset_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                             size_t error_capacity) {
    return qwen3_tts_codec_reset_v1(session, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_cancel_v1(Qwen3TtsCodecSessionV1* session, char* error,
                                                              size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!session) {
        write_error(error, error_capacity, "session is required");
        return kInvalid;
    }
    hipError_t st = hipSetDevice(session->device);
    if (st == hipSuccess) st = hipStreamSynchronize(session->stream);
    if (st != hipSuccess) return hip_error(error, error_capacity, "cancel decoder session", st);
    session->pending_ticket = 0;
    session->pending_frames = session->pending_slot = 0;
    session->device_packet_pending = false;
    session->cancelled = true;
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_state_info_v1(const Qwen3TtsCodecSessionV1* session,
                                                                  Qwen3TtsCodecStateInfoV1* output, char* error,
                                                                  size_t error_capacity) {
    const int32_t r = qwen3_tts_codec_state_info_v1(session, output, error, error_capacity);
    if (r == kOk) output->device_bytes = session_device_bytes(session);
    return r;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_memory_info_v1(const Qwen3TtsCodecSessionV1* session,
                                                                   Qwen3TtsCodecSessionMemoryInfoV1* output,
                                                                   char* error, size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!session || !output) {
        write_error(error, error_capacity, "session and memory output are required");
        return kInvalid;
    }
    const uint64_t codes = (uint64_t)kRingSlots * kMaxFrames * kCodebooks * sizeof(uint16_t);
    const uint64_t pcm = (uint64_t)kRingSlots * kMaxSamples * sizeof(int16_t);
    const uint64_t total = session_device_bytes(session);
    *output = Qwen3TtsCodecSessionMemoryInfoV1{
        total, pcm, session->kv_bytes, session->history_bytes, codes, pcm,
        total - session->kv_bytes - session->history_bytes - codes - pcm, 0,
    };
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_packet_v1(Qwen3TtsCodecSessionV1* session,
                                                                      const uint16_t* codec_frames,
                                                                      uint32_t frame_count, int32_t is_final,
                                                                      int16_t* pcm_output,
                                                                      size_t pcm_capacity_samples,
                                                                      Qwen3TtsCodecPacketResultV1* result,
                                                                      char* error, size_t error_capacity) {
    return qwen3_tts_codec_process_packet_v1(session, codec_frames, frame_count, is_final, pcm_output,
                                             pcm_capacity_samples, result, error, error_capacity);
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_device_packet_begin_v2(
    Qwen3TtsCodecSessionV1* session, const Qwen3TtsCodecDevicePacketBeginV2* request,
    Qwen3TtsCodecDevicePacketBeginResultV2* output, char* error, size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!session || !request || !output) {
        write_error(error, error_capacity, "session, begin request, and output are required");
        return kInvalid;
    }
    if (request->struct_size != sizeof(Qwen3TtsCodecDevicePacketBeginV2) || request->reserved != 0 ||
        request->reserved_2 != 0 || request->reserved_3 != 0 ||
        output->struct_size != sizeof(Qwen3TtsCodecDevicePacketBeginResultV2) || output->reserved != 0 ||
        output->reserved_2 != 0) {
        write_error(error, error_capacity, "device begin structs must have exact struct_size and zero reserved fields");
        return kInvalid;
    }
    output->ticket_id = 0;
    output->codes_consumed_event = nullptr;
    if (!request->device_codec_frames || !request->producer_ready_event) {
        write_error(error, error_capacity, "device codes and producer event are required");
        return kInvalid;
    }
    int32_t r = validate_packet_state(session, request->frame_count, error, error_capacity);
    if (r != kOk) return r;
    if (session->next_ticket == UINT64_MAX) {
        write_error(error, error_capacity, "device packet ticket space is exhausted");
        return kState;
    }
    hipError_t st = hipSetDevice(session->device);
    if (st != hipSuccess) return hip_error(error, error_capacity, "select HIP device", st);
    hipPointerAttribute_t attr{};
    st = hipPointerGetAttributes(&attr, request->device_codec_frames);
    if (st != hipSuccess) return hip_error(error, error_capacity, "inspect device codec pointer", st);
    if (attr.type != hipMemoryTypeDevice || attr.device != session->device) {
        write_error(error, error_capacity, "codec pointer must be device memory on the session HIP device");
        return kInvalid;
    }
    const auto start = std::chrono::steady_clock::now();
    const uint32_t slot = session->next_ring_slot;
    uint16_t* staged = session->code_ring + (size_t)slot * kMaxFrames * kCodebooks;
    st = hipStreamWaitEvent(session->stream, reinterpret_cast<hipEvent_t>(request->producer_ready_event), 0);
    if (st == hipSuccess) st = hipEventRecord(session->start_event, session->stream);
    if (st == hipSuccess)
        st = hipMemcpyAsync(staged, request->device_codec_frames,
                            (size_t)request->frame_count * kCodebooks * sizeof(uint16_t), hipMemcpyDeviceToDevice,
                            session->stream);
    if (st == hipSuccess) st = hipEventRecord(session->consumed_event, session->stream);
    if (st != hipSuccess) {
        const int32_t failure = hip_error(error, error_capacity, "queue device codec snapshot", st);
        (void)hipStreamSynchronize(session->stream);
        session->cancelled = true;
        return failure;
    }
    r = enqueue_staged_packet(session, request->frame_count, slot, error, error_capacity);
    if (r != kOk) {
        (void)hipStreamSynchronize(session->stream);
        session->cancelled = true;
        return r;
    }
    const uint64_t ticket = session->next_ticket++;
    session->pending_ticket = ticket;
    session->pending_frames = request->frame_count;
    session->pending_slot = slot;
    session->pending_start = start;
    session->device_packet_pending = true;
    output->ticket_id = ticket;
    output->codes_consumed_event = reinterpret_cast<void*>(session->consumed_event);
    return kOk;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_device_packet_finish_v2(
    Qwen3TtsCodecSessionV1* session, const Qwen3TtsCodecDevicePacketFinishV2* request, char* error,
    size_t error_capacity) {
    clear_error(error, error_capacity);
    if (!session || !request) {
        write_error(error, error_capacity, "session and finish request are required");
        return kInvalid;
    }
    if (request->struct_size != sizeof(Qwen3TtsCodecDevicePacketFinishV2) || request->reserved != 0 ||
        request->reserved_2 != 0 || request->reserved_3 != 0) {
        write_error(error, error_capacity, "device finish struct must have exact struct_size and zero reserved fields");
        return kInvalid;
    }
    if (request->is_final != 0 && request->is_final != 1) {
        write_error(error, error_capacity, "is_final must be zero or one");
        return kInvalid;
    }
    if (!request->pcm_output || !request->result) {
        write_error(error, error_capacity, "PCM output and packet result are required");
        return kInvalid;
    }
    if (!session->device_packet_pending || request->ticket_id != session->pending_ticket) {
        write_error(error, error_capacity, "device packet ticket is stale or does not match");
        return kState;
    }
    if (request->pcm_capacity_samples < (size_t)session->pending_frames * kSamplesPerFrame) {
        write_error(error, error_capacity, "PCM output capacity is too small");
        return kInvalid;
    }
    hipError_t st = hipSetDevice(session->device);
    if (st != hipSuccess) return hip_error(error, error_capacity, "select HIP device", st);
    const int32_t r = finish_staged_packet(session, session->pending_slot, session->pending_frames,
                                           request->is_final, request->pcm_output, request->result,
                                           session->pending_start, error, error_capacity);
    session->pending_ticket = 0;
    session->pending_frames = session->pending_slot = 0;
    session->device_packet_pending = false;
    if (r != kOk) session->cancelled = true;
    return r;
}

QWEN3_TTS_CODEC_API int32_t qwen3_tts_codec_session_process_batch_v1(Qwen3TtsCodecSessionBatchItemV1* items,
                                                                     uint32_t item_count, char* error,
                                                                     size_t error_capacity) {
    static_assert(sizeof(Qwen3TtsCodecSessionBatchItemV1) == sizeof(Qwen3TtsCodecBatchItemV1), "same layout");
    return qwen3_tts_codec_process_batch_v1(reinterpret_cast<Qwen3TtsCodecBatchItemV1*>(items), item_count, error,
                                            error_capacity);
}

}  // extern "C"
