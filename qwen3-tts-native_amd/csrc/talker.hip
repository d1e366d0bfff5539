// Talker / code-predictor orchestration behind the reference C ABI, gfx950.
//
// Mirrors native/qwen3-tts-native/native/src/talker.cu:
//   TalkerModel (:413-788)  -> q3::Model: bf16 tensor registry with the same
//     names and shape contract, int8 quantization of every decode matrix at
//     finalize, shared and immutable afterwards.
//   TalkerContext (:790-3768) -> q3::Session: per-session KV caches, sampler
//     state, lease protocol, events and one host sync per frame.
//   C ABI (:3815-4087) -> extern "C" functions at the end of this file.
//
// MI355X design (this build's own):
//   * Each decode matrix is quantized into one int8 arena laid out in
//     execution order; q/k/v are stored as one fused [q+2kv][hidden] matrix
//     (per-row quantization makes it identical to three separate ones) and
//     gate/up as one [2I][hidden] matrix, gate rows first.
//   * A decoder layer is 6 launches: QKV GEMV with the input RMSNorm fused as
//     its prologue; one wave per head for q/k RMSNorm + RoPE + KV append;
//     attention; O GEMV with the residual add fused; gate/up GEMV with the
//     post-attention RMSNorm and SiLU-gate fused; down GEMV with the residual
//     add fused.  The reference issues ~19 launches per layer.
//   * Every value that changes between frames (talker position, frame tokens,
//     trailing text token, history count, RNG state) lives in device memory,
//     so the predictor (16 positions) and the talker step are each captured
//     once into a hipGraph and replayed every frame.
//   * Embedding gathers are folded into the consuming GEMV (the GEMV reads
//     its activation row straight from the table through a device-side token).
#include "q3_common.hpp"

#include "../../include/qwen3_tts_native.h"

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <memory>
#include <mutex>
#include <new>
#include <string>
#include <unordered_map>
#include <utility>
#include <vector>

namespace q3 {
namespace {

constexpr int kCodebooks = 16;
constexpr int kResidualCodebooks = 15;
constexpr int kMaxBatch = QWEN3_TTS_MAX_BATCH_SESSIONS;
constexpr int kAttentionCapacity = 8192;  // largest session max_sequence_length
// MFMA (tolerance) batch mode: each talker row's value chains run as this many
// position segments, for more workgroups on long caches (the exact mode keeps
// the reference's one chain)
constexpr int kAttentionSplits = 2;

void write_error(char* destination, size_t capacity, const char* message) {
    if (destination != nullptr && capacity != 0) {
        std::snprintf(destination, capacity, "%s", message);
    }
}

class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) : bytes_(bytes) {
        if (bytes != 0) check_hip(hipMalloc(&pointer_, bytes), "hipMalloc");
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer(DeviceBuffer&& o) noexcept
        : pointer_(std::exchange(o.pointer_, nullptr)), bytes_(std::exchange(o.bytes_, 0)) {}
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            if (pointer_) (void)hipFree(pointer_);
            pointer_ = std::exchange(o.pointer_, nullptr);
            bytes_ = std::exchange(o.bytes_, 0);
        }
        return *this;
    }
    ~DeviceBuffer() {
        if (pointer_) (void)hipFree(pointer_);
    }
    template <typename T>
    T* as() const {
        return static_cast<T*>(pointer_);
    }
    size_t bytes() const { return bytes_; }

private:
    void* pointer_ = nullptr;
    size_t bytes_ = 0;
};

struct Dims {
    int hidden, intermediate, query_heads, key_value_heads, head_dimension, layers;
    int query_width() const { return query_heads * head_dimension; }
    int kv_width() const { return key_value_heads * head_dimension; }
    int qkv_width() const { return query_width() + 2 * kv_width(); }
};

struct Config {
    Dims talker, predictor;
    int talker_vocab, predictor_vocab, text_vocab, codec_eos;
    float eps, theta;
};

Config config_from(const Qwen3TtsModelConfigV1& c) {
    Config r{};
    r.talker = {c.talker_hidden, c.talker_intermediate, c.talker_query_heads,
                c.talker_key_value_heads, c.head_dimension, c.talker_layers};
    r.predictor = {c.predictor_hidden, c.predictor_intermediate, c.predictor_query_heads,
                   c.predictor_key_value_heads, c.head_dimension, c.predictor_layers};
    r.talker_vocab = c.talker_vocabulary;
    r.predictor_vocab = c.predictor_vocabulary;
    r.text_vocab = c.text_vocabulary;
    r.codec_eos = c.codec_eos_token;
    r.eps = c.rms_epsilon;
    r.theta = c.rope_theta;
    return r;
}

void validate_config(const Config& c) {
    for (const Dims* d : {&c.talker, &c.predictor}) {
        if (d->layers <= 0 || d->hidden <= 0 || d->intermediate <= 0 || d->query_heads <= 0 ||
            d->key_value_heads <= 0 || d->head_dimension != 128 ||
            d->query_heads % d->key_value_heads != 0 || d->hidden % 256 != 0 ||
            d->intermediate % 256 != 0) {
            throw std::invalid_argument(
                "model geometry must have head_dimension 128, hidden and intermediate multiples of "
                "256, and query heads divisible by key/value heads");
        }
    }
    if (c.talker_vocab <= 0 || c.talker_vocab > 4096 || c.predictor_vocab <= 0 ||
        c.predictor_vocab > 4096 || c.text_vocab <= 0 || c.codec_eos < 0 ||
        c.codec_eos >= c.talker_vocab) {
        throw std::invalid_argument("model vocabulary sizes are out of range");
    }
}

struct QTensor {
    const int8_t* data = nullptr;
    const float* scales = nullptr;
};

struct Layer {
    const bf16_t* input_norm = nullptr;
    const bf16_t* post_norm = nullptr;
    const bf16_t* q_norm = nullptr;
    const bf16_t* k_norm = nullptr;
    QTensor qkv, o, gate_up, down;
    // bf16 weights ([out][in], as uploaded): the prompt prefill's GEMMs
    const bf16_t *q16 = nullptr, *k16 = nullptr, *v16 = nullptr, *o16 = nullptr;
    const bf16_t *gate16 = nullptr, *up16 = nullptr, *down16 = nullptr;
};

struct DeviceTensor {
    DeviceBuffer storage;
    std::vector<uint64_t> shape;
};

// Host-side RoPE table with the reference's float formula
// (talker_kernels.cu:93-97): angle = float(pos) * powf(theta, -(2d/D)),
// cos/sin rounded to bf16.  Layout [positions][D/2][2].
void build_rope_table(int positions, int head_dimension, float theta, bf16_t* out) {
    const int half = head_dimension / 2;
    for (int p = 0; p < positions; ++p) {
        for (int d = 0; d < half; ++d) {
            const float exponent = static_cast<float>(2 * d) / static_cast<float>(head_dimension);
            const float angle = static_cast<float>(p) * powf(theta, -exponent);
            out[(static_cast<size_t>(p) * half + d) * 2] = f2bf(cosf(angle));
            out[(static_cast<size_t>(p) * half + d) * 2 + 1] = f2bf(sinf(angle));
        }
    }
}

constexpr int kRopePositions = 8192;

bool int8_decode_enabled() {
    const char* value = std::getenv("QWEN3_TTS_INT8_DECODE");
    if (value == nullptr) return true;
    return !(std::strcmp(value, "0") == 0 || std::strcmp(value, "false") == 0);
}

// GEMV mode of the lockstep batch: the exact reference order (VALU) on
// request, otherwise exact for one row and the MFMA skinny GEMM for 2..8.
int batch_gemv_mode() {
    const char* value = std::getenv("QWEN3_TTS_BATCH_GEMV");
    if (value != nullptr && std::strcmp(value, "exact") == 0) return kModeExact;
    return kModeAuto;
}

class Session;
class BatchRunner;

// ---------------------------------------------------------------------------
// Model
// ---------------------------------------------------------------------------
class Model {
public:
    Model(int device_index, const Config& config) : device_(device_index), cfg_(config) {
        validate_config(cfg_);
        check_hip(hipSetDevice(device_), "hipSetDevice(model)");
        check_hip(hipStreamCreateWithFlags(&upload_stream_, hipStreamNonBlocking),
                  "hipStreamCreateWithFlags(model upload)");
    }
    ~Model() {
        (void)hipSetDevice(device_);
        if (upload_stream_) {
            (void)hipStreamSynchronize(upload_stream_);
            (void)hipStreamDestroy(upload_stream_);
        }
    }
    Model(const Model&) = delete;
    Model& operator=(const Model&) = delete;

    // talker.cu:434-482
    void upload_tensor(const char* name, const void* data, uint64_t byte_size, int rank,
                       const uint64_t* shape) {
        if (finalized_) throw std::runtime_error("model weights are already finalized");
        if (name == nullptr || *name == '\0' || data == nullptr || shape == nullptr) {
            throw std::runtime_error("tensor upload received a null argument");
        }
        if (rank <= 0 || rank > 4 || byte_size == 0) {
            throw std::runtime_error("tensor upload has an invalid rank or byte size");
        }
        uint64_t elements = 1;
        std::vector<uint64_t> dims;
        for (int i = 0; i < rank; ++i) {
            if (shape[i] == 0 || elements > std::numeric_limits<uint64_t>::max() / shape[i]) {
                throw std::runtime_error("tensor shape is empty or overflows");
            }
            elements *= shape[i];
            dims.push_back(shape[i]);
        }
        if (elements > std::numeric_limits<uint64_t>::max() / 2 || elements * 2 != byte_size) {
            throw std::runtime_error("tensor byte size does not match BF16 shape");
        }
        const std::string key(name);
        if (tensors_.count(key) != 0) throw std::runtime_error("duplicate tensor upload: " + key);
        check_hip(hipSetDevice(device_), "hipSetDevice(upload)");
        DeviceTensor tensor{DeviceBuffer(static_cast<size_t>(byte_size)), std::move(dims)};
        // hipMemcpyDefault: the source may be host or device memory.
        check_hip(hipMemcpyAsync(tensor.storage.as<void>(), data, static_cast<size_t>(byte_size),
                                 hipMemcpyDefault, upload_stream_),
                  "hipMemcpyAsync(model weight)");
        // Host sources must stay valid until the copy completes.
        check_hip(hipStreamSynchronize(upload_stream_), "hipStreamSynchronize(upload)");
        weight_bytes_ += byte_size;
        tensors_.emplace(key, std::move(tensor));
    }

    size_t expected_tensor_count() const {
        return 8 + 11 * static_cast<size_t>(cfg_.talker.layers) + 3 +
               11 * static_cast<size_t>(cfg_.predictor.layers) + 2 * kResidualCodebooks;
    }

    // talker.cu:484-680
    Qwen3TtsModelMemory finalize() {
        if (finalized_) throw std::runtime_error("model weights are already finalized");
        if (tensors_.size() != expected_tensor_count()) {
            throw std::runtime_error("expected exactly " + std::to_string(expected_tensor_count()) +
                                     " VoiceDesign tensors, found " +
                                     std::to_string(tensors_.size()));
        }
        if (!int8_decode_enabled()) {
            throw std::runtime_error(
                "QWEN3_TTS_INT8_DECODE is disabled, but this library implements only the int8 "
                "weight-only decode path");
        }
        check_hip(hipSetDevice(device_), "hipSetDevice(finalize)");
        const Dims& T = cfg_.talker;
        const Dims& P = cfg_.predictor;
        const uint64_t H = T.hidden;
        codec_embedding_ = require("talker.model.codec_embedding.weight", {uint64_t(cfg_.talker_vocab), H});
        text_embedding_ = require("talker.model.text_embedding.weight", {uint64_t(cfg_.text_vocab), H});
        const bf16_t* fc1 = require("talker.text_projection.linear_fc1.weight", {H, H});
        text_fc1_bias_ = require("talker.text_projection.linear_fc1.bias", {H});
        const bf16_t* fc2 = require("talker.text_projection.linear_fc2.weight", {H, H});
        text_fc2_bias_ = require("talker.text_projection.linear_fc2.bias", {H});
        talker_norm_ = require("talker.model.norm.weight", {H});
        const bf16_t* codec_head = require("talker.codec_head.weight", {uint64_t(cfg_.talker_vocab), H});
        codec_head16_ = codec_head;
        const bf16_t* small = require("talker.code_predictor.small_to_mtp_projection.weight",
                                      {uint64_t(P.hidden), H});
        small_to_mtp_bias_ = require("talker.code_predictor.small_to_mtp_projection.bias", {uint64_t(P.hidden)});
        predictor_norm_ = require("talker.code_predictor.model.norm.weight", {uint64_t(P.hidden)});
        std::array<const bf16_t*, kResidualCodebooks> heads{};
        for (int g = 0; g < kResidualCodebooks; ++g) {
            predictor_embeddings_[g] = require(
                "talker.code_predictor.model.codec_embedding." + std::to_string(g) + ".weight",
                {uint64_t(cfg_.predictor_vocab), H});
            heads[g] = require("talker.code_predictor.lm_head." + std::to_string(g) + ".weight",
                               {uint64_t(cfg_.predictor_vocab), uint64_t(P.hidden)});
        }
        struct LayerSource {
            const bf16_t *q, *k, *v, *o, *gate, *up, *down;
        };
        std::vector<LayerSource> tsrc, psrc;
        auto load = [&](const std::string& prefix, const Dims& d, std::vector<Layer>& layers,
                        std::vector<LayerSource>& sources) {
            const uint64_t h = d.hidden, qw = d.query_width(), kw = d.kv_width(),
                           in = d.intermediate, hd = d.head_dimension;
            Layer l;
            LayerSource s{};
            l.input_norm = require(prefix + ".input_layernorm.weight", {h});
            s.q = require(prefix + ".self_attn.q_proj.weight", {qw, h});
            s.k = require(prefix + ".self_attn.k_proj.weight", {kw, h});
            s.v = require(prefix + ".self_attn.v_proj.weight", {kw, h});
            s.o = require(prefix + ".self_attn.o_proj.weight", {h, qw});
            l.q_norm = require(prefix + ".self_attn.q_norm.weight", {hd});
            l.k_norm = require(prefix + ".self_attn.k_norm.weight", {hd});
            l.post_norm = require(prefix + ".post_attention_layernorm.weight", {h});
            s.gate = require(prefix + ".mlp.gate_proj.weight", {in, h});
            s.up = require(prefix + ".mlp.up_proj.weight", {in, h});
            s.down = require(prefix + ".mlp.down_proj.weight", {h, in});
            l.q16 = s.q;
            l.k16 = s.k;
            l.v16 = s.v;
            l.o16 = s.o;
            l.gate16 = s.gate;
            l.up16 = s.up;
            l.down16 = s.down;
            layers.push_back(l);
            sources.push_back(s);
        };
        for (int i = 0; i < T.layers; ++i) load("talker.model.layers." + std::to_string(i), T, talker_layers_, tsrc);
        for (int i = 0; i < P.layers; ++i)
            load("talker.code_predictor.model.layers." + std::to_string(i), P, predictor_layers_, psrc);

        // ---- int8 arena: every decode matrix, in execution order ----
        struct Job {
            const bf16_t* src;
            int in, out;
            size_t data_offset, scale_offset;
        };
        std::vector<Job> jobs;
        size_t data_bytes = 0, scale_count = 0;
        auto reserve = [&](int in, int out) {
            const size_t offset = data_bytes;
            data_bytes += (static_cast<size_t>(in) * out + 255) / 256 * 256;
            const size_t scale = scale_count;
            scale_count += static_cast<size_t>(out);
            return std::make_pair(offset, scale);
        };
        // A matrix assembled from consecutive row blocks (fused QKV, gate/up).
        auto add_rows = [&](std::initializer_list<std::pair<const bf16_t*, int>> blocks, int in) {
            int total = 0;
            for (auto& b : blocks) total += b.second;
            auto [off, sc] = reserve(in, total);
            int row = 0;
            for (auto& b : blocks) {
                jobs.push_back({b.first, in, b.second, off + static_cast<size_t>(row) * in, sc + row});
                row += b.second;
            }
            return std::make_pair(off, sc);
        };
        struct LayerOffsets {
            std::pair<size_t, size_t> qkv, o, gate_up, down;
        };
        std::vector<LayerOffsets> toff, poff;
        auto plan_layers = [&](const Dims& d, const std::vector<LayerSource>& src, std::vector<LayerOffsets>& out) {
            for (const LayerSource& s : src) {
                LayerOffsets lo;
                lo.qkv = add_rows({{s.q, d.query_width()}, {s.k, d.kv_width()}, {s.v, d.kv_width()}}, d.hidden);
                lo.o = add_rows({{s.o, d.hidden}}, d.query_width());
                lo.gate_up = add_rows({{s.gate, d.intermediate}, {s.up, d.intermediate}}, d.hidden);
                lo.down = add_rows({{s.down, d.hidden}}, d.intermediate);
                out.push_back(lo);
            }
        };
        const auto fc1_off = add_rows({{fc1, T.hidden}}, T.hidden);
        const auto fc2_off = add_rows({{fc2, T.hidden}}, T.hidden);
        const auto small_off = add_rows({{small, P.hidden}}, T.hidden);
        plan_layers(P, psrc, poff);
        std::array<std::pair<size_t, size_t>, kResidualCodebooks> head_off;
        for (int g = 0; g < kResidualCodebooks; ++g) head_off[g] = add_rows({{heads[g], cfg_.predictor_vocab}}, P.hidden);
        plan_layers(T, tsrc, toff);
        const auto codec_head_off = add_rows({{codec_head, cfg_.talker_vocab}}, T.hidden);

        int8_arena_ = DeviceBuffer(data_bytes);
        scale_arena_ = DeviceBuffer(scale_count * sizeof(float));
        for (const Job& j : jobs) {
            check_hip(launch_quantize_weight_rows(j.src, int8_arena_.as<int8_t>() + j.data_offset,
                                                  scale_arena_.as<float>() + j.scale_offset, j.in,
                                                  j.out, upload_stream_),
                      "quantize decode weight");
        }
        auto qt = [&](std::pair<size_t, size_t> o) {
            return QTensor{int8_arena_.as<int8_t>() + o.first, scale_arena_.as<float>() + o.second};
        };
        text_fc1_ = qt(fc1_off);
        text_fc2_ = qt(fc2_off);
        small_to_mtp_ = qt(small_off);
        codec_head_ = qt(codec_head_off);
        for (int g = 0; g < kResidualCodebooks; ++g) predictor_heads_[g] = qt(head_off[g]);
        for (size_t i = 0; i < talker_layers_.size(); ++i) {
            talker_layers_[i].qkv = qt(toff[i].qkv);
            talker_layers_[i].o = qt(toff[i].o);
            talker_layers_[i].gate_up = qt(toff[i].gate_up);
            talker_layers_[i].down = qt(toff[i].down);
        }
        for (size_t i = 0; i < predictor_layers_.size(); ++i) {
            predictor_layers_[i].qkv = qt(poff[i].qkv);
            predictor_layers_[i].o = qt(poff[i].o);
            predictor_layers_[i].gate_up = qt(poff[i].gate_up);
            predictor_layers_[i].down = qt(poff[i].down);
        }
        int8_bytes_ = data_bytes;

        // Embedding tables for the fused next-frame input (codec + 15 residual).
        std::array<const bf16_t*, kCodebooks> tables{};
        tables[0] = codec_embedding_;
        for (int g = 0; g < kResidualCodebooks; ++g) tables[g + 1] = predictor_embeddings_[g];
        embedding_tables_ = DeviceBuffer(sizeof(tables));
        check_hip(hipMemcpyAsync(embedding_tables_.as<void>(), tables.data(), sizeof(tables),
                                 hipMemcpyHostToDevice, upload_stream_),
                  "upload embedding table pointers");

        std::vector<bf16_t> rope(static_cast<size_t>(kRopePositions) * T.head_dimension);
        build_rope_table(kRopePositions, T.head_dimension, cfg_.theta, rope.data());
        rope_table_ = DeviceBuffer(rope.size() * sizeof(bf16_t));
        check_hip(hipMemcpyAsync(rope_table_.as<void>(), rope.data(), rope.size() * sizeof(bf16_t),
                                 hipMemcpyHostToDevice, upload_stream_),
                  "upload RoPE table");
        check_hip(hipStreamSynchronize(upload_stream_), "hipStreamSynchronize(finalize)");
        finalized_ = true;
        Qwen3TtsModelMemory m{};
        m.shared_weight_bytes = weight_bytes_;
        m.tensor_count = static_cast<uint32_t>(tensors_.size());
        m.device_index = device_;
        return m;
    }

    bool finalized() const { return finalized_; }
    int device_index() const { return device_; }
    const Config& config() const { return cfg_; }
    std::mutex& batch_mutex() { return batch_mutex_; }

private:
    friend class Session;
    friend class BatchRunner;

    const bf16_t* require(const std::string& name, std::vector<uint64_t> shape) {
        const auto found = tensors_.find(name);
        if (found == tensors_.end()) throw std::runtime_error("checkpoint is missing required tensor " + name);
        if (found->second.shape != shape) throw std::runtime_error("unexpected shape for tensor " + name);
        return found->second.storage.as<bf16_t>();
    }

    int device_;
    Config cfg_;
    bool finalized_ = false;
    uint64_t weight_bytes_ = 0;
    size_t int8_bytes_ = 0;
    hipStream_t upload_stream_ = nullptr;
    std::unordered_map<std::string, DeviceTensor> tensors_;
    DeviceBuffer int8_arena_, scale_arena_, embedding_tables_, rope_table_;
    std::vector<Layer> talker_layers_, predictor_layers_;
    QTensor text_fc1_, text_fc2_, small_to_mtp_, codec_head_;
    const bf16_t* codec_head16_ = nullptr;
    std::array<QTensor, kResidualCodebooks> predictor_heads_{};
    const bf16_t* codec_embedding_ = nullptr;
    const bf16_t* text_embedding_ = nullptr;
    const bf16_t* text_fc1_bias_ = nullptr;
    const bf16_t* text_fc2_bias_ = nullptr;
    const bf16_t* talker_norm_ = nullptr;
    const bf16_t* small_to_mtp_bias_ = nullptr;
    const bf16_t* predictor_norm_ = nullptr;
    std::array<const bf16_t*, kResidualCodebooks> predictor_embeddings_{};
    std::mutex batch_mutex_;

public:
    std::unique_ptr<BatchRunner, void (*)(BatchRunner*)> batch_{nullptr, nullptr};
};

// ---------------------------------------------------------------------------
// Launch helpers shared by the single-session and batched paths.
// ---------------------------------------------------------------------------
struct Gemv {
    GemvArgs a;
    Gemv(const QTensor& w, const bf16_t* x, int in, int out, int epilogue) {
        a.weight = w.data;
        a.scales = w.scales;
        a.input = x;
        a.in_features = in;
        a.out_features = out;
        a.epilogue = epilogue;
        a.mode = kModeExact;
    }
    Gemv& norm(const bf16_t* g, float eps) {
        a.norm_weight = g;
        a.norm_epsilon = eps;
        return *this;
    }
    Gemv& to(bf16_t* y) {
        a.out16 = y;
        return *this;
    }
    Gemv& bias(const bf16_t* b) {
        a.bias = b;
        return *this;
    }
    Gemv& row_index(const int* index) {
        a.input_row_index = index;
        return *this;
    }
    Gemv& rows(int n, int mode) {
        a.rows = n;
        a.mode = mode;
        return *this;
    }
    void run(hipStream_t s, const char* what) { check_hip(launch_int8_gemv(a, s), what); }
    void run_prompt_rows(hipStream_t s, const char* what) { check_hip(launch_int8_gemv_prompt_rows(a, s), what); }
};

struct SamplingParams {
    int do_sample, top_k;
    float top_p, temperature, penalty;
    bool operator==(const SamplingParams& o) const {
        return do_sample == o.do_sample && top_k == o.top_k && top_p == o.top_p &&
               temperature == o.temperature && penalty == o.penalty;
    }
};

SamplingParams params_of(const Qwen3TtsSamplingConfig& c) {
    // talker.cu:3588-3591
    if (c.top_k < 0 || !(c.top_p > 0.0f) || c.top_p > 1.0f || !(c.temperature > 0.0f) ||
        !(c.repetition_penalty > 0.0f)) {
        throw std::runtime_error("invalid sampling configuration");
    }
    return {c.do_sample, c.top_k, c.top_p, c.temperature, c.repetition_penalty};
}

// ---------------------------------------------------------------------------
// Session
// ---------------------------------------------------------------------------
class Session {
public:
    Session(std::shared_ptr<Model> model, int max_sequence_length, uint64_t seed)
        : model_(std::move(model)), m_(*model_), cfg_(model_->config()),
          device_(model_->device_index()), max_seq_(max_sequence_length) {
        if (max_sequence_length < 16 || max_sequence_length > kAttentionCapacity) {
            throw std::runtime_error("max sequence length must be in [16, 8192]");
        }
        if (!model_->finalized()) {
            throw std::runtime_error("model weights must be finalized before creating a session");
        }
        check_hip(hipSetDevice(device_), "hipSetDevice(session)");
        try {
            check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreateWithFlags(session)");
            for (hipEvent_t* e : {&start_, &stop_, &predictor_start_, &predictor_stop_}) {
                check_hip(hipEventCreate(e), "hipEventCreate");
            }
            check_hip(hipEventCreateWithFlags(&codes_ready_, hipEventDisableTiming), "hipEventCreate(codes ready)");
            check_hip(hipEventCreateWithFlags(&semantic_ready_, hipEventDisableTiming), "hipEventCreate(semantic ready)");
            const Dims& T = cfg_.talker;
            const Dims& P = cfg_.predictor;
            const size_t b = sizeof(bf16_t);
            talker_k_ = DeviceBuffer(static_cast<size_t>(T.layers) * max_seq_ * T.kv_width() * b);
            // value caches blocked dimension-major: [layer][kv_heads][stride / 8][128][8]
            talker_v_ = DeviceBuffer(static_cast<size_t>(T.layers) * value_cache_stride(max_seq_) * T.kv_width() * b);
            pred_k_ = DeviceBuffer(static_cast<size_t>(P.layers) * kCodebooks * P.kv_width() * b);
            pred_v_ = DeviceBuffer(static_cast<size_t>(P.layers) * value_cache_stride(kCodebooks) * P.kv_width() * b);
            const int widest = std::max({T.hidden, P.hidden, T.qkv_width(), P.qkv_width(),
                                         T.intermediate, P.intermediate, cfg_.talker_vocab,
                                         cfg_.predictor_vocab});
            hidden_ = DeviceBuffer(static_cast<size_t>(T.hidden) * b);
            p_hidden_ = DeviceBuffer(static_cast<size_t>(P.hidden) * b);
            qkv_ = DeviceBuffer(static_cast<size_t>(widest) * b);
            attn_ = DeviceBuffer(static_cast<size_t>(std::max(T.query_width(), P.query_width())) * b);
            attn_scratch_ = DeviceBuffer(attention_workspace_bytes(1, std::max(T.query_heads, P.query_heads),
                                                                   std::max(max_seq_, kCodebooks)));
            act_ = DeviceBuffer(static_cast<size_t>(std::max(T.intermediate, P.intermediate)) * b);
            logits_ = DeviceBuffer(static_cast<size_t>(std::max(cfg_.talker_vocab, cfg_.predictor_vocab)) * b);
            proj_ = DeviceBuffer(static_cast<size_t>(T.hidden) * b);
            last_hidden_ = DeviceBuffer(static_cast<size_t>(T.hidden) * b);
            // ints: [0] position, [1] history count, [2] sampled token, [3] text token,
            //       [4..19] frame tokens, [20..35] predictor positions 0..15
            ints_ = DeviceBuffer(64 * sizeof(int));
            history_ = DeviceBuffer(static_cast<size_t>(max_seq_) * sizeof(int));
            codes_ = DeviceBuffer(kCodebooks * sizeof(uint16_t));
            random_state_ = DeviceBuffer(sizeof(uint64_t));
            // KV base pointer tables: [talker K | talker V | pred K | pred V]
            std::vector<bf16_t*> bases;
            for (int l = 0; l < T.layers; ++l) bases.push_back(talker_k_.as<bf16_t>() + static_cast<size_t>(l) * max_seq_ * T.kv_width());
            for (int l = 0; l < T.layers; ++l) bases.push_back(talker_v_.as<bf16_t>() + static_cast<size_t>(l) * value_cache_stride(max_seq_) * T.kv_width());
            for (int l = 0; l < P.layers; ++l) bases.push_back(pred_k_.as<bf16_t>() + static_cast<size_t>(l) * kCodebooks * P.kv_width());
            for (int l = 0; l < P.layers; ++l) bases.push_back(pred_v_.as<bf16_t>() + static_cast<size_t>(l) * value_cache_stride(kCodebooks) * P.kv_width());
            kv_bases_ = DeviceBuffer(bases.size() * sizeof(bf16_t*));
            check_hip(hipMemcpy(kv_bases_.as<void>(), bases.data(), kv_bases_.bytes(), hipMemcpyHostToDevice), "upload KV bases");
            host_bases_ = bases;
            std::vector<int> init(64, 0);
            for (int p = 0; p < kCodebooks; ++p) init[20 + p] = p;
            init[41] = 1;  // predictor pass epoch
            setup_predictor_chain();
            // test switch: the predictor pass starts with its status word
            // set, so every stage wait gives up at once (the frame then
            // reports the failure); no wait is ever unbounded
            const char* give_up = std::getenv("QWEN3_TTS_PREDICTOR_CHAIN_TEST_GIVE_UP");
            if (pred_chain_ && give_up != nullptr && std::strcmp(give_up, "1") == 0) init[40] = 1;
            check_hip(hipMemcpy(ints_.as<void>(), init.data(), init.size() * sizeof(int), hipMemcpyHostToDevice), "init session ints");
            check_hip(hipHostMalloc(reinterpret_cast<void**>(&pinned_), 256, hipHostMallocDefault), "hipHostMalloc(session)");
            std::memset(pinned_, 0, 256);
            reset(seed);
        } catch (...) {
            release();
            throw;
        }
    }
    ~Session() { release(); }
    Session(const Session&) = delete;
    Session& operator=(const Session&) = delete;

    // talker.cu:1008-1034
    void reset(uint64_t seed) {
        check_hip(hipSetDevice(device_), "hipSetDevice(reset)");
        if (frame_in_flight_) throw std::runtime_error("cannot reset while a device frame lease is in flight");
        position_ = 0;
        history_count_ = 0;
        frames_ = 0;
        device_samples_ = 0;
        host_syncs_ = 0;
        semantic_ = 0;
        phase_ = QWEN3_TTS_TALKER_READY;
        const uint64_t state = seed == 0 ? 0x9e3779b97f4a7c15ULL : seed;
        check_hip(hipMemcpyAsync(random_state_.as<void>(), &state, sizeof(state), hipMemcpyHostToDevice, stream_), "reset random state");
        const int zeros[2] = {0, 0};
        check_hip(hipMemcpyAsync(ints_.as<int>(), zeros, sizeof(zeros), hipMemcpyHostToDevice, stream_), "reset counters");
        check_hip(hipStreamSynchronize(stream_), "synchronize reset");
    }

    // Prefill, talker.cu:1036-1093.  By default the reference's bf16 prefill
    // (talker.cu:2750-3249): the prompt's rows through the bf16 weights as
    // MFMA GEMMs.  QWEN3_TTS_PREFILL=decode selects the int8 decode step run
    // once per prompt position instead (the decode path's numerics).
    Qwen3TtsTalkerPrefillResult prefill(const int32_t* text, const int32_t* codec, int count,
                                        const Qwen3TtsSamplingConfig& sampling) {
        check_hip(hipSetDevice(device_), "hipSetDevice(prefill)");
        if (poisoned_) throw std::runtime_error("talker session is poisoned and must be destroyed");
        if (frame_in_flight_) throw std::runtime_error("cannot prefill while a device frame lease is in flight");
        if (text == nullptr || codec == nullptr || count <= 0) {
            throw std::runtime_error("prefill requires non-empty text and codec ID arrays");
        }
        if (count > max_seq_) throw std::runtime_error("prompt exceeds the configured KV-cache capacity");
        for (int i = 0; i < count; ++i) {
            if (text[i] < 0 && codec[i] < 0) throw std::runtime_error("a prompt position must contain text or codec input");
            if (text[i] >= cfg_.text_vocab || codec[i] >= cfg_.talker_vocab) {
                throw std::runtime_error("prompt token is outside the vocabulary");
            }
        }
        const SamplingParams sp = params_of(sampling);
        if (history_count_ >= max_seq_) throw std::runtime_error("semantic history exceeds configured sequence capacity");
        try {
            DeviceBuffer prompt(static_cast<size_t>(count) * 2 * sizeof(int));
            std::vector<int> ids(static_cast<size_t>(count) * 2);
            std::copy(text, text + count, ids.begin());
            std::copy(codec, codec + count, ids.begin() + count);
            check_hip(hipMemcpyAsync(prompt.as<void>(), ids.data(), ids.size() * sizeof(int), hipMemcpyHostToDevice, stream_), "upload prompt");
            const int zeros[2] = {0, 0};
            check_hip(hipMemcpyAsync(ints_.as<int>(), zeros, sizeof(zeros), hipMemcpyHostToDevice, stream_), "reset position");
            position_ = 0;
            history_count_ = 0;
            check_hip(hipEventRecord(start_, stream_), "hipEventRecord(prefill start)");
            const int H = cfg_.talker.hidden;
            const bool bf16 = bf16_prefill_enabled();
            if (bf16) {
                prefill_bf16(count, prompt.as<int>(), prompt.as<int>() + count);
                emit_prefill_logits(count);
            }
            for (int i = 0; !bf16 && i < count; ++i) {
                const int* text_id = prompt.as<int>() + i;
                const int* codec_id = prompt.as<int>() + count + i;
                if (text[i] >= 0) {
                    project_text(text_id, false);
                } else {
                    check_hip(launch_fill_zero(hidden_.as<bf16_t>(), H, stream_), "zero prompt embedding");
                }
                if (codec[i] >= 0) {
                    check_hip(launch_gather_embedding(m_.codec_embedding_, cfg_.talker_vocab, H, codec_id, hidden_.as<bf16_t>(), true, stream_),
                              "add prompt codec embedding");
                }
                run_decoder(false, position_ptr(), 0);
                check_hip(launch_increment(position_ptr(), stream_), "advance position");
            }
            if (!bf16) emit_talker_logits();
            sample_talker(sp);
            check_hip(hipEventRecord(stop_, stream_), "hipEventRecord(prefill stop)");
            position_ = count;
            check_hip(hipMemcpyAsync(pinned_, ints_.as<int>() + 2, sizeof(int), hipMemcpyDeviceToHost, stream_), "copy sampled token");
            check_hip(hipStreamSynchronize(stream_), "synchronize prefill");
            ++host_syncs_;
            const int first = validated_token();
            float ms = 0.0f;
            check_hip(hipEventElapsedTime(&ms, start_, stop_), "hipEventElapsedTime(prefill)");
            semantic_ = static_cast<uint16_t>(first);
            phase_ = first == cfg_.codec_eos ? QWEN3_TTS_TALKER_ENDED : QWEN3_TTS_TALKER_PREFILLED;
            Qwen3TtsTalkerPrefillResult r{};
            r.first_semantic_token = static_cast<uint16_t>(first);
            r.prompt_tokens = static_cast<uint32_t>(count);
            r.talker_gpu_milliseconds = ms;
            return r;
        } catch (...) {
            poisoned_ = true;
            (void)hipStreamSynchronize(stream_);
            throw;
        }
    }

    static bool bf16_prefill_enabled() {
        const char* v = std::getenv("QWEN3_TTS_PREFILL");
        return v == nullptr || std::strcmp(v, "decode") != 0;
    }

    // The prompt's rows through the talker with the bf16 weights
    // (run_decoder_prefill, talker.cu:2854-3202): every projection one MFMA
    // GEMM over all rows; attention through materialized scores and the
    // causal softmax when the prompt fits kPrefillAttentionRows and the
    // session capacity (talker.cu:3035), else the exact per-row kernel.
    // Leaves the rows' final hidden states in prefill_.hidden.
    void prefill_bf16(int rows, const int* text_ids, const int* codec_ids) {
        const Dims& T = cfg_.talker;
        const int H = T.hidden, I = T.intermediate, qw = T.query_width(), kvw = T.kv_width();
        const int qkvw = T.qkv_width(), hd = T.head_dimension;
        const int rp = (rows + 7) / 8 * 8;
        const bool gemm_attention = rows <= std::min(max_seq_, kPrefillAttentionRows);
        PrefillBuffers& w = prefill_;
        w.ensure(rows, H, I, qkvw, qw, T.query_heads, T.key_value_heads, gemm_attention ? rp : 0,
                 gemm_attention ? 0 : max_seq_);
        bf16_t* hidden = w.hidden.as<bf16_t>();
        // prompt embeddings: int8 text projection (exact order, 8 rows a
        // launch), then zero text-less rows and add codec embeddings
        check_hip(launch_gather_text_rows(m_.text_embedding_, text_ids, cfg_.text_vocab, rows, H, w.normalized.as<bf16_t>(),
                                          stream_),
                  "gather prompt text embeddings");
        // (the reference runs 8 rows a launch; each row's exact-order sum is
        // the same whatever rows share its launch, so all rows run in one)
        Gemv(m_.text_fc1_, w.normalized.as<bf16_t>(), H, H, kEpiBiasSilu).bias(m_.text_fc1_bias_)
            .rows(rows, kModeExact).to(w.proj.as<bf16_t>()).run_prompt_rows(stream_, "prompt text fc1");
        Gemv(m_.text_fc2_, w.proj.as<bf16_t>(), H, H, kEpiBias).bias(m_.text_fc2_bias_)
            .rows(rows, kModeExact).to(hidden).run_prompt_rows(stream_, "prompt text fc2");
        check_hip(launch_prompt_rows(hidden, text_ids, codec_ids, m_.codec_embedding_, cfg_.talker_vocab, rows, H, stream_),
                  "prompt rows");
        auto gemm = [&](const bf16_t* a, int lda, const bf16_t* weight, bf16_t* c, int ldc, int n, int k,
                        const char* what, int epilogue = kGemmStore) {
            Bf16GemmArgs g;
            g.epilogue = epilogue;
            g.a = a;
            g.b = weight;
            g.c = c;
            g.m = rows;
            g.n = n;
            g.k = k;
            g.lda = lda;
            g.ldb = k;
            g.ldc = ldc;
            g.partial = w.partial.as<float>();
            g.partial_floats = kPrefillPartialFloats;
            check_hip(launch_bf16_gemm(g, stream_), what);
        };
        bf16_t* xn = w.normalized.as<bf16_t>();
        bf16_t* qkv = w.qkv.as<bf16_t>();
        bf16_t* attn = w.attn.as<bf16_t>();
        bf16_t* gate = w.gate.as<bf16_t>();
        const int vstride = value_cache_stride(max_seq_);
        for (int l = 0; l < T.layers; ++l) {
            const Layer& L = m_.talker_layers_[l];
            bf16_t* kc = host_bases_[l];
            bf16_t* vc = host_bases_[T.layers + l];
            check_hip(launch_rms_norm_rows(hidden, L.input_norm, xn, rows, H, cfg_.eps, stream_), "prefill input norm");
            {  // q, k and v: one GEMM over the three weights as row segments of B
                Bf16GemmArgs g;
                g.a = xn;
                g.b = L.q16;
                g.b2 = L.k16;
                g.b2_row = qw;
                g.b3 = L.v16;
                g.b3_row = qw + kvw;
                g.c = qkv;
                g.m = rows;
                g.n = qkvw;
                g.k = H;
                g.lda = H;
                g.ldb = H;
                g.ldc = qkvw;
                g.partial = w.partial.as<float>();
                g.partial_floats = kPrefillPartialFloats;
                check_hip(launch_bf16_gemm(g, stream_), "prefill q/k/v GEMM");
            }
            check_hip(launch_prefill_qkv_epilogue(qkv, L.q_norm, L.k_norm, m_.rope_table_.as<bf16_t>(), kc, vc, vstride, 0,
                                                  rows, T.query_heads, T.key_value_heads, cfg_.eps, stream_),
                      "prefill q/k norm + RoPE + cache");
            if (gemm_attention) {
                bf16_t* scores = w.scores.as<bf16_t>();
                bf16_t* vt = w.values_t.as<bf16_t>();
                Bf16GemmArgs s;  // scores[h] = q_h k_h^T
                s.a = qkv;
                s.lda = qkvw;
                s.a_batch = hd;
                s.b = qkv + qw;
                s.ldb = qkvw;
                s.b_batch = hd;
                s.b_group = T.query_heads / T.key_value_heads;
                s.c = scores;
                s.ldc = rp;
                s.c_batch = static_cast<long long>(rows) * rp;
                s.m = rows;
                s.n = rows;
                s.k = hd;
                s.batch = T.query_heads;
                s.partial = w.partial.as<float>();
                s.partial_floats = kPrefillPartialFloats;
                check_hip(launch_bf16_gemm(s, stream_), "prefill score GEMM");
                check_hip(launch_causal_softmax(scores, T.query_heads, rows, rp, hd, stream_), "prefill causal softmax");
                check_hip(launch_transpose_values(qkv, qkvw, qw + kvw, rows, rp, T.key_value_heads, vt, stream_),
                          "prefill value transpose");
                Bf16GemmArgs o;  // out_h = p_h v_h
                o.a = scores;
                o.lda = rp;
                o.a_batch = static_cast<long long>(rows) * rp;
                o.b = vt;
                o.ldb = rp;
                o.b_batch = static_cast<long long>(hd) * rp;
                o.b_group = T.query_heads / T.key_value_heads;
                o.c = attn;
                o.ldc = qw;
                o.c_batch = hd;
                o.m = rows;
                o.n = hd;
                o.k = rp;
                o.batch = T.query_heads;
                o.partial = w.partial.as<float>();
                o.partial_floats = kPrefillPartialFloats;
                check_hip(launch_bf16_gemm(o, stream_), "prefill value GEMM");
            } else {
                // the exact kernel, row r over positions 0..r, in chunks that
                // bound the score workspace
                for (int r0 = 0; r0 < rows; r0 += kPrefillChunk) {
                    const int n = std::min(kPrefillChunk, rows - r0);
                    check_hip(launch_attention(true, qkv + static_cast<size_t>(r0) * qkvw, qkvw, nullptr, nullptr, kc, vc,
                                               w.positions.as<int>() + r0, 0, attn + static_cast<size_t>(r0) * qw, n,
                                               T.query_heads, T.key_value_heads, hd, max_seq_, w.workspace.as<float>(),
                                               nullptr, stream_),
                              "prefill exact attention");
                }
            }
            // O GEMM with the residual add (add_in_place) as its epilogue
            gemm(attn, qw, L.o16, hidden, H, H, qw, "prefill O GEMM + residual", kGemmAddInto);
            check_hip(launch_rms_norm_rows(hidden, L.post_norm, xn, rows, H, cfg_.eps, stream_), "prefill post norm");
            gemm(xn, H, L.gate16, gate, I, I, H, "prefill gate GEMM");
            // up GEMM with silu_gate as its epilogue (gate holds the gate product)
            gemm(xn, H, L.up16, gate, I, I, H, "prefill up GEMM + SiLU gate", kGemmSiluGateInto);
            gemm(gate, I, L.down16, hidden, H, H, I, "prefill down GEMM + residual", kGemmAddInto);
        }
    }

    // run_talker_prefill's tail (talker.cu:3204-3231): final norm of the last
    // row into last_hidden, bf16 codec head GEMM into the logits; position =
    // prompt length.
    void emit_prefill_logits(int rows) {
        const int H = cfg_.talker.hidden;
        check_hip(launch_rms_norm_rows(prefill_.hidden.as<bf16_t>() + static_cast<size_t>(rows - 1) * H, m_.talker_norm_,
                                       last_hidden_.as<bf16_t>(), 1, H, cfg_.eps, stream_),
                  "prefill final norm");
        Bf16GemmArgs g;
        g.a = last_hidden_.as<bf16_t>();
        g.b = m_.codec_head16_;
        g.c = logits_.as<bf16_t>();
        g.m = 1;
        g.n = cfg_.talker_vocab;
        g.k = H;
        g.lda = H;
        g.ldb = H;
        g.ldc = cfg_.talker_vocab;
        g.partial = prefill_.partial.as<float>();
        g.partial_floats = kPrefillPartialFloats;
        check_hip(launch_bf16_gemm(g, stream_), "prefill codec head GEMM");
        pinned_[1] = rows;
        check_hip(hipMemcpyAsync(ints_.as<int>(), &pinned_[1], sizeof(int), hipMemcpyHostToDevice, stream_),
                  "set position");
    }

    // begin_frame, talker.cu:1095-1262
    Qwen3TtsDeviceFrameViewV2 begin_frame(uint16_t semantic, int text_token,
                                          const Qwen3TtsSamplingConfig& talker_sampling,
                                          const Qwen3TtsSamplingConfig& predictor_sampling,
                                          bool copy_codes) {
        check_hip(hipSetDevice(device_), "hipSetDevice(begin frame)");
        validate_frame(semantic, text_token);
        const SamplingParams ts = params_of(talker_sampling);
        const SamplingParams ps = params_of(predictor_sampling);
        const uint64_t lease = next_lease_++;
        if (next_lease_ == 0) next_lease_ = 1;
        frame_in_flight_ = true;
        pending_pass_status_ = false;
        pending_copy_ = copy_codes;
        pending_lease_ = lease;
        pending_position_ = static_cast<uint32_t>(position_);
        try {
            pinned_[1] = text_token;
            check_hip(hipMemcpyAsync(ints_.as<int>() + 3, &pinned_[1], sizeof(int), hipMemcpyHostToDevice, stream_), "upload text token");
            if (pred_chain_) {
                // The persistent passes need every CU at once: the passes of
                // all sessions on the device run one after another (a
                // per-device order of their launches; no wait when the last
                // ones were this stream's own).
                PredictorPassOrder order(device_, stream_);
                check_hip(order.status(), "predictor pass order");
                check_hip(hipEventRecord(predictor_start_, stream_), "hipEventRecord(predictor start)");
                launch_graph(predictor_graph_, ps, [&] { enqueue_predictor(ps); });
                check_hip(hipEventRecord(predictor_stop_, stream_), "hipEventRecord(predictor stop)");
                check_hip(order.done(), "predictor pass order");
                check_hip(hipMemcpyAsync(pinned_ + 20, ints_.as<int>() + 40, sizeof(int), hipMemcpyDeviceToHost, stream_),
                          "copy predictor pass status");
                pending_pass_status_ = true;
            } else {
                check_hip(hipEventRecord(predictor_start_, stream_), "hipEventRecord(predictor start)");
                launch_graph(predictor_graph_, ps, [&] { enqueue_predictor(ps); });
                check_hip(hipEventRecord(predictor_stop_, stream_), "hipEventRecord(predictor stop)");
            }
            check_hip(hipEventRecord(codes_ready_, stream_), "hipEventRecord(codes ready)");
            if (copy_codes) {
                check_hip(hipMemcpyAsync(pinned_codes(), codes_.as<void>(), kCodebooks * sizeof(uint16_t), hipMemcpyDeviceToHost, stream_), "copy codec frame");
            }
            check_hip(hipEventRecord(start_, stream_), "hipEventRecord(talker start)");
            launch_graph(talker_graph_, ts, [&] { enqueue_talker(ts); });
            check_hip(hipEventRecord(stop_, stream_), "hipEventRecord(talker stop)");
            ++position_;
            ++history_count_;
            device_samples_ += kCodebooks;  // 15 predictor samples + 1 talker sample
            check_hip(hipMemcpyAsync(pinned_, ints_.as<int>() + 2, sizeof(int), hipMemcpyDeviceToHost, stream_), "copy sampled token");
            check_hip(hipEventRecord(semantic_ready_, stream_), "hipEventRecord(semantic ready)");
        } catch (...) {
            poisoned_ = true;
            (void)hipStreamSynchronize(stream_);
            frame_in_flight_ = false;
            pending_copy_ = false;
            pending_lease_ = 0;
            throw;
        }
        return view(lease);
    }

    // finish_frame, talker.cu:1264-1324
    Qwen3TtsCodecFrameResult finish_frame(uint64_t lease, Qwen3TtsCudaEventHandle consumer_done) {
        check_hip(hipSetDevice(device_), "hipSetDevice(finish frame)");
        if (poisoned_) throw std::runtime_error("talker session is poisoned and must be destroyed");
        if (!frame_in_flight_) throw std::runtime_error("no device frame lease is in flight");
        if (lease == 0 || lease != pending_lease_) throw std::runtime_error("device frame lease ID is stale or invalid");
        if (consumer_done != nullptr) {
            check_hip(hipStreamWaitEvent(stream_, reinterpret_cast<hipEvent_t>(consumer_done), 0), "hipStreamWaitEvent(consumer done)");
        }
        check_hip(hipEventSynchronize(semantic_ready_), "hipEventSynchronize(semantic ready)");
        ++host_syncs_;
        const bool pass_status = pending_pass_status_;  // this frame ran the persistent predictor passes
        pending_pass_status_ = false;
        if (pass_status && pinned_[20] != 0) {
            poisoned_ = true;
            throw DeviceFailure("predictor pass: a stage input did not arrive within its bound");
        }
        const int next = validated_token();
        Qwen3TtsCodecFrameResult r{};
        r.talker_position = pending_position_;
        check_hip(hipEventElapsedTime(&r.predictor_gpu_milliseconds, predictor_start_, predictor_stop_), "hipEventElapsedTime(predictor)");
        check_hip(hipEventElapsedTime(&r.talker_gpu_milliseconds, start_, stop_), "hipEventElapsedTime(talker)");
        if (pending_copy_) std::copy_n(pinned_codes(), kCodebooks, r.codes);
        r.next_semantic_token = static_cast<uint16_t>(next);
        r.ended_by_eos = next == cfg_.codec_eos ? 1 : 0;
        semantic_ = r.next_semantic_token;
        ++frames_;
        phase_ = r.ended_by_eos ? QWEN3_TTS_TALKER_ENDED : QWEN3_TTS_TALKER_PREFILLED;
        frame_in_flight_ = false;
        pending_copy_ = false;
        pending_lease_ = 0;
        return r;
    }

    Qwen3TtsCodecFrameResult next_frame(uint16_t semantic, int text_token,
                                        const Qwen3TtsSamplingConfig& ts,
                                        const Qwen3TtsSamplingConfig& ps) {
        const Qwen3TtsDeviceFrameViewV2 v = begin_frame(semantic, text_token, ts, ps, true);
        return finish_frame(v.lease_id, nullptr);
    }

    uint16_t current_semantic() const { return semantic_; }

    // Diagnostics: the talker's final-normalized hidden state (the predictor's
    // position-0 input and the codec head's input) after the last completed
    // frame or prefill, copied to host memory.
    void read_last_hidden(void* destination, uint64_t bytes) {
        const uint64_t need = static_cast<uint64_t>(cfg_.talker.hidden) * sizeof(bf16_t);
        if (destination == nullptr || bytes != need) throw std::invalid_argument("last hidden needs talker_hidden bf16 values");
        if (frame_in_flight_) throw std::runtime_error("a device frame lease is in flight");
        check_hip(hipSetDevice(device_), "hipSetDevice(read last hidden)");
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize(read last hidden)");
        check_hip(hipMemcpy(destination, last_hidden_.as<void>(), need, hipMemcpyDeviceToHost), "read last hidden");
    }

    // Diagnostics: positions 0..count-1 of talker layer `layer`'s key (which
    // 0) or value (which 1) cache as [position][kv_width] bf16.
    void read_talker_cache(int layer, int which, int count, void* destination, uint64_t bytes) {
        const Dims& T = cfg_.talker;
        const int kvw = T.kv_width();
        if (layer < 0 || layer >= T.layers || (which != 0 && which != 1) || count <= 0 || count > max_seq_ ||
            destination == nullptr || bytes != static_cast<uint64_t>(count) * kvw * sizeof(bf16_t)) {
            throw std::invalid_argument("cache read needs a layer, which (0 key, 1 value) and count * kv_width bf16");
        }
        if (frame_in_flight_) throw std::runtime_error("a device frame lease is in flight");
        check_hip(hipSetDevice(device_), "hipSetDevice(read cache)");
        check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize(read cache)");
        if (which == 0) {
            check_hip(hipMemcpy(destination, host_bases_[layer], bytes, hipMemcpyDeviceToHost), "read key cache");
            return;
        }
        const int stride = value_cache_stride(max_seq_);
        std::vector<bf16_t> blocked(static_cast<size_t>(kvw) * stride);
        check_hip(hipMemcpy(blocked.data(), host_bases_[T.layers + layer], blocked.size() * sizeof(bf16_t),
                            hipMemcpyDeviceToHost),
                  "read value cache");
        bf16_t* out = static_cast<bf16_t*>(destination);
        for (int p = 0; p < count; ++p) {
            for (int c = 0; c < kvw; ++c) {
                out[static_cast<size_t>(p) * kvw + c] =
                    blocked[((static_cast<size_t>(c >> 7) * (stride >> 3) + (p >> 3)) * 128 + (c & 127)) * 8 + (p & 7)];
            }
        }
    }

    Qwen3TtsTalkerStateInfo state_info() const {
        Qwen3TtsTalkerStateInfo r{};
        r.abi_version = QWEN3_TTS_TALKER_ABI_VERSION;
        r.phase = static_cast<uint32_t>(phase_);
        r.talker_position = static_cast<uint32_t>(position_);
        r.semantic_history_count = static_cast<uint32_t>(history_count_);
        r.frames_generated = frames_;
        r.device_sample_count = device_samples_;
        r.host_sync_count = host_syncs_;
        return r;
    }

    Qwen3TtsSessionMemory memory() const {
        Qwen3TtsSessionMemory r{};
        r.talker_kv_bytes = talker_k_.bytes() + talker_v_.bytes();
        r.predictor_kv_bytes = pred_k_.bytes() + pred_v_.bytes();
        r.workspace_bytes = hidden_.bytes() + p_hidden_.bytes() + qkv_.bytes() + attn_.bytes() + attn_scratch_.bytes() +
                            act_.bytes() + logits_.bytes() + proj_.bytes() + last_hidden_.bytes() +
                            ints_.bytes() + history_.bytes() + codes_.bytes() + random_state_.bytes() +
                            kv_bases_.bytes();
        r.max_sequence_length = static_cast<uint32_t>(max_seq_);
        return r;
    }

    const Model* model() const { return model_.get(); }

private:
    friend class BatchRunner;

    int* position_ptr() const { return ints_.as<int>(); }
    int* history_count_ptr() const { return ints_.as<int>() + 1; }
    int* sampled_ptr() const { return ints_.as<int>() + 2; }
    int* text_token_ptr() const { return ints_.as<int>() + 3; }
    int* frame_tokens() const { return ints_.as<int>() + 4; }
    int* pred_positions() const { return ints_.as<int>() + 20; }
    uint16_t* pinned_codes() const { return reinterpret_cast<uint16_t*>(pinned_ + 8); }

    void validate_frame(uint16_t semantic, int text_token) {
        if (poisoned_) throw std::runtime_error("talker session is poisoned and must be destroyed");
        if (frame_in_flight_) throw std::runtime_error("a device frame lease is already in flight");
        if (phase_ != QWEN3_TTS_TALKER_PREFILLED) throw std::runtime_error("talker must be prefilled before frame generation");
        if (semantic == cfg_.codec_eos) throw std::runtime_error("EOS must not be expanded into a codec frame");
        if (semantic >= cfg_.talker_vocab) throw std::runtime_error("semantic token is outside the talker vocabulary");
        if (semantic != semantic_) throw std::runtime_error("semantic token does not match talker session state");
        if (text_token < 0 || text_token >= cfg_.text_vocab) throw std::runtime_error("next-frame text token is outside the text vocabulary");
        if (position_ >= max_seq_) throw std::runtime_error("talker KV cache is full");
        if (history_count_ >= max_seq_) throw std::runtime_error("semantic history exceeds configured sequence capacity");
    }

    int validated_token() const {
        const int t = pinned_[0];
        if (t < 0 || t >= cfg_.talker_vocab) throw std::runtime_error("device sampler returned an invalid token");
        return t;
    }

    Qwen3TtsDeviceFrameViewV2 view(uint64_t lease) const {
        Qwen3TtsDeviceFrameViewV2 v{};
        v.struct_size = sizeof(Qwen3TtsDeviceFrameViewV2);
        v.code_count = kCodebooks;
        v.device_codes = codes_.as<uint16_t>();
        v.ready_event = reinterpret_cast<Qwen3TtsCudaEventHandle>(codes_ready_);
        v.lease_id = lease;
        v.device_index = device_;
        return v;
    }

    // Row buffers of the bf16 prefill, grown on demand and kept.
    static constexpr int kPrefillChunk = 128;  // rows per exact-attention launch
    // split-K partial sums of the prefill GEMMs (short prompts), 16 MB
    static constexpr size_t kPrefillPartialFloats = size_t{4} << 20;
    struct PrefillBuffers {
        DeviceBuffer hidden, normalized, qkv, attn, proj, gate, scores, values_t, positions, workspace, partial;
        int rows = 0, score_stride = 0, capacity = 0;
        void ensure(int r, int H, int I, int qkvw, int qw, int query_heads, int kv_heads, int rp, int exact_capacity) {
            const size_t b = sizeof(bf16_t);
            if (partial.as<void>() == nullptr) partial = DeviceBuffer(kPrefillPartialFloats * sizeof(float));
            if (r > rows) {
                hidden = DeviceBuffer(static_cast<size_t>(r) * H * b);
                normalized = DeviceBuffer(static_cast<size_t>(r) * H * b);
                qkv = DeviceBuffer(static_cast<size_t>(r) * qkvw * b);
                attn = DeviceBuffer(static_cast<size_t>(r) * qw * b);
                proj = DeviceBuffer(static_cast<size_t>(r) * H * b);
                gate = DeviceBuffer(static_cast<size_t>(r) * I * b);
                rows = r;
            }
            if (rp > score_stride) {  // GEMM attention: scores, transposed values
                scores = DeviceBuffer(static_cast<size_t>(query_heads) * rp * rp * b);
                values_t = DeviceBuffer(static_cast<size_t>(kv_heads) * 128 * rp * b);
                score_stride = rp;
            }
            if (exact_capacity > capacity) {  // exact attention: positions, score workspace
                std::vector<int> ids(static_cast<size_t>(exact_capacity));
                for (int i = 0; i < exact_capacity; ++i) ids[i] = i;
                positions = DeviceBuffer(ids.size() * sizeof(int));
                check_hip(hipMemcpy(positions.as<void>(), ids.data(), ids.size() * sizeof(int), hipMemcpyHostToDevice),
                          "upload prefill positions");
                workspace = DeviceBuffer(attention_workspace_bytes(kPrefillChunk, query_heads, exact_capacity));
                capacity = exact_capacity;
            }
        }
    };

    struct Graph {
        hipGraphExec_t exec = nullptr;
        bool have_key = false;
        SamplingParams key{};
        int eager_runs = 0;
    };

    // Capture on the second use of a sampling configuration, replay after.
    // The work runs on `exec` (default: the session's stream); a capture is
    // always taken on the session's own stream.
    template <typename Enqueue>
    void launch_graph(Graph& g, const SamplingParams& key, Enqueue&& enqueue, hipStream_t exec = nullptr) {
        if (exec == nullptr) exec = stream_;
        if (g.have_key && !(g.key == key)) {
            // the old graph may still be queued on the stream
            if (g.exec) check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize(replace graph)");
            if (g.exec) (void)hipGraphExecDestroy(g.exec);
            g.exec = nullptr;
            g.eager_runs = 0;
        }
        g.have_key = true;
        g.key = key;
        if (g.exec != nullptr) {
            check_hip(hipGraphLaunch(g.exec, exec), "hipGraphLaunch");
            return;
        }
        if (g.eager_runs < 1 || !graphs_enabled()) {
            const hipStream_t own = stream_;
            stream_ = exec;  // the enqueue functions launch on stream_
            try {
                enqueue();
            } catch (...) {
                stream_ = own;
                throw;
            }
            stream_ = own;
            ++g.eager_runs;
            return;
        }
        check_hip(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
        try {
            enqueue();
        } catch (...) {
            hipGraph_t aborted = nullptr;
            (void)hipStreamEndCapture(stream_, &aborted);
            if (aborted) (void)hipGraphDestroy(aborted);
            throw;
        }
        hipGraph_t graph = nullptr;
        check_hip(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture");
        const hipError_t inst = hipGraphInstantiate(&g.exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        check_hip(inst, "hipGraphInstantiate");
        check_hip(hipGraphLaunch(g.exec, exec), "hipGraphLaunch");
    }

    static bool graphs_enabled() {
        const char* v = std::getenv("QWEN3_TTS_DISABLE_GRAPHS");
        return v == nullptr || std::strcmp(v, "1") != 0;
    }


    // One decoder stack step (talker.cu:3251-3456) at the position held in
    // *position (device).  predictor selects the 5-layer code predictor.
    void run_decoder(bool predictor, const int* position, int) {
        const Dims& d = predictor ? cfg_.predictor : cfg_.talker;
        const std::vector<Layer>& layers = predictor ? m_.predictor_layers_ : m_.talker_layers_;
        bf16_t* hidden = predictor ? p_hidden_.as<bf16_t>() : hidden_.as<bf16_t>();
        const int cache_rows = predictor ? kCodebooks : max_seq_;
        for (int l = 0; l < d.layers; ++l) {
            const Layer& L = layers[l];
            Gemv(L.qkv, hidden, d.hidden, d.qkv_width(), kEpiStore).norm(L.input_norm, cfg_.eps).to(qkv_.as<bf16_t>()).run(stream_, "QKV GEMV");
            const bf16_t* kc = host_bases_[(predictor ? 2 * cfg_.talker.layers : 0) + l];
            const bf16_t* vc = host_bases_[(predictor ? 2 * cfg_.talker.layers : 0) + d.layers + l];
            check_hip(launch_decode_attention(true, qkv_.as<bf16_t>(), d.qkv_width(), L.q_norm, L.k_norm,
                                              m_.rope_table_.as<bf16_t>(), cfg_.eps, nullptr, nullptr, kc, vc, position,
                                              attn_.as<bf16_t>(), 1, d.query_heads, d.key_value_heads,
                                              d.head_dimension, cache_rows, attn_scratch_.as<float>(), nullptr, stream_),
                      "q/k norm + RoPE + KV append + attention");
            Gemv(L.o, attn_.as<bf16_t>(), d.query_width(), d.hidden, kEpiAddRounded).to(hidden).run(stream_, "O GEMV");
            Gemv(L.gate_up, hidden, d.hidden, d.intermediate, kEpiSiluRounded).norm(L.post_norm, cfg_.eps).to(act_.as<bf16_t>()).run(stream_, "gate/up GEMV");
            Gemv(L.down, act_.as<bf16_t>(), d.intermediate, d.hidden, kEpiAddRounded).to(hidden).run(stream_, "down GEMV");
        }
    }

    // project_text (talker.cu:2676-2719).  into_hidden: hidden += projection
    // (prepare_generated_embedding, :3572-3580); otherwise hidden = projection.
    void project_text(const int* token, bool into_hidden) {
        const int H = cfg_.talker.hidden;
        Gemv(m_.text_fc1_, m_.text_embedding_, H, H, kEpiBiasSilu).row_index(token).bias(m_.text_fc1_bias_).to(proj_.as<bf16_t>()).run(stream_, "text fc1");
        Gemv(m_.text_fc2_, proj_.as<bf16_t>(), H, H, into_hidden ? kEpiBiasAdd : kEpiBias).bias(m_.text_fc2_bias_).to(hidden_.as<bf16_t>()).run(stream_, "text fc2");
    }

    // Final norm -> last_hidden, codec head -> logits (talker.cu:3458-3495).
    void emit_talker_logits() {
        const int H = cfg_.talker.hidden;
        check_hip(launch_rms_norm_rows(hidden_.as<bf16_t>(), m_.talker_norm_, last_hidden_.as<bf16_t>(), 1, H, cfg_.eps, stream_), "talker final norm");
        Gemv(m_.codec_head_, last_hidden_.as<bf16_t>(), H, cfg_.talker_vocab, kEpiStore).to(logits_.as<bf16_t>()).run(stream_, "codec head");
    }

    // Talker sample: store into frame_tokens[0] (next frame's semantic token),
    // append to the history, advance nothing else (talker.cu:3583-3627).
    void sample_talker(const SamplingParams& s) {
        check_hip(launch_sample_logits_ex(logits_.as<bf16_t>(), cfg_.talker_vocab, true, cfg_.codec_eos, history_.as<int>(),
                                          history_count_ptr(), 0, s.do_sample, s.top_k, s.top_p, s.temperature, s.penalty,
                                          random_state_.as<uint64_t>(), sampled_ptr(), frame_tokens(), nullptr, 0,
                                          history_.as<int>(), history_count_ptr(), stream_),
                  "talker sample");
        ++device_samples_;
        ++history_count_;
    }

    // The persistent predictor pass runs the predictor at the geometry it is
    // built for (the reference's: talker hidden 2048; predictor 1024 / 3072,
    // 16 / 8 heads, 5 layers, 2048-entry codebooks) on a device where all
    // its workgroups fit at once; QWEN3_TTS_DISABLE_PREDICTOR_CHAIN=1 keeps
    // the per-kernel sequence.  Both give the same bits.
    void setup_predictor_chain() {
        const Dims& P = cfg_.predictor;
        const char* off = std::getenv("QWEN3_TTS_DISABLE_PREDICTOR_CHAIN");
        bool supported = false;
        if (off != nullptr && std::strcmp(off, "1") == 0) return;
        if (cfg_.talker.hidden != 2048 || P.hidden != 1024 || P.intermediate != 3072 || P.query_heads != 16 ||
            P.key_value_heads != 8 || P.head_dimension != 128 || P.layers != 5 || cfg_.predictor_vocab != 2048) {
            return;
        }
        check_hip(predictor_pass_supported(device_, &supported), "predictor pass support");
        if (!supported) return;
        pred_words_ = DeviceBuffer(predictor_pass_words() * sizeof(unsigned long long));
        check_hip(hipMemset(pred_words_.as<void>(), 0, pred_words_.bytes()), "zero predictor words");
        const int T2 = 2 * cfg_.talker.layers;
        PredictorPassArgs& c = pass_;
        c.s2m_w = m_.small_to_mtp_.data;
        c.s2m_s = m_.small_to_mtp_.scales;
        c.s2m_bias = m_.small_to_mtp_bias_;
        for (int l = 0; l < P.layers; ++l) {
            const Layer& L = m_.predictor_layers_[l];
            PredLayerArgs& d = c.layer[l];
            d.qkv_w = L.qkv.data;
            d.qkv_s = L.qkv.scales;
            d.o_w = L.o.data;
            d.o_s = L.o.scales;
            d.gu_w = L.gate_up.data;
            d.gu_s = L.gate_up.scales;
            d.d_w = L.down.data;
            d.d_s = L.down.scales;
            d.input_norm = L.input_norm;
            d.post_norm = L.post_norm;
            d.q_norm = L.q_norm;
            d.k_norm = L.k_norm;
            d.key_cache = host_bases_[T2 + l];
            d.value_cache = host_bases_[T2 + P.layers + l];
        }
        c.final_norm = m_.predictor_norm_;
        c.logits = logits_.as<bf16_t>();
        c.rope_table = m_.rope_table_.as<bf16_t>();
        c.words = pred_words_.as<unsigned long long>();
        c.epoch = reinterpret_cast<unsigned*>(ints_.as<int>() + 41);
        c.status = ints_.as<int>() + 40;
        c.hidden = P.hidden;
        c.intermediate = P.intermediate;
        c.query_heads = P.query_heads;
        c.key_value_heads = P.key_value_heads;
        c.input_width = cfg_.talker.hidden;
        c.vocabulary = cfg_.predictor_vocab;
        c.layers = P.layers;
        c.capacity = kCodebooks;
        c.epsilon = cfg_.eps;
        pred_chain_ = true;
    }

    // Predictor: 16 positions (talker.cu:1153-1220).
    void enqueue_predictor(const SamplingParams& ps) {
        if (pred_chain_) {
            enqueue_predictor_chain(ps);
            return;
        }
        const int H = cfg_.talker.hidden;
        const int PH = cfg_.predictor.hidden;
        const int PV = cfg_.predictor_vocab;
        for (int p = 0; p < kCodebooks; ++p) {
            // small_to_mtp projection + bias on: last hidden (p = 0), the
            // semantic token's codec embedding (p = 1) or the previous
            // residual code's embedding (p >= 2), read straight from the table.
            Gemv g(m_.small_to_mtp_, last_hidden_.as<bf16_t>(), H, PH, kEpiBias);
            if (p == 1) {
                g.a.input = m_.codec_embedding_;
                g.row_index(frame_tokens());
            } else if (p >= 2) {
                g.a.input = m_.predictor_embeddings_[p - 2];
                g.row_index(frame_tokens() + p - 1);
            }
            g.bias(m_.small_to_mtp_bias_).to(p_hidden_.as<bf16_t>()).run(stream_, "small_to_mtp");
            run_decoder(true, pred_positions() + p, p);
            if (p >= 1) {
                Gemv(m_.predictor_heads_[p - 1], p_hidden_.as<bf16_t>(), PH, PV, kEpiStore)
                    .norm(m_.predictor_norm_, cfg_.eps).to(logits_.as<bf16_t>()).run(stream_, "predictor head");
                check_hip(launch_sample_logits_ex(logits_.as<bf16_t>(), PV, false, cfg_.codec_eos, history_.as<int>(),
                                                  history_count_ptr(), 0, ps.do_sample, ps.top_k, ps.top_p, ps.temperature,
                                                  ps.penalty, random_state_.as<uint64_t>(), sampled_ptr(), frame_tokens(),
                                                  nullptr, p, nullptr, nullptr, stream_),
                          "predictor sample");
            }
        }
        check_hip(launch_pack_frame_codes(frame_tokens(), codes_.as<uint16_t>(), kCodebooks, stream_), "pack frame codes");
    }

    // The same 16 passes, one persistent launch each (the inputs of
    // small_to_mtp as above), each followed by its sampler.
    void enqueue_predictor_chain(const SamplingParams& ps) {
        const int PV = cfg_.predictor_vocab;
        for (int p = 0; p < kCodebooks; ++p) {
            PredictorPassArgs c = pass_;
            c.input = p == 0 ? last_hidden_.as<bf16_t>() : p == 1 ? m_.codec_embedding_ : m_.predictor_embeddings_[p - 2];
            c.input_row = p == 0 ? nullptr : frame_tokens() + (p == 1 ? 0 : p - 1);
            c.position = pred_positions() + p;
            if (p >= 1) {
                c.head_w = m_.predictor_heads_[p - 1].data;
                c.head_s = m_.predictor_heads_[p - 1].scales;
            }
            check_hip(launch_predictor_pass(c, stream_), "predictor pass");
            if (p >= 1) {
                check_hip(launch_sample_logits_ex(logits_.as<bf16_t>(), PV, false, cfg_.codec_eos, history_.as<int>(),
                                                  history_count_ptr(), 0, ps.do_sample, ps.top_k, ps.top_p, ps.temperature,
                                                  ps.penalty, random_state_.as<uint64_t>(), sampled_ptr(), frame_tokens(),
                                                  nullptr, p, nullptr, nullptr, stream_),
                          "predictor sample");
            }
        }
        check_hip(launch_pack_frame_codes(frame_tokens(), codes_.as<uint16_t>(), kCodebooks, stream_), "pack frame codes");
    }

    // Next talker input + talker step + sample (talker.cu:1222-1244,3546-3581).
    void enqueue_talker(const SamplingParams& ts) {
        const int H = cfg_.talker.hidden;
        check_hip(launch_sum_embeddings(m_.embedding_tables_.as<const bf16_t*>(), kCodebooks, cfg_.talker_vocab,
                                        cfg_.predictor_vocab, H, frame_tokens(), hidden_.as<bf16_t>(), stream_),
                  "sum codec embeddings");
        project_text(text_token_ptr(), true);
        run_decoder(false, position_ptr(), 0);
        emit_talker_logits();
        check_hip(launch_sample_logits_ex(logits_.as<bf16_t>(), cfg_.talker_vocab, true, cfg_.codec_eos, history_.as<int>(),
                                          history_count_ptr(), 0, ts.do_sample, ts.top_k, ts.top_p, ts.temperature, ts.penalty,
                                          random_state_.as<uint64_t>(), sampled_ptr(), frame_tokens(), nullptr, 0,
                                          history_.as<int>(), history_count_ptr(), stream_),
                  "talker sample");
        check_hip(launch_increment(position_ptr(), stream_), "advance position");
    }

    void release() {
        (void)hipSetDevice(device_);
        if (stream_) (void)hipStreamSynchronize(stream_);
        for (Graph* g : {&predictor_graph_, &talker_graph_}) {
            if (g->exec) (void)hipGraphExecDestroy(g->exec);
            g->exec = nullptr;
        }
        if (pinned_) (void)hipHostFree(pinned_);
        pinned_ = nullptr;
        for (hipEvent_t* e : {&start_, &stop_, &predictor_start_, &predictor_stop_, &codes_ready_, &semantic_ready_}) {
            if (*e) (void)hipEventDestroy(*e);
            *e = nullptr;
        }
        if (stream_) (void)hipStreamDestroy(stream_);
        stream_ = nullptr;
    }

    std::shared_ptr<Model> model_;
    Model& m_;
    Config cfg_;
    int device_;
    int max_seq_;
    hipStream_t stream_ = nullptr;
    hipEvent_t start_ = nullptr, stop_ = nullptr, predictor_start_ = nullptr, predictor_stop_ = nullptr;
    hipEvent_t codes_ready_ = nullptr, semantic_ready_ = nullptr;
    DeviceBuffer talker_k_, talker_v_, pred_k_, pred_v_;
    DeviceBuffer hidden_, p_hidden_, qkv_, attn_, attn_scratch_, act_, logits_, proj_, last_hidden_;
    DeviceBuffer ints_, history_, codes_, random_state_, kv_bases_;
    // Persistent predictor pass (pred_chain.hip): its tagged words, and the
    // static part of its arguments; ints_[40] status, ints_[41] epoch.
    DeviceBuffer pred_words_;
    PredictorPassArgs pass_{};
    bool pred_chain_ = false;
    std::vector<bf16_t*> host_bases_;
    int* pinned_ = nullptr;  // [0] sampled token, [1] text token, [8..] codes (u16), [20] predictor pass status
    Graph predictor_graph_, talker_graph_;
    PrefillBuffers prefill_;
    int position_ = 0;
    int history_count_ = 0;
    uint64_t frames_ = 0, device_samples_ = 0, host_syncs_ = 0;
    uint16_t semantic_ = 0;
    Qwen3TtsTalkerPhase phase_ = QWEN3_TTS_TALKER_CREATED;
    bool frame_in_flight_ = false, pending_copy_ = false, poisoned_ = false, pending_pass_status_ = false;
    uint64_t next_lease_ = 1, pending_lease_ = 0;
    uint32_t pending_position_ = 0;

public:
    // Batched-frame hooks (lockstep batch runner).
    bool poisoned() const { return poisoned_; }
    void poison() {
        poisoned_ = true;
        frame_in_flight_ = false;
        pending_copy_ = false;
        pending_lease_ = 0;
    }
};

using ModelBox = std::shared_ptr<Model>;

ModelBox& model_of(Qwen3TtsModelHandle h) {
    if (h == nullptr) throw std::runtime_error("model handle is null");
    return *static_cast<ModelBox*>(h);
}

Session* session_of(Qwen3TtsSessionHandle h) {
    if (h == nullptr) throw std::runtime_error("session handle is null");
    return static_cast<Session*>(h);
}

// protect, talker.cu:3791-3812
template <typename Op>
int32_t protect(Op&& op, int32_t failure, char* error, size_t capacity) {
    try {
        op();
        write_error(error, capacity, "");
        return QWEN3_TTS_TALKER_STATUS_OK;
    } catch (const DeviceFailure& e) {
        write_error(error, capacity, e.what());
        return QWEN3_TTS_TALKER_STATUS_CUDA;
    } catch (const std::bad_alloc& e) {
        write_error(error, capacity, e.what());
        return QWEN3_TTS_TALKER_STATUS_ALLOCATION;
    } catch (const std::invalid_argument& e) {
        write_error(error, capacity, e.what());
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    } catch (const std::exception& e) {
        write_error(error, capacity, e.what());
        return failure;
    }
}

Qwen3TtsModelConfigV1 default_config() {
    Qwen3TtsModelConfigV1 c{};
    c.struct_size = sizeof(c);
    // talker.cu:29-52
    c.talker_layers = 28;
    c.talker_hidden = 2048;
    c.talker_intermediate = 6144;
    c.talker_query_heads = 16;
    c.talker_key_value_heads = 8;
    c.predictor_layers = 5;
    c.predictor_hidden = 1024;
    c.predictor_intermediate = 3072;
    c.predictor_query_heads = 16;
    c.predictor_key_value_heads = 8;
    c.head_dimension = 128;
    c.talker_vocabulary = 3072;
    c.predictor_vocabulary = 2048;
    c.text_vocabulary = 151936;
    c.codec_eos_token = 2150;
    c.rms_epsilon = 1.0e-6f;
    c.rope_theta = 1.0e6f;
    return c;
}


// ---------------------------------------------------------------------------
// Lockstep batch of up to 8 sessions (talker.cu:1352-1969): one frame for all
// sessions with every weight matrix read once.  Row semantics are those of
// the reference's batched int8 decoder (talker.cu:2038-2334): fused QKV,
// fast attention, fma residual epilogue, fused gate/up SiLU.  KV caches,
// sampler state, histories and events stay session-local; per-frame values
// reach the (graph-captured) kernels through device tables refreshed from
// pinned host memory before each launch.
// ---------------------------------------------------------------------------
class BatchRunner {
public:
    static constexpr int kCapacity = kMaxBatch;
    static constexpr int kSlots = kCodebooks + 1;  // predictor positions 0..15, talker

    explicit BatchRunner(Model& m) : m_(m), cfg_(m.config()), device_(m.device_index()) {
        check_hip(hipSetDevice(device_), "hipSetDevice(batch)");
        check_hip(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate(batch)");
        for (hipEvent_t& e : join_) check_hip(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate(join)");
        const Dims& T = cfg_.talker;
        const Dims& P = cfg_.predictor;
        const size_t b = sizeof(bf16_t);
        const size_t R = kCapacity;
        hidden_ = DeviceBuffer(R * T.hidden * b);
        normalized_ = DeviceBuffer(R * T.hidden * b);
        p_hidden_ = DeviceBuffer(R * P.hidden * b);
        text_input_ = DeviceBuffer(R * T.hidden * b);
        proj_ = DeviceBuffer(R * T.hidden * b);
        qkv_ = DeviceBuffer(R * std::max(T.qkv_width(), P.qkv_width()) * b);
        attn_ = DeviceBuffer(R * std::max(T.query_width(), P.query_width()) * b);
        attn_scratch_ = DeviceBuffer(attention_split_workspace_bytes(static_cast<int>(R),
                                                                     std::max(T.query_heads, P.query_heads),
                                                                     kAttentionCapacity, kAttentionSplits));
        act_ = DeviceBuffer(R * std::max(T.intermediate, P.intermediate) * b);
        logits_ = DeviceBuffer(R * std::max(cfg_.talker_vocab, cfg_.predictor_vocab) * b);
        layers_ = T.layers + P.layers;
        table_bytes_ = off_codes() + kCapacity * sizeof(void*);
        tables_ = DeviceBuffer(table_bytes_);
        for (int k = 0; k < kStaging; ++k) {
            check_hip(hipHostMalloc(&staging_[k], table_bytes_, hipHostMallocDefault), "hipHostMalloc(batch tables)");
            std::memset(staging_[k], 0, table_bytes_);
            check_hip(hipEventCreateWithFlags(&staged_[k], hipEventDisableTiming), "hipEventCreate(batch tables)");
        }
    }
    ~BatchRunner() {
        (void)hipSetDevice(device_);
        if (stream_) (void)hipStreamSynchronize(stream_);
        destroy_graphs();
        for (int k = 0; k < kStaging; ++k) {
            if (staging_[k]) (void)hipHostFree(staging_[k]);
            if (staged_[k]) (void)hipEventDestroy(staged_[k]);
        }
        for (hipEvent_t e : join_) if (e) (void)hipEventDestroy(e);
        if (stream_) (void)hipStreamDestroy(stream_);
    }

    void begin(Session** s, int n, const int* trailing, const Qwen3TtsSamplingConfig* ts,
               const Qwen3TtsSamplingConfig* ps, Qwen3TtsDeviceFrameViewV2* views) {
        check_hip(hipSetDevice(device_), "hipSetDevice(batch frame)");
        std::vector<SamplingParams> tp(n), pp(n);
        for (int i = 0; i < n; ++i) {
            if (s[i]->model() != &m_) throw std::runtime_error("batched session belongs to a different model");
            for (int j = 0; j < i; ++j) {
                if (s[j] == s[i]) throw std::runtime_error("a session appears twice in the batch");
            }
            s[i]->validate_frame(s[i]->semantic_, trailing[i]);
            tp[i] = params_of(ts[i]);
            pp[i] = params_of(ps[i]);
        }
        for (int i = 0; i < n; ++i) {
            Session* c = s[i];
            const uint64_t lease = c->next_lease_++;
            if (c->next_lease_ == 0) c->next_lease_ = 1;
            c->frame_in_flight_ = true;
            c->pending_pass_status_ = false;
            c->pending_copy_ = false;
            c->pending_lease_ = lease;
            c->pending_position_ = static_cast<uint32_t>(c->position_);
        }
        // The host tables are staged in a ring of pinned buffers: the upload
        // of an earlier batch may still wait behind its sessions' work, so a
        // buffer is refilled only after its own upload has completed.
        current_ = next_staging_;
        next_staging_ = (next_staging_ + 1) % kStaging;
        if (staged_used_[current_]) check_hip(hipEventSynchronize(staged_[current_]), "hipEventSynchronize(batch tables)");
        fill_tables(s, n, trailing, tp, pp);
        // A captured frame bakes only the row count, the GEMV mode and the
        // largest session capacity (attention grid and bound); everything
        // session-specific reaches the kernels through the tables.  Graph
        // sets for a few such keys are kept, so batches of different
        // compositions alternate without re-capture.
        int max_capacity = kCodebooks;
        for (int i = 0; i < n; ++i) max_capacity = std::max(max_capacity, s[i]->max_seq_);
        const GraphKey key{n, batch_gemv_mode(), max_capacity};
        try {
            for (int i = 0; i < n; ++i) {
                check_hip(hipEventRecord(join_[i], s[i]->stream_), "hipEventRecord(join)");
                check_hip(hipStreamWaitEvent(stream_, join_[i], 0), "hipStreamWaitEvent(join)");
            }
            GraphSet& graphs = graph_set(key);
            check_hip(hipMemcpyAsync(tables_.as<void>(), staging_[current_], table_bytes_, hipMemcpyHostToDevice, stream_),
                      "upload batch tables");
            check_hip(hipEventRecord(staged_[current_], stream_), "hipEventRecord(batch tables)");
            staged_used_[current_] = true;
            for (int i = 0; i < n; ++i) check_hip(hipEventRecord(s[i]->predictor_start_, stream_), "hipEventRecord");
            run_graph(graphs, graphs.predictor, [&] { enqueue_predictor(n, key.mode); });
            for (int i = 0; i < n; ++i) {
                check_hip(hipEventRecord(s[i]->predictor_stop_, stream_), "hipEventRecord");
                check_hip(hipEventRecord(s[i]->codes_ready_, stream_), "hipEventRecord");
                check_hip(hipEventRecord(s[i]->start_, stream_), "hipEventRecord");
            }
            run_graph(graphs, graphs.talker, [&] { enqueue_talker(n, key.mode, key.capacity); });
            for (int i = 0; i < n; ++i) {
                Session* c = s[i];
                check_hip(hipEventRecord(c->stop_, stream_), "hipEventRecord");
                check_hip(hipMemcpyAsync(c->pinned_, c->sampled_ptr(), sizeof(int), hipMemcpyDeviceToHost, stream_),
                          "copy sampled token");
                check_hip(hipEventRecord(c->semantic_ready_, stream_), "hipEventRecord(semantic ready)");
                check_hip(hipStreamWaitEvent(c->stream_, c->semantic_ready_, 0), "hipStreamWaitEvent(session)");
                c->device_samples_ += kCodebooks;
                ++c->history_count_;
                ++c->position_;
            }
        } catch (...) {
            for (int i = 0; i < n; ++i) s[i]->poison();
            (void)hipStreamSynchronize(stream_);
            destroy_graphs();
            throw;
        }
        for (int i = 0; i < n; ++i) views[i] = s[i]->view(s[i]->pending_lease_);
    }

private:
    // Table layout (identical in pinned host memory and in device memory):
    // positions int[kSlots][8] | K/V bases ptr[2*layers][8] | token bases ptr[8] |
    // trailing-token ptrs ptr[8] | last_hidden ptrs ptr[8] | position ptrs ptr[8] |
    // trailing tokens int[8] | talker value-cache strides int[8] |
    // sampler arguments SampleArgs[16 samples per frame][8] | code rows uint16_t*[8]
    size_t off_kv() const { return kSlots * kCapacity * sizeof(int); }
    size_t off_tokens() const { return off_kv() + 2 * layers_ * kCapacity * sizeof(void*); }
    size_t off_trail_ptrs() const { return off_tokens() + kCapacity * sizeof(void*); }
    size_t off_last() const { return off_trail_ptrs() + kCapacity * sizeof(void*); }
    size_t off_pos_ptrs() const { return off_last() + kCapacity * sizeof(void*); }
    size_t off_trail_values() const { return off_pos_ptrs() + kCapacity * sizeof(void*); }
    size_t off_strides() const { return off_trail_values() + kCapacity * sizeof(int); }
    size_t off_samples() const {
        return (off_strides() + kCapacity * sizeof(int) + alignof(SampleArgs) - 1) / alignof(SampleArgs) *
               alignof(SampleArgs);
    }
    size_t off_codes() const {
        return (off_samples() + static_cast<size_t>(kCodebooks) * kCapacity * sizeof(SampleArgs) + alignof(void*) - 1) /
               alignof(void*) * alignof(void*);
    }
    template <typename T>
    T* dev_at(size_t offset) const { return reinterpret_cast<T*>(tables_.as<char>() + offset); }
    template <typename T>
    T* host_at(size_t offset) const { return reinterpret_cast<T*>(static_cast<char*>(staging_[current_]) + offset); }

    int* positions(int slot) const { return dev_at<int>(0) + slot * kCapacity; }
    bf16_t* const* kv_table(int layer_slot, bool value) const {
        return dev_at<bf16_t*>(off_kv()) + (2 * layer_slot + (value ? 1 : 0)) * kCapacity;
    }
    const int* const* token_bases() const { return dev_at<const int*>(off_tokens()); }
    const int* const* trailing_ptrs() const { return dev_at<const int*>(off_trail_ptrs()); }
    bf16_t* const* last_hidden_ptrs() const { return dev_at<bf16_t*>(off_last()); }
    int* const* position_ptrs() const { return dev_at<int*>(off_pos_ptrs()); }
    const int* value_strides() const { return dev_at<int>(off_strides()); }
    // sampler rows of sample `slot` (0: talker, 1..15: predictor codebooks)
    const SampleArgs* sample_rows(int slot) const {
        return dev_at<SampleArgs>(off_samples()) + static_cast<size_t>(slot) * kCapacity;
    }

    void fill_tables(Session** s, int n, const int* trailing, const std::vector<SamplingParams>& tp,
                     const std::vector<SamplingParams>& pp) {
        int* pos = host_at<int>(0);
        for (int slot = 0; slot < kCodebooks; ++slot)
            for (int i = 0; i < kCapacity; ++i) pos[slot * kCapacity + i] = slot;
        for (int i = 0; i < kCapacity; ++i) pos[kCodebooks * kCapacity + i] = i < n ? s[i]->position_ : 0;
        bf16_t** kv = host_at<bf16_t*>(off_kv());
        const int TL = cfg_.talker.layers, PL = cfg_.predictor.layers;
        const int* trail_dev = dev_at<int>(off_trail_values());
        for (int i = 0; i < n; ++i) {
            const std::vector<bf16_t*>& hb = s[i]->host_bases_;
            for (int l = 0; l < TL; ++l) {
                kv[(2 * l) * kCapacity + i] = hb[l];
                kv[(2 * l + 1) * kCapacity + i] = hb[TL + l];
            }
            for (int l = 0; l < PL; ++l) {
                kv[(2 * (TL + l)) * kCapacity + i] = hb[2 * TL + l];
                kv[(2 * (TL + l) + 1) * kCapacity + i] = hb[2 * TL + PL + l];
            }
            host_at<const int*>(off_tokens())[i] = s[i]->frame_tokens();
            host_at<uint16_t*>(off_codes())[i] = s[i]->codes_.as<uint16_t>();
            host_at<const int*>(off_trail_ptrs())[i] = trail_dev + i;
            host_at<bf16_t*>(off_last())[i] = s[i]->last_hidden_.as<bf16_t>();
            host_at<int*>(off_pos_ptrs())[i] = s[i]->position_ptr();
            host_at<int>(off_trail_values())[i] = trailing[i];
            host_at<int>(off_strides())[i] = value_cache_stride(s[i]->max_seq_);
            // sampler rows: the talker's sample (mask, penalty, history
            // append) and the 15 predictor samples (frame token p)
            SampleArgs* rows = host_at<SampleArgs>(off_samples());
            Session* c = s[i];
            for (int slot = 0; slot < kCodebooks; ++slot) {
                const bool talker = slot == 0;
                const SamplingParams& q = talker ? tp[i] : pp[i];
                const int vocab = talker ? cfg_.talker_vocab : cfg_.predictor_vocab;
                SampleArgs a{};
                a.logits = logits_.as<bf16_t>() + static_cast<size_t>(i) * vocab;
                a.vocabulary = vocab;
                a.suppress = talker;
                a.eos = cfg_.codec_eos;
                a.history = c->history_.as<int>();
                a.history_count = c->history_count_ptr();
                a.do_sample = q.do_sample;
                a.top_k = q.top_k;
                a.top_p = q.top_p;
                a.temperature = q.temperature;
                a.penalty = q.penalty;
                a.random_state = c->random_state_.as<uint64_t>();
                a.selected = c->sampled_ptr();
                a.store_tokens = c->frame_tokens();
                a.store_index_fallback = slot;
                a.append_history = talker ? c->history_.as<int>() : nullptr;
                a.append_count = talker ? c->history_count_ptr() : nullptr;
                if (!sample_args_valid(a)) throw std::invalid_argument("invalid sampler arguments");
                rows[static_cast<size_t>(slot) * kCapacity + i] = a;
            }
        }
    }

    struct GraphKey {
        int rows, mode, capacity;
        bool operator==(const GraphKey& o) const { return rows == o.rows && mode == o.mode && capacity == o.capacity; }
    };
    struct GraphSet {
        GraphKey key;
        hipGraphExec_t predictor = nullptr, talker = nullptr;
        int uncaptured = 0;  // eager enqueues so far (the first frame runs eagerly)
        uint64_t last_use = 0;
    };
    static constexpr size_t kGraphSets = 4;

    // The graph set of `key`, created on first use; the least recently used
    // set is evicted when kGraphSets are held (after the stream has drained:
    // its graphs may still be queued).
    GraphSet& graph_set(const GraphKey& key) {
        for (GraphSet& g : graphs_) {
            if (g.key == key) {
                g.last_use = ++use_clock_;
                return g;
            }
        }
        if (graphs_.size() >= kGraphSets) {
            auto victim = std::min_element(graphs_.begin(), graphs_.end(),
                                           [](const GraphSet& a, const GraphSet& b) { return a.last_use < b.last_use; });
            check_hip(hipStreamSynchronize(stream_), "hipStreamSynchronize(evict batch graphs)");
            destroy(*victim);
            graphs_.erase(victim);
        }
        graphs_.push_back(GraphSet{key});
        graphs_.back().last_use = ++use_clock_;
        return graphs_.back();
    }

    static void destroy(GraphSet& g) {
        for (hipGraphExec_t* e : {&g.predictor, &g.talker}) {
            if (*e) (void)hipGraphExecDestroy(*e);
            *e = nullptr;
        }
    }

    template <typename Enqueue>
    void run_graph(GraphSet& set, hipGraphExec_t& exec, Enqueue&& enqueue) {
        if (exec != nullptr) {
            check_hip(hipGraphLaunch(exec, stream_), "hipGraphLaunch(batch)");
            return;
        }
        if (set.uncaptured < 2 || !Session::graphs_enabled()) {
            enqueue();
            ++set.uncaptured;
            return;
        }
        check_hip(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture(batch)");
        try {
            enqueue();
        } catch (...) {
            hipGraph_t aborted = nullptr;
            (void)hipStreamEndCapture(stream_, &aborted);
            if (aborted) (void)hipGraphDestroy(aborted);
            throw;
        }
        hipGraph_t graph = nullptr;
        check_hip(hipStreamEndCapture(stream_, &graph), "hipStreamEndCapture(batch)");
        const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        (void)hipGraphDestroy(graph);
        check_hip(st, "hipGraphInstantiate(batch)");
        check_hip(hipGraphLaunch(exec, stream_), "hipGraphLaunch(batch)");
    }

    void destroy_graphs() {
        for (GraphSet& g : graphs_) destroy(g);
        graphs_.clear();
    }

    void run_decoder(bool predictor, int n, int mode, const int* pos, int capacity) {
        const Dims& d = predictor ? cfg_.predictor : cfg_.talker;
        const std::vector<Layer>& layers = predictor ? m_.predictor_layers_ : m_.talker_layers_;
        bf16_t* hidden = predictor ? p_hidden_.as<bf16_t>() : hidden_.as<bf16_t>();
        const int slot0 = predictor ? cfg_.talker.layers : 0;
        for (int l = 0; l < d.layers; ++l) {
            const Layer& L = layers[l];
            Gemv(L.qkv, hidden, d.hidden, d.qkv_width(), kEpiStore).norm(L.input_norm, cfg_.eps).rows(n, mode)
                .to(qkv_.as<bf16_t>()).run(stream_, "batch QKV GEMV");
            check_hip(launch_decode_attention(false, qkv_.as<bf16_t>(), d.qkv_width(), L.q_norm, L.k_norm,
                                              m_.rope_table_.as<bf16_t>(), cfg_.eps, kv_table(slot0 + l, false),
                                              kv_table(slot0 + l, true), nullptr, nullptr, pos, attn_.as<bf16_t>(), n,
                                              d.query_heads, d.key_value_heads, d.head_dimension, capacity,
                                              attn_scratch_.as<float>(), predictor ? nullptr : value_strides(), stream_,
                                              (mode == kModeMfma || (mode == kModeAuto && n >= 2)) ? kAttentionSplits : 1),
                      "batch q/k norm + RoPE + KV append + attention");
            Gemv(L.o, attn_.as<bf16_t>(), d.query_width(), d.hidden, kEpiAddFma).rows(n, mode).to(hidden)
                .run(stream_, "batch O GEMV");
            Gemv(L.gate_up, hidden, d.hidden, d.intermediate, kEpiSiluFused).norm(L.post_norm, cfg_.eps).rows(n, mode)
                .to(act_.as<bf16_t>()).run(stream_, "batch gate/up GEMV");
            Gemv(L.down, act_.as<bf16_t>(), d.intermediate, d.hidden, kEpiAddFma).rows(n, mode).to(hidden)
                .run(stream_, "batch down GEMV");
        }
    }

    void enqueue_predictor(int n, int mode) {
        const int H = cfg_.talker.hidden, PH = cfg_.predictor.hidden, PV = cfg_.predictor_vocab;
        bf16_t* input = text_input_.as<bf16_t>();
        for (int p = 0; p < kCodebooks; ++p) {
            if (p == 0) {
                check_hip(launch_gather_rows(reinterpret_cast<const bf16_t* const*>(last_hidden_ptrs()), n, H, input, stream_),
                          "gather last hidden");
            } else if (p == 1) {
                check_hip(launch_gather_embedding_rows(m_.codec_embedding_, cfg_.talker_vocab, H, token_bases(), 0, input, n, stream_),
                          "gather semantic embedding");
            } else {
                check_hip(launch_gather_embedding_rows(m_.predictor_embeddings_[p - 2], PV, H, token_bases(), p - 1, input, n, stream_),
                          "gather residual embedding");
            }
            Gemv(m_.small_to_mtp_, input, H, PH, kEpiBias).bias(m_.small_to_mtp_bias_).rows(n, mode)
                .to(p_hidden_.as<bf16_t>()).run(stream_, "batch small_to_mtp");
            run_decoder(true, n, mode, positions(p), kCodebooks);
            if (p >= 1) {
                Gemv(m_.predictor_heads_[p - 1], p_hidden_.as<bf16_t>(), PH, PV, kEpiStore).norm(m_.predictor_norm_, cfg_.eps)
                    .rows(n, mode).to(logits_.as<bf16_t>()).run(stream_, "batch predictor head");
                check_hip(launch_sample_rows(sample_rows(p), n, stream_), "batch predictor sample");
            }
        }
        check_hip(launch_pack_frame_codes_rows(token_bases(), dev_at<uint16_t* const>(off_codes()), kCodebooks, n, stream_),
                  "pack frame codes");
    }

    void enqueue_talker(int n, int mode, int max_capacity) {
        const int H = cfg_.talker.hidden, TV = cfg_.talker_vocab;
        check_hip(launch_sum_embeddings_rows(m_.embedding_tables_.as<const bf16_t*>(), kCodebooks, TV, cfg_.predictor_vocab, H,
                                             token_bases(), hidden_.as<bf16_t>(), n, stream_),
                  "batch codec embeddings");
        check_hip(launch_gather_embedding_rows(m_.text_embedding_, cfg_.text_vocab, H, trailing_ptrs(), 0,
                                               text_input_.as<bf16_t>(), n, stream_),
                  "gather text embedding");
        Gemv(m_.text_fc1_, text_input_.as<bf16_t>(), H, H, kEpiBiasSilu).bias(m_.text_fc1_bias_).rows(n, mode)
            .to(proj_.as<bf16_t>()).run(stream_, "batch text fc1");
        Gemv(m_.text_fc2_, proj_.as<bf16_t>(), H, H, kEpiBiasAdd).bias(m_.text_fc2_bias_).rows(n, mode)
            .to(hidden_.as<bf16_t>()).run(stream_, "batch text fc2");
        run_decoder(false, n, mode, positions(kCodebooks), max_capacity);
        check_hip(launch_rms_norm_rows(hidden_.as<bf16_t>(), m_.talker_norm_, normalized_.as<bf16_t>(), n, H, cfg_.eps, stream_),
                  "batch talker final norm");
        check_hip(launch_scatter_rows(normalized_.as<bf16_t>(), last_hidden_ptrs(), n, H, stream_), "scatter last hidden");
        Gemv(m_.codec_head_, normalized_.as<bf16_t>(), H, TV, kEpiStore).rows(n, mode).to(logits_.as<bf16_t>())
            .run(stream_, "batch codec head");
        check_hip(launch_sample_rows(sample_rows(0), n, stream_), "batch talker sample");
        check_hip(launch_increment_each(position_ptrs(), n, stream_), "advance positions");
    }

    Model& m_;
    Config cfg_;
    int device_;
    int layers_ = 0;
    hipStream_t stream_ = nullptr;
    std::array<hipEvent_t, kCapacity> join_{};
    DeviceBuffer hidden_, normalized_, p_hidden_, text_input_, proj_, qkv_, attn_, attn_scratch_, act_, logits_, tables_;
    size_t table_bytes_ = 0;
    static constexpr int kStaging = 2;
    void* staging_[kStaging] = {};
    hipEvent_t staged_[kStaging] = {};
    bool staged_used_[kStaging] = {};
    int current_ = 0, next_staging_ = 0;
    std::vector<GraphSet> graphs_;
    uint64_t use_clock_ = 0;
};

void delete_batch_runner(BatchRunner* r) { delete r; }

void batch_begin_frames(Model* model, Session** s, int n, const int* trailing,
                        const Qwen3TtsSamplingConfig* ts, const Qwen3TtsSamplingConfig* ps,
                        Qwen3TtsDeviceFrameViewV2* views) {
    if (model == nullptr || s == nullptr || n <= 0 || n > kMaxBatch) {
        throw std::invalid_argument("invalid batch frame arguments");
    }
    if (!model->finalized()) throw std::runtime_error("model weights must be finalized");
    std::lock_guard<std::mutex> lock(model->batch_mutex());
    if (!model->batch_) {
        model->batch_ = std::unique_ptr<BatchRunner, void (*)(BatchRunner*)>(new BatchRunner(*model), delete_batch_runner);
    }
    model->batch_->begin(s, n, trailing, ts, ps, views);
}

}  // namespace

}  // namespace q3

using namespace q3;

extern "C" {

QWEN3_TTS_API uint32_t qwen3_tts_talker_abi_version(void) { return QWEN3_TTS_TALKER_ABI_VERSION; }

QWEN3_TTS_API void qwen3_tts_model_config_default(Qwen3TtsModelConfigV1* output) {
    if (output != nullptr) *output = default_config();
}

QWEN3_TTS_API int32_t qwen3_tts_model_create_with_config(int32_t device_index, const Qwen3TtsModelConfigV1* config,
                                                         Qwen3TtsModelHandle* output, char* error, size_t cap) {
    if (output == nullptr || config == nullptr || config->struct_size != sizeof(Qwen3TtsModelConfigV1)) {
        write_error(error, cap, "model output handle or config is null or has the wrong struct_size");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] { *output = new ModelBox(std::make_shared<Model>(device_index, config_from(*config))); },
                   QWEN3_TTS_TALKER_STATUS_MODEL, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_model_create(int32_t device_index, Qwen3TtsModelHandle* output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "model output handle pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    const Qwen3TtsModelConfigV1 c = default_config();
    return qwen3_tts_model_create_with_config(device_index, &c, output, error, cap);
}

QWEN3_TTS_API void qwen3_tts_model_destroy(Qwen3TtsModelHandle handle) { delete static_cast<ModelBox*>(handle); }

QWEN3_TTS_API int32_t qwen3_tts_model_upload_tensor(Qwen3TtsModelHandle handle, const char* name, const void* data,
                                                    uint64_t byte_size, int32_t rank, const uint64_t* shape,
                                                    char* error, size_t cap) {
    return protect([&] { model_of(handle)->upload_tensor(name, data, byte_size, rank, shape); },
                   QWEN3_TTS_TALKER_STATUS_MODEL, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_model_finalize(Qwen3TtsModelHandle handle, Qwen3TtsModelMemory* memory, char* error,
                                               size_t cap) {
    if (memory == nullptr) {
        write_error(error, cap, "talker memory output pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] { *memory = model_of(handle)->finalize(); }, QWEN3_TTS_TALKER_STATUS_MODEL, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_create(Qwen3TtsModelHandle model, int32_t max_sequence_length, uint64_t seed,
                                               Qwen3TtsSessionHandle* output, Qwen3TtsSessionMemory* memory,
                                               char* error, size_t cap) {
    if (output == nullptr || memory == nullptr) {
        write_error(error, cap, "session output or memory pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] {
        auto created = std::make_unique<Session>(model_of(model), max_sequence_length, seed);
        *memory = created->memory();
        *output = created.release();
    }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API void qwen3_tts_session_destroy(Qwen3TtsSessionHandle handle) { delete static_cast<Session*>(handle); }

QWEN3_TTS_API int32_t qwen3_tts_session_reset(Qwen3TtsSessionHandle handle, uint64_t seed, char* error, size_t cap) {
    return protect([&] { session_of(handle)->reset(seed); }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_prefill(Qwen3TtsSessionHandle handle, const int32_t* text, const int32_t* codec,
                                                int32_t count, Qwen3TtsSamplingConfig sampling,
                                                Qwen3TtsTalkerPrefillResult* output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "prefill output pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] { *output = session_of(handle)->prefill(text, codec, count, sampling); },
                   QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_next_frame(Qwen3TtsSessionHandle handle, uint16_t semantic, int32_t text_token,
                                                   Qwen3TtsSamplingConfig ts, Qwen3TtsSamplingConfig ps,
                                                   uint16_t* codes, size_t code_capacity, uint16_t* next_semantic,
                                                   Qwen3TtsCodecFrameInfo* info, char* error, size_t cap) {
    if (codes == nullptr || code_capacity < kCodebooks || next_semantic == nullptr || info == nullptr) {
        write_error(error, cap, "codec-frame outputs are null or undersized");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] {
        const Qwen3TtsCodecFrameResult f = session_of(handle)->next_frame(semantic, text_token, ts, ps);
        std::copy_n(f.codes, kCodebooks, codes);
        *next_semantic = f.next_semantic_token;
        info->talker_position = f.talker_position;
        info->ended_by_eos = f.ended_by_eos;
        info->predictor_gpu_milliseconds = f.predictor_gpu_milliseconds;
        info->talker_gpu_milliseconds = f.talker_gpu_milliseconds;
    }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_next_frame_begin_v2(Qwen3TtsSessionHandle handle, int32_t text_token,
                                                            Qwen3TtsSamplingConfig ts, Qwen3TtsSamplingConfig ps,
                                                            Qwen3TtsDeviceFrameViewV2* output, char* error,
                                                            size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "device-frame output is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    if (output->struct_size != sizeof(Qwen3TtsDeviceFrameViewV2) || output->reserved != 0) {
        write_error(error, cap, "device-frame output has an unsupported size or nonzero reserved field");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] {
        Session* s = session_of(handle);
        *output = s->begin_frame(s->current_semantic(), text_token, ts, ps, false);
    }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_next_frame_finish_v2(Qwen3TtsSessionHandle handle, uint64_t lease,
                                                             Qwen3TtsCudaEventHandle consumer_done,
                                                             uint16_t* next_semantic, Qwen3TtsCodecFrameInfo* info,
                                                             char* error, size_t cap) {
    if (next_semantic == nullptr || info == nullptr) {
        write_error(error, cap, "device-frame finish outputs are null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] {
        const Qwen3TtsCodecFrameResult f = session_of(handle)->finish_frame(lease, consumer_done);
        *next_semantic = f.next_semantic_token;
        info->talker_position = f.talker_position;
        info->ended_by_eos = f.ended_by_eos;
        info->predictor_gpu_milliseconds = f.predictor_gpu_milliseconds;
        info->talker_gpu_milliseconds = f.talker_gpu_milliseconds;
    }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_model_batch_next_frame_begin_v2(
    Qwen3TtsModelHandle model_handle, Qwen3TtsSessionHandle* sessions, int32_t count, const int32_t* trailing,
    const Qwen3TtsSamplingConfig* ts, const Qwen3TtsSamplingConfig* ps, Qwen3TtsDeviceFrameViewV2* outputs,
    char* error, size_t cap) {
    if (sessions == nullptr || count <= 0 || count > QWEN3_TTS_MAX_BATCH_SESSIONS || trailing == nullptr ||
        ts == nullptr || ps == nullptr || outputs == nullptr) {
        write_error(error, cap, "batch frame arguments are null or out of range");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    for (int32_t i = 0; i < count; ++i) {
        if (sessions[i] == nullptr || outputs[i].struct_size != sizeof(Qwen3TtsDeviceFrameViewV2) ||
            outputs[i].reserved != 0) {
            write_error(error, cap, "batch frame outputs have an unsupported size or nonzero reserved field");
            return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
        }
    }
    return protect([&] {
        Session* s[QWEN3_TTS_MAX_BATCH_SESSIONS];
        for (int32_t i = 0; i < count; ++i) s[i] = session_of(sessions[i]);
        batch_begin_frames(model_of(model_handle).get(), s, count, trailing, ts, ps, outputs);
    }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_state_info(Qwen3TtsSessionHandle handle, Qwen3TtsTalkerStateInfo* output,
                                                   char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "session state output pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return protect([&] { *output = session_of(handle)->state_info(); }, QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_read_talker_cache_v1(Qwen3TtsSessionHandle handle, int32_t layer, int32_t which,
                                                             int32_t count, void* destination, uint64_t bytes,
                                                             char* error, size_t cap) {
    return protect([&] { session_of(handle)->read_talker_cache(layer, which, count, destination, bytes); },
                   QWEN3_TTS_TALKER_STATUS_STATE, error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_session_read_last_hidden_v1(Qwen3TtsSessionHandle handle, void* destination,
                                                            uint64_t bytes, char* error, size_t cap) {
    return protect([&] { session_of(handle)->read_last_hidden(destination, bytes); }, QWEN3_TTS_TALKER_STATUS_STATE,
                   error, cap);
}

}  // extern "C"
