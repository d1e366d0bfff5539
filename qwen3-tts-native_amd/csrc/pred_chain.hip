// Persistent code-predictor pass for gfx950: one pass of the 15-step code
// predictor (native/qwen3-tts-native/native/src/talker.cu:1153-1220) in ONE
// launch -- the small_to_mtp projection, the five decoder layers (QKV +
// RMSNorm, q/k norm + RoPE + KV append + exact attention, O + residual,
// gate/up + RMSNorm + SiLU, down + residual) and the codebook head with the
// final RMSNorm -- bit-identical to the per-kernel sequence of the same pass
// (gemv_exact_fixed for every GEMV, attention_short_kernel's arithmetic for
// the attention).  The sampler that follows each head stays its own launch.
//
// Why: the predictor's weights (about 15 MB per layer) stay in the Infinity
// Cache, so each of the ~23 kernels of a pass sits at a launch-latency floor
// of 3-5 us.  Here a stage hands its outputs to the next through tagged
// words (csrc/chain_device.hpp) and the weights of the next layer are
// already in registers when its input arrives.
//
// Layout: 256 workgroups (one per CU, all resident), 12 waves each.
//   * 8 compute waves own fixed output rows of every GEMV, with the
//     reference's k-assignment (int8_gemv.cu:67-125: lane l of 32 owns the
//     16-byte vectors l, l+32, ...; fresh 16-term fmaf chains added in
//     order; shuffle-down fold 16..1):
//       small_to_mtp  rows 4b..4b+3, one per wave 0-3 (K = 2048: the two
//                     halves of the wave take vectors j = 0,1 and 2,3)
//       QKV           rows 16b..16b+15, one per half-wave (K = 1024)
//       O             rows 4b..4b+3, as small_to_mtp (K = 2048)
//       gate/up       units 12b..12b+11 (gate row u, up row 3072 + u), one
//                     per half-wave 0-11
//       down          rows 4b..4b+3, one per wave 0-3 (K = 3072: halves take
//                     j = 0..2 and 3..5)
//       head          rows 8b..8b+7, one per half-wave 0-7
//     and in workgroups 0-15, wave 0 runs the attention of query head b.
//   * 4 waves poll the stage inputs, compute the RMSNorm statistic in the
//     reference's 256-thread order and apply the epilogues.
// Every wait is bounded: a poll that sees no progress for ~0.1 s sets the
// status word and every later poll gives up, so the grid always drains.
#include <mutex>

#include "chain_device.hpp"
#include "short_attention.hpp"

// Build-time diagnostic: -DQ3_PRED_TRACE records, for workgroup 0, the
// wall-clock time at which each stage's input was staged and its outputs
// published (q3_pred_trace, read by qwen3_tts_debug_pred_trace).  Off in the
// library build.
#ifdef Q3_PRED_TRACE
__device__ unsigned long long q3_pred_trace[128];
#define PRED_STAMP(i)                                                              \
    do {                                                                           \
        if (blockIdx.x == 0 && (threadIdx.x & 255) == 0) q3_pred_trace[i] = wall_clock64(); \
    } while (0)
#else
#define PRED_STAMP(i) \
    do {              \
    } while (0)
#endif

namespace q3 {
namespace {

using namespace gemv_detail;
using namespace chain_detail;

constexpr int kGrid = 256;
constexpr int kComputeWaves = 8;
constexpr int kPassThreads = 64 * kComputeWaves + kPollThreads;
constexpr int kPH = 1024;     // predictor hidden
constexpr int kPI = 3072;     // predictor intermediate
constexpr int kQkv = 4096;    // fused q|k|v rows
constexpr int kQW = 2048;     // query width (16 heads x 128)
constexpr int kKvW = 1024;    // key/value width (8 heads x 128)
constexpr int kTH = 2048;     // talker hidden: small_to_mtp input width
constexpr int kVocab = 2048;  // codebook head rows
constexpr int kLayers = 5;
constexpr int kHeads = 16;
constexpr int kGroup = 2;     // query heads per kv head
// Tagged word areas (two bf16 values per word).
constexpr int kWordsH = kPH / 2, kWordsQkv = kQkv / 2, kWordsAtt = kQW / 2, kWordsAct = kPI / 2;
constexpr int kOffHA = 0, kOffHB = kOffHA + kWordsH, kOffQkv = kOffHB + kWordsH, kOffAtt = kOffQkv + kWordsQkv,
              kOffAct = kOffAtt + kWordsAtt;
constexpr int kWordsTotal = kOffAct + kWordsAct;
// Tags: small_to_mtp base; layer l: QKV base+1+5l, attention +2, O +3,
// gate/up +4, down +5; the epoch advances by kTagsPerPass per launch.
constexpr unsigned kTagsPerPass = 27;

struct PredArgs {
    const int8_t* s2m_w;
    const float* s2m_s;
    const bf16_t* s2m_bias;
    const bf16_t* input;      // [rows][2048]
    const int* input_row;     // row of `input` (nullable: row 0)
    PredLayerArgs layer[kLayers];
    const int8_t* head_w;     // null: no head in this pass
    const float* head_s;
    const bf16_t* final_norm;
    bf16_t* logits;           // [2048]
    const bf16_t* rope_table;  // [positions][64][cos, sin]
    const int* position;
    float epsilon;
    float scale;
    unsigned long long* words;
    unsigned* epoch;
    int* status;
};

struct PassLds {
    float x[kPI];            // stage input as fp32 (normalized for QKV, gate/up, head)
    float partial[256];      // RMSNorm statistic partials
    float y[32];             // scaled dot products of this workgroup's rows
    float residual[4];       // hidden rows 4b..4b+3 (fp32 of the bf16 value)
    uint4 att_rows[48];      // attention workgroups: the head's q, its kv head's k and v (bf16)
};

__device__ __forceinline__ void barrier() { __syncthreads(); }

__device__ __forceinline__ const int4* vec_ptr(const int8_t* m, size_t byte_offset) {
    return reinterpret_cast<const int4*>(m + byte_offset);
}

// ------------------------------------------------------------ compute waves

struct Wide2 { int4 w[2]; float s; };          // K = 2048 row per wave (small_to_mtp, O)
struct Narrow { int4 w[2]; float s; };         // K = 1024 row per half-wave (QKV, head)
struct Unit { int4 w[4]; float s[2]; };        // gate and up rows of a unit per half-wave
struct Wide3 { int4 w[3]; float s; };          // K = 3072 row per wave (down)

// Row per wave, K = 2048: half h loads vectors l + 32 (2h + j), j = 0, 1.
__device__ __forceinline__ void issue_wide2(Wide2& r, const int8_t* m, const float* s, int row) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < 2; ++j) r.w[j] = stream_load(vec_ptr(m, static_cast<size_t>(row) * 2048 + 16 * (l + 32 * (2 * h + j))));
    r.s = s[row];
}
__device__ __forceinline__ void issue_narrow(Narrow& r, const int8_t* m, const float* s, int row) {
    const int l = threadIdx.x & 31;
#pragma unroll
    for (int j = 0; j < 2; ++j) r.w[j] = stream_load(vec_ptr(m, static_cast<size_t>(row) * 1024 + 16 * (l + 32 * j)));
    r.s = s[row];
}
__device__ __forceinline__ void issue_unit(Unit& r, const int8_t* m, const float* s, int unit) {
    const int l = threadIdx.x & 31;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int row = k == 0 ? unit : kPI + unit;
#pragma unroll
        for (int j = 0; j < 2; ++j) r.w[2 * k + j] = stream_load(vec_ptr(m, static_cast<size_t>(row) * 1024 + 16 * (l + 32 * j)));
        r.s[k] = s[row];
    }
}
__device__ __forceinline__ void issue_wide3(Wide3& r, const int8_t* m, const float* s, int row) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
#pragma unroll
    for (int j = 0; j < 3; ++j) r.w[j] = stream_load(vec_ptr(m, static_cast<size_t>(row) * 3072 + 16 * (l + 32 * (3 * h + j))));
    r.s = s[row];
}

// Row per wave over K = 2048: the halves' chains, then acc = c0 + c1 + c2 + c3
// in the reference's vector order.
__device__ __forceinline__ float dot_wide2(const Wide2& r, const float* x) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
    const float c0 = chain_at<2048>(r.w[0], x, l + 32 * (2 * h));
    const float c1 = chain_at<2048>(r.w[1], x, l + 32 * (2 * h + 1));
    const float c2 = from_upper_half(c0), c3 = from_upper_half(c1);
    float acc = 0.0f;
    acc += c0;
    acc += c1;
    acc += c2;
    acc += c3;
    return fold32(acc);
}
__device__ __forceinline__ float dot_narrow(const int4 (&w)[2], const float* x) {
    const int l = threadIdx.x & 31;
    float acc = 0.0f;
    acc += chain_at<1024>(w[0], x, l);
    acc += chain_at<1024>(w[1], x, l + 32);
    return fold32(acc);
}
__device__ __forceinline__ float dot_wide3(const Wide3& r, const float* x) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
    float c[3];
#pragma unroll
    for (int j = 0; j < 3; ++j) c[j] = chain_at<3072>(r.w[j], x, l + 32 * (3 * h + j));
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 3; ++j) acc += c[j];
#pragma unroll
    for (int j = 0; j < 3; ++j) acc += from_upper_half(c[j]);
    return fold32(acc);
}

// The attention of query head b (workgroups 0-15, wave 0): operands from
// the polled q/k/v rows (LDS), the gains, the rope rows and the caches; the
// outputs published as attention words.  The group's first query head
// appends the key and value to the caches for the later passes.
struct AttnOperandsGlobal {
    uint4 qgain, kgain;
    uint4 rv[4], kv4[4];
    uint4 vg0[2], vg1[2];
};

__device__ __forceinline__ void issue_attention(AttnOperandsGlobal& g, const PredLayerArgs& L, const PredArgs& a,
                                                int head) {
    const int lane = threadIdx.x & 63, chunk = lane & 15;
    const int kvh = head / kGroup;
    g.qgain = *reinterpret_cast<const uint4*>(L.q_norm + chunk * 8);
    g.kgain = *reinterpret_cast<const uint4*>(L.k_norm + chunk * 8);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = 4 * i + (lane >> 4);
        g.rv[i] = *reinterpret_cast<const uint4*>(a.rope_table + static_cast<size_t>(p) * 128 + chunk * 8);
        g.kv4[i] = *reinterpret_cast<const uint4*>(L.key_cache + static_cast<size_t>(p) * kKvW + kvh * 128 + chunk * 8);
    }
    const bf16_t* vrun0 = L.value_cache + (static_cast<size_t>(kvh) * 2 * 128 + lane) * 8;
    const bf16_t* vrun1 = vrun0 + 64 * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        g.vg0[i] = *reinterpret_cast<const uint4*>(vrun0 + i * short_attn::kGroupStep);
        g.vg1[i] = *reinterpret_cast<const uint4*>(vrun1 + i * short_attn::kGroupStep);
    }
}

__device__ __forceinline__ void run_attention(const AttnOperandsGlobal& g, const PredLayerArgs& L, const PredArgs& a,
                                              const PassLds& s, int head, unsigned tag) {
    const int lane = threadIdx.x & 63, chunk = lane & 15, part = lane >> 4;
    const int kvh = head / kGroup;
    const int position = *a.position;
    short_attn::Operands in;
    in.hv0 = part < 3 ? s.att_rows[16 * part + chunk] : g.qgain;
    in.hv1 = g.kgain;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        in.rv[i] = g.rv[i];
        in.kv4[i] = g.kv4[i];
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        in.vg0[i] = g.vg0[i];
        in.vg1[i] = g.vg1[i];
    }
    bf16_t* vrun0 = L.value_cache + (static_cast<size_t>(kvh) * 2 * 128 + lane) * 8;
    bf16_t* kdst = head % kGroup == 0 ? L.key_cache + static_cast<size_t>(position) * kKvW + kvh * 128 : nullptr;
    float acc0, acc1;
#ifdef Q3_PRED_TRACE
    const int trace_base = 64 + 8 * static_cast<int>((tag - 2u - *a.epoch) / 5u);
    PRED_STAMP(trace_base);
    struct Stamp {
        int base;
        __device__ void operator()(int k) const { PRED_STAMP(base + k); }
    };
    short_attn::core<true>(in, position, a.epsilon, a.scale, kdst, vrun0, vrun0 + 64 * 8, acc0, acc1,
                           Stamp{trace_base});
#else
    short_attn::core<true>(in, position, a.epsilon, a.scale, kdst, vrun0, vrun0 + 64 * 8, acc0, acc1);
#endif
    // dimensions (lane, lane + 1) and (lane + 64, lane + 65) from the even lanes
    const unsigned b0 = f2bf(acc0), b1 = f2bf(acc1);
    const unsigned n0 = static_cast<unsigned>(__shfl_xor(static_cast<int>(b0), 1, 64));
    const unsigned n1 = static_cast<unsigned>(__shfl_xor(static_cast<int>(b1), 1, 64));
    if ((lane & 1) == 0) {
        unsigned long long* att = a.words + kOffAtt + 64 * head;
        publish(att + lane / 2, pack_word(b0, n0, tag));
        publish(att + 32 + lane / 2, pack_word(b1, n1, tag));
    }
#ifdef Q3_PRED_TRACE
    PRED_STAMP(trace_base + 5);  // attention outputs published
#endif
}

struct ComputeRegs {
    Narrow q;
    Wide2 o;
    Unit gu;
    Wide3 d;
};

__device__ __forceinline__ void issue_layer_qkv(ComputeRegs& r, const PredLayerArgs& L, int b, int hw) {
    issue_narrow(r.q, L.qkv_w, L.qkv_s, 16 * b + hw);
}
__device__ __forceinline__ void issue_layer_o(ComputeRegs& r, const PredLayerArgs& L, int b, int wave) {
    if (wave < 4) issue_wide2(r.o, L.o_w, L.o_s, 4 * b + wave);
}
__device__ __forceinline__ void issue_layer_gu(ComputeRegs& r, const PredLayerArgs& L, int b, int hw) {
    if (hw < 12) issue_unit(r.gu, L.gu_w, L.gu_s, 12 * b + hw);
}
__device__ __forceinline__ void issue_layer_d(ComputeRegs& r, const PredLayerArgs& L, int b, int wave) {
    if (wave < 4) issue_wide3(r.d, L.d_w, L.d_s, 4 * b + wave);
}

// Barriers per stage, matched by the poller path: norm stages B1a, B1,
// B2; plain stages B1, B2; the attention (workgroups 0-15) one more.
template <int kL>
__device__ __forceinline__ void compute_layer(const PredArgs& a, PassLds& s, ComputeRegs& r, int b, int wave, int hw,
                                              unsigned base) {
    const PredLayerArgs& L = a.layer[kL];
    const int lane = threadIdx.x & 63, l = lane & 31;
    // QKV
    AttnOperandsGlobal g;
    if (b < kHeads && wave == 0) issue_attention(g, L, a, b);  // independent of this pass's QKV
    barrier();  // input staged
    barrier();  // input normalized
    {
        const float acc = dot_narrow(r.q.w, s.x);
        if (l == 0) s.y[hw] = acc * r.q.s;
    }
    if constexpr (kL + 1 < kLayers) issue_layer_qkv(r, a.layer[kL + 1], b, hw);
    barrier();
    // attention
    if (b < kHeads) {
        barrier();
        if (wave == 0) run_attention(g, L, a, s, b, base + 2u + 5u * kL);
    }
    // O
    barrier();
    if (wave < 4) {
        const float acc = dot_wide2(r.o, s.x);
        if (lane == 0) s.y[wave] = acc * r.o.s;
    }
    if constexpr (kL + 1 < kLayers) issue_layer_o(r, a.layer[kL + 1], b, wave);
    barrier();
    // gate/up
    barrier();  // input staged
    barrier();  // input normalized
    if (hw < 12) {
        const int4 wg[2] = {r.gu.w[0], r.gu.w[1]};
        const int4 wu[2] = {r.gu.w[2], r.gu.w[3]};
        const float g0 = dot_narrow(wg, s.x);
        const float u0 = dot_narrow(wu, s.x);
        if (l == 0) {
            s.y[2 * hw] = g0 * r.gu.s[0];
            s.y[2 * hw + 1] = u0 * r.gu.s[1];
        }
    }
    if constexpr (kL + 1 < kLayers) issue_layer_gu(r, a.layer[kL + 1], b, hw);
    barrier();
    // down
    barrier();
    if (wave < 4) {
        const float acc = dot_wide3(r.d, s.x);
        if (lane == 0) s.y[wave] = acc * r.d.s;
    }
    if constexpr (kL + 1 < kLayers) issue_layer_d(r, a.layer[kL + 1], b, wave);
    barrier();
}

template <int kL>
__device__ __forceinline__ void compute_layers(const PredArgs& a, PassLds& s, ComputeRegs& r, int b, int wave, int hw,
                                               unsigned base) {
    compute_layer<kL>(a, s, r, b, wave, hw, base);
    if constexpr (kL + 1 < kLayers) compute_layers<kL + 1>(a, s, r, b, wave, hw, base);
}

__device__ __forceinline__ void compute_path(const PredArgs& a, PassLds& s) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31;
    const int b = blockIdx.x, hw = 2 * wave + (lane >> 5);
    const unsigned base = *a.epoch;  // read at the start; workgroup 0 advances it at its end
    Wide2 s2m;
    Narrow head;
    ComputeRegs r;
    if (wave < 4) issue_wide2(s2m, a.s2m_w, a.s2m_s, 4 * b + wave);
    issue_layer_qkv(r, a.layer[0], b, hw);
    issue_layer_o(r, a.layer[0], b, wave);
    issue_layer_gu(r, a.layer[0], b, hw);
    issue_layer_d(r, a.layer[0], b, wave);
    const bool with_head = a.head_w != nullptr;
    if (with_head && hw < 8) issue_narrow(head, a.head_w, a.head_s, 8 * b + hw);
    // small_to_mtp
    barrier();
    if (wave < 4) {
        const float acc = dot_wide2(s2m, s.x);
        if (lane == 0) s.y[wave] = acc * s2m.s;
    }
    barrier();
    compute_layers<0>(a, s, r, b, wave, hw, base);
    if (with_head) {
        barrier();
        barrier();
        if (hw < 8) {
            const float acc = dot_narrow(head.w, s.x);
            if (l == 0) s.y[hw] = acc * head.s;
        }
        barrier();
    }
}

// ------------------------------------------------------------- poller waves

// RMSNorm of the staged 1024-wide input in place, after poll_norm_input
// (input and partials staged):
// the partials fold in the tree of fold_partials256, then each thread
// normalizes elements 4t..4t+3 with the gain chunk it loaded ahead.
__device__ __forceinline__ void norm_stage(PassLds& s, int pt, const uint2& gain, float epsilon) {
    barrier();  // B1a: input staged, partials written
    {
        const float inverse = fold_partials256(s.partial, kPH, epsilon);
        float4* c = reinterpret_cast<float4*>(s.x + x_index<kPH>(4 * pt));
        const float4 in = *c;
        const uint32_t g[2] = {gain.x, gain.y};
        *c = make_float4(normalize_one(in.x, inverse, __uint_as_float(g[0] << 16)),
                         normalize_one(in.y, inverse, __uint_as_float(g[0] & 0xffff0000u)),
                         normalize_one(in.z, inverse, __uint_as_float(g[1] << 16)),
                         normalize_one(in.w, inverse, __uint_as_float(g[1] & 0xffff0000u)));
    }
    barrier();  // B1: input ready
}

// Residual-add epilogue of rows 4b..4b+3 (pollers 0 and 1, two rows each):
// out = bf16(residual + bf16(y)), published as words 2b + pt.
__device__ __forceinline__ void residual_epilogue(PassLds& s, unsigned long long* area, int b, int pt, unsigned tag) {
    if (pt < 2) {
        unsigned r[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = 2 * pt + i;
            r[i] = f2bf(s.residual[row] + round_bf(s.y[row]));
            s.residual[row] = bf2f(static_cast<bf16_t>(r[i]));
        }
        publish(area + 2 * b + pt, pack_word(r[0], r[1], tag));
    }
}

__device__ __forceinline__ void poll_path(const PredArgs& a, PassLds& s) {
    const int pt = threadIdx.x - 64 * kComputeWaves;  // 0..255
    const int b = blockIdx.x;
    const unsigned base = *a.epoch;
    unsigned long long* HA = a.words + kOffHA;
    unsigned long long* HB = a.words + kOffHB;
    unsigned long long* Q = a.words + kOffQkv;
    unsigned long long* AT = a.words + kOffAtt;
    unsigned long long* AC = a.words + kOffAct;
    // ---- small_to_mtp: x = the input row (ready before the launch), + bias
    {
        const bf16_t* row = a.input + static_cast<size_t>(a.input_row != nullptr ? *a.input_row : 0) * kTH;
        const uint4 v = reinterpret_cast<const uint4*>(row)[pt];
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        float4* chunk0 = reinterpret_cast<float4*>(s.x + x_index<kTH>(8 * pt));
        float4* chunk1 = reinterpret_cast<float4*>(s.x + x_index<kTH>(8 * pt + 4));
        *chunk0 = make_float4(__uint_as_float(w[0] << 16), __uint_as_float(w[0] & 0xffff0000u),
                              __uint_as_float(w[1] << 16), __uint_as_float(w[1] & 0xffff0000u));
        *chunk1 = make_float4(__uint_as_float(w[2] << 16), __uint_as_float(w[2] & 0xffff0000u),
                              __uint_as_float(w[3] << 16), __uint_as_float(w[3] & 0xffff0000u));
    }
    float bias[2] = {0.0f, 0.0f};
    if (pt < 2) {
        bias[0] = bf2f(a.s2m_bias[4 * b + 2 * pt]);
        bias[1] = bf2f(a.s2m_bias[4 * b + 2 * pt + 1]);
    }
    PRED_STAMP(0);
    barrier();  // B1
    barrier();  // B2
    if (pt < 2) {  // bf16(bf16(y) + bias)
        unsigned r[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = 2 * pt + i;
            r[i] = f2bf(round_bf(s.y[row]) + bias[i]);
            s.residual[row] = bf2f(static_cast<bf16_t>(r[i]));
        }
        publish(HA + 2 * b + pt, pack_word(r[0], r[1], base));
    }
    PRED_STAMP(1);
#pragma unroll 1
    for (int layer = 0; layer < kLayers; ++layer) {
        const PredLayerArgs& L = a.layer[layer];
        const unsigned t = base + 1u + 5u * layer;  // this layer's QKV tag
        const uint2 gq = reinterpret_cast<const uint2*>(L.input_norm)[pt];
        const uint2 gg = reinterpret_cast<const uint2*>(L.post_norm)[pt];
        // ---- QKV: x = hidden (RMSNorm)
        poll_norm_input<kPH>(HA, t - 1u, s.x, s.partial, pt, a.status);
        PRED_STAMP(2 + 10 * layer);
        norm_stage(s, pt, gq, a.epsilon);
        barrier();  // B2
        if (pt < 8) publish(Q + 8 * b + pt, pack_word(f2bf(s.y[2 * pt]), f2bf(s.y[2 * pt + 1]), t));
        PRED_STAMP(3 + 10 * layer);
        // ---- attention (workgroups 0-15): the head's q, its kv head's k, v
        if (b < kHeads) {
            if (pt < 192) {
                const int kvh = b / kGroup;
                const int part = pt >> 6, i = pt & 63;
                const int word = part == 0 ? 64 * b + i : part == 1 ? 1024 + 64 * kvh + i : 1536 + 64 * kvh + i;
                unsigned long long v = read_word(Q + word);
                unsigned long long t0 = 0;
                int spins = 0;
                while (static_cast<unsigned>(v >> 32) != t) {
                    if (give_up(spins, t0, a.status)) break;
                    v = read_word(Q + word);
                }
                reinterpret_cast<uint32_t*>(s.att_rows)[pt] = static_cast<uint32_t>(v);
            }
            PRED_STAMP(4 + 10 * layer);
            barrier();
        }
        // ---- O: x = attention output, residual add
        poll_words<kWordsAtt>(AT, t + 1u, s.x, pt, a.status);
        PRED_STAMP(5 + 10 * layer);
        barrier();  // B1
        barrier();  // B2
        residual_epilogue(s, HB, b, pt, t + 2u);
        PRED_STAMP(6 + 10 * layer);
        // ---- gate/up: x = hidden after O (RMSNorm), SiLU gate
        poll_norm_input<kPH>(HB, t + 2u, s.x, s.partial, pt, a.status);
        PRED_STAMP(7 + 10 * layer);
        norm_stage(s, pt, gg, a.epsilon);
        barrier();  // B2
        if (pt < 6) {
            unsigned r[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int u = 2 * pt + i;  // local unit: gate y[2u], up y[2u + 1]
                const float gate16 = round_bf(s.y[2 * u]);
                const float up16 = round_bf(s.y[2 * u + 1]);
                const float activated = round_bf(gate16 / (1.0f + q3_expf(-gate16)));
                r[i] = f2bf(activated * up16);
            }
            publish(AC + 6 * b + pt, pack_word(r[0], r[1], t + 3u));
        }
        PRED_STAMP(8 + 10 * layer);
        // ---- down: x = activation, residual add
        poll_words<kWordsAct>(AC, t + 3u, s.x, pt, a.status);
        PRED_STAMP(9 + 10 * layer);
        barrier();  // B1
        barrier();  // B2
        residual_epilogue(s, HA, b, pt, t + 4u);
        PRED_STAMP(10 + 10 * layer);
    }
    // ---- head: final RMSNorm + codebook logits
    if (a.head_w != nullptr) {
        const uint2 gf = reinterpret_cast<const uint2*>(a.final_norm)[pt];
        poll_norm_input<kPH>(HA, base + 5u * kLayers, s.x, s.partial, pt, a.status);
        PRED_STAMP(52);
        norm_stage(s, pt, gf, a.epsilon);
        barrier();  // B2
        if (pt < 8) a.logits[8 * b + pt] = f2bf(s.y[pt]);
        PRED_STAMP(53);
    }
    if (b == 0 && pt == 0) {
        __hip_atomic_store(a.epoch, base + kTagsPerPass, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ __launch_bounds__(kPassThreads, 1) void predictor_pass_kernel(PredArgs a) {
    __shared__ PassLds s;
    if (threadIdx.x < 64 * kComputeWaves) {
        compute_path(a, s);
    } else {
        poll_path(a, s);
    }
}

}  // namespace

size_t predictor_pass_words() { return kWordsTotal; }

#ifdef Q3_PRED_TRACE
extern "C" __attribute__((visibility("default"))) int qwen3_tts_debug_pred_trace(unsigned long long* out) {
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(q3_pred_trace), sizeof(q3_pred_trace)) == hipSuccess ? 0 : -1;
}
#endif

hipError_t launch_predictor_pass(const PredictorPassArgs& c, hipStream_t stream) {
    if (c.hidden != kPH || c.intermediate != kPI || c.query_heads != kHeads || c.key_value_heads != kHeads / kGroup ||
        c.input_width != kTH || c.vocabulary != kVocab || c.layers != kLayers || c.capacity != short_attn::kCapacity ||
        c.s2m_w == nullptr || c.s2m_s == nullptr || c.s2m_bias == nullptr || c.input == nullptr ||
        c.rope_table == nullptr || c.position == nullptr || c.words == nullptr || c.epoch == nullptr ||
        c.status == nullptr || (c.head_w != nullptr && (c.head_s == nullptr || c.final_norm == nullptr || c.logits == nullptr))) {
        return hipErrorInvalidValue;
    }
    PredArgs a{};
    a.s2m_w = c.s2m_w;
    a.s2m_s = c.s2m_s;
    a.s2m_bias = c.s2m_bias;
    a.input = c.input;
    a.input_row = c.input_row;
    for (int l = 0; l < kLayers; ++l) {
        const PredLayerArgs& L = c.layer[l];
        if (L.qkv_w == nullptr || L.o_w == nullptr || L.gu_w == nullptr || L.d_w == nullptr || L.qkv_s == nullptr ||
            L.o_s == nullptr || L.gu_s == nullptr || L.d_s == nullptr || L.input_norm == nullptr ||
            L.post_norm == nullptr || L.q_norm == nullptr || L.k_norm == nullptr || L.key_cache == nullptr ||
            L.value_cache == nullptr) {
            return hipErrorInvalidValue;
        }
        a.layer[l] = L;
    }
    a.head_w = c.head_w;
    a.head_s = c.head_s;
    a.final_norm = c.final_norm;
    a.logits = c.logits;
    a.rope_table = c.rope_table;
    a.position = c.position;
    a.epsilon = c.epsilon;
    a.scale = 1.0f / sqrtf(128.0f);
    a.words = c.words;
    a.epoch = c.epoch;
    a.status = c.status;
    hipLaunchKernelGGL(predictor_pass_kernel, dim3(kGrid), dim3(kPassThreads), 0, stream, a);
    return hipGetLastError();
}

struct PassOrderSlot {
    std::mutex lock;
    hipEvent_t done = nullptr;  // after the device's last predictor launches
    hipStream_t stream = nullptr;
    bool recorded = false;
};
namespace {
PassOrderSlot pass_order[64];
}  // namespace

PredictorPassOrder::PredictorPassOrder(int device, hipStream_t stream) : stream_(stream) {
    if (device < 0 || device >= 64) {
        status_ = hipErrorInvalidDevice;
        return;
    }
    slot_ = &pass_order[device];
    slot_->lock.lock();
    if (slot_->done == nullptr) status_ = hipEventCreateWithFlags(&slot_->done, hipEventDisableTiming);
    if (status_ == hipSuccess && slot_->recorded && slot_->stream != stream)
        status_ = hipStreamWaitEvent(stream, slot_->done, 0);
}

hipError_t PredictorPassOrder::done() {
    if (slot_ == nullptr || status_ != hipSuccess) return status_;
    status_ = hipEventRecord(slot_->done, stream_);
    if (status_ == hipSuccess) {
        slot_->stream = stream_;
        slot_->recorded = true;
    }
    return status_;
}

PredictorPassOrder::~PredictorPassOrder() {
    if (slot_ != nullptr) slot_->lock.unlock();
}

hipError_t predictor_pass_supported(int device, bool* supported) {
    hipDeviceProp_t p;
    hipError_t st = hipGetDeviceProperties(&p, device);
    if (st != hipSuccess) return st;
    int blocks = 0;
    st = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(predictor_pass_kernel),
                                                      kPassThreads, 0);
    if (st != hipSuccess) return st;
    *supported = p.multiProcessorCount >= kGrid && blocks >= 1;
    return hipSuccess;
}

}  // namespace q3
