// Persistent talker-step GEMV chain for gfx950: the 28 x {QKV + RMSNorm,
// O + residual, gate/up + RMSNorm + SiLU, down + residual} GEMVs of one
// batch-1 decode step in ONE launch, bit-identical to
// the per-GEMV exact kernels (gemv_exact_fixed, which reproduce
// native/qwen3-tts-native/native/src/int8_gemv.cu:58-293 and the layer
// sequence of talker.cu:3251-3456 without the attention).
//
// Why one launch: at batch 1 a GEMV streams 4-25 MB, 1.3-3.9 us of HBM time,
// and a dependent kernel boundary in a hipGraph costs ~1.1 us of idle GPU plus
// ~1 us of HBM ramp.  Here the weights of the next three GEMVs are already in
// flight (registers) while the dependency between two GEMVs resolves, so the
// weight stream does not stop at the 112 boundaries of a step.
//
// Layout: 256 workgroups (one per CU, all resident), 12 waves each.
//   * 8 compute waves own fixed output rows of every GEMV: QKV rows
//     16b..16b+15 (one per half-wave), O rows 8b..8b+7 (one per wave, the
//     row's 32-lane vectors split between the two halves of the wave),
//     gate/up units 24b..24b+23 (48 rows, three per half-wave) and down rows
//     8b..8b+7 (as O).  Each lane keeps the reference's k-assignment (vectors
//     l, l+32, ...; fresh 16-term fmaf chains added in order; shuffle-down
//     fold 16..1), so every sum is the reference's, bit for bit.  Their only
//     global memory operations are weight and scale loads, issued three
//     GEMVs ahead, so the compiler's in-order wait counts never stall a
//     GEMV on later GEMVs' weights.
//   * 4 waves poll and publish.  A GEMV's outputs travel between workgroups
//     as tagged 64-bit words (two bf16 values + a 32-bit epoch tag written by
//     one store), so a consumer needs no counter or fence: it re-reads a word
//     until the tag is the current stage's.  These waves also compute the
//     RMSNorm statistic of the reference's 256-thread block_sum
//     (talker_kernels.cu:14-48) and apply the epilogues (scale, residual add,
//     SiLU gate) in the reference's rounding order.
// Every wait is bounded: a poll that sees no progress for ~0.1 s sets the
// status word and every later poll gives up, so the grid always drains.
#include "chain_device.hpp"

// Build-time diagnostic: -DQ3_CHAIN_TRACE records per-GEMV timestamps of
// workgroup 0 (poll start / poll done / dot products start / done / outputs
// published) into ChainArgs::trace.  Off in the library build.
#ifdef Q3_CHAIN_TRACE
#define CHAIN_TRACE(...) __VA_ARGS__
__device__ int chain_nosync = 0;  // diagnostic: skip every poll (timing of the weight stream alone)
#else
#define CHAIN_TRACE(...)
#endif

namespace q3 {
namespace {

using namespace gemv_detail;

constexpr int kChainGrid = 256;
constexpr int kComputeWaves = 8;
constexpr int kPollWaves = 4;
constexpr int kChainThreads = 64 * (kComputeWaves + kPollWaves);
constexpr int kH = 2048;      // hidden
constexpr int kI = 6144;      // intermediate
constexpr int kQkv = 4096;    // fused q|k|v rows
constexpr int kQ = 2048;      // O input width (the query part)
// Tagged word areas (two bf16 values per word).
constexpr int kWordsH = kH / 2, kWordsQkv = kQkv / 2, kWordsAct = kI / 2;
constexpr int kOffH = 0, kOffQkv = kOffH + kWordsH, kOffH2 = kOffQkv + kWordsQkv, kOffAct = kOffH2 + kWordsH;
constexpr int kWordsTotal = kOffAct + kWordsAct;


struct ChainArgs {
    const int8_t* weights;       // per layer: qkv [4096][2048], o [2048][2048], gate/up [12288][2048], down [2048][6144]
    const float* scales;         // per layer: 4096 + 2048 + 12288 + 2048
    size_t weight_layer_stride;  // bytes
    size_t scale_layer_stride;   // floats
    const bf16_t* gain_qkv;      // RMSNorm gains [2048] before QKV
    const bf16_t* gain_gu;       // and before gate/up
    size_t gain_layer_stride;    // elements (0: shared by all layers)
    bf16_t* hidden;              // [2048] in / out
    bf16_t* qkv;                 // [4096] out: last layer's QKV
    bf16_t* act;                 // [6144] out: last layer's gate/up activation
    unsigned long long* words;   // kWordsTotal tagged words
    unsigned* epoch;             // tag base; advanced by 4 * layers + 1 per launch
    int* status;                 // 0 ok; 1 a poll timed out (outputs invalid)
    int layers;
    float epsilon;
    CHAIN_TRACE(unsigned long long* trace;)
};

// ----------------------------------------------------------------- helpers

using chain_detail::chain_at;
using chain_detail::from_upper_half;
using chain_detail::pack_word;
using chain_detail::publish;
using chain_detail::x_index;

template <int kWords>
__device__ __forceinline__ void poll_words(const unsigned long long* src, unsigned tag, float* x, int pt,
                                           int* status) {
    CHAIN_TRACE(if (chain_nosync) return;)
    chain_detail::poll_words<kWords>(src, tag, x, pt, status);
}

template <int kK>
__device__ __forceinline__ void poll_norm_input(const unsigned long long* src, unsigned tag, float* x, float* partial,
                                                int pt, int* status) {
    CHAIN_TRACE(if (chain_nosync) return;)
    chain_detail::poll_norm_input<kK>(src, tag, x, partial, pt, status);
}

// ------------------------------------------------------------ compute waves

struct RowOffsets {
    int qkv;      // byte offset of this lane's first vector within a layer's QKV matrix
    int o;        // ... O
    int gu[3];    // ... gate/up rows (three per half-wave)
    int down;     // ... down
    int sq, so, sgu[3], sd;  // scale indices
};

// Weight (and scale) registers of one GEMV kind.
struct QkvRegs { int4 w[4]; float s; };
struct ORegs { int4 w[2]; float s; };
struct GuRegs { int4 w[12]; float s[3]; };
struct DownRegs { int4 w[6]; float s; };

__device__ __forceinline__ const int4* vec_ptr(const int8_t* base, int byte_offset) {
    return reinterpret_cast<const int4*>(base + byte_offset);
}

__device__ __forceinline__ void issue_qkv(QkvRegs& r, const int8_t* w, const float* s, const RowOffsets& o) {
#pragma unroll
    for (int j = 0; j < 4; ++j) r.w[j] = stream_load(vec_ptr(w, o.qkv + 512 * j));
    r.s = s[o.sq];
}
__device__ __forceinline__ void issue_o(ORegs& r, const int8_t* w, const float* s, const RowOffsets& o) {
    const int8_t* m = w + static_cast<size_t>(kQkv) * kH;
#pragma unroll
    for (int j = 0; j < 2; ++j) r.w[j] = stream_load(vec_ptr(m, o.o + 512 * j));
    r.s = s[kQkv + o.so];
}
template <int kRow>
__device__ __forceinline__ void issue_gu(GuRegs& r, const int8_t* w, const float* s, const RowOffsets& o) {
    const int8_t* m = w + static_cast<size_t>(kQkv) * kH + static_cast<size_t>(kH) * kQ;
#pragma unroll
    for (int j = 0; j < 4; ++j) r.w[4 * kRow + j] = stream_load(vec_ptr(m, o.gu[kRow] + 512 * j));
    r.s[kRow] = s[kQkv + kH + o.sgu[kRow]];
}
__device__ __forceinline__ void issue_down(DownRegs& r, const int8_t* w, const float* s, const RowOffsets& o) {
    const int8_t* m = w + static_cast<size_t>(kQkv) * kH + static_cast<size_t>(kH) * kQ + 2ull * kI * kH;
#pragma unroll
    for (int j = 0; j < 6; ++j) r.w[j] = stream_load(vec_ptr(m, o.down + 512 * j));
    r.s = s[kQkv + kH + 2 * kI + o.sd];
}

struct ChainLds {
    float x[kI];               // stage input as fp32 (normalized for QKV and gate/up)
    float partial[256];        // RMSNorm statistic partials
    float y[48];               // scaled dot products of this workgroup's rows
    float residual[8];         // hidden rows 8b..8b+7 (fp32 of the bf16 value)
    CHAIN_TRACE(unsigned long long ts[8];)
    CHAIN_TRACE(unsigned long long tw[4][8];)  // each compute wave's end of its dot products
};

__device__ __forceinline__ void compute_qkv(const QkvRegs& r, ChainLds& s) {
    const int lane = threadIdx.x & 63, l = lane & 31, hw = 2 * (threadIdx.x >> 6) + (lane >> 5);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) acc += chain_at<kH>(r.w[j], s.x, l + 32 * j);
    acc = fold32(acc);
    if (l == 0) s.y[hw] = acc * r.s;
}

__device__ __forceinline__ void compute_o(const ORegs& r, ChainLds& s) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
    const float c0 = chain_at<kQ>(r.w[0], s.x, l + 32 * (2 * h));
    const float c1 = chain_at<kQ>(r.w[1], s.x, l + 32 * (2 * h + 1));
    const float c2 = from_upper_half(c0), c3 = from_upper_half(c1);
    float acc = 0.0f;
    acc += c0;
    acc += c1;
    acc += c2;
    acc += c3;
    acc = fold32(acc);
    if (lane == 0) s.y[threadIdx.x >> 6] = acc * r.s;
}

__device__ __forceinline__ void compute_gu(const GuRegs& r, ChainLds& s) {
    const int lane = threadIdx.x & 63, l = lane & 31, hw = 2 * (threadIdx.x >> 6) + (lane >> 5);
    float acc[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {  // per row the order is j = 0..3
#pragma unroll
        for (int k = 0; k < 3; ++k) acc[k] += chain_at<kH>(r.w[4 * k + j], s.x, l + 32 * j);
    }
#pragma unroll
    for (int k = 0; k < 3; ++k) acc[k] = fold32(acc[k]);
    if (l == 0) {
#pragma unroll
        for (int k = 0; k < 3; ++k) s.y[3 * hw + k] = acc[k] * r.s[k];
    }
}

__device__ __forceinline__ void compute_down(const DownRegs& r, ChainLds& s) {
    const int lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
    float c[6];
#pragma unroll
    for (int j = 0; j < 6; ++j) c[j] = chain_at<kI>(r.w[j], s.x, l + 32 * (6 * h + j));
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 6; ++j) acc += c[j];
#pragma unroll
    for (int j = 0; j < 6; ++j) acc += from_upper_half(c[j]);
    acc = fold32(acc);
    if (lane == 0) s.y[threadIdx.x >> 6] = acc * r.s;
}

// Barriers per GEMV on both paths: for the normalized inputs (QKV,
// gate/up) B1a (input and norm partials staged), B1 (normalized input
// ready), B2 (dot products in LDS); for O and down B1 (input staged), B2.
__device__ __forceinline__ void barrier() { __syncthreads(); }

// Per GEMV: [B1a,] B1 (input ready), the loads of the GEMV three ahead, the
// dot products, B2.
template <bool kLast>
__device__ __forceinline__ void compute_layer(const ChainArgs& a, int layer, const RowOffsets& o, ChainLds& s,
                                              QkvRegs& rq, ORegs& ro, GuRegs& rg, DownRegs& rd) {
    const int8_t* wl = a.weights + a.weight_layer_stride * layer;
    const float* sl = a.scales + a.scale_layer_stride * layer;
    const int8_t* wn = wl + a.weight_layer_stride;
    const float* sn = sl + a.scale_layer_stride;
    barrier();  // B1a
    barrier();  // B1
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[0] = wall_clock64();)
    issue_down(rd, wl, sl, o);
    compute_qkv(rq, s);
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[1] = wall_clock64();)
    CHAIN_TRACE(if ((threadIdx.x & 63) == 0) s.tw[0][threadIdx.x >> 6] = wall_clock64();)
    barrier();  // B2
    barrier();  // B1
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[2] = wall_clock64();)
    if constexpr (!kLast) issue_qkv(rq, wn, sn, o);
    compute_o(ro, s);
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[3] = wall_clock64();)
    CHAIN_TRACE(if ((threadIdx.x & 63) == 0) s.tw[1][threadIdx.x >> 6] = wall_clock64();)
    barrier();  // B2
    barrier();  // B1a
    barrier();  // B1
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[4] = wall_clock64();)
    if constexpr (!kLast) issue_o(ro, wn, sn, o);
    compute_gu(rg, s);
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[5] = wall_clock64();)
    CHAIN_TRACE(if ((threadIdx.x & 63) == 0) s.tw[2][threadIdx.x >> 6] = wall_clock64();)
    barrier();  // B2
    barrier();  // B1
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[6] = wall_clock64();)
    if constexpr (!kLast) {
        issue_gu<0>(rg, wn, sn, o);
        issue_gu<1>(rg, wn, sn, o);
        issue_gu<2>(rg, wn, sn, o);
    }
    compute_down(rd, s);
    CHAIN_TRACE(if (threadIdx.x == 0) s.ts[7] = wall_clock64();)
    CHAIN_TRACE(if ((threadIdx.x & 63) == 0) s.tw[3][threadIdx.x >> 6] = wall_clock64();)
    barrier();
}

__device__ __forceinline__ void compute_path(const ChainArgs& a, ChainLds& s) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31, h = lane >> 5;
    const int b = blockIdx.x, hw = 2 * wave + h;
    RowOffsets o;
    o.sq = 16 * b + hw;
    o.qkv = o.sq * kH + 16 * l;
    o.so = 8 * b + wave;
    o.o = o.so * kQ + 16 * (l + 64 * h);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const int idx = 3 * hw + k;
        const int unit = 24 * b + idx / 2;
        o.sgu[k] = (idx & 1) ? kI + unit : unit;
        o.gu[k] = o.sgu[k] * kH + 16 * l;
    }
    o.sd = 8 * b + wave;
    o.down = o.sd * kI + 16 * (l + 192 * h);
    QkvRegs rq;
    ORegs ro;
    GuRegs rg;
    DownRegs rd;
    issue_qkv(rq, a.weights, a.scales, o);
    issue_o(ro, a.weights, a.scales, o);
    issue_gu<0>(rg, a.weights, a.scales, o);
    issue_gu<1>(rg, a.weights, a.scales, o);
    issue_gu<2>(rg, a.weights, a.scales, o);
    for (int layer = 0; layer + 1 < a.layers; ++layer) compute_layer<false>(a, layer, o, s, rq, ro, rg, rd);
    compute_layer<true>(a, a.layers - 1, o, s, rq, ro, rg, rd);
}

// ------------------------------------------------------------- poller waves

// RMSNorm of the staged input in place, after poll_norm_input (input and the
// reference's 256-thread partials staged, talker_kernels.cu:14-48): the
// partials fold in the tree of fold_partials256, then each thread
// normalizes its own 16-byte chunk with the gain chunk it loaded ahead.
__device__ __forceinline__ void norm_stage(ChainLds& s, int pt, const uint4& gain, float epsilon) {
    barrier();  // B1a: input and partials staged
    {
        const float inverse = fold_partials256(s.partial, kH, epsilon);
        // elements 8pt..8pt+7: quarters 2(pt%2), 2(pt%2)+1 of vector pt/2
        float4* c0 = reinterpret_cast<float4*>(s.x + x_index<kH>(8 * pt));
        float4* c1 = reinterpret_cast<float4*>(s.x + x_index<kH>(8 * pt + 4));
        const float4 a = *c0, b = *c1;
        const uint32_t g[4] = {gain.x, gain.y, gain.z, gain.w};
        const float in[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float out[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            out[2 * i] = normalize_one(in[2 * i], inverse, __uint_as_float(g[i] << 16));
            out[2 * i + 1] = normalize_one(in[2 * i + 1], inverse, __uint_as_float(g[i] & 0xffff0000u));
        }
        *c0 = make_float4(out[0], out[1], out[2], out[3]);
        *c1 = make_float4(out[4], out[5], out[6], out[7]);
    }
    barrier();  // B1: input ready
}

__device__ __forceinline__ void poll_path(const ChainArgs& a, ChainLds& s) {
    const int pt = threadIdx.x - 64 * kComputeWaves;  // 0..255
    const int b = blockIdx.x;
    const unsigned base = *a.epoch;
    unsigned long long* H = a.words + kOffH;
    unsigned long long* Q = a.words + kOffQkv;
    unsigned long long* H2 = a.words + kOffH2;
    unsigned long long* A = a.words + kOffAct;
    for (int layer = 0; layer < a.layers; ++layer) {

        const bool last = layer + 1 == a.layers;
        const unsigned t = base + 4u * layer;  // tag of this layer's QKV input (layer > 0)
        // Gain chunks of this layer's two norms, requested before the polls
        // (vector memory returns in order, so they are not behind them).
        const uint4 gq = reinterpret_cast<const uint4*>(a.gain_qkv + a.gain_layer_stride * layer)[pt];
        const uint4 gg = reinterpret_cast<const uint4*>(a.gain_gu + a.gain_layer_stride * layer)[pt];
        // ---- QKV: x = hidden
        if (layer == 0) {
            if (pt < 128) {
                const uint32_t* row = reinterpret_cast<const uint32_t*>(a.hidden);
                uint32_t pairs[kH / 256];
#pragma unroll
                for (int i = 0; i < kH / 256; ++i) pairs[i] = row[pt + 128 * i];
                chain_detail::stage_norm_pairs<kH>(pairs, s.x, s.partial, pt);
            }
            if (pt == b) {  // this workgroup's residual rows 8b..8b+7
                const uint4 v = reinterpret_cast<const uint4*>(a.hidden)[b];
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    s.residual[2 * i] = __uint_as_float(w[i] << 16);
                    s.residual[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
                }
            }
        } else {
            CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 0 + 0] = wall_clock64();)
            poll_norm_input<kH>(H, t, s.x, s.partial, pt, a.status);
        }
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 0 + 1] = wall_clock64();)
        norm_stage(s, pt, gq, a.epsilon);
        barrier();  // B2: QKV dot products
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) { a.trace[64 * layer + 8 * 0 + 2] = s.ts[0]; a.trace[64 * layer + 8 * 0 + 3] = s.ts[1]; a.trace[64 * layer + 8 * 0 + 4] = wall_clock64(); unsigned long long mx = 0, mn = ~0ull; for (int w = 0; w < kComputeWaves; ++w) { mx = max(mx, s.tw[0][w]); mn = min(mn, s.tw[0][w]); } a.trace[64 * layer + 8 * 0 + 5] = mx; a.trace[64 * layer + 8 * 0 + 6] = mn; })
        if (pt < 8) {
            const unsigned lo = f2bf(s.y[2 * pt]), hi = f2bf(s.y[2 * pt + 1]);
            publish(Q + 8 * b + pt, pack_word(lo, hi, t + 1));
            if (last) {
                a.qkv[16 * b + 2 * pt] = static_cast<bf16_t>(lo);
                a.qkv[16 * b + 2 * pt + 1] = static_cast<bf16_t>(hi);
            }
        }
        // ---- O: x = q (QKV words 0..1023), residual add
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 1 + 0] = wall_clock64();)
        poll_words<kWordsH>(Q, t + 1, s.x, pt, a.status);
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 1 + 1] = wall_clock64();)
        barrier();  // B1
        barrier();  // B2
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) { a.trace[64 * layer + 8 * 1 + 2] = s.ts[2]; a.trace[64 * layer + 8 * 1 + 3] = s.ts[3]; a.trace[64 * layer + 8 * 1 + 4] = wall_clock64(); unsigned long long mx = 0, mn = ~0ull; for (int w = 0; w < kComputeWaves; ++w) { mx = max(mx, s.tw[1][w]); mn = min(mn, s.tw[1][w]); } a.trace[64 * layer + 8 * 1 + 5] = mx; a.trace[64 * layer + 8 * 1 + 6] = mn; })
        if (pt < 4) {
            unsigned r[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = 2 * pt + i;
                r[i] = f2bf(s.residual[row] + round_bf(s.y[row]));
                s.residual[row] = bf2f(static_cast<bf16_t>(r[i]));
            }
            publish(H2 + 4 * b + pt, pack_word(r[0], r[1], t + 2));
        }
        // ---- gate/up: x = hidden after O, RMSNorm, SiLU gate
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 2 + 0] = wall_clock64();)
        poll_norm_input<kH>(H2, t + 2, s.x, s.partial, pt, a.status);
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 2 + 1] = wall_clock64();)
        norm_stage(s, pt, gg, a.epsilon);
        barrier();  // B2
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) { a.trace[64 * layer + 8 * 2 + 2] = s.ts[4]; a.trace[64 * layer + 8 * 2 + 3] = s.ts[5]; a.trace[64 * layer + 8 * 2 + 4] = wall_clock64(); unsigned long long mx = 0, mn = ~0ull; for (int w = 0; w < kComputeWaves; ++w) { mx = max(mx, s.tw[2][w]); mn = min(mn, s.tw[2][w]); } a.trace[64 * layer + 8 * 2 + 5] = mx; a.trace[64 * layer + 8 * 2 + 6] = mn; })
        if (pt < 12) {
            unsigned r[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int u = 2 * pt + i;  // local unit: gate row 2u, up row 2u + 1
                const float gate16 = round_bf(s.y[2 * u]);
                const float up16 = round_bf(s.y[2 * u + 1]);
                const float activated = round_bf(gate16 / (1.0f + q3_expf(-gate16)));
                r[i] = f2bf(activated * up16);
                if (last) a.act[24 * b + u] = static_cast<bf16_t>(r[i]);
            }
            publish(A + 12 * b + pt, pack_word(r[0], r[1], t + 3));
        }
        // ---- down: x = activation, residual add
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 3 + 0] = wall_clock64();)
        poll_words<kWordsAct>(A, t + 3, s.x, pt, a.status);
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) a.trace[64 * layer + 8 * 3 + 1] = wall_clock64();)
        barrier();  // B1
        barrier();  // B2
        CHAIN_TRACE(if (a.trace && b == 0 && pt == 0) { a.trace[64 * layer + 8 * 3 + 2] = s.ts[6]; a.trace[64 * layer + 8 * 3 + 3] = s.ts[7]; a.trace[64 * layer + 8 * 3 + 4] = wall_clock64(); unsigned long long mx = 0, mn = ~0ull; for (int w = 0; w < kComputeWaves; ++w) { mx = max(mx, s.tw[3][w]); mn = min(mn, s.tw[3][w]); } a.trace[64 * layer + 8 * 3 + 5] = mx; a.trace[64 * layer + 8 * 3 + 6] = mn; })
        if (pt < 4) {
            unsigned r[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int row = 2 * pt + i;
                r[i] = f2bf(s.residual[row] + round_bf(s.y[row]));
                s.residual[row] = bf2f(static_cast<bf16_t>(r[i]));
                if (last) a.hidden[8 * b + row] = static_cast<bf16_t>(r[i]);
            }
            if (!last) publish(H + 4 * b + pt, pack_word(r[0], r[1], t + 4));
        }
    }
    if (b == 0 && pt == 0) {
        __hip_atomic_store(a.epoch, base + 4u * a.layers + 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__global__ __launch_bounds__(kChainThreads, 1) void talker_step_chain_kernel(ChainArgs a) {
    __shared__ ChainLds s;
    if (threadIdx.x < 64 * kComputeWaves) {
        compute_path(a, s);
    } else {
        poll_path(a, s);
    }
}

}  // namespace

size_t talker_step_chain_words() { return kWordsTotal; }

hipError_t launch_talker_step_chain(const StepChainArgs& c, hipStream_t stream) {
    if (c.hidden_size != kH || c.intermediate != kI || c.qkv_rows != kQkv || c.query_width != kQ ||
        c.layers < 1 || c.weights == nullptr || c.scales == nullptr || c.hidden == nullptr ||
        c.qkv == nullptr || c.act == nullptr || c.words == nullptr || c.epoch == nullptr ||
        c.status == nullptr || c.gain_qkv == nullptr || c.gain_gu == nullptr) {
        return hipErrorInvalidValue;
    }
    ChainArgs a;
    a.weights = c.weights;
    a.scales = c.scales;
    a.weight_layer_stride = c.weight_layer_stride;
    a.scale_layer_stride = c.scale_layer_stride;
    a.gain_qkv = c.gain_qkv;
    a.gain_gu = c.gain_gu;
    a.gain_layer_stride = c.gain_layer_stride;
    a.hidden = c.hidden;
    a.qkv = c.qkv;
    a.act = c.act;
    a.words = c.words;
    a.epoch = c.epoch;
    a.status = c.status;
    a.layers = c.layers;
    a.epsilon = c.epsilon;
    hipLaunchKernelGGL(talker_step_chain_kernel, dim3(kChainGrid), dim3(kChainThreads), 0, stream, a);
    return hipGetLastError();
}

hipError_t talker_step_chain_supported(int device, bool* supported) {
    hipDeviceProp_t p;
    hipError_t st = hipGetDeviceProperties(&p, device);
    if (st != hipSuccess) return st;
    int blocks = 0;
    st = hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, reinterpret_cast<const void*>(talker_step_chain_kernel),
                                                      kChainThreads, 0);
    if (st != hipSuccess) return st;
    *supported = p.multiProcessorCount >= kChainGrid && blocks >= 1;
    return hipSuccess;
}

}  // namespace q3
