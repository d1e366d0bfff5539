// Device helpers of the int8 GEMV family (gemv.hip).
//
// The exact order reproduces native/qwen3-tts-native/native/src/int8_gemv.cu:
// 67-125: lane l of a 32-lane group owns the 16-byte weight vectors
// l, l+32, ...; each vector is a fresh 16-term fmaf chain added to the lane
// accumulator; lanes fold by shuffle-down 16, 8, 4, 2, 1.
#pragma once

#include "q3_common.hpp"
#include "q3_math.h"

namespace q3 {
namespace gemv_detail {

constexpr int kThreads = 256;
constexpr int kHalfWaves = kThreads / 32;

__device__ __forceinline__ float byte_f(int word, int b) {
    return static_cast<float>(static_cast<int8_t>(word >> (8 * b)));
}

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Streaming 128-bit weight load (nontemporal: weights are read once per step).
__device__ __forceinline__ int4 stream_load(const void* p) {
    const i32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const i32x4_t*>(p));
    return make_int4(v.x, v.y, v.z, v.w);
}

// Reference 32-lane shuffle-down fold, offsets 16..1 (int8_gemv.cu:114-118).
// The sum is valid in lane 0 of each half-wave.
__device__ __forceinline__ float fold32(float value) { return wave_sum_down<32>(value); }

// Lane 0's value, for every lane (the whole wave must be active).
__device__ __forceinline__ float from_lane0(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}

// inv_rms of x[0..width) with the exact 256-thread tree of the reference's
// block_sum (talker_kernels.cu:14-25,36-41), computed by one wave64.
__device__ inline float wave_inverse_rms(const bf16_t* x, int width, float epsilon) {
    const int lane = threadIdx.x & 63;
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float s = 0.0f;
        for (int i = lane + 64 * j; i < width; i += 256) {
            const float v = bf2f(x[i]);
            s = fmaf(v, v, s);
        }
        part[j] = s;
    }
    part[0] += part[2];
    part[1] += part[3];
    float value = part[0] + part[1];
    const float total = from_lane0(wave_sum_down<64>(value));
    return 1.0f / sqrtf(total / static_cast<float>(width) + epsilon);
}

// Cooperative RMSNorm statistic of a 256-thread block, identical to the
// reference's 256-thread block_sum (talker_kernels.cu:36-41): thread t's
// partial is sum(x[i]^2, i = t, t+256, ...) as one fma chain, written to
// partial[t]; after a barrier every wave folds the 256 partials in the tree
// order of wave_inverse_rms and gets the same inverse.
template <int kWidth>
__device__ __forceinline__ float block_partial_sq(const bf16_t* x) {
    static_assert(kWidth % 256 == 0, "whole rounds of 256 threads");
    constexpr int kCount = kWidth / 256;
    float v[kCount];
#pragma unroll
    for (int j = 0; j < kCount; ++j) v[j] = bf2f(x[threadIdx.x + 256 * j]);  // all reads first
    float s = 0.0f;
#pragma unroll
    for (int j = 0; j < kCount; ++j) s = fmaf(v[j], v[j], s);
    return s;
}

__device__ __forceinline__ float fold_partials256(const float* partial, int width, float epsilon) {
    const int lane = threadIdx.x & 63;
    float p0 = partial[lane], p1 = partial[lane + 64];
    const float p2 = partial[lane + 128], p3 = partial[lane + 192];
    p0 += p2;
    p1 += p3;
    float value = p0 + p1;
    const float total = from_lane0(wave_sum_down<64>(value));
    return 1.0f / sqrtf(total / static_cast<float>(width) + epsilon);
}

__device__ __forceinline__ float normalize_one(float x, float inverse, float gain) {
    return round_bf(round_bf(x * inverse) * gain);
}

// Normalize one 16-byte chunk (8 bf16 activations with their gains).  The
// result of normalize_one is a bf16 value, so its top half is exact.
__device__ __forceinline__ uint4 normalize_chunk(const uint4 x, const uint4 g, float inverse) {
    const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lo = normalize_one(__uint_as_float(xw[i] << 16), inverse, __uint_as_float(gw[i] << 16));
        const float hi = normalize_one(__uint_as_float(xw[i] & 0xffff0000u), inverse,
                                       __uint_as_float(gw[i] & 0xffff0000u));
        o[i] = (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// normalize_chunk with the hardware float -> bf16 conversion (round to
// nearest even, as round_bf for every finite value; only a NaN's payload can
// differ).  Used by the batched MFMA path, whose results follow the
// reference's batched (non-exact-order) semantics.
__device__ __forceinline__ uint4 normalize_chunk_hw(const uint4 x, const uint4 g, float inverse) {
    const uint32_t xw[4] = {x.x, x.y, x.z, x.w};
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = __builtin_bit_cast(uint16_t, static_cast<__bf16>(__uint_as_float(xw[i] << 16) * inverse)) |
                           (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(
                                __uint_as_float(xw[i] & 0xffff0000u) * inverse))) << 16);
        const float lo = __uint_as_float(a << 16) * __uint_as_float(gw[i] << 16);
        const float hi = __uint_as_float(a & 0xffff0000u) * __uint_as_float(gw[i] & 0xffff0000u);
        o[i] = __builtin_bit_cast(uint16_t, static_cast<__bf16>(lo)) |
               (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, static_cast<__bf16>(hi))) << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// Load the 16 activations of vector `v` (bf16) as fp32, normalized if needed.
template <bool kNorm>
__device__ __forceinline__ void load_x16(const bf16_t* x, const bf16_t* gain, int v,
                                         float inverse, float* out) {
    const uint4* p = reinterpret_cast<const uint4*>(x + static_cast<size_t>(v) * 16);
    const uint4 a = p[0];
    const uint4 b = p[1];
    const uint32_t words[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        out[2 * i] = __uint_as_float(words[i] << 16);
        out[2 * i + 1] = __uint_as_float(words[i] & 0xffff0000u);
    }
    if constexpr (kNorm) {
        const uint4* g = reinterpret_cast<const uint4*>(gain + static_cast<size_t>(v) * 16);
        const uint4 ga = g[0];
        const uint4 gb = g[1];
        const uint32_t gw[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            out[2 * i] = normalize_one(out[2 * i], inverse, __uint_as_float(gw[i] << 16));
            out[2 * i + 1] =
                normalize_one(out[2 * i + 1], inverse, __uint_as_float(gw[i] & 0xffff0000u));
        }
    }
}

// One 16-byte weight vector against 16 fp32 activations: the reference's
// fresh fmaf chain (int8_gemv.cu:99-112).
__device__ __forceinline__ float chain16(const int4 w, const float* x) {
    const int words[4] = {w.x, w.y, w.z, w.w};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            sum = fmaf(byte_f(words[i], b), x[4 * i + b], sum);
        }
    }
    return sum;
}

// Packed-activation variant: x as 8 words of bf16 pairs.
__device__ __forceinline__ float chain16_packed(const int4 w, const uint32_t* xp) {
    const int words[4] = {w.x, w.y, w.z, w.w};
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const uint32_t pair = xp[(4 * i + b) >> 1];
            const float xv = ((b & 1) == 0) ? __uint_as_float(pair << 16)
                                            : __uint_as_float(pair & 0xffff0000u);
            sum = fmaf(byte_f(words[i], b), xv, sum);
        }
    }
    return sum;
}

// Epilogue operands of one output channel (or gate/up pair): the scale(s),
// the residual or bias.  Loaded before the dot products so their memory
// latency overlaps the weight stream instead of following it.
struct EpiInputs {
    float scale0 = 0.0f;
    float scale1 = 0.0f;
    float extra = 0.0f;  // residual (add epilogues) or bias
    float prior = 0.0f;  // residual of bias-add
};

template <int kEpi>
__device__ __forceinline__ EpiInputs prefetch_epi(const GemvArgs& a, int channel) {
    EpiInputs e;
    e.scale0 = a.scales[channel];
    if constexpr (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded) {
        e.scale1 = a.scales[a.out_features + channel];
    } else if constexpr (kEpi == kEpiAddFma || kEpi == kEpiAddRounded) {
        e.extra = bf2f(a.out16[channel]);
    } else if constexpr (kEpi == kEpiBias || kEpi == kEpiBiasSilu) {
        e.extra = bf2f(a.bias[channel]);
    } else if constexpr (kEpi == kEpiBiasAdd) {
        e.extra = bf2f(a.bias[channel]);
        e.prior = bf2f(a.out16[channel]);
    }
    return e;
}

// Half-wave lane 0 epilogue for the plain / residual / bias epilogues.
template <int kEpi>
__device__ __forceinline__ void finish_channel(const GemvArgs& a, int channel, float value, const EpiInputs& e) {
    const float scale = e.scale0;
    bf16_t* out = a.out16 + channel;
    if constexpr (kEpi == kEpiStore) {
        const float y = value * scale;
        if (a.out32 != nullptr) a.out32[channel] = y;
        if (a.out16 != nullptr) *out = f2bf(y);
    } else if constexpr (kEpi == kEpiAddFma) {
        *out = f2bf(fmaf(value, scale, e.extra));
    } else if constexpr (kEpi == kEpiAddRounded) {
        const float projected = round_bf(value * scale);
        *out = f2bf(e.extra + projected);
    } else if constexpr (kEpi == kEpiBias) {
        *out = f2bf(round_bf(value * scale) + e.extra);
    } else if constexpr (kEpi == kEpiBiasSilu) {
        float v = round_bf(value * scale) + e.extra;
        v *= 1.0f / (1.0f + q3_expf(-v));
        *out = f2bf(v);
    } else if constexpr (kEpi == kEpiBiasAdd) {
        const float projected = round_bf(round_bf(value * scale) + e.extra);
        *out = f2bf(e.prior + projected);
    }
}

// Gate/up pair epilogue (int8_gemv.cu:284-288 fused; separate SiLU-gate
// rounding for the single-session path).
template <int kEpi>
__device__ __forceinline__ void finish_gate_up(const GemvArgs& a, int channel, float g, float u, const EpiInputs& e) {
    const float gate = g * e.scale0;
    const float up = u * e.scale1;
    if constexpr (kEpi == kEpiSiluFused) {
        const float activated = gate / (1.0f + q3_expf(-gate));
        a.out16[channel] = f2bf(activated * up);
    } else {
        const float gate16 = round_bf(gate);
        const float up16 = round_bf(up);
        const float activated = round_bf(gate16 / (1.0f + q3_expf(-gate16)));
        a.out16[channel] = f2bf(activated * up16);
    }
}

template <int kEpi>
__device__ __forceinline__ void store_channel(const GemvArgs& a, int channel, float value) {
    finish_channel<kEpi>(a, channel, value, prefetch_epi<kEpi>(a, channel));
}

template <int kEpi>
__device__ __forceinline__ void store_gate_up(const GemvArgs& a, int channel, float g, float u) {
    finish_gate_up<kEpi>(a, channel, g, u, prefetch_epi<kEpi>(a, channel));
}

}  // namespace gemv_detail
}  // namespace q3
