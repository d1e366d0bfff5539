// Device helpers of the persistent GEMV chains (step_chain.hip: the talker
// step; pred_chain.hip: a code-predictor pass).  Stage outputs travel
// between workgroups as tagged 64-bit words: two bf16 values and a 32-bit
// tag written by one store, so a consumer needs no counter or fence -- it
// re-reads a word until its tag is the stage's.
#pragma once

#include "gemv_device.hpp"

namespace q3 {
namespace chain_detail {

using gemv_detail::chain16;

constexpr int kPollThreads = 256;                      // 4 poller waves
constexpr unsigned long long kPollLimit = 10000000ull;  // 0.1 s of the 100 MHz clock

__device__ __forceinline__ unsigned long long pack_word(unsigned lo, unsigned hi, unsigned tag) {
    return (static_cast<unsigned long long>(tag) << 32) | (hi << 16) | (lo & 0xffffu);
}

__device__ __forceinline__ void publish(unsigned long long* dst, unsigned long long word) {
    __hip_atomic_store(dst, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ unsigned long long read_word(const unsigned long long* src) {
    return __hip_atomic_load(src, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// LDS layout of a stage input of K values as fp32: element k of vector
// v = k / 16 sits in quarter q = (k % 16) / 4 at [q][v][k % 4], so the
// 16-byte reads of one quarter by consecutive lanes (consecutive vectors)
// are contiguous: no bank conflicts.
template <int kK>
__device__ __forceinline__ int x_index(int k) {
    return ((k & 15) >> 2) * (kK / 4) + (k >> 4) * 4 + (k & 3);
}

// Bounded wait bookkeeping: true when the caller should stop waiting (the
// status word is set, or this wait saw no progress for kPollLimit).
__device__ __forceinline__ bool give_up(int& spins, unsigned long long& t0, int* status) {
    if (t0 == 0) t0 = wall_clock64();
    if ((++spins & 63) != 0) return false;
    if (__hip_atomic_load(status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) return true;
    if (wall_clock64() - t0 > kPollLimit) {
        __hip_atomic_store(status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        return true;
    }
    return false;
}

// Poll kWords tagged words (this poller thread's share: words pt + 256 i)
// until all carry `tag`, then store their payloads to LDS as fp32 in the
// x_index layout.  All loads of a round are in flight together; only stale
// words are re-read.
template <int kWords>
__device__ __forceinline__ void poll_words(const unsigned long long* src, unsigned tag, float* x, int pt,
                                           int* status) {
    constexpr int kPer = kWords / kPollThreads;
    static_assert(kPer * kPollThreads == kWords, "whole rounds");
    unsigned long long v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = read_word(src + pt + kPollThreads * i);
    unsigned long long t0 = 0;
    int spins = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int i = 0; i < kPer; ++i) stale |= static_cast<unsigned>(v[i] >> 32) != tag;
        if (!stale) break;
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (static_cast<unsigned>(v[i] >> 32) != tag) v[i] = read_word(src + pt + kPollThreads * i);
        if (give_up(spins, t0, status)) break;
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const uint32_t pair = static_cast<uint32_t>(v[i]);
        *reinterpret_cast<float2*>(x + x_index<2 * kWords>(2 * (pt + kPollThreads * i))) =
            make_float2(__uint_as_float(pair << 16), __uint_as_float(pair & 0xffff0000u));
    }
}

// Stage one RMSNorm input element pair per word and write the reference's
// 256-thread sum-of-squares partials (talker_kernels.cu:14-48: thread t's
// partial is the fma chain of x[t + 256 i]^2 in i order).  Thread q < 128
// holds words q + 128 i, i.e. elements 2q + 256 i and 2q + 1 + 256 i: the
// inputs of partials t = 2q and t = 2q + 1, so no barrier separates the
// staging from the partials.
template <int kK>
__device__ __forceinline__ void stage_norm_pairs(const uint32_t (&pairs)[kK / 256], float* x, float* partial,
                                                 int q) {
    float even = 0.0f, odd = 0.0f;
#pragma unroll
    for (int i = 0; i < kK / 256; ++i) {
        const float lo = __uint_as_float(pairs[i] << 16), hi = __uint_as_float(pairs[i] & 0xffff0000u);
        *reinterpret_cast<float2*>(x + x_index<kK>(2 * q + 256 * i)) = make_float2(lo, hi);
        even = fmaf(lo, lo, even);
        odd = fmaf(hi, hi, odd);
    }
    *reinterpret_cast<float2*>(partial + 2 * q) = make_float2(even, odd);
}

// poll_words for an RMSNorm input of kK values (kK / 2 words), staged with
// its partials by stage_norm_pairs: poller threads 0-127 poll kK / 256 words
// each, the others return at once.
template <int kK>
__device__ __forceinline__ void poll_norm_input(const unsigned long long* src, unsigned tag, float* x,
                                                float* partial, int pt, int* status) {
    constexpr int kPer = kK / 256;
    if (pt >= 128) return;
    unsigned long long v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) v[i] = read_word(src + pt + 128 * i);
    unsigned long long t0 = 0;
    int spins = 0;
    while (true) {
        bool stale = false;
#pragma unroll
        for (int i = 0; i < kPer; ++i) stale |= static_cast<unsigned>(v[i] >> 32) != tag;
        if (!stale) break;
#pragma unroll
        for (int i = 0; i < kPer; ++i)
            if (static_cast<unsigned>(v[i] >> 32) != tag) v[i] = read_word(src + pt + 128 * i);
        if (give_up(spins, t0, status)) break;
    }
    uint32_t pairs[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) pairs[i] = static_cast<uint32_t>(v[i]);
    stage_norm_pairs<kK>(pairs, x, partial, pt);
}

// One 16-byte weight vector against its 16 activations (fp32 in LDS, the
// exact values of the bf16 inputs): the reference's fresh 16-term fmaf chain
// (chain16, int8_gemv.cu:99-112).
template <int kK>
__device__ __forceinline__ float chain_at(const int4& w, const float* x, int vec) {
    float v[16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float4 q = reinterpret_cast<const float4*>(x + i * (kK / 4))[vec];
        v[4 * i] = q.x;
        v[4 * i + 1] = q.y;
        v[4 * i + 2] = q.z;
        v[4 * i + 3] = q.w;
    }
    return chain16(w, v);
}

// Lanes 0-31 receive lanes 32-63's value.
__device__ __forceinline__ float from_upper_half(float v) {
    const unsigned bits = __float_as_uint(v);
    return __uint_as_float(__builtin_amdgcn_permlane32_swap(bits, bits, false, false)[1]);
}

}  // namespace chain_detail
}  // namespace q3
