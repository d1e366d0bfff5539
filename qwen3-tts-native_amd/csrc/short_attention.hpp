// The code predictor's attention over caches of <= 16 positions, one wave
// per query head: head RMSNorm + RoPE of the query head and the new key,
// the append of the key and value, the scores, the softmax and the value
// chains, in the exact order of the reference's causal_gqa_attention_kernel
// (talker_kernels.cu:287-357) or, with kExact = false, of its batched
// causal_gqa_attention_fast (talker_kernels.cu:506-595).  Shared by the
// attention kernel (csrc/attention.hip) and the predictor pass chain
// (csrc/pred_chain.hip); each caller brings the operands into registers.
#pragma once

#include "head_device.hpp"
#include "q3_common.hpp"
#include "q3_math.h"

namespace q3 {
namespace short_attn {

constexpr int kDim = 128;
constexpr int kCapacity = 16;
constexpr int kGroupStep = kDim * 8;  // blocked value cache: elements between 8-position groups

__device__ __forceinline__ int value_offset(int position) { return (position >> 3) * kGroupStep + (position & 7); }
__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float wave_max(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_max_down(v))));
}

// Operands, in the lane layout the arithmetic reads them from (chunk =
// lane % 16, 8 bf16 per 16-byte chunk):
//   hv0   lanes 0-15: query head chunk; 16-31: new key chunk; 32-47: new
//         value chunk; 48-63: query-norm gain chunk
//   hv1   lanes 0-15: key-norm gain chunk
//   rv[i], kv4[i]   rope-table row and cached key row of position
//         4 i + lane / 16, chunk `chunk`
//   vg0[i], vg1[i]  the value-cache groups i (positions 8i..8i+7) of
//         dimensions lane and lane + 64 (zeros past the capacity)
struct Operands {
    uint4 hv0, hv1;
    uint4 rv[4], kv4[4];
    uint4 vg0[kCapacity / 8], vg1[kCapacity / 8];
};

// acc0 / acc1: the head's outputs for dimensions lane and lane + 64 (fp32,
// before the bf16 store).  key_dst (this kv head's 128 keys of row
// `position`) non-null: the normalized, rotated key is written there and the
// value into the blocked value runs vrun0 / vrun1 (group 0 of dimensions
// lane and lane + 64).  One wave; no barrier.
// Stage hook of core (a diagnostic build's stamps); the default does nothing.
struct NoHook {
    __device__ void operator()(int) const {}
};

template <bool kExact, typename Hook = NoHook>
__device__ __forceinline__ void core(const Operands& in, int position, float epsilon, float scale, bf16_t* key_dst,
                                     bf16_t* vrun0, bf16_t* vrun1, float& acc0, float& acc1, Hook hook = Hook()) {
    __shared__ uint4 rows_lds[2][kCapacity][kDim / 8];  // rope, keys
    __shared__ uint4 head_lds[5][kDim / 8];             // q, k, v, q gain, k gain
    const int lane = threadIdx.x & 63;
    const int chunk = lane & 15;
    const uint4 hv0 = in.hv0, hv1 = in.hv1;
    const uint4* rv = in.rv;
    const uint4* kv4 = in.kv4;
    const uint4* vg0 = in.vg0;
    const uint4* vg1 = in.vg1;
    head_lds[lane >> 4][chunk] = hv0;
    if (lane < 16) head_lds[4][chunk] = hv1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = 4 * i + (lane >> 4);
        rows_lds[0][p][chunk] = rv[i];
        rows_lds[1][p][chunk] = kv4[i];
    }
    // one wave: its LDS writes precede its reads
    const bf16_t* hl = reinterpret_cast<const bf16_t*>(head_lds);
    head_detail::HeadInputs q_in, k_in;
    q_in.x0 = bf2f(hl[lane]);
    q_in.x1 = bf2f(hl[lane + 64]);
    k_in.x0 = bf2f(hl[kDim + lane]);
    k_in.x1 = bf2f(hl[kDim + lane + 64]);
    const float v_new0 = bf2f(hl[2 * kDim + lane]);
    const float v_new1 = bf2f(hl[2 * kDim + lane + 64]);
    q_in.g0 = bf2f(hl[3 * kDim + lane]);
    q_in.g1 = bf2f(hl[3 * kDim + lane + 64]);
    k_in.g0 = bf2f(hl[4 * kDim + lane]);
    k_in.g1 = bf2f(hl[4 * kDim + lane + 64]);
    const bf16_t* rl = reinterpret_cast<const bf16_t*>(rows_lds[0][position]);
    q_in.c = k_in.c = bf2f(rl[2 * lane]);
    q_in.s = k_in.s = bf2f(rl[2 * lane + 1]);
    float v0[kCapacity], v1[kCapacity];
#pragma unroll
    for (int i = 0; i < kCapacity / 8; ++i) {
        const uint32_t w0[4] = {vg0[i].x, vg0[i].y, vg0[i].z, vg0[i].w};
        const uint32_t w1[4] = {vg1[i].x, vg1[i].y, vg1[i].z, vg1[i].w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            v0[8 * i + 2 * j] = lo_bf(w0[j]);
            v0[8 * i + 2 * j + 1] = hi_bf(w0[j]);
            v1[8 * i + 2 * j] = lo_bf(w1[j]);
            v1[8 * i + 2 * j + 1] = hi_bf(w1[j]);
        }
    }

    hook(1);
    // 2. head norm + RoPE of the query head and the new key; the append
    bf16_t q0b, q1b, kn0, kn1;
    head_detail::norm_rope_from(q_in, epsilon, q0b, q1b);
    head_detail::norm_rope_from(k_in, epsilon, kn0, kn1);
    if (key_dst != nullptr) {
        key_dst[lane] = kn0;
        key_dst[lane + 64] = kn1;
        vrun0[value_offset(position)] = f2bf(v_new0);
        vrun1[value_offset(position)] = f2bf(v_new1);
    }
    // the current position's key and value come from qkv, not the cache
    bf16_t* q_l = reinterpret_cast<bf16_t*>(head_lds[0]);
    bf16_t* k_l = reinterpret_cast<bf16_t*>(rows_lds[1][position]);
    q_l[lane] = q0b;
    q_l[lane + 64] = q1b;
    k_l[lane] = kn0;
    k_l[lane + 64] = kn1;
#pragma unroll
    for (int p = 0; p < kCapacity; ++p) {
        if (p == position) {
            v0[p] = v_new0;
            v1[p] = v_new1;
        }
    }

    hook(2);
    // 3. scores.  Lane L = 16 j + p works on position p and the tree's
    //    entries t = 8 j + i (i < 8) of level 32: it forms
    //    (P[t] + P[t+64]) + (P[t+32] + P[t+96]) itself (P = q*k), receives
    //    level 16's partner (t + 16, lane L + 32) and level 8's (t + 8, lane
    //    L + 16) through lane swaps, and folds levels 4, 2, 1 in registers --
    //    the reference tree's additions in its order.  Lane p ends with
    //    position p's dot.
    const int length = position + 1;
    const bool live = lane < length;
    float score;
    if constexpr (!kExact) {
        // batched semantics (causal_gqa_attention_fast): lane p < 16 forms
        // position p's dot as one fma chain over the dimensions in order
        const uint4* qv = reinterpret_cast<const uint4*>(head_lds[0]);
        const uint4* kv = rows_lds[1][lane & 15];
        float dot = 0.0f;
#pragma unroll
        for (int c = 0; c < kDim / 8; ++c) {
            const uint4 qa = qv[c], ka = kv[c];
            const uint32_t qw[4] = {qa.x, qa.y, qa.z, qa.w};
            const uint32_t kw[4] = {ka.x, ka.y, ka.z, ka.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dot = fmaf(lo_bf(qw[i]), lo_bf(kw[i]), dot);
                dot = fmaf(hi_bf(qw[i]), hi_bf(kw[i]), dot);
            }
        }
        score = live ? dot * scale : -INFINITY;
    } else {
        const int sp = lane & 15;
        const int j = lane >> 4;
        const uint4* qv = reinterpret_cast<const uint4*>(head_lds[0]);
        const uint4* kv = rows_lds[1][sp];
        float t8[8];
        const uint4 qa = qv[j], qb = qv[4 + j], qc = qv[8 + j], qd = qv[12 + j];  // t, t+32, t+64, t+96
        const uint4 ka = kv[j], kb = kv[4 + j], kc = kv[8 + j], kd = kv[12 + j];
        const uint32_t qw[4][4] = {{qa.x, qa.y, qa.z, qa.w}, {qb.x, qb.y, qb.z, qb.w},
                                   {qc.x, qc.y, qc.z, qc.w}, {qd.x, qd.y, qd.z, qd.w}};
        const uint32_t kw4[4][4] = {{ka.x, ka.y, ka.z, ka.w}, {kb.x, kb.y, kb.z, kb.w},
                                    {kc.x, kc.y, kc.z, kc.w}, {kd.x, kd.y, kd.z, kd.w}};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            auto el = [&](const uint32_t (&w)[4][4], int part) {
                return (i & 1) ? hi_bf(w[part][i >> 1]) : lo_bf(w[part][i >> 1]);
            };
            const float lo = fmaf(el(qw, 0), el(kw4, 0), 0.0f) + fmaf(el(qw, 2), el(kw4, 2), 0.0f);  // level 64, t
            const float hi = fmaf(el(qw, 1), el(kw4, 1), 0.0f) + fmaf(el(qw, 3), el(kw4, 3), 0.0f);  // level 64, t+32
            t8[i] = lo + hi;                                                                            // level 32
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // level 16: lanes 0-31 add lanes 32-63
            const unsigned b = __float_as_uint(t8[i]);
            t8[i] += __uint_as_float(__builtin_amdgcn_permlane32_swap(b, b, false, false)[1]);
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // level 8: row 0 adds row 1
            const unsigned b = __float_as_uint(t8[i]);
            t8[i] += __uint_as_float(__builtin_amdgcn_permlane16_swap(b, b, false, false)[1]);
        }
#pragma unroll
        for (int w = 4; w > 0; w >>= 1) {
#pragma unroll
            for (int i = 0; i < w; ++i) t8[i] += t8[i + w];
        }
        score = live ? round_bf(round_bf(t8[0]) * scale) : -INFINITY;
    }

    // 4. softmax, lane = position; the normalizer in position order.  The 16
    //    exponentials and then the 16 probabilities reach every lane as
    //    scalar operands (lane reads); entries past the current position are
    //    0, and adding them leaves the sequential sum as it is.
    //    Batched semantics: the normalizer is the 256-thread tree, whose
    //    levels 128 and 64 only add zeros here (a wave shuffle-down tree),
    //    the value chains take the unnormalized exponentials, and the
    //    output is scaled by the inverse once.
    hook(3);
    const float maximum = wave_max(score);
    const float e = live ? q3_expf(score - maximum) : 0.0f;
    float inverse;
    if constexpr (kExact) {
        float denominator = 0.0f;
#pragma unroll
        for (int p = 0; p < kCapacity; ++p) {
            denominator += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p));
        }
        inverse = 1.0f / denominator;
    } else {
        const float total = wave_sum_down<64>(e);
        inverse = 1.0f / __int_as_float(__builtin_amdgcn_readlane(__float_as_int(total), 0));
    }
    const float prob = kExact ? (live ? round_bf(e * inverse) : 0.0f) : e;
    float pv[kCapacity];
#pragma unroll
    for (int p = 0; p < kCapacity; ++p) pv[p] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(prob), p));

    hook(4);
    // 5. value chains for dimensions lane and lane + 64, positions in order.
    //    Past the current position the value is replaced by 0 (and its
    //    probability is 0): fmaf(0, 0, acc) == acc exactly, for every acc the
    //    chain can hold (it starts at +0 and never becomes -0).
    acc0 = 0.0f;
    acc1 = 0.0f;
#pragma unroll
    for (int p = 0; p < kCapacity; ++p) {
        const bool inside = p <= position;
        acc0 = fmaf(pv[p], inside ? v0[p] : 0.0f, acc0);
        acc1 = fmaf(pv[p], inside ? v1[p] : 0.0f, acc1);
    }
    if constexpr (!kExact) {
        acc0 *= inverse;
        acc1 *= inverse;
    }
}

}  // namespace short_attn
}  // namespace q3
