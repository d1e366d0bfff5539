// Per-head device helpers shared by the QKV epilogue and decode attention.
#pragma once

#include "q3_common.hpp"

namespace q3 {
namespace head_detail {

// Exact emulation of the reference's 256-thread block_sum tree
// (talker_kernels.cu:14-25) by one wave64: `p<j>` is virtual thread
// lane + 64*j.  Result is broadcast to every lane (whole wave active).
__device__ __forceinline__ float wave_tree256(float p0, float p1, float p2, float p3) {
    p0 += p2;
    p1 += p3;
    float value = p0 + p1;
    value = wave_sum_down<64>(value);
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(value)));
}

// Head RMSNorm (talker_kernels.cu:50-70) followed by rotate-half RoPE
// (talker_kernels.cu:72-114) of one 128-wide head, by one full wave: lane l
// owns elements l and l+64.  cs: this position's row of the rope table,
// [64][cos, sin] bf16.  Split into the loads and the arithmetic so a caller
// can request the operands ahead of other memory traffic.
struct HeadInputs {
    float x0, x1, g0, g1, c, s;
};

__device__ __forceinline__ HeadInputs load_head(const bf16_t* head, const bf16_t* gain, const bf16_t* cs) {
    const int lane = threadIdx.x & 63;
    HeadInputs in;
    in.x0 = bf2f(head[lane]);
    in.x1 = bf2f(head[lane + 64]);
    in.g0 = bf2f(gain[lane]);
    in.g1 = bf2f(gain[lane + 64]);
    in.c = bf2f(cs[2 * lane]);
    in.s = bf2f(cs[2 * lane + 1]);
    return in;
}

__device__ __forceinline__ void norm_rope_from(const HeadInputs& in, float epsilon, bf16_t& out0, bf16_t& out1) {
    constexpr int kDim = 128;
    // 256-thread tree over 128 squares; virtual threads 128..255 hold 0.
    const float total = wave_tree256(fmaf(in.x0, in.x0, 0.0f), fmaf(in.x1, in.x1, 0.0f), 0.0f, 0.0f);
    const float inverse = 1.0f / sqrtf(total / static_cast<float>(kDim) + epsilon);
    const float first = round_bf(round_bf(in.x0 * inverse) * in.g0);
    const float second = round_bf(round_bf(in.x1 * inverse) * in.g1);
    const float fc = round_bf(first * in.c);
    const float ss = round_bf(second * in.s);
    const float sc = round_bf(second * in.c);
    const float fs = round_bf(first * in.s);
    out0 = f2bf(fc - ss);
    out1 = f2bf(sc + fs);
}

__device__ __forceinline__ void norm_rope_head(const bf16_t* head, const bf16_t* gain, const bf16_t* cs,
                                               float epsilon, bf16_t& out0, bf16_t& out1) {
    norm_rope_from(load_head(head, gain, cs), epsilon, out0, out1);
}

}  // namespace head_detail
}  // namespace q3
