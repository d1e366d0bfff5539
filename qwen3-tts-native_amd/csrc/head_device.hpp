// Per-head device helpers shared by the QKV epilogue and decode attention.
#pragma once

#include "q3_common.hpp"

namespace q3 {
namespace head_detail {

// Exact emulation of the reference's 256-thread block_sum tree
// (talker_kernels.cu:14-25) by one wave64: `p<j>` is virtual thread
// lane + 64*j.  Result is broadcast to every lane.
__device__ __forceinline__ float wave_tree256(float p0, float p1, float p2, float p3) {
    p0 += p2;
    p1 += p3;
    float value = p0 + p1;
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) {
        value += __shfl_down(value, offset, 64);
    }
    return __shfl(value, 0, 64);
}

// Head RMSNorm (talker_kernels.cu:50-70) followed by rotate-half RoPE
// (talker_kernels.cu:72-114) of one 128-wide head, by one full wave: lane l
// owns elements l and l+64.  cs: this position's row of the rope table,
// [64][cos, sin] bf16.  Returns the two rotated bf16 values of the lane.
__device__ __forceinline__ void norm_rope_head(const bf16_t* head, const bf16_t* gain, const bf16_t* cs,
                                               float epsilon, bf16_t& out0, bf16_t& out1) {
    constexpr int kDim = 128;
    constexpr int kHalf = 64;
    const int lane = threadIdx.x & 63;
    const float x0 = bf2f(head[lane]);
    const float x1 = bf2f(head[lane + kHalf]);
    // 256-thread tree over 128 squares; virtual threads 128..255 hold 0.
    const float total = wave_tree256(fmaf(x0, x0, 0.0f), fmaf(x1, x1, 0.0f), 0.0f, 0.0f);
    const float inverse = 1.0f / sqrtf(total / static_cast<float>(kDim) + epsilon);
    const float first = round_bf(round_bf(x0 * inverse) * bf2f(gain[lane]));
    const float second = round_bf(round_bf(x1 * inverse) * bf2f(gain[lane + kHalf]));
    const float c = bf2f(cs[2 * lane]);
    const float s = bf2f(cs[2 * lane + 1]);
    const float fc = round_bf(first * c);
    const float ss = round_bf(second * s);
    const float sc = round_bf(second * c);
    const float fs = round_bf(first * s);
    out0 = f2bf(fc - ss);
    out1 = f2bf(sc + fs);
}

}  // namespace head_detail
}  // namespace q3
