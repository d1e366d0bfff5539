// Decode attention over a bf16 KV cache, head dimension 128, as three
// kernels so that every phase runs on many compute units:
//
//   scores   one lane per (row, kv head, position): the key row is read once
//            and dotted with every query head of the GQA group.
//   softmax  one block per (row, query head): maximum, exponentials and the
//            normalizer; writes the probabilities (exact) or the unnormalized
//            weights plus 1/sum (fast) back over the scores.
//   values   one wave per (row, kv head, slice of the head dimension): lanes
//            are (query head of the group, dimension) pairs, each running the
//            reference's sequential fma chain over positions.  Value rows are
//            streamed through a 32-deep register ring (16-byte loads, 32 KB
//            in flight per wave) and transposed through LDS.
//
// Caches of at most 64 positions (the code predictor's) run all three phases
// in one kernel.
//
// Two arithmetic variants, each the reference's own operation order:
//   exact  causal_gqa_attention_kernel (talker_kernels.cu:287-357):
//          dot = 256-thread block_sum tree of the 128 products (threads
//          128..255 contribute zeros), rounded to bf16; score =
//          bf16(dot * scale); thread 0 takes the max, exponentials and their
//          sum sequentially; p = bf16(e * (1/sum)); out = bf16(sequential
//          fmaf(p, v) over positions).
//   fast   batch_causal_gqa_attention_fast_kernel (talker_kernels.cu:506-595):
//          fp32 score from a sequential fmaf over d, times scale; 256-thread
//          strided partial sums of the exponentials and a tree; out =
//          bf16(sequential fmaf(w, v) * (1/sum)).
// The max is order independent, and every exponential is q3_expf of the same
// operands as the oracle's, so splitting the phases over kernels changes no
// bit of the result.
#include "q3_common.hpp"
#include "q3_math.h"

namespace q3 {
namespace {

constexpr int kDim = 128;
constexpr int kScoreLanes = 64;   // positions per score block
constexpr int kSoftmaxThreads = 256;
constexpr int kRing = 32;         // value loads in flight per lane
constexpr int kMaxCapacity = 12288;

struct AttnArgs {
    const bf16_t* query;
    int query_stride;
    bf16_t* const* key_bases;
    bf16_t* const* value_bases;
    const bf16_t* key_cache;
    const bf16_t* value_cache;
    const int* positions;
    int fixed_length;
    bf16_t* output;
    int query_heads;
    int key_value_heads;
    int capacity;
    float scale;
    float* scores;   // [rows][query_heads][capacity]
    float* inverse;  // [rows][query_heads] (fast variant)
};

__device__ __forceinline__ int row_length(const AttnArgs& a, int row) {
    return a.positions != nullptr ? a.positions[row] + 1 : a.fixed_length;
}

__device__ __forceinline__ const bf16_t* row_keys(const AttnArgs& a, int row) {
    return a.key_bases != nullptr ? a.key_bases[row] : a.key_cache;
}

__device__ __forceinline__ const bf16_t* row_values(const AttnArgs& a, int row) {
    return a.value_bases != nullptr ? a.value_bases[row] : a.value_cache;
}

// Cache rows are reached through pointer tables, which the compiler cannot
// place in the global address space by itself; a flat load would also count
// against the LDS counter and serialize with the LDS traffic.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_global16(const void* p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)(reinterpret_cast<uintptr_t>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// ---------------------------------------------------------------------------
// scores: grid (position blocks, kv heads, rows), 64 threads, lane = position
// ---------------------------------------------------------------------------
template <bool kExact, int kG>
__global__ __launch_bounds__(kScoreLanes) void attention_scores_kernel(AttnArgs a) {
    const int row = blockIdx.z;
    const int kvh = blockIdx.y;
    const int length = row_length(a, row);
    const int p0 = blockIdx.x * kScoreLanes;
    if (p0 >= length) return;
    __shared__ float q_lds[kG][kDim];
    const int lane = threadIdx.x;
    const bf16_t* q = a.query + static_cast<size_t>(row) * a.query_stride + static_cast<size_t>(kvh) * kG * kDim;
    for (int i = lane; i < kG * kDim; i += kScoreLanes) q_lds[i / kDim][i % kDim] = bf2f(q[i]);
    __syncthreads();
    const int p = p0 + lane;
    if (p >= length) return;
    const int kv_width = a.key_value_heads * kDim;
    const uint4* k4 = reinterpret_cast<const uint4*>(row_keys(a, row) + static_cast<size_t>(p) * kv_width +
                                                     static_cast<size_t>(kvh) * kDim);
    uint32_t kw[64];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
        const uint4 t = load_global16(k4 + v);
        kw[4 * v + 0] = t.x;
        kw[4 * v + 1] = t.y;
        kw[4 * v + 2] = t.z;
        kw[4 * v + 3] = t.w;
    }
    float* out = a.scores + (static_cast<size_t>(row) * a.query_heads + static_cast<size_t>(kvh) * kG) * a.capacity + p;
#pragma unroll
    for (int g = 0; g < kG; ++g) {
        const float* qg = q_lds[g];
        float score;
        if constexpr (kExact) {
            // block_sum over 256 threads: thread t < 128 holds q[t]k[t],
            // the rest zero.  Level 128 adds zeros (a no-op up to the sign of
            // a zero dot, which no later step can observe); level 64 pairs
            // t with t+64; then halves down to 1.
            float s[64];
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                const float kl = (t & 1) ? hi_bf(kw[t >> 1]) : lo_bf(kw[t >> 1]);
                const float kh = (t & 1) ? hi_bf(kw[32 + (t >> 1)]) : lo_bf(kw[32 + (t >> 1)]);
                s[t] = fmaf(qg[t], kl, 0.0f) + fmaf(qg[t + 64], kh, 0.0f);
            }
#pragma unroll
            for (int w = 32; w > 0; w >>= 1) {
#pragma unroll
                for (int t = 0; t < w; ++t) s[t] += s[t + w];
            }
            score = round_bf(round_bf(s[0]) * a.scale);
        } else {
            float dot = 0.0f;
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                dot = fmaf(qg[2 * t], lo_bf(kw[t]), dot);
                dot = fmaf(qg[2 * t + 1], hi_bf(kw[t]), dot);
            }
            score = dot * a.scale;
        }
        out[static_cast<size_t>(g) * a.capacity] = score;
    }
}

// ---------------------------------------------------------------------------
// softmax: grid (query heads, rows), 256 threads
// ---------------------------------------------------------------------------
template <bool kExact>
__global__ __launch_bounds__(kSoftmaxThreads) void attention_softmax_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float e_lds[];
    __shared__ float reduction[kSoftmaxThreads];
    __shared__ float broadcast;
    const int row = blockIdx.y;
    const int head = blockIdx.x;
    const int tid = threadIdx.x;
    const int length = row_length(a, row);
    float* s = a.scores + (static_cast<size_t>(row) * a.query_heads + head) * a.capacity;

    float local_max = -INFINITY;
    for (int p = tid; p < length; p += kSoftmaxThreads) {
        const float v = s[p];
        if constexpr (kExact) e_lds[p] = v;
        local_max = fmaxf(local_max, v);
    }
    reduction[tid] = local_max;
    __syncthreads();
    for (int w = kSoftmaxThreads / 2; w > 0; w >>= 1) {
        if (tid < w) reduction[tid] = fmaxf(reduction[tid], reduction[tid + w]);
        __syncthreads();
    }
    const float maximum = reduction[0];
    __syncthreads();
    if constexpr (kExact) {
        for (int p = tid; p < length; p += kSoftmaxThreads) e_lds[p] = q3_expf(e_lds[p] - maximum);
        __syncthreads();
        if (tid == 0) {
            float denominator = 0.0f;
            int p = 0;
#pragma unroll 4
            for (; p + 4 <= length; p += 4) {
                const float4 v = *reinterpret_cast<const float4*>(e_lds + p);
                denominator += v.x;
                denominator += v.y;
                denominator += v.z;
                denominator += v.w;
            }
            for (; p < length; ++p) denominator += e_lds[p];
            broadcast = 1.0f / denominator;
        }
        __syncthreads();
        const float inverse = broadcast;
        for (int p = tid; p < length; p += kSoftmaxThreads) s[p] = round_bf(e_lds[p] * inverse);
    } else {
        float local = 0.0f;
        for (int p = tid; p < length; p += kSoftmaxThreads) {
            const float w = q3_expf(s[p] - maximum);
            s[p] = w;
            local += w;
        }
        reduction[tid] = local;
        __syncthreads();
        for (int w = kSoftmaxThreads / 2; w > 0; w >>= 1) {
            if (tid < w) reduction[tid] += reduction[tid + w];
            __syncthreads();
        }
        if (tid == 0) a.inverse[static_cast<size_t>(row) * a.query_heads + head] = 1.0f / reduction[0];
    }
}

// Row stride of the probability table in LDS: 16-byte aligned and offset by
// four banks between query heads.
__host__ __device__ constexpr int lds_stride(int capacity) { return (capacity + 3) / 4 * 4 + 4; }

// ---------------------------------------------------------------------------
// values: grid (kv heads * 2G slices, rows), one wave.  Lane = (g, dim):
// g = lane / (64/G), dim = slice * (64/G) + lane % (64/G).  One 16-byte load
// per lane covers 8 dims of one position, so one wave load covers 8G
// positions ("a chunk").
// ---------------------------------------------------------------------------
template <bool kExact, int kG>
__global__ __launch_bounds__(64) void attention_values_kernel(AttnArgs a) {
    constexpr int kSliceDims = 64 / kG;
    constexpr int kLanesPerPos = kSliceDims / 8;
    constexpr int kPosPerChunk = 64 / kLanesPerPos;
    extern __shared__ __align__(16) float p_lds[];  // [kG][stride] probabilities
    __shared__ __align__(16) bf16_t v_lds[2][kPosPerChunk * kSliceDims];
    const int row = blockIdx.y;
    const int kvh = blockIdx.x / (2 * kG);
    const int slice = blockIdx.x % (2 * kG);
    const int lane = threadIdx.x;
    const int g = lane / kSliceDims;
    const int dl = lane % kSliceDims;
    const int length = row_length(a, row);
    const int stride = lds_stride(a.capacity);
    const float* scores = a.scores + (static_cast<size_t>(row) * a.query_heads + static_cast<size_t>(kvh) * kG) *
                                         a.capacity;
    // Probabilities into LDS, 16 loads in flight per lane.
    for (int gg = 0; gg < kG; ++gg) {
        const float* src = scores + static_cast<size_t>(gg) * a.capacity;
        for (int base = 0; base < length; base += 16 * 64) {
            float t[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int p = base + u * 64 + lane;
                t[u] = src[p < length ? p : length - 1];
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const int p = base + u * 64 + lane;
                if (p < length) p_lds[gg * stride + p] = t[u];
            }
        }
    }
    __syncthreads();

    const int kv_width = a.key_value_heads * kDim;
    const bf16_t* vbase = row_values(a, row) + static_cast<size_t>(kvh) * kDim + slice * kSliceDims +
                          (lane % kLanesPerPos) * 8;
    const int lane_pos = lane / kLanesPerPos;
    const int chunks = (length + kPosPerChunk - 1) / kPosPerChunk;
    auto load = [&](int c) {
        int pos = c * kPosPerChunk + lane_pos;
        pos = pos < length ? pos : length - 1;  // never past this row's last written position
        return load_global16(vbase + static_cast<size_t>(pos) * kv_width);
    };
    uint4 ring[kRing];
#pragma unroll
    for (int k = 0; k < kRing; ++k) ring[k] = load(k);

    const float* pg = p_lds + g * stride;
    float acc = 0.0f;
    for (int base = 0; base < chunks; base += kRing) {
#pragma unroll
        for (int k = 0; k < kRing; ++k) {
            const int c = base + k;
            bf16_t* slot = v_lds[k & 1];
            reinterpret_cast<uint4*>(slot)[lane] = ring[k];
            ring[k] = load(c + kRing);
            // issue the refill here, not where its value is next needed
            asm volatile("" ::: "memory");
            const int first = c * kPosPerChunk;
            if (first + kPosPerChunk <= length) {
#pragma unroll
                for (int j = 0; j < kPosPerChunk; j += 4) {
                    const float4 pv = *reinterpret_cast<const float4*>(pg + first + j);
                    acc = fmaf(pv.x, bf2f(slot[(j + 0) * kSliceDims + dl]), acc);
                    acc = fmaf(pv.y, bf2f(slot[(j + 1) * kSliceDims + dl]), acc);
                    acc = fmaf(pv.z, bf2f(slot[(j + 2) * kSliceDims + dl]), acc);
                    acc = fmaf(pv.w, bf2f(slot[(j + 3) * kSliceDims + dl]), acc);
                }
            } else if (first < length) {
                for (int j = 0; first + j < length; ++j) {
                    acc = fmaf(pg[first + j], bf2f(slot[j * kSliceDims + dl]), acc);
                }
            }
        }
    }
    const int head = kvh * kG + g;
    const int dim = slice * kSliceDims + dl;
    float y = acc;
    if constexpr (!kExact) y = acc * a.inverse[static_cast<size_t>(row) * a.query_heads + head];
    a.output[(static_cast<size_t>(row) * a.query_heads + head) * kDim + dim] = f2bf(y);
}

// ---------------------------------------------------------------------------
// Short caches (capacity <= 64, the code predictor's 16 positions): the three
// phases in one kernel, one block of G*128 threads per (kv head, row).  Same
// operation order as the split kernels.
// ---------------------------------------------------------------------------
constexpr int kSmallCapacity = 64;

template <bool kExact, int kG>
__global__ __launch_bounds__(kG * kDim) void attention_small_kernel(AttnArgs a) {
    __shared__ float q_lds[kG][kDim];
    __shared__ float prob[kG][kSmallCapacity];
    __shared__ float partial[kG][256];
    __shared__ float inverse_lds[kG];
    const int row = blockIdx.y;
    const int kvh = blockIdx.x;
    const int tid = threadIdx.x;
    const int length = row_length(a, row);
    const int kv_width = a.key_value_heads * kDim;
    const bf16_t* q = a.query + static_cast<size_t>(row) * a.query_stride + static_cast<size_t>(kvh) * kG * kDim;
    q_lds[tid / kDim][tid % kDim] = bf2f(q[tid]);
    __syncthreads();
    if (tid < kG * length) {
        const int g = tid / length;
        const int p = tid % length;
        const uint4* k4 = reinterpret_cast<const uint4*>(row_keys(a, row) + static_cast<size_t>(p) * kv_width +
                                                         static_cast<size_t>(kvh) * kDim);
        uint32_t kw[64];
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint4 t = load_global16(k4 + v);
            kw[4 * v + 0] = t.x;
            kw[4 * v + 1] = t.y;
            kw[4 * v + 2] = t.z;
            kw[4 * v + 3] = t.w;
        }
        const float* qg = q_lds[g];
        float score;
        if constexpr (kExact) {
            float sv[64];
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                const float kl = (t & 1) ? hi_bf(kw[t >> 1]) : lo_bf(kw[t >> 1]);
                const float kh = (t & 1) ? hi_bf(kw[32 + (t >> 1)]) : lo_bf(kw[32 + (t >> 1)]);
                sv[t] = fmaf(qg[t], kl, 0.0f) + fmaf(qg[t + 64], kh, 0.0f);
            }
#pragma unroll
            for (int w = 32; w > 0; w >>= 1) {
#pragma unroll
                for (int t = 0; t < w; ++t) sv[t] += sv[t + w];
            }
            score = round_bf(round_bf(sv[0]) * a.scale);
        } else {
            float dot = 0.0f;
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                dot = fmaf(qg[2 * t], lo_bf(kw[t]), dot);
                dot = fmaf(qg[2 * t + 1], hi_bf(kw[t]), dot);
            }
            score = dot * a.scale;
        }
        prob[g][p] = score;
    }
    __syncthreads();
    const int g = tid / kDim;
    const int d = tid % kDim;
    if (d == 0) {
        float* sg = prob[g];
        float maximum = -INFINITY;
        for (int p = 0; p < length; ++p) maximum = fmaxf(maximum, sg[p]);
        if constexpr (kExact) {
            float denominator = 0.0f;
            for (int p = 0; p < length; ++p) {
                sg[p] = q3_expf(sg[p] - maximum);
                denominator += sg[p];
            }
            const float inverse = 1.0f / denominator;
            for (int p = 0; p < length; ++p) sg[p] = round_bf(sg[p] * inverse);
        } else {
            // 256 strided partials (one term each here) and their tree
            float* part = partial[g];
            for (int t = 0; t < 256; ++t) part[t] = 0.0f;
            for (int p = 0; p < length; ++p) {
                sg[p] = q3_expf(sg[p] - maximum);
                part[p] += sg[p];
            }
            for (int w = 128; w > 0; w >>= 1) {
                for (int t = 0; t < w; ++t) part[t] += part[t + w];
            }
            inverse_lds[g] = 1.0f / part[0];
        }
    }
    __syncthreads();
    const bf16_t* vcol = row_values(a, row) + static_cast<size_t>(kvh) * kDim + d;
    float acc = 0.0f;
    int p = 0;
    for (; p + 8 <= length; p += 8) {
        float vv[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) vv[u] = bf2f(vcol[static_cast<size_t>(p + u) * kv_width]);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc = fmaf(prob[g][p + u], vv[u], acc);
    }
    for (; p < length; ++p) acc = fmaf(prob[g][p], bf2f(vcol[static_cast<size_t>(p) * kv_width]), acc);
    const int head = kvh * kG + g;
    float y = acc;
    if constexpr (!kExact) y = acc * inverse_lds[g];
    a.output[(static_cast<size_t>(row) * a.query_heads + head) * kDim + d] = f2bf(y);
}

template <bool kExact, int kG>
hipError_t launch_variant(const AttnArgs& a, int rows, hipStream_t stream) {
    const size_t softmax_lds = kExact ? static_cast<size_t>(a.capacity) * sizeof(float) : 0;
    const size_t values_lds = static_cast<size_t>(kG) * lds_stride(a.capacity) * sizeof(float);
    // LDS: up to 160 KB per workgroup on gfx950 (the value ring's 2 KB
    // static slots included).
    constexpr size_t kLdsLimit = 160 * 1024 - 2048 - 64;
    if (softmax_lds > kLdsLimit || values_lds > kLdsLimit) return hipErrorInvalidValue;
    static bool configured = false;
    if (!configured) {
        hipError_t st = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_softmax_kernel<kExact>),
                                            hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsLimit));
        if (st != hipSuccess) return st;
        st = hipFuncSetAttribute(reinterpret_cast<const void*>(attention_values_kernel<kExact, kG>),
                                 hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(kLdsLimit));
        if (st != hipSuccess) return st;
        configured = true;
    }
    if (a.capacity <= kSmallCapacity) {
        attention_small_kernel<kExact, kG><<<dim3(a.key_value_heads, rows), kG * kDim, 0, stream>>>(a);
        return hipGetLastError();
    }
    const dim3 score_grid((a.capacity + kScoreLanes - 1) / kScoreLanes, a.key_value_heads, rows);
    attention_scores_kernel<kExact, kG><<<score_grid, kScoreLanes, 0, stream>>>(a);
    attention_softmax_kernel<kExact><<<dim3(a.query_heads, rows), kSoftmaxThreads, softmax_lds, stream>>>(a);
    attention_values_kernel<kExact, kG><<<dim3(a.key_value_heads * 2 * kG, rows), 64, values_lds, stream>>>(a);
    return hipGetLastError();
}

}  // namespace

size_t attention_workspace_bytes(int rows, int query_heads, int capacity) {
    return static_cast<size_t>(rows) * query_heads * (static_cast<size_t>(capacity) + 1) * sizeof(float);
}

hipError_t launch_attention(bool exact, const bf16_t* query, int query_stride, bf16_t* const* key_bases,
                            bf16_t* const* value_bases, const bf16_t* key_cache, const bf16_t* value_cache,
                            const int* positions, int fixed_sequence_length, bf16_t* output, int rows,
                            int query_heads, int key_value_heads, int head_dimension, int max_sequence_length,
                            float* workspace, hipStream_t stream) {
    if (head_dimension != kDim || key_value_heads <= 0 || query_heads % key_value_heads != 0 || rows <= 0 ||
        max_sequence_length <= 0 || max_sequence_length > kMaxCapacity || workspace == nullptr ||
        query == nullptr || output == nullptr) {
        return hipErrorInvalidValue;
    }
    if ((key_bases == nullptr) != (value_bases == nullptr)) return hipErrorInvalidValue;
    if (key_bases == nullptr && (key_cache == nullptr || value_cache == nullptr)) return hipErrorInvalidValue;
    if (positions == nullptr && (fixed_sequence_length <= 0 || fixed_sequence_length > max_sequence_length)) {
        return hipErrorInvalidValue;
    }
    AttnArgs a;
    a.query = query;
    a.query_stride = query_stride;
    a.key_bases = key_bases;
    a.value_bases = value_bases;
    a.key_cache = key_cache;
    a.value_cache = value_cache;
    a.positions = positions;
    a.fixed_length = fixed_sequence_length;
    a.output = output;
    a.query_heads = query_heads;
    a.key_value_heads = key_value_heads;
    a.capacity = max_sequence_length;
    a.scale = 1.0f / sqrtf(static_cast<float>(head_dimension));
    a.scores = workspace;
    a.inverse = workspace + static_cast<size_t>(rows) * query_heads * max_sequence_length;
    const int group = query_heads / key_value_heads;
    switch (group) {
        case 1: return exact ? launch_variant<true, 1>(a, rows, stream) : launch_variant<false, 1>(a, rows, stream);
        case 2: return exact ? launch_variant<true, 2>(a, rows, stream) : launch_variant<false, 2>(a, rows, stream);
        case 4: return exact ? launch_variant<true, 4>(a, rows, stream) : launch_variant<false, 4>(a, rows, stream);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace q3
