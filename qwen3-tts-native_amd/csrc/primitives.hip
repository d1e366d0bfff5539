// Decode-step transformer primitives around the int8 GEMVs, gfx950.
//
// Arithmetic follows native/qwen3-tts-native/native/src/talker_kernels.cu
// (cited per kernel) with its operation order reproduced exactly, so results
// are bit-identical to the CPU restatement; the layouts and launch shapes are
// this build's own (wave64 reductions, one wave per head, device-resident
// positions so a frame can be replayed as a hipGraph).
#include <algorithm>
#include <mutex>

#include "q3_common.hpp"
#include "q3_math.h"
#include "head_device.hpp"

namespace q3 {
namespace {

constexpr int kThreads = 256;

using head_detail::wave_tree256;

// rms_norm_kernel (talker_kernels.cu:27-48), one wave64 per row.
__global__ __launch_bounds__(64) void rms_norm_rows_kernel(const bf16_t* input, const bf16_t* weight,
                                                           bf16_t* output, int width, float epsilon) {
    const bf16_t* in = input + static_cast<size_t>(blockIdx.x) * width;
    bf16_t* out = output + static_cast<size_t>(blockIdx.x) * width;
    const int lane = threadIdx.x;
    float part[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float s = 0.0f;
        for (int i = lane + 64 * j; i < width; i += 256) {
            const float v = bf2f(in[i]);
            s = fmaf(v, v, s);
        }
        part[j] = s;
    }
    const float total = wave_tree256(part[0], part[1], part[2], part[3]);
    const float inverse = 1.0f / sqrtf(total / static_cast<float>(width) + epsilon);
    for (int i = lane; i < width; i += 64) {
        const float normalized = round_bf(bf2f(in[i]) * inverse);
        out[i] = f2bf(normalized * bf2f(weight[i]));
    }
}

// The same for rows whose width is a multiple of 8 up to kNormMaxWidth: 256
// threads, the row staged into LDS with 16-byte loads, thread t's partial
// over x[t], x[t+256], ... in that order, the 256 partials folded in the
// block_sum tree order, then each thread normalizes 8-element chunks.
constexpr int kNormMaxWidth = 8192;

__global__ __launch_bounds__(kThreads) void rms_norm_rows_vec_kernel(const bf16_t* input, const bf16_t* weight,
                                                                     bf16_t* output, int width, float epsilon) {
    __shared__ uint4 x_lds[kNormMaxWidth / 8];
    __shared__ float partial_lds[kThreads];
    const uint4* in = reinterpret_cast<const uint4*>(input + static_cast<size_t>(blockIdx.x) * width);
    uint4* out = reinterpret_cast<uint4*>(output + static_cast<size_t>(blockIdx.x) * width);
    const uint4* gain = reinterpret_cast<const uint4*>(weight);
    const int chunks = width / 8;
    for (int c = threadIdx.x; c < chunks; c += kThreads) x_lds[c] = in[c];
    __syncthreads();
    const bf16_t* xs = reinterpret_cast<const bf16_t*>(x_lds);
    float s = 0.0f;
    for (int i = threadIdx.x; i < width; i += kThreads) {
        const float v = bf2f(xs[i]);
        s = fmaf(v, v, s);
    }
    partial_lds[threadIdx.x] = s;
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const float total = wave_tree256(partial_lds[lane], partial_lds[lane + 64], partial_lds[lane + 128],
                                     partial_lds[lane + 192]);
    const float inverse = 1.0f / sqrtf(total / static_cast<float>(width) + epsilon);
    for (int c = threadIdx.x; c < chunks; c += kThreads) {
        const uint4 xv = x_lds[c];
        const uint4 gv = gain[c];
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
        const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float lo = round_bf(__uint_as_float(xw[i] << 16) * inverse) * __uint_as_float(gw[i] << 16);
            const float hi = round_bf(__uint_as_float(xw[i] & 0xffff0000u) * inverse) *
                             __uint_as_float(gw[i] & 0xffff0000u);
            o[i] = static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
        }
        out[c] = make_uint4(o[0], o[1], o[2], o[3]);
    }
}

// Fused QKV epilogue, one wave64 per head:
//   q/k heads: head RMSNorm (talker_kernels.cu:50-70) then rotate-half RoPE
//   (talker_kernels.cu:72-114) with cos/sin read from a bf16 table built on
//   the host with the same float formula; k heads are then appended to the
//   cache, v heads are copied to the cache (the reference's two D2D copies,
//   talker.cu:3343-3364).  Supports head_dimension == 128.
// rope_table: [max_positions][head_dim/2][2] bf16 (cos, sin).
__global__ __launch_bounds__(64) void qk_norm_rope_kv_kernel(
    bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, bf16_t* const* key_bases,
    bf16_t* const* value_bases, const int* positions, const bf16_t* rope_table, int query_heads,
    int key_value_heads, float epsilon) {
    constexpr int kDim = 128;
    constexpr int kHalf = 64;
    const int heads = query_heads + 2 * key_value_heads;
    const int row = blockIdx.x / heads;
    const int head = blockIdx.x % heads;
    const int lane = threadIdx.x;
    const int q_width = query_heads * kDim;
    const int kv_width = key_value_heads * kDim;
    bf16_t* base = qkv + static_cast<size_t>(row) * (q_width + 2 * kv_width) +
                   static_cast<size_t>(head) * kDim;
    const int position = positions[row];
    if (head >= query_heads + key_value_heads) {
        const int vh = head - query_heads - key_value_heads;
        bf16_t* dst = value_bases[row] + static_cast<size_t>(position) * kv_width +
                      static_cast<size_t>(vh) * kDim;
        dst[lane] = base[lane];
        dst[lane + kHalf] = base[lane + kHalf];
        return;
    }
    const bool is_query = head < query_heads;
    const bf16_t* gain = is_query ? q_norm : k_norm;
    bf16_t out0, out1;
    head_detail::norm_rope_head(base, gain, rope_table + static_cast<size_t>(position) * kDim, epsilon, out0, out1);
    if (is_query) {
        base[lane] = out0;
        base[lane + kHalf] = out1;
    } else {
        const int kh = head - query_heads;
        bf16_t* dst = key_bases[row] + static_cast<size_t>(position) * kv_width +
                      static_cast<size_t>(kh) * kDim;
        dst[lane] = out0;
        dst[lane + kHalf] = out1;
    }
}

// Head RMSNorm alone (talker_kernels.cu:50-70), one wave per head, d = 128.
__global__ __launch_bounds__(64) void head_rms_norm_kernel(bf16_t* values, const bf16_t* weight,
                                                           float epsilon) {
    bf16_t* head = values + static_cast<size_t>(blockIdx.x) * 128;
    const int lane = threadIdx.x;
    const float x0 = bf2f(head[lane]);
    const float x1 = bf2f(head[lane + 64]);
    const float total = wave_tree256(fmaf(x0, x0, 0.0f), fmaf(x1, x1, 0.0f), 0.0f, 0.0f);
    const float inverse = 1.0f / sqrtf(total / 128.0f + epsilon);
    head[lane] = f2bf(round_bf(x0 * inverse) * bf2f(weight[lane]));
    head[lane + 64] = f2bf(round_bf(x1 * inverse) * bf2f(weight[lane + 64]));
}

// RoPE alone (talker_kernels.cu:72-114) with the reference's in-kernel
// powf/cosf/sinf angle.  Used only by the primitive self-test export; the
// decode path uses the host-built table above.
__global__ void rope_kernel(bf16_t* values, int rows, int heads, int head_dimension,
                            const int* positions, int first_position, float theta) {
    const int half = head_dimension / 2;
    const int pair = blockIdx.x * blockDim.x + threadIdx.x;
    const int row_pairs = heads * half;
    if (pair >= rows * row_pairs) return;
    const int row = pair / row_pairs;
    const int head = (pair % row_pairs) / half;
    const int d = pair % half;
    const int position = positions ? positions[row] : first_position + row;
    bf16_t* base = values + (static_cast<size_t>(row) * heads + head) * head_dimension;
    const float exponent = static_cast<float>(2 * d) / static_cast<float>(head_dimension);
    const float angle = static_cast<float>(position) * powf(theta, -exponent);
    const float c = round_bf(cosf(angle));
    const float s = round_bf(sinf(angle));
    const float first = bf2f(base[d]);
    const float second = bf2f(base[d + half]);
    const float fc = round_bf(first * c);
    const float ss = round_bf(second * s);
    const float sc = round_bf(second * c);
    const float fs = round_bf(first * s);
    base[d] = f2bf(fc - ss);
    base[d + half] = f2bf(sc + fs);
}

__global__ void kv_scatter_rows_kernel(const bf16_t* rows_data, bf16_t* const* cache_bases,
                                       const int* positions, int rows, int width, int row_stride) {
    const int index = blockIdx.x * blockDim.x + threadIdx.x;
    if (index >= rows * width) return;
    const int row = index / width;
    const int column = index % width;
    cache_bases[row][static_cast<size_t>(positions[row]) * width + column] =
        rows_data[static_cast<size_t>(row) * row_stride + column];
}

__global__ void add_in_place_kernel(bf16_t* destination, const bf16_t* source, int width) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < width) destination[i] = f2bf(bf2f(destination[i]) + bf2f(source[i]));
}

__global__ void bias_activation_rows_kernel(bf16_t* values, const bf16_t* bias, int total,
                                            int width, bool silu) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= total) return;
    float value = bf2f(values[i]) + bf2f(bias[i % width]);
    if (silu) value *= 1.0f / (1.0f + q3_expf(-value));
    values[i] = f2bf(value);
}

__global__ void silu_gate_kernel(bf16_t* gate, const bf16_t* up, int width) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width) return;
    const float g = bf2f(gate[i]);
    const float activated = round_bf(g / (1.0f + q3_expf(-g)));
    gate[i] = f2bf(activated * bf2f(up[i]));
}

__global__ void fill_zero_kernel(bf16_t* values, int width) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < width) values[i] = 0;
}

__global__ void increment_kernel(int* counter) {
    if (threadIdx.x == 0) *counter += 1;
}

// Deterministic N(mean, stddev) bf16 fill: Box-Muller on two 24-bit uniforms
// taken from a splitmix64 hash of (seed, index).
__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

__global__ void fill_normal_kernel(bf16_t* out, uint64_t count, uint64_t seed, float mean,
                                   float stddev) {
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const uint64_t h = splitmix64(seed * 0x100000001b3ULL + i);
        const float u1 = (static_cast<float>(h >> 40) + 1.0f) * (1.0f / 16777217.0f);
        const float u2 = static_cast<float>((h >> 16) & 0xffffffu) * (1.0f / 16777216.0f);
        const float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
        out[i] = f2bf(mean + stddev * z);
    }
}

int blocks_for(int n) { return (n + kThreads - 1) / kThreads; }

}  // namespace

hipError_t launch_increment(int* counter, hipStream_t stream) {
    increment_kernel<<<1, 64, 0, stream>>>(counter);
    return hipGetLastError();
}

hipError_t launch_fill_bf16_normal(bf16_t* destination, uint64_t count, uint64_t seed, float mean,
                                   float stddev, hipStream_t stream) {
    if (count == 0) return hipSuccess;
    uint64_t blocks = (count + kThreads - 1) / kThreads;
    if (blocks > 65536) blocks = 65536;
    fill_normal_kernel<<<static_cast<int>(blocks), kThreads, 0, stream>>>(destination, count, seed,
                                                                          mean, stddev);
    return hipGetLastError();
}

hipError_t launch_rms_norm_rows(const bf16_t* input, const bf16_t* weight, bf16_t* output, int rows,
                                int width, float epsilon, hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    const bool vec = width % 8 == 0 && width <= kNormMaxWidth &&
                     ((reinterpret_cast<uintptr_t>(input) | reinterpret_cast<uintptr_t>(weight) |
                       reinterpret_cast<uintptr_t>(output)) & 15u) == 0;
    if (vec) {
        rms_norm_rows_vec_kernel<<<rows, kThreads, 0, stream>>>(input, weight, output, width, epsilon);
    } else {
        rms_norm_rows_kernel<<<rows, 64, 0, stream>>>(input, weight, output, width, epsilon);
    }
    return hipGetLastError();
}

hipError_t launch_head_rms_norm_rows(bf16_t* values, const bf16_t* weight, int rows, int heads,
                                     int head_dimension, float epsilon, hipStream_t stream) {
    if (head_dimension != 128 || rows <= 0 || heads <= 0) return hipErrorInvalidValue;
    head_rms_norm_kernel<<<rows * heads, 64, 0, stream>>>(values, weight, epsilon);
    return hipGetLastError();
}

hipError_t launch_rope_rows(bf16_t* values, int rows, int heads, int head_dimension,
                            int first_position, float theta, hipStream_t stream) {
    if (head_dimension % 2 != 0 || rows <= 0) return hipErrorInvalidValue;
    const int pairs = rows * heads * head_dimension / 2;
    rope_kernel<<<blocks_for(pairs), kThreads, 0, stream>>>(values, rows, heads, head_dimension,
                                                            nullptr, first_position, theta);
    return hipGetLastError();
}

hipError_t launch_rope_rows_at(bf16_t* values, int rows, int heads, int head_dimension,
                               const int* positions, float theta, hipStream_t stream) {
    if (head_dimension % 2 != 0 || rows <= 0) return hipErrorInvalidValue;
    const int pairs = rows * heads * head_dimension / 2;
    rope_kernel<<<blocks_for(pairs), kThreads, 0, stream>>>(values, rows, heads, head_dimension,
                                                            positions, 0, theta);
    return hipGetLastError();
}

hipError_t launch_qk_norm_rope_kv_append(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm,
                                         bf16_t* const* key_bases, bf16_t* const* value_bases,
                                         const int* positions, const bf16_t* rope_table, int rows,
                                         int query_heads, int key_value_heads, int head_dimension,
                                         float epsilon, hipStream_t stream) {
    if (head_dimension != 128 || rows <= 0 || key_value_heads <= 0) return hipErrorInvalidValue;
    const int heads = query_heads + 2 * key_value_heads;
    qk_norm_rope_kv_kernel<<<rows * heads, 64, 0, stream>>>(qkv, q_norm, k_norm, key_bases,
                                                            value_bases, positions, rope_table,
                                                            query_heads, key_value_heads, epsilon);
    return hipGetLastError();
}

// Stand-alone forms (primitive self-test and op exports).  Their value caches
// have the reference's layout, [position][kv_width] per row; the attention
// kernels read blocked dimension-major values, so each call copies the written
// positions of every row into a stream-ordered temporary of that form (and,
// for the decode form, the appended position back).

// Blocked dimension-major index of element (position p, column c = kv head
// * 128 + dimension) in a row's value cache of the given stride.
__device__ __forceinline__ size_t blocked_value_index(int c, int p, int stride) {
    return ((static_cast<size_t>(c >> 7) * (stride >> 3) + (p >> 3)) * 128 + (c & 127)) * 8 + (p & 7);
}

// temporary[row] = cache(row) in the blocked layout for p < length(row), 0
// beyond; value_table[row] = the row's temporary.
__global__ __launch_bounds__(256) void values_to_dimension_major_kernel(
    bf16_t* const* value_bases, const bf16_t* value_cache, const int* positions, int fixed_length, int kv_width,
    int stride, bf16_t* temporary, bf16_t** value_table) {
    const int row = blockIdx.y;
    const size_t per_row = static_cast<size_t>(kv_width) * stride;
    bf16_t* dst = temporary + row * per_row;
    if (blockIdx.x == 0 && threadIdx.x == 0) value_table[row] = dst;
    const bf16_t* src = value_bases != nullptr ? value_bases[row] : value_cache;
    const int length = positions != nullptr ? positions[row] + 1 : fixed_length;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < per_row;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int c = static_cast<int>(t % kv_width);
        const int p = static_cast<int>(t / kv_width);
        dst[blocked_value_index(c, p, stride)] = p < length ? src[static_cast<size_t>(p) * kv_width + c] : f2bf(0.0f);
    }
}

// cache(row)[positions[row] * kv_width + c] = the temporary's element at
// (positions[row], c)
__global__ __launch_bounds__(256) void appended_value_back_kernel(bf16_t* const* value_bases, const int* positions,
                                                                  int kv_width, int stride,
                                                                  const bf16_t* temporary) {
    const int row = blockIdx.y;
    const int position = positions[row];
    const bf16_t* src = temporary + static_cast<size_t>(row) * kv_width * stride;
    for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < kv_width; c += gridDim.x * blockDim.x) {
        value_bases[row][static_cast<size_t>(position) * kv_width + c] = src[blocked_value_index(c, position, stride)];
    }
}

namespace {

struct ValueTemporary {
    void* memory = nullptr;
    bf16_t** table = nullptr;
    bf16_t* values = nullptr;
    int stride = 0;
};

size_t value_temporary_bytes(int rows, int kv_width, int capacity) {
    const size_t table_bytes = (static_cast<size_t>(rows) * sizeof(bf16_t*) + 255) / 256 * 256;
    return table_bytes + static_cast<size_t>(rows) * kv_width * value_cache_stride(capacity) * sizeof(bf16_t);
}

// Lays the temporary out in `memory` (value_temporary_bytes of it) and fills
// it: a table of per-row pointers, then each row's values dimension-major.
hipError_t fill_value_temporary(ValueTemporary& t, void* memory, bf16_t* const* value_bases,
                                const bf16_t* value_cache, const int* positions, int fixed_length, int rows,
                                int kv_width, int capacity, hipStream_t stream) {
    t.stride = value_cache_stride(capacity);
    const size_t table_bytes = (static_cast<size_t>(rows) * sizeof(bf16_t*) + 255) / 256 * 256;
    t.table = static_cast<bf16_t**>(memory);
    t.values = reinterpret_cast<bf16_t*>(static_cast<char*>(memory) + table_bytes);
    const size_t per_row = static_cast<size_t>(kv_width) * t.stride;
    const int blocks = static_cast<int>(std::min<size_t>((per_row + 255) / 256, 1024));
    values_to_dimension_major_kernel<<<dim3(blocks, rows), 256, 0, stream>>>(
        value_bases, value_cache, positions, fixed_length, kv_width, t.stride, t.values, t.table);
    return hipGetLastError();
}

hipError_t make_value_temporary(ValueTemporary& t, bf16_t* const* value_bases, const bf16_t* value_cache,
                                const int* positions, int fixed_length, int rows, int kv_width, int capacity,
                                hipStream_t stream) {
    hipError_t st = hipMallocAsync(&t.memory, value_temporary_bytes(rows, kv_width, capacity), stream);
    if (st != hipSuccess) return st;
    return fill_value_temporary(t, t.memory, value_bases, value_cache, positions, fixed_length, rows, kv_width,
                                capacity, stream);
}

hipError_t free_value_temporary(ValueTemporary& t, hipStream_t stream, hipError_t st) {
    if (t.memory == nullptr) return st;
    const hipError_t freed = hipFreeAsync(t.memory, stream);
    return st != hipSuccess ? st : freed;
}

}  // namespace

static hipError_t attention_with_temporary(bool exact, const bf16_t* query, int query_stride,
                                           bf16_t* const* key_bases, bf16_t* const* value_bases,
                                           const bf16_t* key_cache, const bf16_t* value_cache,
                                           const int* positions, int fixed_length, bf16_t* output, int rows,
                                           int query_heads, int key_value_heads, int head_dimension, int capacity,
                                           hipStream_t stream) {
    if (rows <= 0 || query_heads <= 0 || key_value_heads <= 0 || capacity <= 0) return hipErrorInvalidValue;
    if (value_bases == nullptr && value_cache == nullptr) return hipErrorInvalidValue;
    void* workspace = nullptr;
    hipError_t st = hipMallocAsync(&workspace, attention_workspace_bytes(rows, query_heads, capacity), stream);
    if (st != hipSuccess) return st;
    ValueTemporary values;
    st = make_value_temporary(values, value_bases, value_cache, positions, fixed_length, rows,
                              key_value_heads * head_dimension, capacity, stream);
    if (st == hipSuccess) {
        st = launch_attention(exact, query, query_stride, key_bases, value_bases != nullptr ? values.table : nullptr,
                              key_cache, values.values, positions, fixed_length, output, rows, query_heads,
                              key_value_heads, head_dimension, capacity, static_cast<float*>(workspace), nullptr,
                              stream);
    }
    st = free_value_temporary(values, stream, st);
    const hipError_t freed = hipFreeAsync(workspace, stream);
    return st != hipSuccess ? st : freed;
}

hipError_t launch_causal_gqa_attention(const bf16_t* query, const bf16_t* key_cache,
                                       const bf16_t* value_cache, bf16_t* output, int query_heads,
                                       int key_value_heads, int head_dimension,
                                       int sequence_length, int query_stride, hipStream_t stream) {
    return attention_with_temporary(true, query, query_stride, nullptr, nullptr, key_cache, value_cache, nullptr,
                                    sequence_length, output, 1, query_heads, key_value_heads, head_dimension,
                                    sequence_length, stream);
}

hipError_t launch_batch_causal_gqa_attention_fast(const bf16_t* query, bf16_t* const* key_bases,
                                                  bf16_t* const* value_bases, const int* positions,
                                                  bf16_t* output, int rows, int query_heads,
                                                  int key_value_heads, int head_dimension,
                                                  int max_sequence_length, int query_stride,
                                                  hipStream_t stream) {
    return attention_with_temporary(false, query, query_stride, key_bases, value_bases, nullptr, nullptr,
                                    positions, 0, output, rows, query_heads, key_value_heads, head_dimension,
                                    max_sequence_length, stream);
}

hipError_t launch_attention_op(bool exact, const bf16_t* query, int query_stride, bf16_t* const* key_bases,
                               bf16_t* const* value_bases, const int* positions, bf16_t* output, int rows,
                               int query_heads, int key_value_heads, int head_dimension, int max_sequence_length,
                               hipStream_t stream) {
    if (key_bases == nullptr || value_bases == nullptr || positions == nullptr) return hipErrorInvalidValue;
    return attention_with_temporary(exact, query, query_stride, key_bases, value_bases, nullptr, nullptr, positions,
                                    0, output, rows, query_heads, key_value_heads, head_dimension,
                                    max_sequence_length, stream);
}

hipError_t launch_prompt_attention_op(bool exact, const bf16_t* query, int query_stride, const bf16_t* key_cache,
                                      const bf16_t* value_cache, const int* positions, bf16_t* output, int rows,
                                      int query_heads, int key_value_heads, int head_dimension, int capacity,
                                      hipStream_t stream) {
    if (key_cache == nullptr || value_cache == nullptr || positions == nullptr || rows <= 0 || query_heads <= 0 ||
        key_value_heads <= 0 || capacity <= 0) {
        return hipErrorInvalidValue;
    }
    void* workspace = nullptr;
    hipError_t st = hipMallocAsync(&workspace, attention_workspace_bytes(rows, query_heads, capacity), stream);
    if (st != hipSuccess) return st;
    // the one shared cache, all of its positions, dimension-major
    ValueTemporary values;
    st = make_value_temporary(values, nullptr, value_cache, nullptr, capacity, 1, key_value_heads * head_dimension,
                              capacity, stream);
    if (st == hipSuccess) {
        st = launch_attention(exact, query, query_stride, nullptr, nullptr, key_cache, values.values, positions, 0,
                              output, rows, query_heads, key_value_heads, head_dimension, capacity,
                              static_cast<float*>(workspace), nullptr, stream);
    }
    st = free_value_temporary(values, stream, st);
    const hipError_t freed = hipFreeAsync(workspace, stream);
    return st != hipSuccess ? st : freed;
}

// File-scope scratch of the allocation-free decode attention entry point:
// each device holds its own copy for the life of the process.  In host code
// the name is only a stand-in; the device address comes from
// hipGetSymbolAddress, once per device, and only that address is used.
constexpr size_t kNoAllocScratchBytes = size_t{32} << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

bool decode_attention_args_ok(int rows, int query_heads, int key_value_heads, int head_dimension,
                              int max_sequence_length, bf16_t* const* key_bases, bf16_t* const* value_bases,
                              const int* positions) {
    return rows > 0 && query_heads > 0 && max_sequence_length > 0 && key_bases != nullptr && value_bases != nullptr &&
           key_value_heads > 0 && head_dimension == 128 && positions != nullptr;
}

size_t aligned256(size_t bytes) { return (bytes + 255) / 256 * 256; }

// The fused decode step on caller-provided scratch memory: the score
// workspace, then the dimension-major value temporary.  Nothing in it needs
// to start at zero (every element is written before it is read).
hipError_t decode_attention_in(void* scratch, bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                               const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                               bf16_t* const* key_bases, bf16_t* const* value_bases, const int* positions,
                               bf16_t* output, int rows, int query_heads, int key_value_heads, int head_dimension,
                               int max_sequence_length, hipStream_t stream) {
    const int kv_width = key_value_heads * head_dimension;
    float* workspace = static_cast<float*>(scratch);
    void* temporary =
        static_cast<char*>(scratch) + aligned256(attention_workspace_bytes(rows, query_heads, max_sequence_length));
    ValueTemporary values;
    hipError_t st = fill_value_temporary(values, temporary, value_bases, nullptr, positions, 0, rows, kv_width,
                                         max_sequence_length, stream);
    if (st == hipSuccess) {
        st = launch_decode_attention(exact, qkv, qkv_stride, q_norm, k_norm, rope_table, epsilon, key_bases,
                                     values.table, nullptr, nullptr, positions, output, rows, query_heads,
                                     key_value_heads, head_dimension, max_sequence_length, workspace, nullptr, stream);
    }
    if (st == hipSuccess) {
        appended_value_back_kernel<<<dim3((kv_width + 255) / 256, rows), 256, 0, stream>>>(
            value_bases, positions, kv_width, values.stride, values.values);
        st = hipGetLastError();
    }
    return st;
}

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_address[kMaxDevices] = {};
// Stream-order guard of each device's scratch: the last eager call's stream
// and an event recorded after its kernels.
struct ScratchUse {
    hipEvent_t done = nullptr;
    hipStream_t stream = nullptr;
    bool recorded = false;
};
ScratchUse scratch_use[kMaxDevices];

hipError_t scratch_for_current_device(void** out) {
    int device = 0;
    hipError_t st = hipGetDevice(&device);
    if (st != hipSuccess) return st;
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    if (scratch_address[device] == nullptr) {
        void* ptr = nullptr;
        st = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (st != hipSuccess) return st;
        scratch_address[device] = ptr;
    }
    *out = scratch_address[device];
    return hipSuccess;
}

}  // namespace

size_t decode_attention_scratch_bytes(int rows, int query_heads, int key_value_heads, int head_dimension,
                                      int max_sequence_length) {
    return aligned256(attention_workspace_bytes(rows, query_heads, max_sequence_length)) +
           value_temporary_bytes(rows, key_value_heads * head_dimension, max_sequence_length);
}

size_t decode_attention_scratch_limit() { return kNoAllocScratchBytes; }

hipError_t launch_decode_attention_op(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                      const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                      bf16_t* const* key_bases, bf16_t* const* value_bases, const int* positions,
                                      bf16_t* output, int rows, int query_heads, int key_value_heads,
                                      int head_dimension, int max_sequence_length, hipStream_t stream) {
    if (!decode_attention_args_ok(rows, query_heads, key_value_heads, head_dimension, max_sequence_length, key_bases,
                                  value_bases, positions)) {
        return hipErrorInvalidValue;
    }
    void* memory = nullptr;
    hipError_t st = hipMallocAsync(
        &memory, decode_attention_scratch_bytes(rows, query_heads, key_value_heads, head_dimension, max_sequence_length),
        stream);
    if (st != hipSuccess) return st;
    st = decode_attention_in(memory, exact, qkv, qkv_stride, q_norm, k_norm, rope_table, epsilon, key_bases,
                             value_bases, positions, output, rows, query_heads, key_value_heads, head_dimension,
                             max_sequence_length, stream);
    const hipError_t freed = hipFreeAsync(memory, stream);
    return st != hipSuccess ? st : freed;
}

hipError_t launch_decode_attention_op_noalloc(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                              const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                              bf16_t* const* key_bases, bf16_t* const* value_bases,
                                              const int* positions, bf16_t* output, int rows, int query_heads,
                                              int key_value_heads, int head_dimension, int max_sequence_length,
                                              hipStream_t stream) {
    if (!decode_attention_args_ok(rows, query_heads, key_value_heads, head_dimension, max_sequence_length, key_bases,
                                  value_bases, positions)) {
        return hipErrorInvalidValue;
    }
    if (decode_attention_scratch_bytes(rows, query_heads, key_value_heads, head_dimension, max_sequence_length) >
        kNoAllocScratchBytes) {
        return hipErrorInvalidValue;
    }
    void* memory = nullptr;
    hipError_t st = scratch_for_current_device(&memory);
    if (st != hipSuccess) return st;
    auto enqueue = [&] {
        return decode_attention_in(memory, exact, qkv, qkv_stride, q_norm, k_norm, rope_table, epsilon, key_bases,
                                   value_bases, positions, output, rows, query_heads, key_value_heads,
                                   head_dimension, max_sequence_length, stream);
    };
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    st = hipStreamIsCapturing(stream, &capture);
    if (st != hipSuccess) return st;
    if (capture != hipStreamCaptureStatusNone) {
        // Under capture the graph orders the call; replays of graphs that hold
        // it must not overlap on one device (documented in the header).
        return enqueue();
    }
    // Eager calls share the device's scratch in stream order: a call on
    // another stream than the previous one first waits for the previous
    // call's kernels, then marks its own end.
    int device = 0;
    st = hipGetDevice(&device);
    if (st != hipSuccess) return st;
    std::lock_guard<std::mutex> lock(scratch_mutex);
    ScratchUse& use = scratch_use[device];
    if (use.done == nullptr) {
        st = hipEventCreateWithFlags(&use.done, hipEventDisableTiming);
        if (st != hipSuccess) return st;
    }
    if (use.recorded && use.stream != stream) {
        st = hipStreamWaitEvent(stream, use.done, 0);
        if (st != hipSuccess) return st;
    }
    st = enqueue();
    if (st != hipSuccess) return st;
    st = hipEventRecord(use.done, stream);
    if (st != hipSuccess) return st;
    use.stream = stream;
    use.recorded = true;
    return hipSuccess;
}

hipError_t launch_kv_scatter_rows(const bf16_t* rows_data, bf16_t* const* cache_bases,
                                  const int* positions, int rows, int width, int row_stride,
                                  hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    kv_scatter_rows_kernel<<<blocks_for(rows * width), kThreads, 0, stream>>>(
        rows_data, cache_bases, positions, rows, width, row_stride);
    return hipGetLastError();
}

hipError_t launch_add_in_place(bf16_t* destination, const bf16_t* source, int width,
                               hipStream_t stream) {
    if (width <= 0) return hipErrorInvalidValue;
    add_in_place_kernel<<<blocks_for(width), kThreads, 0, stream>>>(destination, source, width);
    return hipGetLastError();
}

hipError_t launch_bias_activation_rows(bf16_t* values, const bf16_t* bias, int rows, int width,
                                       bool silu, hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    bias_activation_rows_kernel<<<blocks_for(rows * width), kThreads, 0, stream>>>(
        values, bias, rows * width, width, silu);
    return hipGetLastError();
}

hipError_t launch_silu_gate(bf16_t* gate, const bf16_t* up, int width, hipStream_t stream) {
    if (width <= 0) return hipErrorInvalidValue;
    silu_gate_kernel<<<blocks_for(width), kThreads, 0, stream>>>(gate, up, width);
    return hipGetLastError();
}

hipError_t launch_fill_zero(bf16_t* values, int width, hipStream_t stream) {
    if (width <= 0) return hipErrorInvalidValue;
    fill_zero_kernel<<<blocks_for(width), kThreads, 0, stream>>>(values, width);
    return hipGetLastError();
}

}  // namespace q3
