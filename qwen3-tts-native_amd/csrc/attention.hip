// Decode attention over a bf16 KV cache, head dimension 128.  Four main kernels:
//
//   scores  (caches > 64 positions) one wave per (64 positions, query head,
//           row), lane = position: the query head and the new key are
//           RMSNormed and rotated in-lane, the group's first head appends the
//           new key and value to the caches, then each lane runs the
//           reference's dot tree over the 128 dimensions for its position.
//   head    (caches > 64 positions) one wave per (row, query head, half of
//           the head dimension), lane = dimension: the softmax of the head's
//           scores (maximum, exponentials, normalizer) runs under a 16-deep
//           register ring of 16-byte value loads from the blocked
//           dimension-major value cache, then each lane runs the reference's
//           sequential chain over positions.
//   short   (the code predictor's <= 16 positions) one wave per query head:
//           append, scores, softmax and values fused, with the QKV epilogue.
//   small   (other caches <= 64 positions) one block of G*128 threads per
//           (kv head, row), the phases in one kernel.
// and two for particular callers: prompt-row score tiles (many prompt rows on
// one shared, complete cache: each key row loaded once for a tile of rows and
// the heads of its group), and the combine of the batched (non-exact) value
// chains when they run as position segments (tolerance mode only).
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
#include <cstdlib>
#include <cstring>
#include <type_traits>

#include "q3_common.hpp"
#include "q3_math.h"
#include "head_device.hpp"
#include "short_attention.hpp"

namespace q3 {
namespace {

constexpr int kDim = 128;
constexpr int kScoreLanes = 64;   // positions per score block
constexpr int kRing = 16;         // value loads in flight per lane
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
    // Fused QKV epilogue: `query` is the raw fused q|k|v row; the query heads
    // are normalized and rotated here, and the current position's key
    // (normalized, rotated) and value are appended to the caches and used
    // directly.  Null q_norm: `query` is final and the caches are complete.
    const bf16_t* q_norm;
    const bf16_t* k_norm;
    const bf16_t* rope_table;  // [positions][64][cos, sin] bf16
    float epsilon;
    // Value caches are blocked dimension-major: element (position p, kv head
    // h, dimension d) at [((h * stride / 8 + p / 8) * 128 + d) * 8 + p % 8]:
    // 16-byte groups of 8 positions of one (head, dimension), the 128
    // dimensions of a head side by side for each 8 positions (so a wave's
    // 64 dimensions read 1 KB in one piece).  stride >= capacity, a multiple
    // of 8; per row from value_strides when that is set.
    int value_stride;
    const int* value_strides;
    // Batched (non-exact) value chains split over position_splits segments
    // (tolerance semantics only): unnormalized partial chains in `partials`
    // [rows][query_heads][splits][128], added in segment order by a second
    // launch, which applies the inverse (`inverse`).
    int position_splits;
    float* partials;
    // Factor on the exact kernel's provisional normalizer (1 in production;
    // QWEN3_TTS_ATTENTION_SKEW_PROVISIONAL=1 sets 1 + 2^-7 so that the
    // provisional probabilities differ and the rerun path runs).
    float provisional_scale;
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

__device__ __forceinline__ int row_value_stride(const AttnArgs& a, int row) {
    return a.value_strides != nullptr ? a.value_strides[row] : a.value_stride;
}

// Elements between consecutive 8-position groups of one (head, dimension).
constexpr int kGroupStep = kDim * 8;

// Group 0 (positions 0..7) of (kv head kvh, dimension d) in row's value
// cache; group g is kGroupStep * g elements further.
__device__ __forceinline__ bf16_t* value_run(const AttnArgs& a, int row, int kvh, int d) {
    return const_cast<bf16_t*>(row_values(a, row)) +
           (static_cast<size_t>(kvh) * (row_value_stride(a, row) / 8) * kDim + d) * 8;
}

__device__ __forceinline__ int value_offset(int position) { return (position >> 3) * kGroupStep + (position & 7); }

// Value of the current position, dimensions lane and lane + 64 of kv head
// kvh, into the blocked cache.
__device__ __forceinline__ void append_value(const AttnArgs& a, int row, int kvh, int position, int lane, bf16_t v0,
                                             bf16_t v1) {
    value_run(a, row, kvh, lane)[value_offset(position)] = v0;
    value_run(a, row, kvh, lane + 64)[value_offset(position)] = v1;
}

// Cache rows are reached through pointer tables, which the compiler cannot
// place in the global address space by itself; a flat load would also count
// against the LDS counter and serialize with the LDS traffic.
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 load_global16(const void* p) {
    const u32x4 v = *(const __attribute__((address_space(1))) u32x4*)(reinterpret_cast<uintptr_t>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// Appends the current position's key and value of kv head `kvh` (one full
// wave); returns this lane's key and value elements lane and lane+64.
__device__ __forceinline__ void append_kv(const AttnArgs& a, int row, int kvh, int position, bf16_t& k0,
                                          bf16_t& k1, bf16_t& v0, bf16_t& v1) {
    constexpr int kDim = 128;
    const int lane = threadIdx.x & 63;
    const int kv_width = a.key_value_heads * kDim;
    const bf16_t* raw = a.query + static_cast<size_t>(row) * a.query_stride +
                        static_cast<size_t>(a.query_heads) * kDim;
    head_detail::norm_rope_head(raw + static_cast<size_t>(kvh) * kDim, a.k_norm,
                                a.rope_table + static_cast<size_t>(position) * kDim, a.epsilon, k0, k1);
    const bf16_t* vraw = raw + kv_width + static_cast<size_t>(kvh) * kDim;
    v0 = vraw[lane];
    v1 = vraw[lane + 64];
    bf16_t* kdst = (a.key_bases != nullptr ? a.key_bases[row] : const_cast<bf16_t*>(a.key_cache)) +
                   static_cast<size_t>(position) * kv_width + static_cast<size_t>(kvh) * kDim;
    kdst[lane] = k0;
    kdst[lane + 64] = k1;
    append_value(a, row, kvh, position, lane, v0, v1);
}

__device__ __forceinline__ float lo_bf(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Exact score of one (query head, position): the reference's block_sum over
// 256 threads where thread t < 128 holds q[t]k[t] and the rest zero.  Level
// 128 adds zeros (a no-op up to the sign of a zero dot, which no later step
// can observe); level 64 pairs t with t+64; then halves down to 1.  The dot
// is rounded to bf16, scaled and rounded again.  kw: the key row as 64
// packed bf16 pairs.
__device__ __forceinline__ float exact_score(const float* qg, const uint32_t (&kw)[64], float scale) {
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
    return round_bf(round_bf(s[0]) * scale);
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// The key pair (k[t], k[t + 64]) of a key row held as 64 packed bf16 pairs
// (kw[j] = (k[2j], k[2j + 1]), kw[32 + j] = (k[64 + 2j], k[65 + 2j])).
__device__ __forceinline__ uint32_t key_pair(const uint32_t (&kw)[64], int t) {
    const uint32_t lo = kw[t >> 1], hi = kw[32 + (t >> 1)];
    return (t & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
}

// exact_score's arithmetic on bf16 pairs: leaf t = q[t] k[t] + q[t+64] k[t+64]
// as one bf16 dot2 on (q[t], q[t+64]) x (k[t], k[t+64]) -- both products of
// bf16 values are exact in fp32, so the sum rounds once, as the two fmas and
// the add do -- then the same tree (s[t] += s[t + w], w = 32..1) evaluated
// as a stack over the leaves in post-order (bit-reversed index order): at
// most six partial sums live.  Bit-identical to exact_score.  kp(t): the
// key pair of leaf t.
template <typename KeyPair>
__device__ __forceinline__ float exact_score_pairs(const uint32_t* qp, KeyPair kp, float scale) {
    float stack[6];
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        const int t = static_cast<int>(__builtin_bitreverse32(static_cast<unsigned>(i)) >> 26);
        float v = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, qp[t]), __builtin_bit_cast(bf16x2_t, kp(t)),
                                                  0.0f, false);
#pragma unroll
        for (int b = 0; b < 6; ++b) {
            if (((i >> b) & 1) == 0) break;
            v = stack[b] + v;  // earlier (left) subtree + this one
        }
        stack[__builtin_ctz(~static_cast<unsigned>(i)) < 6 ? __builtin_ctz(~static_cast<unsigned>(i)) : 0] = v;
    }
    return round_bf(round_bf(stack[0]) * scale);
}

// ---------------------------------------------------------------------------
// scores: grid (position blocks, kv heads, rows), 64 threads, lane = position
// ---------------------------------------------------------------------------
template <bool kExact, int kG>
__global__ __launch_bounds__(kScoreLanes) void attention_scores_kernel(AttnArgs a) {
    // one wave per (64 positions, query head, row)
    const int row = blockIdx.z;
    const int head = blockIdx.y;
    const int kvh = head / kG;
    const int length = row_length(a, row);
    const int p0 = blockIdx.x * kScoreLanes;
    if (p0 >= length) return;
    __shared__ float q_lds[kDim];
    __shared__ uint32_t q_pairs[kDim / 2];  // (q[t], q[t + 64]) bf16 pairs for the exact score
    __shared__ uint32_t knew_lds[kDim / 2];
    const int lane = threadIdx.x;
    const int position = length - 1;
    const int p = p0 + lane;
    const int kv_width = a.key_value_heads * kDim;
    // key row first (independent of the query)
    const int prow = p < length ? p : position;
    const uint4* k4 = reinterpret_cast<const uint4*>(row_keys(a, row) + static_cast<size_t>(prow) * kv_width +
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
    const bf16_t* q = a.query + static_cast<size_t>(row) * a.query_stride + static_cast<size_t>(head) * kDim;
    const bool fused = a.q_norm != nullptr;
    if (fused) {
        const bf16_t* cs = a.rope_table + static_cast<size_t>(position) * kDim;
        bf16_t q0, q1;
        head_detail::norm_rope_head(q, a.q_norm, cs, a.epsilon, q0, q1);
        q_lds[lane] = bf2f(q0);
        q_lds[lane + 64] = bf2f(q1);
        q_pairs[lane] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, q0)) |
                        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, q1)) << 16);
        if (position >= p0 && position < p0 + kScoreLanes) {
            // the current key; the group's first query head appends it (and
            // the value) to the caches
            bf16_t k0, k1, v0, v1;
            if (head % kG == 0) {
                append_kv(a, row, kvh, position, k0, k1, v0, v1);
            } else {
                const bf16_t* kraw = a.query + static_cast<size_t>(row) * a.query_stride +
                                     static_cast<size_t>(a.query_heads + kvh) * kDim;
                head_detail::norm_rope_head(kraw, a.k_norm, cs, a.epsilon, k0, k1);
            }
            reinterpret_cast<bf16_t*>(knew_lds)[lane] = k0;
            reinterpret_cast<bf16_t*>(knew_lds)[lane + 64] = k1;
        }
    } else {
        q_lds[lane] = bf2f(q[lane]);
        q_lds[lane + 64] = bf2f(q[lane + 64]);
        q_pairs[lane] = static_cast<uint32_t>(__builtin_bit_cast(uint16_t, q[lane])) |
                        (static_cast<uint32_t>(__builtin_bit_cast(uint16_t, q[lane + 64])) << 16);
    }
    __syncthreads();
    if (p >= length) return;
    if (fused && p == position) {
#pragma unroll
        for (int i = 0; i < 64; ++i) kw[i] = knew_lds[i];
    }
    float score;
    if constexpr (kExact) {
        score = exact_score_pairs(q_pairs, [&](int t) { return key_pair(kw, t); }, a.scale);
    } else {
        float dot = 0.0f;
#pragma unroll
        for (int t = 0; t < 64; ++t) {
            dot = fmaf(q_lds[2 * t], lo_bf(kw[t]), dot);
            dot = fmaf(q_lds[2 * t + 1], hi_bf(kw[t]), dot);
        }
        score = dot * a.scale;
    }
    a.scores[(static_cast<size_t>(row) * a.query_heads + head) * a.capacity + p] = score;
}


// Prompt rows against one shared, complete key cache (the prefill's exact
// attention for long prompts: queries already normalized and rotated):
// grid (position blocks, kv heads, tiles of kRows rows), one wave, lane =
// position.  The key row is loaded once for the kRows rows and kG query
// heads of the tile (the per-row kernel loads it once per row and head).
// Each score is exact_score's arithmetic: leaf t = q[t] k[t] + q[t+64]
// k[t+64], here one bf16 dot2 on the pairs (q[t], q[t+64]) and (k[t],
// k[t+64]) -- both products of bf16 values are exact in fp32, so the sum
// rounds once, as the two fmas and the add do -- then the same tree
// (s[t] += s[t + w], w = 32..1), evaluated as a stack over the leaves in
// post-order (bit-reversed index order), so at most six partial sums are
// live.  Scores are bit-identical to attention_scores_kernel's.
template <int kG, int kRows>
__global__ __launch_bounds__(kScoreLanes) void attention_scores_rows_kernel(AttnArgs a, int rows) {
    const int r0 = blockIdx.z * kRows;
    const int kvh = blockIdx.y;
    const int p0 = blockIdx.x * kScoreLanes;
    const int last = min(r0 + kRows, rows) - 1;
    int longest = 0;
    for (int r = r0; r <= last; ++r) longest = max(longest, row_length(a, r));
    if (p0 >= longest) return;
    __shared__ uint32_t q_pairs[kRows][kG][kDim / 2];  // (q[t], q[t + 64]) bf16 pairs
    const int lane = threadIdx.x;
    const int p = p0 + lane;
    const int kv_width = a.key_value_heads * kDim;
    const int prow = p < longest ? p : longest - 1;
    const uint4* k4 = reinterpret_cast<const uint4*>(a.key_cache + static_cast<size_t>(prow) * kv_width +
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
    for (int i = lane; i < kRows * kG * (kDim / 2); i += kScoreLanes) {
        const int r = i / (kG * (kDim / 2));
        const int h = (i / (kDim / 2)) % kG;
        const int t = i % (kDim / 2);
        const int row = min(r0 + r, last);
        const uint16_t* q = reinterpret_cast<const uint16_t*>(a.query) + static_cast<size_t>(row) * a.query_stride +
                            static_cast<size_t>(kvh * kG + h) * kDim;
        q_pairs[r][h][t] = static_cast<uint32_t>(q[t]) | (static_cast<uint32_t>(q[t + 64]) << 16);
    }
    // key pairs (k[t], k[t + 64]), once for the tile's rows and heads
    uint32_t kp[64];
#pragma unroll
    for (int t = 0; t < 64; ++t) kp[t] = key_pair(kw, t);
    __syncthreads();
    for (int r = 0; r < kRows && r0 + r <= last; ++r) {
        const int row = r0 + r;
        if (p >= row_length(a, row)) continue;
#pragma unroll
        for (int h = 0; h < kG; ++h) {
            a.scores[(static_cast<size_t>(row) * a.query_heads + kvh * kG + h) * a.capacity + p] =
                exact_score_pairs(q_pairs[r][h], [&](int t) { return kp[t]; }, a.scale);
        }
    }
}

// Prompt rows per tile of attention_scores_rows_kernel.
constexpr int kPromptTileRows = 4;

// Row stride of the probability table in LDS: whole 64-position blocks plus
// one (the exact normalizer's look-ahead block), 16-byte aligned, and offset
// by four banks between query heads.
__host__ __device__ constexpr int lds_stride(int capacity) { return (capacity + 127) / 128 * 128 + 64; }

// Wave-wide max (order independent).
// Maximum over the wave, in every lane (the whole wave must be active).
__device__ __forceinline__ float wave_max(float v) {
    return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_max_down(v))));
}

// ---------------------------------------------------------------------------
// softmax + values: grid (query heads * 2, rows), one wave per (row, query
// head, half of the head dimension); lane = dimension.
//   1. the lane's value run (blocked dimension-major cache) is requested first,
//      8 positions per 16-byte load, kRing loads ahead;
//   2. the head's scores into LDS, the maximum;
//   3. exponentials and the normalizer (exact: the sequential sum of one
//      thread, overlapped with the exponentials of the next block; fast: the
//      256-thread strided partials and tree), then the probabilities (exact:
//      bf16, stored as one half of a bf16 pair);
//   4. the chain over positions: every lane reads the probabilities by LDS
//      broadcast (four per read) and applies them to its own value loads --
//      one VALU operation per position when exact (a bf16 dot2 on the packed
//      value pair), two otherwise (unpack, fma).
// Positions past the length carry probability 0 up to the end of the last
// ring round; full rounds run in a loop without side exits, the last partial
// round masks its values.
// ---------------------------------------------------------------------------

// acc = fmaf(p[e], v[e], acc) for the 8 positions of a group (fp32
// weights, values unpacked from bf16; values past `live` read 0).
__device__ __forceinline__ float chain8(float acc, const uint4& w, const float* p, int live) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float v = e < live ? __uint_as_float((e & 1) ? (words[e >> 1] & 0xffff0000u) : (words[e >> 1] << 16))
                                 : 0.0f;
        acc = fmaf(p[e], v, acc);
    }
    return acc;
}

// The exact chain with bf16 probabilities: acc = p * v + acc for each of the
// 8 positions of a group as a bf16 dot2 whose other product is 0 * (the
// neighbouring value).  A product of two bf16 values is exact in fp32, so
// the dot2 rounds once, like the fma (values past `live` are masked to 0).
__device__ __forceinline__ float chain8_pairs(float acc, const uint4& w, const float* p, int live) {
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        uint32_t word = words[e >> 1];
        const int first = e & ~1;  // the pair's even position
        word = first + 1 < live ? word : (first < live ? (word & 0xffffu) : 0u);
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, __float_as_uint(p[e])),
                                              __builtin_bit_cast(bf16x2_t, word), acc, false);
    }
    return acc;
}

// The head's scores (fp32, `length` of them) into LDS, 16 loads in flight
// per lane; returns their maximum in every lane.
__device__ __forceinline__ float scores_to_lds(const float* src, int length, float* p_lds, int lane) {
    float m = -INFINITY;
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
            if (p < length) {
                p_lds[p] = t[u];
                m = fmaxf(m, t[u]);
            }
        }
    }
    return wave_max(m);
}

// Exact softmax over the scores in p_lds (one wave): thread 0 of the
// reference's block takes one sequential sum (every lane runs the same
// additions on the same values).  Blocks of 64 positions: the sum over block
// b is interleaved with the exponentials of block b+1; exponentials past the
// length are 0 (x + 0 == x for the non-negative running sum).  Then the
// probabilities bf16(e * (1/sum)), each stored as one half of a bf16 pair
// (the half of the position's parity, the other 0) up to `padded` (a
// multiple of 128 >= length); p_lds holds at least ceil(length / 128) * 128
// + 64 floats (the look-ahead block's exponentials are written as zeros).
__device__ __forceinline__ void exact_probabilities(float* p_lds, int length, int padded, float maximum, int lane) {
    auto exps = [&](int block) {
        const int p = block * 64 + lane;
        const float t = p_lds[p < length ? p : length - 1];
        p_lds[p] = p < length ? q3_expf(t - maximum) : 0.0f;
    };
    const int blocks = (length + 63) / 64;
    const float4* all = reinterpret_cast<const float4*>(p_lds);
    float denominator = 0.0f;
    exps(0);
    for (int b = 0; b < blocks; ++b) {
        float4 v[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) v[u] = all[b * 16 + u];  // block b, requested first
        exps(b + 1);
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            denominator += v[u].x;
            denominator += v[u].y;
            denominator += v[u].z;
            denominator += v[u].w;
        }
    }
    const float inverse = 1.0f / denominator;
    // reads first, then the conversions
    auto convert = [&](int base, auto count) {
        constexpr int kCount = decltype(count)::value;
        float t[kCount];
#pragma unroll
        for (int u = 0; u < kCount; ++u) t[u] = p_lds[base + u * 64 + lane];
#pragma unroll
        for (int u = 0; u < kCount; ++u) {
            const uint32_t bits = __float_as_uint(round_bf(t[u] * inverse));
            p_lds[base + u * 64 + lane] = __uint_as_float((lane & 1) ? (bits & 0xffff0000u) : (bits >> 16));
        }
    };
    int base = 0;
    for (; base + 512 <= padded; base += 512) convert(base, std::integral_constant<int, 8>());
    for (; base < padded; base += 128) convert(base, std::integral_constant<int, 2>());
}

template <bool kExact, int kG, bool kSplit = false>
__global__ __launch_bounds__(64) void attention_head_kernel(AttnArgs a) {
    extern __shared__ __align__(16) float p_lds[];  // scores, then exponentials, then probabilities
    const int row = blockIdx.y;
    const int head = blockIdx.x >> 1;
    const int half = blockIdx.x & 1;
    const int kvh = head / kG;
    const int lane = threadIdx.x;
    const int length = row_length(a, row);
    // kSplit: this workgroup's segment of the value chain (whole ring rounds)
    constexpr int kRound = kRing * 8;
    int chain_begin = 0, chain_end = length;
    if constexpr (kSplit) {
        const int per = ((length + gridDim.z - 1) / gridDim.z + kRound - 1) / kRound * kRound;
        chain_begin = min(length, static_cast<int>(blockIdx.z) * per);
        chain_end = min(length, chain_begin + per);
    }

    // 1. value ring
    const bf16_t* vrun = value_run(a, row, kvh, half * 64 + lane);
    const int last_group = row_value_stride(a, row) / 8 - 1;
    auto load = [&](int i) { return load_global16(vrun + kGroupStep * (i < last_group ? i : last_group)); };
    uint4 ring[kRing];
#pragma unroll
    for (int k = 0; k < kRing; ++k) ring[k] = load(chain_begin / 8 + k);
    asm volatile("" ::: "memory");  // in flight before the scores are requested

    // 2. this head's scores into LDS, 16 loads in flight per lane
    const float* src = a.scores + (static_cast<size_t>(row) * a.query_heads + head) * a.capacity;
    const float maximum = scores_to_lds(src, length, p_lds, lane);
    const int padded = (length + kRing * 8 - 1) / (kRing * 8) * (kRing * 8);  // end of the last ring round

    // 3. exponentials, normalizer, probabilities
    float inverse = 1.0f;
    if constexpr (kExact) {
        exact_probabilities(p_lds, length, padded, maximum, lane);
    } else {
        // 256 strided partials: lane l holds those of threads l, l+64,
        // l+128, l+192; the block_sum tree's levels 128 and 64 are lane
        // local, the rest a wave tree.  The weights stay unnormalized; the
        // chain's result is scaled by 1/sum.
        float partial[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int base = 0; base < padded; base += 8 * 64) {
            float t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = base + u * 64 + lane;
                t[u] = p_lds[p < length ? p : length - 1];
            }
#pragma unroll
            for (int u = 0; u < 8; ++u) {
                const int p = base + u * 64 + lane;
                if (p < padded) {
                    const float w = p < length ? q3_expf(t[u] - maximum) : 0.0f;
                    p_lds[p] = w;
                    if (p < length) partial[(p >> 6) & 3] += w;  // thread (p mod 256)'s partial
                }
            }
        }
        const float p0 = partial[0] + partial[2];
        const float p1 = partial[1] + partial[3];
        inverse = 1.0f / __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(wave_sum_down<64>(p0 + p1))));
    }

    // 4. the value chain, rounds of kRing loads (8 positions each); the last,
    //    partial round replaces values past the length by 0 (positions
    //    there were never written for this sequence), so each fmaf adds
    //    0 * 0 -- the running sum starts at +0 and never becomes -0.
    float acc = 0.0f;
    auto round = [&](int base, int live) {
#pragma unroll
        for (int k = 0; k < kRing; k += 2) {
            const int i = base / 8 + k;  // groups i and i+1: positions 8i .. 8i+15
            float pv[16];  // the 16 positions' probability words, LDS broadcast reads
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float4 t = reinterpret_cast<const float4*>(p_lds)[2 * i + j];
                pv[4 * j] = t.x;
                pv[4 * j + 1] = t.y;
                pv[4 * j + 2] = t.z;
                pv[4 * j + 3] = t.w;
            }
            const uint4 w0 = ring[k];
            const uint4 w1 = ring[k + 1];
            if constexpr (kExact) {
                acc = chain8_pairs(acc, w0, pv, live - 8 * k);
                acc = chain8_pairs(acc, w1, pv + 8, live - 8 * k - 8);
            } else {
                acc = chain8(acc, w0, pv, live - 8 * k);
                acc = chain8(acc, w1, pv + 8, live - 8 * k - 8);
            }
            // refilled after use, so each slot keeps its registers
            ring[k] = load(i + kRing);
            ring[k + 1] = load(i + 1 + kRing);
        }
    };
    int base = chain_begin;
    for (; base + kRing * 8 <= chain_end; base += kRing * 8) round(base, kRing * 8);
    if (base < chain_end) round(base, chain_end - base);
    if constexpr (kSplit) {
        const size_t slot = (static_cast<size_t>(row) * a.query_heads + head) * gridDim.z + blockIdx.z;
        a.partials[slot * kDim + half * 64 + lane] = acc;
        if (blockIdx.z == 0 && half == 0 && lane == 0) a.inverse[static_cast<size_t>(row) * a.query_heads + head] = inverse;
        return;
    }
    const float y = kExact ? acc : acc * inverse;
    a.output[(static_cast<size_t>(row) * a.query_heads + head) * kDim + half * 64 + lane] = f2bf(y);
}

// The split value chains: out = bf16((partial_0 + .. + partial_{S-1}) * inverse),
// segments added in order.  One workgroup per (row, query head), lane =
// dimension.
__global__ __launch_bounds__(kDim) void attention_combine_kernel(AttnArgs a, int splits) {
    const size_t rh = blockIdx.x;
    const float* p = a.partials + rh * splits * kDim + threadIdx.x;
    float acc = p[0];
    for (int s = 1; s < splits; ++s) acc += p[static_cast<size_t>(s) * kDim];
    a.output[rh * kDim + threadIdx.x] = f2bf(acc * a.inverse[rh]);
}

// ---------------------------------------------------------------------------
// Exact softmax + values with the value slice staged in LDS (caches whose
// slice fits): grid (kv heads * 2G slices, rows), 8 waves.
// Workgroup (kv head, slice, row) covers the kD = 64 / G dimensions
// [slice * kD, slice * kD + kD) of the kv head for all G query heads of its
// group; the chain wave (wave G) runs the chain of query head h, dimension
// slice * kD + j in lane h * kD + j.
//   1. waves G .. 7 request the slice's values from the blocked cache; wave
//      h < G brings the scores of query head h into LDS and takes their
//      maximum;
//   2. all waves: every exponential of the G heads and a provisional sum of
//      them (any order);
//   3. in parallel: wave h < G takes the reference's sequential normalizer
//      of head h (thread 0's sum in position order, every lane on LDS
//      broadcast reads kept 48 positions ahead), the exact probabilities
//      bf16(e * (1/sum)) (once the staging waves are done with the
//      exponentials) and the first position where one differs from the
//      provisional one; waves G .. 7 write the provisional probabilities,
//      store the values (zeros past the length) and stage the rest, each
//      then adding itself to an LDS count; the chain wave, once the count
//      is complete, runs the sequential chains with the provisional
//      probabilities (one bf16 dot2 per position, as in
//      attention_head_kernel, 32 positions read ahead), keeping the chain's
//      value at the start of every 64-position block;
//   4. the chain wave: lanes of a head with a differing position rerun their
//      chain from the start of its 64-position block with the exact
//      probabilities.
// The probabilities are rounded to bf16, so the provisional ones almost
// always equal the exact ones and the sequential sum and the chain (the
// kernel's two long dependent sequences, about 4.6 cycles per step) run
// side by side.  Every output is the chain over the exact probabilities:
// bit-identical to attention_head_kernel<true, G> (positions past the length
// add +0).
// ---------------------------------------------------------------------------
// Waves per workgroup: G softmax waves, the others (the first of them the
// chain wave) stage values.
constexpr int kGroupWaves = 8;

// Positions held per head: whole 128-position blocks (the chain and the sum
// run over whole 64-position blocks) plus the reads ahead.
__host__ __device__ constexpr int group_p_stride(int capacity) { return (capacity + 127) / 128 * 128 + 64; }

// LDS: exponentials / exact probabilities [G][p_stride]; provisional
// probabilities [G][p_stride]; chain checkpoints [64-position blocks][64];
// the staged value slice [groups of 8 positions + 4 read ahead][kD] x 16 B.
template <int kG>
constexpr size_t group_lds_bytes(int capacity) {
    return 2 * static_cast<size_t>(kG) * group_p_stride(capacity) * sizeof(float) +
           static_cast<size_t>((capacity + 63) / 64) * 64 * sizeof(float) +
           static_cast<size_t>((capacity + 127) / 128 * 16 + 4) * (64 / kG) * 16;
}

#ifdef Q3_ATT_TRACE
__device__ unsigned long long q3_att_trace[64];
#define ATT_STAMP(i) \
    do { \
        if (blockIdx.x == 0 && blockIdx.y == 0 && (threadIdx.x & 63) == 0 && threadIdx.x < 256) { \
            q3_att_trace[(i) + 8 * (threadIdx.x >> 6)] = wall_clock64(); \
            if (threadIdx.x == 128) q3_att_trace[32 + (i)] = clock64(); \
        } \
    } while (0)
#else
#define ATT_STAMP(i) \
    do { \
    } while (0)
#endif

// Sequential fp32 sum of e[0 .. count) (count a multiple of 64) in index
// order, every lane the same; LDS broadcast reads of 8 positions per
// buffer, six buffers (48 positions, 12 reads) ahead of the additions.  e
// holds at least count + 64 floats (the reads ahead stay inside).
__device__ __forceinline__ float sequential_sum(const float* e, int count) {
    const float4* all = static_cast<const float4*>(__builtin_assume_aligned(e, 16));
    float4 buf[8][2];
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        buf[k][0] = all[2 * k];
        buf[k][1] = all[2 * k + 1];
    }
    float s = 0.0f;
    for (int b4 = 0; b4 < count / 4; b4 += 16) {
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            buf[(k + 6) & 7][0] = all[b4 + 2 * (k + 6)];
            buf[(k + 6) & 7][1] = all[b4 + 2 * (k + 6) + 1];
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                s += buf[k][r].x;
                s += buf[k][r].y;
                s += buf[k][r].z;
                s += buf[k][r].w;
            }
            __builtin_amdgcn_sched_barrier(0);
        }
    }
    return s;
}

// Waits until `count` (LDS) reaches `target` (bounded: the staging waves
// always add themselves).
__device__ __forceinline__ void wait_for_staging(int& count, int target) {
    for (int spin = 0; spin < (1 << 22); ++spin) {
        if (__hip_atomic_load(&count, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) == target) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// Minimum over the wave (every lane active), in every lane.
__device__ __forceinline__ int wave_min_int(int v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
    return v;
}

// One bf16 dot2 step per position of an 8-position group: the position's
// probability word (p, 0) or (0, p) against the value pair holding it.
__device__ __forceinline__ float chain_group8(float acc, const uint4& w, const float4& pa, const float4& pb) {
    const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int e = 0; e < 8; ++e)
        acc = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, __float_as_uint(pv[e])),
                                              __builtin_bit_cast(bf16x2_t, words[e >> 1]), acc, false);
    return acc;
}

// bf16(e * inverse) as the half of a bf16 pair of position p's parity.
__device__ __forceinline__ float probability_word(float e, float inverse, int p) {
    const uint32_t bits = __float_as_uint(round_bf(e * inverse));
    return __uint_as_float((p & 1) ? (bits & 0xffff0000u) : (bits >> 16));
}

template <int kG>
__global__ __launch_bounds__(64 * kGroupWaves) void attention_group_kernel(AttnArgs a) {
    constexpr int kD = 64 / kG;
    constexpr int kThreads = 64 * kGroupWaves;
    constexpr int kChainWave = kG;
    extern __shared__ __align__(16) float lds[];
    __shared__ float head_max[kG];
    __shared__ int first_mismatch[kG];
    __shared__ float provisional_sum[kG];
    __shared__ int staged_waves;
    const int row = blockIdx.y;
    const int kvh = blockIdx.x / (2 * kG);
    const int d0 = (blockIdx.x % (2 * kG)) * kD;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int length = row_length(a, row);
    const int p_stride = group_p_stride(a.capacity);
    float* provisional = lds + kG * p_stride;
    float* checkpoints = provisional + kG * p_stride;
    uint4* staged = reinterpret_cast<uint4*>(checkpoints + (a.capacity + 63) / 64 * 64);
    const int blocks = (length + 63) / 64;  // 64-position blocks of the sum and the chain
    const int padded = (length + 127) / 128 * 128;
    const int units = blocks * 8 * kD;  // staged units, zeros past the length
    const int live_units = (length + 7) / 8 * kD;
    const bf16_t* vbase = value_run(a, row, kvh, d0);
    constexpr int kStride = 64 * (kGroupWaves - kG);
    const int stager = tid - 64 * kG;
    ATT_STAMP(0);
    if (tid < kG) provisional_sum[tid] = 0.0f;
    if (tid == 0) staged_waves = 0;

    // 1. value requests; scores and maxima
    uint4 t[16];
    auto request = [&](int first) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int u = min(min(first + j * kStride, units - 1), live_units - 1);
            t[j] = load_global16(vbase + static_cast<size_t>(u / kD) * kGroupStep + (u % kD) * 8);
        }
    };
    auto store = [&](int first) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int u = first + j * kStride;
            if (u < units) {
                const int live = length - (u / kD) * 8;  // positions of the group inside the length
                uint4 w = t[j];
                if (live < 8) {
                    uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int k = 0; k < 4; ++k)
                        words[k] = 2 * k + 1 < live ? words[k] : (2 * k < live ? (words[k] & 0xffffu) : 0u);
                    w = make_uint4(words[0], words[1], words[2], words[3]);
                }
                staged[u] = w;
            }
        }
    };
    if (wave < kG) {
        const int head = kvh * kG + wave;
        const float* src = a.scores + (static_cast<size_t>(row) * a.query_heads + head) * a.capacity;
        const float m = scores_to_lds(src, length, lds + wave * p_stride, lane);
        if (lane == 0) head_max[wave] = m;
    } else {
        request(stager);
    }
    __syncthreads();
    ATT_STAMP(1);

    // 2. exponentials (zeros past the length, up to `padded`) and their
    //    provisional sums (any order); values
#pragma unroll
    for (int h = 0; h < kG; ++h) {
        float* e = lds + h * p_stride;
        const float m = head_max[h];
        constexpr int kPer = 4;
        float part = 0.0f;
        for (int first = tid; first < padded; first += kPer * kThreads) {
            float x[kPer];
#pragma unroll
            for (int k = 0; k < kPer; ++k) x[k] = e[min(first + k * kThreads, length - 1)];
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                const int p = first + k * kThreads;
                if (p < padded) {
                    const float ex = p < length ? q3_expf(x[k] - m) : 0.0f;
                    e[p] = ex;
                    part += ex;
                }
            }
        }
        part = wave_sum_down<64>(part);
        if (lane == 0) atomicAdd(&provisional_sum[h], part);
    }
    ATT_STAMP(6);
    __syncthreads();
    ATT_STAMP(2);
    // 3. exact normalizers || provisional probabilities and chains
    const int h = lane / kD;
    const int j = lane % kD;
    const int groups = blocks * 8;
    float acc = 0.0f;
    if (wave < kG) {
        // the exact probabilities of head `wave` and the first position
        // where one differs from the provisional one
        float* e = lds + wave * p_stride;
        const float* q = provisional + wave * p_stride;
        const float inverse = 1.0f / sequential_sum(e, blocks * 64);
        // the staging waves have read the exponentials and written the
        // provisional probabilities before they are overwritten / compared
        wait_for_staging(staged_waves, kGroupWaves - kG);
        int mismatch = 0x7fffffff;
        for (int base = 0; base < padded; base += 4 * 64) {
            float x[4], y[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int p = min(base + k * 64 + lane, padded - 1);
                x[k] = e[p];
                y[k] = q[p];
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int p = base + k * 64 + lane;
                if (p < padded) {
                    const float word = probability_word(x[k], inverse, p);
                    e[p] = word;
                    if (__float_as_uint(word) != __float_as_uint(y[k])) mismatch = min(mismatch, p);
                }
            }
        }
        mismatch = wave_min_int(mismatch);
        if (lane == 0) first_mismatch[wave] = mismatch;
    } else {
        // provisional probabilities; the values; then the chain wave waits
        // for every staging wave (an LDS count, bounded)
#pragma unroll
        for (int hh = 0; hh < kG; ++hh) {
            const float* e = lds + hh * p_stride;
            float* q = provisional + hh * p_stride;
            const float inverse = a.provisional_scale / provisional_sum[hh];
            constexpr int kPer = 4;
            for (int first = stager; first < padded; first += kPer * kStride) {
                float x[kPer];
#pragma unroll
                for (int k = 0; k < kPer; ++k) x[k] = e[min(first + k * kStride, padded - 1)];
#pragma unroll
                for (int k = 0; k < kPer; ++k) {
                    const int p = first + k * kStride;
                    if (p < padded) q[p] = probability_word(x[k], inverse, p);
                }
            }
        }
        store(stager);
        for (int first = stager + 16 * kStride; first < units; first += 16 * kStride) {
            request(first);
            store(first);
        }
        __threadfence_block();  // this wave's LDS writes before its count
        if (lane == 0) atomicAdd(&staged_waves, 1);
    }
    if (wave == kChainWave) {
        wait_for_staging(staged_waves, kGroupWaves - kG);
        ATT_STAMP(4);
        // the chains: one 8-position group per buffer, four buffers (12
        // reads) ahead; the reads ahead stay inside the slice and the rows
        const float4* p4 = static_cast<const float4*>(__builtin_assume_aligned(provisional + h * p_stride, 16));
        const uint4* v = staged + j;
        uint4 w[8];
        float4 pa[8], pb[8];
        auto issue = [&](int slot, int g) {
            w[slot] = v[g * kD];
            pa[slot] = p4[2 * g];
            pb[slot] = p4[2 * g + 1];
        };
#pragma unroll
        for (int k = 0; k < 4; ++k) issue(k, k);
        for (int g0 = 0; g0 < groups; g0 += 8) {
            checkpoints[g0 * 8 + lane] = acc;  // the chain before block g0 / 8
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                issue((k + 4) & 7, g0 + k + 4);
                __builtin_amdgcn_sched_barrier(0);
                acc = chain_group8(acc, w[k], pa[k], pb[k]);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    __syncthreads();
    ATT_STAMP(3);

    if (wave != kChainWave) return;

    // 4. rerun from the block of the first mismatch with the exact
    //    probabilities (lanes of heads without one keep their chain)
    const int bad = first_mismatch[h];
    const int start = bad < length ? bad / 64 : blocks;
    int earliest = blocks;
#pragma unroll
    for (int hh = 0; hh < kG; ++hh) {
        const int m = first_mismatch[hh];
        earliest = min(earliest, m < length ? m / 64 : blocks);
    }
    if (earliest < blocks) {
        const float4* p4 = reinterpret_cast<const float4*>(lds + h * p_stride);
        const uint4* v = staged + j;
        for (int b = earliest; b < blocks; ++b) {
            if (b == start) acc = checkpoints[b * 64 + lane];
            if (b >= start) {
                for (int g = b * 8; g < b * 8 + 8; ++g) acc = chain_group8(acc, v[g * kD], p4[2 * g], p4[2 * g + 1]);
            }
        }
    }
    a.output[(static_cast<size_t>(row) * a.query_heads + kvh * kG + h) * kDim + d0 + j] = f2bf(acc);
    ATT_STAMP(5);
}

// ---------------------------------------------------------------------------
// Short caches (capacity <= 64, the code predictor's 16 positions): the three
// phases in one kernel, one block of G*128 threads per (kv head, row).  Same
// operation order as the split kernels.
// ---------------------------------------------------------------------------
constexpr int kSmallCapacity = 64;

template <bool kExact, int kG>
__global__ __launch_bounds__(kG * kDim) void attention_small_kernel(AttnArgs a) {
    constexpr int kPrefetch = 16;  // value rows each lane requests up front
    __shared__ float q_lds[kG][kDim];
    __shared__ float prob[kG][kSmallCapacity];
    __shared__ float inverse_lds[kG];
    __shared__ uint32_t knew_lds[kDim / 2];
    __shared__ bf16_t vnew_lds[kDim];
    const int row = blockIdx.y;
    const int kvh = blockIdx.x;
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int length = row_length(a, row);
    const int kv_width = a.key_value_heads * kDim;
    const int position = length - 1;
    const bool fused = a.q_norm != nullptr;
    // With the QKV epilogue fused, the current position's key and value come
    // from qkv (and are written to the caches here), not from the caches.
    const int cached = fused ? position : length;
    const bf16_t* q = a.query + static_cast<size_t>(row) * a.query_stride + static_cast<size_t>(kvh) * kG * kDim;
    const bf16_t* cs = a.rope_table + static_cast<size_t>(position) * kDim;

    // 1. everything this block reads, requested up front in the order it is
    //    needed: the head-norm operands, the key rows, the value columns.
    head_detail::HeadInputs head_in{};
    if (fused) {
        if (wave < kG) {
            head_in = head_detail::load_head(q + wave * kDim, a.q_norm, cs);
        } else if (wave == kG) {
            const bf16_t* kraw = a.query + static_cast<size_t>(row) * a.query_stride +
                                 static_cast<size_t>(a.query_heads + kvh) * kDim;
            head_in = head_detail::load_head(kraw, a.k_norm, cs);
        }
    }
    const int g_score = tid / length;
    const int p_score = tid % length;
    const bool scores_lane = tid < kG * length;
    uint32_t kw[64];
    if (scores_lane && p_score < cached) {
        const uint4* k4 = reinterpret_cast<const uint4*>(row_keys(a, row) + static_cast<size_t>(p_score) * kv_width +
                                                         static_cast<size_t>(kvh) * kDim);
#pragma unroll
        for (int v = 0; v < 16; ++v) {
            const uint4 t = load_global16(k4 + v);
            kw[4 * v + 0] = t.x;
            kw[4 * v + 1] = t.y;
            kw[4 * v + 2] = t.z;
            kw[4 * v + 3] = t.w;
        }
    }
    const int g = tid / kDim;
    const int d = tid % kDim;
    const bf16_t* vcol = value_run(a, row, kvh, d);
    float vpre[kPrefetch];
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
        vpre[p] = p < cached ? bf2f(vcol[value_offset(p)]) : 0.0f;
    }

    // 2. head norms, RoPE, KV append
    if (fused) {
        if (wave < kG) {
            bf16_t q0, q1;
            head_detail::norm_rope_from(head_in, a.epsilon, q0, q1);
            q_lds[wave][lane] = bf2f(q0);
            q_lds[wave][lane + 64] = bf2f(q1);
        } else if (wave == kG) {
            bf16_t k0, k1;
            head_detail::norm_rope_from(head_in, a.epsilon, k0, k1);
            const bf16_t* vraw = a.query + static_cast<size_t>(row) * a.query_stride +
                                 static_cast<size_t>(a.query_heads) * kDim + kv_width + static_cast<size_t>(kvh) * kDim;
            const bf16_t v0 = vraw[lane];
            const bf16_t v1 = vraw[lane + 64];
            bf16_t* kdst = (a.key_bases != nullptr ? a.key_bases[row] : const_cast<bf16_t*>(a.key_cache)) +
                           static_cast<size_t>(position) * kv_width + static_cast<size_t>(kvh) * kDim;
            kdst[lane] = k0;
            kdst[lane + 64] = k1;
            append_value(a, row, kvh, position, lane, v0, v1);
            reinterpret_cast<bf16_t*>(knew_lds)[lane] = k0;
            reinterpret_cast<bf16_t*>(knew_lds)[lane + 64] = k1;
            vnew_lds[lane] = v0;
            vnew_lds[lane + 64] = v1;
        }
    } else {
        q_lds[tid / kDim][tid % kDim] = bf2f(q[tid]);
    }
    __syncthreads();

    // 3. scores, lane = (g, p)
    if (scores_lane) {
        if (p_score >= cached) {
#pragma unroll
            for (int i = 0; i < 64; ++i) kw[i] = knew_lds[i];
        }
        const float* qg = q_lds[g_score];
        float score;
        if constexpr (kExact) {
            score = exact_score(qg, kw, a.scale);
        } else {
            float dot = 0.0f;
#pragma unroll
            for (int t = 0; t < 64; ++t) {
                dot = fmaf(qg[2 * t], lo_bf(kw[t]), dot);
                dot = fmaf(qg[2 * t + 1], hi_bf(kw[t]), dot);
            }
            score = dot * a.scale;
        }
        prob[g_score][p_score] = score;
    }
    __syncthreads();

    // 4. softmax per head, one wave per head, lane = position: the max is
    //    order independent, the exponentials are per element, and the
    //    normalizer keeps the reference's order (exact: a sequential sum read
    //    lane by lane; fast: the 256-thread tree, whose levels 128 and 64
    //    only add zeros here).
    if (wave < kG) {
        float* sg = prob[wave];
        const bool live = lane < length;
        const float s = live ? sg[lane] : -INFINITY;
        float maximum = s;
#pragma unroll
        for (int offset = 32; offset > 0; offset >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, offset, 64));
        const float e = live ? q3_expf(s - maximum) : 0.0f;
        if constexpr (kExact) {
            float denominator = 0.0f;
            for (int p = 0; p < length; ++p) denominator += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e), p));
            const float inverse = 1.0f / denominator;
            if (live) sg[lane] = round_bf(e * inverse);
        } else {
            const float value = wave_sum_down<64>(e);
            if (live) sg[lane] = e;
            if (lane == 0) inverse_lds[wave] = 1.0f / value;
        }
    }
    __syncthreads();

    // 5. value chain, lane = (g, d)
    float acc = 0.0f;
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
        if (p < cached) acc = fmaf(prob[g][p], vpre[p], acc);
    }
    for (int p = kPrefetch; p < cached; ++p) acc = fmaf(prob[g][p], bf2f(vcol[value_offset(p)]), acc);
    if (fused) acc = fmaf(prob[g][position], bf2f(vnew_lds[d]), acc);
    const int head = kvh * kG + g;
    float y = acc;
    if constexpr (!kExact) y = acc * inverse_lds[g];
    a.output[(static_cast<size_t>(row) * a.query_heads + head) * kDim + d] = f2bf(y);
}

// ---------------------------------------------------------------------------
// The code predictor's caches (<= 16 positions), fused QKV epilogue, in the
// exact order (kExact) or the batched path's order (kExact = false; the
// reference's causal_gqa_attention_fast): one wave per (query head, row)
// does everything, with no block barrier.  Lane l holds elements l and l+64 of every 128-wide vector, which
// is the layout the reference's tree needs: the exact score's
// s[t] = q[t]k[t] + q[t+64]k[t+64] sits in lane t and its halving tree is a
// wave shuffle-down tree (wave_sum_down).  The wave normalizes and rotates its
// query head and (redundantly with the other waves of its GQA group) the new
// key; the group's first wave appends the key and value to the caches.  All
// key and value rows (the cache holds <= 16), and the rope rows of every
// position, are requested before the position is known, so no load waits
// for another.
// ---------------------------------------------------------------------------
constexpr int kShortCapacity = 16;

template <bool kExact, int kG>
__global__ __launch_bounds__(64) void attention_short_kernel(AttnArgs a) {
    const int row = blockIdx.y;
    const int head = blockIdx.x;
    const int kvh = head / kG;
    const int lane = threadIdx.x;
    const int kv_width = a.key_value_heads * kDim;
    const bf16_t* raw = a.query + static_cast<size_t>(row) * a.query_stride;
    const bf16_t* kraw = raw + static_cast<size_t>(a.query_heads + kvh) * kDim;
    const bf16_t* vraw = raw + static_cast<size_t>(a.query_heads) * kDim + kv_width + static_cast<size_t>(kvh) * kDim;
    const bf16_t* keys = row_keys(a, row) + static_cast<size_t>(kvh) * kDim;
    const bf16_t* vrun0 = value_run(a, row, kvh, lane);
    const bf16_t* vrun1 = value_run(a, row, kvh, lane + 64);

    // 1. every operand, with 16-byte loads: the query/key rows (lane l:
    //    chunk l % 16 of row 4i + l / 16) staged through LDS into the
    //    lane-l / lane-(l+64) layout; the values straight from the lane's two
    //    dimension runs.  Only the selections below depend on the position.
    const int position = a.positions[row];
    const int chunk = lane & 15;
    uint4 hv0, hv1 = make_uint4(0, 0, 0, 0);
    {
        const int part = lane >> 4;  // q, k, v, q gain
        const bf16_t* src = part == 0 ? raw + head * kDim : part == 1 ? kraw : part == 2 ? vraw : a.q_norm;
        hv0 = load_global16(src + chunk * 8);
        if (lane < 16) hv1 = load_global16(a.k_norm + chunk * 8);
    }
    uint4 rv[4], kv4[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int p = 4 * i + (lane >> 4);
        const int pc = p < a.capacity ? p : a.capacity - 1;  // rows past the capacity: a valid row, unused
        rv[i] = load_global16(a.rope_table + static_cast<size_t>(pc) * kDim + chunk * 8);
        kv4[i] = load_global16(keys + static_cast<size_t>(pc) * kv_width + chunk * 8);
    }
    // value runs: groups of 8 positions inside the (8-aligned) stride
    uint4 vg0[kShortCapacity / 8], vg1[kShortCapacity / 8];
#pragma unroll
    for (int i = 0; i < kShortCapacity / 8; ++i) {
        const bool in = i * 8 < a.capacity;
        vg0[i] = in ? load_global16(vrun0 + i * kGroupStep) : make_uint4(0, 0, 0, 0);
        vg1[i] = in ? load_global16(vrun1 + i * kGroupStep) : make_uint4(0, 0, 0, 0);
    }
    short_attn::Operands in;
    in.hv0 = hv0;
    in.hv1 = hv1;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        in.rv[i] = rv[i];
        in.kv4[i] = kv4[i];
    }
#pragma unroll
    for (int i = 0; i < kShortCapacity / 8; ++i) {
        in.vg0[i] = vg0[i];
        in.vg1[i] = vg1[i];
    }
    // the group's first query head appends the key and value
    bf16_t* kdst = head % kG == 0 ? (a.key_bases != nullptr ? a.key_bases[row] : const_cast<bf16_t*>(a.key_cache)) +
                                        static_cast<size_t>(position) * kv_width + static_cast<size_t>(kvh) * kDim
                                  : nullptr;
    float acc0, acc1;
    short_attn::core<kExact>(in, position, a.epsilon, a.scale, kdst, const_cast<bf16_t*>(vrun0),
                             const_cast<bf16_t*>(vrun1), acc0, acc1);
    bf16_t* out = a.output + (static_cast<size_t>(row) * a.query_heads + head) * kDim;
    out[lane] = f2bf(acc0);
    out[lane + 64] = f2bf(acc1);
}

template <bool kExact, int kG>
hipError_t launch_variant(const AttnArgs& a, int rows, hipStream_t stream) {
    const size_t head_lds = static_cast<size_t>(lds_stride(a.capacity)) * sizeof(float);
    // LDS: up to 160 KB per workgroup on gfx950
    constexpr size_t kLdsLimit = 160 * 1024;
    if (head_lds > kLdsLimit) return hipErrorInvalidValue;
    static std::atomic<unsigned long long> configured{0};
    const hipError_t st = set_dynamic_lds_once(configured, reinterpret_cast<const void*>(attention_head_kernel<kExact, kG>),
                                               static_cast<int>(kLdsLimit));
    if (st != hipSuccess) return st;
    if (a.capacity <= kShortCapacity && a.q_norm != nullptr) {
        attention_short_kernel<kExact, kG><<<dim3(a.query_heads, rows), 64, 0, stream>>>(a);
        return hipGetLastError();
    }
    if (a.capacity <= kSmallCapacity) {
        attention_small_kernel<kExact, kG><<<dim3(a.key_value_heads, rows), kG * kDim, 0, stream>>>(a);
        return hipGetLastError();
    }
    // many prompt rows on one complete cache (the prefill's exact attention)
    const bool prompt_rows = kExact && a.key_bases == nullptr && a.q_norm == nullptr && rows >= 2 * kPromptTileRows;
    if (prompt_rows) {
        // the key rows are shared
        const dim3 grid((a.capacity + kScoreLanes - 1) / kScoreLanes, a.key_value_heads,
                        (rows + kPromptTileRows - 1) / kPromptTileRows);
        attention_scores_rows_kernel<kG, kPromptTileRows><<<grid, kScoreLanes, 0, stream>>>(a, rows);
    } else {
        const dim3 score_grid((a.capacity + kScoreLanes - 1) / kScoreLanes, a.query_heads, rows);
        attention_scores_kernel<kExact, kG><<<score_grid, kScoreLanes, 0, stream>>>(a);
    }
    if constexpr (!kExact) {
        if (a.position_splits > 1 && a.partials != nullptr) {
            static std::atomic<unsigned long long> configured_split{0};
            const hipError_t sst = set_dynamic_lds_once(
                configured_split, reinterpret_cast<const void*>(attention_head_kernel<kExact, kG, true>),
                static_cast<int>(kLdsLimit));
            if (sst != hipSuccess) return sst;
            attention_head_kernel<kExact, kG, true>
                <<<dim3(a.query_heads * 2, rows, a.position_splits), 64, head_lds, stream>>>(a);
            const hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            attention_combine_kernel<<<rows * a.query_heads, kDim, 0, stream>>>(a, a.position_splits);
            return hipGetLastError();
        }
    }
    // The staged-slice kernel shortens one row's latency with a whole CU per
    // (kv head, slice); prompt chunks (thousands of workgroups) run the
    // one-wave head kernel, which fills the GPU with many per CU (801-row
    // prefill: 15.5 ms against 28.7 ms with the staged-slice kernel).
    if (kExact && !prompt_rows) {
        const size_t group_lds = group_lds_bytes<kG>(a.capacity);
        if (group_lds + 256 <= kLdsLimit) {  // + the static maxima and normalizers
            static std::atomic<unsigned long long> configured_group{0};
            const hipError_t gst = set_dynamic_lds_once(
                configured_group, reinterpret_cast<const void*>(attention_group_kernel<kG>),
                static_cast<int>(kLdsLimit - 256));
            if (gst != hipSuccess) return gst;
            attention_group_kernel<kG>
                <<<dim3(a.key_value_heads * 2 * kG, rows), 64 * kGroupWaves, group_lds, stream>>>(a);
            return hipGetLastError();
        }
    }
    attention_head_kernel<kExact, kG><<<dim3(a.query_heads * 2, rows), 64, head_lds, stream>>>(a);
    return hipGetLastError();
}

}  // namespace


int value_cache_stride(int capacity) { return (capacity + 7) / 8 * 8; }

size_t attention_workspace_bytes(int rows, int query_heads, int capacity) {
    return static_cast<size_t>(rows) * query_heads * (static_cast<size_t>(capacity) + 1) * sizeof(float);
}

size_t attention_split_workspace_bytes(int rows, int query_heads, int capacity, int splits) {
    return attention_workspace_bytes(rows, query_heads, capacity) +
           static_cast<size_t>(rows) * query_heads * splits * kDim * sizeof(float);
}

namespace {

hipError_t dispatch(bool exact, const AttnArgs& a, int rows, hipStream_t stream) {
    switch (a.query_heads / a.key_value_heads) {
        case 1: return exact ? launch_variant<true, 1>(a, rows, stream) : launch_variant<false, 1>(a, rows, stream);
        case 2: return exact ? launch_variant<true, 2>(a, rows, stream) : launch_variant<false, 2>(a, rows, stream);
        case 4: return exact ? launch_variant<true, 4>(a, rows, stream) : launch_variant<false, 4>(a, rows, stream);
        default: return hipErrorInvalidValue;
    }
}

bool valid_shape(int rows, int query_heads, int key_value_heads, int head_dimension, int capacity,
                 const float* workspace) {
    return head_dimension == kDim && key_value_heads > 0 && query_heads % key_value_heads == 0 && rows > 0 &&
           capacity > 0 && capacity <= kMaxCapacity && workspace != nullptr;
}

float provisional_scale() {
    static const float scale = [] {
        const char* v = std::getenv("QWEN3_TTS_ATTENTION_SKEW_PROVISIONAL");
        return v != nullptr && std::strcmp(v, "1") == 0 ? 1.0f + 0.0078125f : 1.0f;
    }();
    return scale;
}

AttnArgs base_args(const bf16_t* query, int query_stride, bf16_t* const* key_bases, bf16_t* const* value_bases,
                   const bf16_t* key_cache, const bf16_t* value_cache, const int* positions, int fixed_length,
                   bf16_t* output, int rows, int query_heads, int key_value_heads, int capacity, float* workspace,
                   const int* value_strides) {
    AttnArgs a{};
    a.query = query;
    a.query_stride = query_stride;
    a.key_bases = key_bases;
    a.value_bases = value_bases;
    a.key_cache = key_cache;
    a.value_cache = value_cache;
    a.positions = positions;
    a.fixed_length = fixed_length;
    a.output = output;
    a.query_heads = query_heads;
    a.key_value_heads = key_value_heads;
    a.capacity = capacity;
    a.scale = 1.0f / sqrtf(static_cast<float>(kDim));
    a.scores = workspace;
    a.inverse = workspace + static_cast<size_t>(rows) * query_heads * capacity;
    a.value_stride = value_cache_stride(capacity);
    a.value_strides = value_strides;
    a.provisional_scale = provisional_scale();
    return a;
}

}  // namespace

hipError_t launch_attention(bool exact, const bf16_t* query, int query_stride, bf16_t* const* key_bases,
                            bf16_t* const* value_bases, const bf16_t* key_cache, const bf16_t* value_cache,
                            const int* positions, int fixed_sequence_length, bf16_t* output, int rows,
                            int query_heads, int key_value_heads, int head_dimension, int max_sequence_length,
                            float* workspace, const int* value_strides, hipStream_t stream) {
    if (!valid_shape(rows, query_heads, key_value_heads, head_dimension, max_sequence_length, workspace) ||
        query == nullptr || output == nullptr) {
        return hipErrorInvalidValue;
    }
    if ((key_bases == nullptr) != (value_bases == nullptr)) return hipErrorInvalidValue;
    if (key_bases == nullptr && (key_cache == nullptr || value_cache == nullptr)) return hipErrorInvalidValue;
    if (positions == nullptr && (fixed_sequence_length <= 0 || fixed_sequence_length > max_sequence_length)) {
        return hipErrorInvalidValue;
    }
    const AttnArgs a = base_args(query, query_stride, key_bases, value_bases, key_cache, value_cache, positions,
                                 fixed_sequence_length, output, rows, query_heads, key_value_heads,
                                 max_sequence_length, workspace, value_strides);
    return dispatch(exact, a, rows, stream);
}

hipError_t launch_decode_attention(bool exact, const bf16_t* qkv, int qkv_stride, const bf16_t* q_norm,
                                   const bf16_t* k_norm, const bf16_t* rope_table, float epsilon,
                                   bf16_t* const* key_bases, bf16_t* const* value_bases, const bf16_t* key_cache,
                                   const bf16_t* value_cache, const int* positions, bf16_t* output, int rows,
                                   int query_heads, int key_value_heads, int head_dimension, int capacity,
                                   float* workspace, const int* value_strides, hipStream_t stream,
                                   int position_splits) {
    if (position_splits < 1 || position_splits > 8) return hipErrorInvalidValue;
    if (!valid_shape(rows, query_heads, key_value_heads, head_dimension, capacity, workspace) || qkv == nullptr ||
        output == nullptr || q_norm == nullptr || k_norm == nullptr || rope_table == nullptr ||
        positions == nullptr) {
        return hipErrorInvalidValue;
    }
    if ((key_bases == nullptr) != (value_bases == nullptr)) return hipErrorInvalidValue;
    if (key_bases == nullptr && (key_cache == nullptr || value_cache == nullptr)) return hipErrorInvalidValue;
    AttnArgs a = base_args(qkv, qkv_stride, key_bases, value_bases, key_cache, value_cache, positions, 0, output,
                           rows, query_heads, key_value_heads, capacity, workspace, value_strides);
    a.q_norm = q_norm;
    a.k_norm = k_norm;
    a.rope_table = rope_table;
    a.epsilon = epsilon;
    if (position_splits > 1) {
        a.position_splits = position_splits;
        a.partials = workspace + static_cast<size_t>(rows) * query_heads * (static_cast<size_t>(capacity) + 1);
    }
    return dispatch(exact, a, rows, stream);
}

}  // namespace q3
