// bf16 prompt prefill for gfx950: the reference's prefill runs the talker's
// bf16 weights through cuBLAS GEMMs with fp32 accumulation and bf16 outputs
// (native/qwen3-tts-native/native/src/talker.cu:2637-2674, 2750-3249).  Here
// every such product is one MFMA kernel, gemm_bf16_kernel:
//
//   C[m][n] = bf16( sum_k A[m][k] * B[n][k] )      (fp32 accumulation)
//
// with A and B row-major and K contiguous in both (activations x weights^T,
// queries x keys^T, probabilities x values^T), batched over heads through
// gridDim.z with a grouped B index for GQA.  A 128x128 (or, when that leaves
// CUs idle, 64x64 or 32x32) block tile of 256 threads (4 waves in 2x2, each a grid of
// v_mfma_f32_16x16x32_bf16 tiles), K in steps of 64 to 256 (by tile and
// prompt length) staged through double-buffered LDS (padded rows), the
// global loads of the next one or two steps in flight under each step's
// MFMAs.  Deep products and under-filled grids split K into slices (fp32
// partial sums, added in slice order by a second launch).  Epilogues fold
// the reference's residual add_in_place and silu_gate into the products, and
// B may come in three row segments (the q, k and v weights as one GEMM).
//
// The summation order of an fp32 GEMM is not the reference's (cuBLAS leaves
// it unspecified), so this path is compared with tolerances; everything
// around the GEMMs (causal softmax, head norm, RoPE, residual adds, SiLU
// gate) reproduces the reference's operation order exactly.
#include <algorithm>

#include "q3_common.hpp"
#include "q3_math.h"
#include "head_device.hpp"

namespace q3 {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4& v) { return __builtin_bit_cast(bf16x8_t, v); }

// One 16-byte chunk (8 consecutive k) of row `row` at column `col`, zero past
// the matrix (rows >= limit or k >= k_limit; K is a multiple of 8).
__device__ __forceinline__ uint4 load_chunk(const bf16_t* base, int ld, int row, int limit, int col, int k_limit) {
    uint4 v{0u, 0u, 0u, 0u};
    if (row < limit && col < k_limit) v = *reinterpret_cast<const uint4*>(base + static_cast<size_t>(row) * ld + col);
    return v;
}

// The product's bf16 value v = bf16(sum) into C, as the epilogue says: kept
// (store), added into C as the reference's add_in_place after the GEMM
// (C = bf16(C + v)), or as its silu_gate with C holding the gate GEMM's
// output and v the up GEMM's (C = bf16(bf16(g / (1 + exp(-g))) * v)).
__device__ __forceinline__ void gemm_store(bf16_t* out, float sum, int epilogue) {
    const bf16_t v = f2bf(sum);
    if (epilogue == kGemmAddInto) {
        *out = f2bf(bf2f(*out) + bf2f(v));
    } else if (epilogue == kGemmSiluGateInto) {
        const float g = bf2f(*out);
        const float activated = round_bf(g / (1.0f + q3_expf(-g)));
        *out = f2bf(activated * bf2f(v));
    } else {
        *out = v;
    }
}

// Block tile kBM x kBN, four waves in 2 x 2, each (kBM/2) x (kBN/2) as
// (kBM/32) x (kBN/32) 16x16 MFMA tiles.
// gridDim.z = batch * splits: slice `split` covers K steps
// [split * steps_per_split, ...) and writes fp32 partial sums when splits > 1.
// kDeep: two register sets of global loads, so the loads of steps s + 1 and
// s + 2 are in flight while step s runs its MFMAs (each step otherwise waits
// one memory latency); beyond the slice the loads still issue (masked past
// the matrix, unused) so that every wait counts the same loads.
template <int kBM, int kBN, int kBK, bool kDeep = false>
__global__ __launch_bounds__(kGemmThreads) void gemm_bf16_kernel(Bf16GemmArgs g, int splits, int steps_per_split) {
    constexpr int kLdsRow = kBK + 8;  // bf16 per LDS row: 16-byte pad against bank conflicts
    constexpr int kRowChunks = kBK / 8;  // 16-byte chunks per row and K step
    constexpr int kTM = kBM / 32;                 // MFMA tiles per wave along M
    constexpr int kTN = kBN / 32;                 // and along N
    constexpr int kChunksA = kBM * kRowChunks / kGemmThreads;  // 16-byte chunks per thread per K step
    constexpr int kChunksB = kBN * kRowChunks / kGemmThreads;
    constexpr int kSets = kDeep ? 2 : 1;
    __shared__ __align__(16) bf16_t as[2][kBM * kLdsRow];
    __shared__ __align__(16) bf16_t bs[2][kBN * kLdsRow];
    const int tid = threadIdx.x;
    const int wave = tid >> 6;
    const int lane = tid & 63;
    const int m0 = blockIdx.y * kBM;
    const int n0 = blockIdx.x * kBN;
    const int z = blockIdx.z % g.batch;
    const int split = blockIdx.z / g.batch;
    const bf16_t* a = g.a + static_cast<size_t>(z) * g.a_batch;
    const bf16_t* b = g.b + static_cast<size_t>(z / g.b_group) * g.b_batch;
    bf16_t* c = g.c + static_cast<size_t>(z) * g.c_batch;

    uint4 ra[kSets][kChunksA], rb[kSets][kChunksB];
    auto fetch = [&](int set, int k0) {
#pragma unroll
        for (int i = 0; i < kChunksA; ++i) {
            const int chunk = tid + i * kGemmThreads;
            ra[set][i] = load_chunk(a, g.lda, m0 + chunk / kRowChunks, g.m, k0 + (chunk % kRowChunks) * 8, g.k);
        }
#pragma unroll
        for (int i = 0; i < kChunksB; ++i) {
            const int chunk = tid + i * kGemmThreads;
            const int row = n0 + chunk / kRowChunks;
            // B may come in up to three row segments (the q, k and v weights)
            const bf16_t* bseg = b;
            int brow = row;
            if (g.b3 != nullptr && row >= g.b3_row) {
                bseg = g.b3;
                brow = row - g.b3_row;
            } else if (g.b2 != nullptr && row >= g.b2_row) {
                bseg = g.b2;
                brow = row - g.b2_row;
            }
            rb[set][i] = row < g.n ? load_chunk(bseg, g.ldb, brow, g.n, k0 + (chunk % kRowChunks) * 8, g.k)
                                   : uint4{0u, 0u, 0u, 0u};
        }
    };
    auto stage = [&](int set, int buffer) {
#pragma unroll
        for (int i = 0; i < kChunksA; ++i) {
            const int chunk = tid + i * kGemmThreads;
            *reinterpret_cast<uint4*>(&as[buffer][(chunk / kRowChunks) * kLdsRow + (chunk % kRowChunks) * 8]) =
                ra[set][i];
        }
#pragma unroll
        for (int i = 0; i < kChunksB; ++i) {
            const int chunk = tid + i * kGemmThreads;
            *reinterpret_cast<uint4*>(&bs[buffer][(chunk / kRowChunks) * kLdsRow + (chunk % kRowChunks) * 8]) =
                rb[set][i];
        }
    };

    const int wm = (wave >> 1) * (kBM / 2);  // wave tile origin inside the block tile
    const int wn = (wave & 1) * (kBN / 2);
    const int m = lane & 15;
    const int group = lane >> 4;
    floatx4_t acc[kTM][kTN];
#pragma unroll
    for (int i = 0; i < kTM; ++i)
#pragma unroll
        for (int j = 0; j < kTN; ++j) acc[i][j] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    auto compute = [&](int buffer) {
#pragma unroll
        for (int kk = 0; kk < kBK; kk += 32) {
            bf16x8_t af[kTM], bfr[kTN];
#pragma unroll
            for (int i = 0; i < kTM; ++i) {
                af[i] = as_bf16x8(*reinterpret_cast<const uint4*>(&as[buffer][(wm + 16 * i + m) * kLdsRow + kk + 8 * group]));
            }
#pragma unroll
            for (int j = 0; j < kTN; ++j) {
                bfr[j] = as_bf16x8(*reinterpret_cast<const uint4*>(&bs[buffer][(wn + 16 * j + m) * kLdsRow + kk + 8 * group]));
            }
#pragma unroll
            for (int i = 0; i < kTM; ++i)
#pragma unroll
                for (int j = 0; j < kTN; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
    };

    const int first = split * steps_per_split;
    const int steps = min((g.k + kBK - 1) / kBK - first, steps_per_split);
    const int k_base = first * kBK;
    if constexpr (kDeep) {
        // step j's loads live in set (j + 1) % 2 after the prologue: step 0
        // staged from set 0, then step 1 in set 1 and step 2 in set 0
        fetch(0, k_base);
        stage(0, 0);
        fetch(1, k_base + kBK);
        fetch(0, k_base + 2 * kBK);
        __syncthreads();
        for (int s = 0; s < steps; s += 2) {
            compute(0);  // step s
            if (s + 1 >= steps) break;
            stage(1, 1);  // step s + 1
            fetch(1, k_base + (s + 3) * kBK);
            __syncthreads();
            compute(1);  // step s + 1
            if (s + 2 >= steps) break;
            stage(0, 0);  // step s + 2
            fetch(0, k_base + (s + 4) * kBK);
            __syncthreads();
        }
    } else {
        fetch(0, k_base);
        stage(0, 0);
        __syncthreads();
        for (int s = 0; s < steps; ++s) {
            const int buffer = s & 1;
            if (s + 1 < steps) fetch(0, k_base + (s + 1) * kBK);  // in flight under the MFMAs
            compute(buffer);
            if (s + 1 < steps) {
                stage(0, buffer ^ 1);
                __syncthreads();
            }
        }
    }
    // acc[i][j][r] = C[wm + 16 i + 4 group + r][wn + 16 j + m]
    if (splits > 1) {
        float* p = g.partial + (static_cast<size_t>(split) * g.batch + z) * g.m * g.n;
#pragma unroll
        for (int i = 0; i < kTM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm + 16 * i + 4 * group + r;
                if (row >= g.m) continue;
#pragma unroll
                for (int j = 0; j < kTN; ++j) {
                    const int col = n0 + wn + 16 * j + m;
                    if (col < g.n) p[static_cast<size_t>(row) * g.n + col] = acc[i][j][r];
                }
            }
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < kTM; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = m0 + wm + 16 * i + 4 * group + r;
            if (row >= g.m) continue;
#pragma unroll
            for (int j = 0; j < kTN; ++j) {
                const int col = n0 + wn + 16 * j + m;
                if (col < g.n) gemm_store(c + static_cast<size_t>(row) * g.ldc + col, acc[i][j][r], g.epilogue);
            }
        }
    }
}

// Split-K reduction: C[z][row][col] = bf16(sum over slices, in slice order,
// of the fp32 partials).  Block (column block, row, batch entry), one thread
// per column.
__global__ __launch_bounds__(256) void gemm_bf16_reduce_kernel(Bf16GemmArgs g, int splits) {
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= g.n) return;
    const int row = blockIdx.y;
    const int z = blockIdx.z;
    const size_t slice = static_cast<size_t>(g.m) * g.n * g.batch;
    const float* p = g.partial + (static_cast<size_t>(z) * g.m + row) * g.n + col;
    float sum = p[0];
    for (int s = 1; s < splits; ++s) sum += p[s * slice];
    gemm_store(g.c + static_cast<size_t>(z) * g.c_batch + static_cast<size_t>(row) * g.ldc + col, sum, g.epilogue);
}

// causal_softmax_kernel (talker_kernels.cu:232-260) on bf16 scores
// [heads][rows][stride]: scaled = bf16(s * (1/sqrt(d))); maximum over keys
// 0..query; denominator = sequential fp32 sum of exp(scaled - max); p =
// bf16(exp(scaled - max) * (1/denominator)); keys query+1 .. stride-1 = 0.
// One wave per (head, query) row: the wave computes the exponentials in
// parallel (into LDS), lane 0 sums them in key order.
__global__ __launch_bounds__(64) void causal_softmax_kernel(bf16_t* scores, int rows, int stride, float scale) {
    __shared__ float e[kPrefillAttentionRows];
    __shared__ float inverse_lds;
    const int query = blockIdx.x;
    bf16_t* row = scores + (static_cast<size_t>(blockIdx.y) * rows + query) * stride;
    const int lane = threadIdx.x;
    const int count = query + 1;
    float maximum = -__int_as_float(0x7f800000);
    for (int key = lane; key < count; key += 64) {
        const float scaled = round_bf(bf2f(row[key]) * scale);
        e[key] = scaled;
        maximum = fmaxf(maximum, scaled);
    }
#pragma unroll
    for (int offset = 32; offset > 0; offset >>= 1) maximum = fmaxf(maximum, __shfl_xor(maximum, offset, 64));
    for (int key = lane; key < count; key += 64) e[key] = q3_expf(e[key] - maximum);
    __syncthreads();
    if (lane == 0) {
        float denominator = 0.0f;
        for (int key = 0; key < count; ++key) denominator += e[key];
        inverse_lds = 1.0f / denominator;
    }
    __syncthreads();
    const float inverse = inverse_lds;
    for (int key = lane; key < stride; key += 64) row[key] = key < count ? f2bf(e[key] * inverse) : f2bf(0.0f);
}

// The QKV epilogue of a prompt of `rows` positions starting at `first`: per
// (row, head) of the fused [rows][q | k | v] projection, head RMSNorm and
// RoPE on q and k heads in place (the decode path's exact arithmetic and
// RoPE table); k heads also to the key cache ([position][kv_width]), v heads
// to the blocked dimension-major value cache.  One wave per head.
__global__ __launch_bounds__(64) void prefill_qkv_epilogue_kernel(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm,
                                                                  const bf16_t* rope_table, bf16_t* key_cache,
                                                                  bf16_t* value_cache, int value_stride, int first,
                                                                  int query_heads, int key_value_heads, float epsilon) {
    constexpr int kDim = 128;
    const int heads = query_heads + 2 * key_value_heads;
    const int row = blockIdx.x / heads;
    const int head = blockIdx.x % heads;
    const int lane = threadIdx.x;
    const int q_width = query_heads * kDim;
    const int kv_width = key_value_heads * kDim;
    const int position = first + row;
    bf16_t* base = qkv + static_cast<size_t>(row) * (q_width + 2 * kv_width) + static_cast<size_t>(head) * kDim;
    if (head >= query_heads + key_value_heads) {
        const int vh = head - query_heads - key_value_heads;
        for (int d = lane; d < kDim; d += 64) {
            const size_t index = ((static_cast<size_t>(vh) * (value_stride >> 3) + (position >> 3)) * kDim + d) * 8 +
                                 (position & 7);
            value_cache[index] = base[d];
        }
        return;
    }
    const bool is_query = head < query_heads;
    bf16_t out0, out1;
    head_detail::norm_rope_head(base, is_query ? q_norm : k_norm, rope_table + static_cast<size_t>(position) * kDim,
                                epsilon, out0, out1);
    base[lane] = out0;
    base[lane + 64] = out1;
    if (!is_query) {
        bf16_t* dst = key_cache + static_cast<size_t>(position) * kv_width + static_cast<size_t>(head - query_heads) * kDim;
        dst[lane] = out0;
        dst[lane + 64] = out1;
    }
}

// vt[h][d][j] = v(row j, head h, dim d) for j < rows, 0 for rows <= j < stride.
__global__ __launch_bounds__(256) void transpose_values_kernel(const bf16_t* qkv, int qkv_width, int v_offset, int rows,
                                                               int stride, int key_value_heads, bf16_t* vt) {
    const size_t total = static_cast<size_t>(key_value_heads) * 128 * stride;
    for (size_t t = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; t < total;
         t += static_cast<size_t>(gridDim.x) * blockDim.x) {
        const int j = static_cast<int>(t % stride);
        const int hd = static_cast<int>(t / stride);  // h * 128 + d
        vt[t] = j < rows ? qkv[static_cast<size_t>(j) * qkv_width + v_offset + hd] : f2bf(0.0f);
    }
}

// Prompt rows: out[r] = (text[r] >= 0 ? projected[r] : 0), then + the codec
// embedding of codec[r] when codec[r] >= 0 (bf16 add), as the reference's
// prepare_prompt_embedding (talker.cu:2721-2748).
__global__ __launch_bounds__(256) void prompt_rows_kernel(bf16_t* rows_data, const int* text, const int* codec,
                                                          const bf16_t* codec_embedding, int codec_vocabulary,
                                                          int width) {
    const int r = blockIdx.y;
    bf16_t* out = rows_data + static_cast<size_t>(r) * width;
    const bool has_text = text[r] >= 0;
    const int token = codec[r];
    const bool has_codec = token >= 0 && token < codec_vocabulary;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += gridDim.x * blockDim.x) {
        float v = has_text ? bf2f(out[i]) : 0.0f;
        if (has_codec) v = round_bf(v + bf2f(codec_embedding[static_cast<size_t>(token) * width + i]));
        out[i] = f2bf(v);
    }
}

// Text-embedding rows of the prompt (row 0 for positions without text; their
// projection is discarded by prompt_rows_kernel).
__global__ __launch_bounds__(256) void gather_text_rows_kernel(const bf16_t* table, const int* text, int vocabulary,
                                                               int width, bf16_t* out) {
    const int r = blockIdx.y;
    const int token = text[r] >= 0 && text[r] < vocabulary ? text[r] : 0;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += gridDim.x * blockDim.x) {
        out[static_cast<size_t>(r) * width + i] = table[static_cast<size_t>(token) * width + i];
    }
}

}  // namespace

hipError_t launch_bf16_gemm(const Bf16GemmArgs& g, hipStream_t stream) {
    if (g.a == nullptr || g.b == nullptr || g.c == nullptr || g.m <= 0 || g.n <= 0 || g.k <= 0 || g.batch <= 0 ||
        g.b_group <= 0 || g.k % 8 != 0 || g.lda % 8 != 0 || g.ldb % 8 != 0 || g.lda < g.k || g.ldb < g.k ||
        g.ldc < g.n) {
        return hipErrorInvalidValue;
    }
    if (g.epilogue != kGemmStore && g.epilogue != kGemmAddInto && g.epilogue != kGemmSiluGateInto) {
        return hipErrorInvalidValue;
    }
    if ((g.b2 != nullptr || g.b3 != nullptr) &&
        (g.batch != 1 || (g.b2 != nullptr && (g.b2_row <= 0 || g.b2_row >= g.n)) ||
         (g.b3 != nullptr && (g.b3_row <= (g.b2 != nullptr ? g.b2_row : 0) || g.b3_row >= g.n)) ||
         ((reinterpret_cast<uintptr_t>(g.b2) | reinterpret_cast<uintptr_t>(g.b3)) & 15u) != 0)) {
        return hipErrorInvalidValue;
    }
    const uintptr_t align = reinterpret_cast<uintptr_t>(g.a) | reinterpret_cast<uintptr_t>(g.b);
    if ((align & 15u) != 0 || (g.a_batch % 8) != 0 || (g.b_batch % 8) != 0) return hipErrorInvalidValue;
    // Tiles, K steps and K slices, measured on MI355X over the prefill's
    // shapes (prompts of 16..801 rows, N 1024..6144, K 2048 / 6144): 128-square
    // only where it still gives two workgroups per CU; else 32-square up to
    // 256 rows (K steps of 256 up to 64 rows, else 128: the 256-step tile's
    // 66 KB of LDS halves occupancy), 64-square above (K steps of 128 up to
    // 2048 columns, else 64).  Each K step waits one memory latency, so deep
    // products (K >= 4096) split K into slices (4 for the 32-square tile, 8
    // for the 64-square one up to 256 rows, 2 above while the grid has under
    // 384 workgroups), and a 32-square grid of
    // under 128 workgroups spreads to about 512 (two steps a slice at least).
    auto blocks = [&](int t) { return static_cast<long long>((g.n + t - 1) / t) * ((g.m + t - 1) / t) * g.batch; };
    const bool deep = g.k >= 4096;
    int tile = g.force_tile;
    if (tile == 0) tile = blocks(128) >= 512 ? 128 : (g.m <= 128 || (g.m <= 256 && !deep)) ? 32 : 64;
    if (tile != 32 && tile != 64 && tile != 128) return hipErrorInvalidValue;
    int bk = g.force_k_step;
    if (bk == 0) {
        if (tile == 32) bk = g.m <= 64 ? 256 : 128;
        else if (tile == 64) bk = (g.n >= 3072 || (deep && g.m <= 256)) ? 64 : 128;
        else bk = 64;
    }
    if (!((tile == 32 && (bk == 64 || bk == 128 || bk == 256)) || (tile == 64 && (bk == 64 || bk == 128)) ||
          (tile == 128 && bk == 64))) {
        return hipErrorInvalidValue;
    }
    const int steps = (g.k + bk - 1) / bk;
    int splits = g.force_splits;
    if (splits == 0) {
        const long long tiles = blocks(tile);
        if (tile == 32) {
            splits = deep ? 4 : 1;
            if (tiles < 128) {
                splits = std::max<long long>(splits, std::min<long long>((512 + tiles - 1) / tiles, steps / 2));
            }
        } else {
            splits = deep ? (g.m <= 256 ? 8 : tiles < 384 ? 2 : 1) : 1;
        }
    }
    splits = std::max(1, std::min(splits, steps));
    const size_t plane = static_cast<size_t>(g.m) * g.n * g.batch;
    if (g.partial == nullptr) {
        splits = 1;
    } else {
        splits = std::min<size_t>(splits, g.partial_floats / plane);
        if (splits < 1) splits = 1;
    }
    const int per = (steps + splits - 1) / splits;
    splits = (steps + per - 1) / per;  // no empty slice
    const dim3 grid((g.n + tile - 1) / tile, (g.m + tile - 1) / tile, g.batch * splits);
    if (tile == 128) {
        gemm_bf16_kernel<128, 128, 64><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
    } else if (tile == 64) {
        if (bk == 128) gemm_bf16_kernel<64, 64, 128, true><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
        else gemm_bf16_kernel<64, 64, 64, true><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
    } else {
        if (bk == 256) gemm_bf16_kernel<32, 32, 256, true><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
        else if (bk == 128) gemm_bf16_kernel<32, 32, 128, true><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
        else gemm_bf16_kernel<32, 32, 64, true><<<grid, kGemmThreads, 0, stream>>>(g, splits, per);
    }
    if (splits > 1) {
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        gemm_bf16_reduce_kernel<<<dim3((g.n + 255) / 256, g.m, g.batch), 256, 0, stream>>>(g, splits);
    }
    return hipGetLastError();
}

hipError_t launch_causal_softmax(bf16_t* scores, int heads, int rows, int stride, int head_dimension,
                                 hipStream_t stream) {
    if (scores == nullptr || heads <= 0 || rows <= 0 || rows > kPrefillAttentionRows || stride < rows ||
        head_dimension <= 0) {
        return hipErrorInvalidValue;
    }
    const float scale = 1.0f / sqrtf(static_cast<float>(head_dimension));
    causal_softmax_kernel<<<dim3(rows, heads), 64, 0, stream>>>(scores, rows, stride, scale);
    return hipGetLastError();
}

hipError_t launch_prefill_qkv_epilogue(bf16_t* qkv, const bf16_t* q_norm, const bf16_t* k_norm, const bf16_t* rope_table,
                                       bf16_t* key_cache, bf16_t* value_cache, int value_stride, int first, int rows,
                                       int query_heads, int key_value_heads, float epsilon, hipStream_t stream) {
    if (rows <= 0 || query_heads <= 0 || key_value_heads <= 0 || value_stride % 8 != 0) return hipErrorInvalidValue;
    const int heads = query_heads + 2 * key_value_heads;
    prefill_qkv_epilogue_kernel<<<rows * heads, 64, 0, stream>>>(qkv, q_norm, k_norm, rope_table, key_cache, value_cache,
                                                                 value_stride, first, query_heads, key_value_heads,
                                                                 epsilon);
    return hipGetLastError();
}

hipError_t launch_transpose_values(const bf16_t* qkv, int qkv_width, int v_offset, int rows, int stride,
                                   int key_value_heads, bf16_t* vt, hipStream_t stream) {
    if (rows <= 0 || stride < rows || key_value_heads <= 0) return hipErrorInvalidValue;
    const size_t total = static_cast<size_t>(key_value_heads) * 128 * stride;
    const int blocks = static_cast<int>(std::min<size_t>((total + 255) / 256, 4096));
    transpose_values_kernel<<<blocks, 256, 0, stream>>>(qkv, qkv_width, v_offset, rows, stride, key_value_heads, vt);
    return hipGetLastError();
}

hipError_t launch_prompt_rows(bf16_t* rows_data, const int* text, const int* codec, const bf16_t* codec_embedding,
                              int codec_vocabulary, int rows, int width, hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    prompt_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(rows_data, text, codec, codec_embedding,
                                                                            codec_vocabulary, width);
    return hipGetLastError();
}

hipError_t launch_gather_text_rows(const bf16_t* table, const int* text, int vocabulary, int rows, int width,
                                   bf16_t* out, hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    gather_text_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(table, text, vocabulary, width, out);
    return hipGetLastError();
}

}  // namespace q3
