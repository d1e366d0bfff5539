// Kernels of the speech-tokenizer decoder (reference:
// native/qwen3-tts-native-codec/native/src/codec_state.cu, cited CS:line).
//
// The reference runs cuBLAS SGEMM plus one elementwise kernel per operation.
// Here the convolutions are one fp32 MFMA GEMM kernel whose A operand is read
// straight from the extended (history + packet) buffer -- no im2col copy --
// and whose epilogue applies bias, GELU, ConvNeXt's gamma residual or the
// residual-unit add, and the following SnakeBeta, writing the next layer's
// input directly.  The transformer's 1..4-row products are a GEMV kernel with
// RMSNorm fused on its input.
#include "codec.hpp"

#include "../q3_math.h"

#include <algorithm>

namespace q3c {

namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float wave_sum(float v) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

__device__ __forceinline__ float4 load4(const float* p) { return *reinterpret_cast<const float4*>(p); }

inline unsigned blocks_for(size_t count, unsigned threads = 256) {
    const size_t b = (count + threads - 1) / threads;
    return (unsigned)std::min<size_t>(std::max<size_t>(b, 1), 65535u * 16);
}

// ---------------------------------------------------------------------------
// Epilogue of one output element (CS:407-412 bias, CS:860-866 GELU,
// CS:1115-1124 residual add, ConvNeXt gamma CS:1432-1667, SnakeBeta CS:882-898)
// ---------------------------------------------------------------------------
__device__ __forceinline__ void conv_epilogue(const ConvGemmArgs& g, int p, int col, int ch, float acc) {
    float v = g.bias ? acc + g.bias[ch] : acc;
    const size_t idx = (size_t)p * g.n + col;
    if (g.epilogue == kEpGelu) {
        v = 0.5f * v * (1.0f + erff(v * 0.7071067811865475f));
    } else if (g.epilogue == kEpGammaResidual) {
        v = g.residual[idx] + v * g.gamma[ch];
    } else if (g.epilogue == kEpResidual) {
        v = v + g.residual[idx];
    }
    if (g.out) g.out[idx] = v;
    if (g.snake_out) {
        const float s = sinf(v * g.snake_alpha[ch]);
        g.snake_out[idx] = v + (s * s) / g.snake_beta_den[ch];
    }
}

// ---------------------------------------------------------------------------
// fp32 MFMA convolution GEMM.
//
// 256 threads = 4 waves in a WM x WN grid; each wave owns TM x TN tiles of
// 16 x 16 (v_mfma_f32_16x16x4_f32).  K advances 32 floats per step through
// two LDS buffers: the block's threads read the next step's A rows (from the
// extended buffer, at the tap's row offset) and W rows from global memory into
// registers -- 128 contiguous bytes per row, 8 threads per row -- while the
// waves run the current step's MFMAs from LDS, then store them into the other
// buffer; one barrier per step.  In a step, lane (row = lane & 15,
// group = lane >> 4) reads 8 consecutive floats at k = 8 * group of its A row
// and of its W row, and MFMA e (0..7) takes element e, so one MFMA's four
// k-slots are 8g + e for g = 0..3: the same k for A and W, a valid
// (reordered) dot product.  Rows are padded to 36 floats in LDS.
//
// Split-K: slice z of Z covers a contiguous range of the steps and stores its
// partial tile; conv_gemm_reduce_kernel then sums them.  (An in-kernel
// last-arriver fix-up needs device-scope release/acquire fences, which write
// back and invalidate L2 and cost ~100 us per launch here.)
// ---------------------------------------------------------------------------
template <int TM, int TN>
__device__ __forceinline__ float* partial_slot(const ConvGemmArgs& g, size_t tiles, size_t tile, int z, int wave, int i,
                                               int j, int lane) {
    return g.partial + ((((size_t)z * tiles + tile) * 4 + wave) * (TM * TN) + (i * TN + j)) * 256 + lane * 4;
}

// Lane (row16 = lane & 15, group = lane >> 4) of wave `wave` holds, for its
// 16 x 16 sub-tile (i, j), rows 4 * group + r (r = 0..3) of column row16.
template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void subtile_epilogue(const ConvGemmArgs& g, const floatx4& acc, int tile_m, int tile_n,
                                                 int wave, int i, int j, int lane) {
    constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
    const int wm = wave / WN, wn = wave % WN;
    const int col0 = tile_n * BN + (wn * TN + j) * 16;
    if (col0 >= g.n) return;  // wave-uniform (n % 16 == 0)
    const int col = col0 + (lane & 15);
    const int ch = col % g.channels_out;
    const int p0 = tile_m * BM + (wm * TM + i) * 16 + 4 * (lane >> 4);
#pragma unroll
    for (int r = 0; r < 4; ++r)
        if (p0 + r < g.m) conv_epilogue(g, p0 + r, col, ch, acc[r]);
}

template <int TM, int TN, int WM, int WN>
__device__ __forceinline__ void tile_epilogue(const ConvGemmArgs& g, const floatx4 (&acc)[TM][TN], int tile_m,
                                              int tile_n, int wave, int lane) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
        for (int i = 0; i < TM; ++i) subtile_epilogue<TM, TN, WM, WN>(g, acc[i][j], tile_m, tile_n, wave, i, j, lane);
}

template <int TM, int TN, int WM, int WN, int BK>
__global__ __launch_bounds__(256) void conv_gemm_kernel(ConvGemmArgs g) {
    static_assert(WM * WN == 4, "4 waves");
    static_assert(BK == 32 || BK == 64, "K step");
    constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
    constexpr int VPR = BK / 4;      // float4 per row per step
    constexpr int ROW = BK + 4;      // LDS row pitch (floats)
    constexpr int A_VEC = BM * VPR, W_VEC = BN * VPR;
    constexpr int A_PER = (A_VEC + 255) / 256, W_PER = (W_VEC + 255) / 256;
    // every thread copies A_PER + W_PER vectors; rows past the tile (small
    // tiles) are loaded from clamped addresses into spare LDS rows, unused
    __shared__ float lds_a[2][A_PER * (256 / VPR) * ROW];
    __shared__ float lds_w[2][W_PER * (256 / VPR) * ROW];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int row16 = lane & 15, group = lane >> 4;

    // global -> LDS copy assignment: vector v = tid + 256 * r covers row v / VPR, float4 v % VPR
    const float* a_src[A_PER];
    const float* w_src[W_PER];
#pragma unroll
    for (int r = 0; r < A_PER; ++r) {
        const int v = tid + 256 * r;
        const int p = min((int)(blockIdx.y * BM) + v / VPR, g.m - 1);
        a_src[r] = g.a + (size_t)p * g.channels_in + (v % VPR) * 4;
    }
#pragma unroll
    for (int r = 0; r < W_PER; ++r) {
        const int v = tid + 256 * r;
        const int col = min((int)(blockIdx.x * BN) + v / VPR, g.n - 1);
        w_src[r] = g.w + (size_t)col * g.k + (v % VPR) * 4;
    }

    const int steps = g.k / BK;
    const int s0 = (int)((long long)steps * blockIdx.z / g.splits);
    const int s1 = (int)((long long)steps * (blockIdx.z + 1) / g.splits);
    // (tap, channel) of the next step to load (channels_in % BK == 0)
    int tap = (s0 * BK) / g.channels_in;
    int chan = s0 * BK - tap * g.channels_in;
    int s_load = s0;
    const size_t tap_stride = (size_t)g.dilation * g.channels_in;

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    float4 a_reg[A_PER], w_reg[W_PER];
    auto fetch = [&]() {
        const size_t a_off = (size_t)tap * tap_stride + chan;
        const size_t w_off = (size_t)s_load * BK;
#pragma unroll
        for (int r = 0; r < A_PER; ++r) a_reg[r] = load4(a_src[r] + a_off);
#pragma unroll
        for (int r = 0; r < W_PER; ++r) w_reg[r] = load4(w_src[r] + w_off);
        ++s_load;
        chan += BK;
        if (chan == g.channels_in) {
            chan = 0;
            ++tap;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int r = 0; r < A_PER; ++r) {
            const int v = tid + 256 * r;
            *reinterpret_cast<float4*>(&lds_a[buf][(v / VPR) * ROW + (v % VPR) * 4]) = a_reg[r];
        }
#pragma unroll
        for (int r = 0; r < W_PER; ++r) {
            const int v = tid + 256 * r;
            *reinterpret_cast<float4*>(&lds_w[buf][(v / VPR) * ROW + (v % VPR) * 4]) = w_reg[r];
        }
    };
    auto compute = [&](int buf) {
#pragma unroll
        for (int kh = 0; kh < BK / 32; ++kh) {
            float4 av[TM][2], wv[TN][2];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const float* src = &lds_a[buf][((wm * TM + i) * 16 + row16) * ROW + kh * 32 + 8 * group];
                av[i][0] = *reinterpret_cast<const float4*>(src);
                av[i][1] = *reinterpret_cast<const float4*>(src + 4);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const float* src = &lds_w[buf][((wn * TN + j) * 16 + row16) * ROW + kh * 32 + 8 * group];
                wv[j][0] = *reinterpret_cast<const float4*>(src);
                wv[j][1] = *reinterpret_cast<const float4*>(src + 4);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const float4& a4 = av[i][e >> 2];
                    const float x = (e & 3) == 0 ? a4.x : (e & 3) == 1 ? a4.y : (e & 3) == 2 ? a4.z : a4.w;
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        const float4& w4 = wv[j][e >> 2];
                        const float y = (e & 3) == 0 ? w4.x : (e & 3) == 1 ? w4.y : (e & 3) == 2 ? w4.z : w4.w;
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(x, y, acc[i][j], 0, 0, 0);
                    }
                }
            }
        }
    };
    if (s0 < s1) {
        fetch();
        stash(0);
        __syncthreads();
        for (int s = s0; s < s1; ++s) {
            const int buf = (s - s0) & 1;
            const bool more = s + 1 < s1;
            if (more) fetch();
            compute(buf);
            if (more) stash(buf ^ 1);
            __syncthreads();
        }
    }
    if (g.splits > 1) {
        // partial tile of slice z, lane-major: the reduction kernel reads it back
        // with the same thread mapping
        const size_t tiles = (size_t)gridDim.x * gridDim.y;
        const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                *reinterpret_cast<floatx4*>(partial_slot<TM, TN>(g, tiles, tile, blockIdx.z, wave, i, j, lane)) =
                    acc[i][j];
        return;
    }
    tile_epilogue<TM, TN, WM, WN>(g, acc, blockIdx.y, blockIdx.x, wave, lane);
}

// Split-K reduction: one 64-lane block per 16 x 16 sub-tile (the lanes of the
// wave that computed it) sums the slices' partials in slice order
// (deterministic) and runs the epilogue.
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(64) void conv_gemm_reduce_kernel(ConvGemmArgs g) {
    const int lane = threadIdx.x;
    const int sub = blockIdx.z;  // (wave, i, j)
    const int wave = sub / (TM * TN), i = (sub / TN) % TM, j = sub % TN;
    const size_t tiles = (size_t)gridDim.x * gridDim.y;
    const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    floatx4 sum = *reinterpret_cast<const floatx4*>(partial_slot<TM, TN>(g, tiles, tile, 0, wave, i, j, lane));
    // eight slices' loads in flight together, added in slice order
    for (int z0 = 1; z0 < g.splits; z0 += 8) {
        floatx4 v[8];
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const int z = min(z0 + d, g.splits - 1);
            v[d] = *reinterpret_cast<const floatx4*>(partial_slot<TM, TN>(g, tiles, tile, z, wave, i, j, lane));
        }
#pragma unroll
        for (int d = 0; d < 8; ++d)
            if (z0 + d < g.splits) sum += v[d];
    }
    subtile_epilogue<TM, TN, WM, WN>(g, sum, blockIdx.y, blockIdx.x, wave, i, j, lane);
}

// ---------------------------------------------------------------------------
// Rows GEMV for 1..4 rows (transformer projections, RVQ projection, causal
// pre-convolution).  One wave per block computes one output channel: its
// lanes hold the rows in registers (float4 at k = 256 * c + 4 * lane, read
// from L2), apply RMSNorm there when asked (CS:414-434: each wave reduces the
// row's squares itself), stream each channel's weight row with float4 loads
// and finish with a butterfly sum.  No LDS and no barrier: the launch's
// latency is one weight read plus one reduction.
// ---------------------------------------------------------------------------
constexpr int kMaxRows = 4;

template <int kChunks>
__global__ __launch_bounds__(64) void rows_gemv_kernel(RowsGemvArgs g) {
    const int lane = threadIdx.x;
    const int ch = blockIdx.x;
    const bool pair = g.epilogue == kRowsSiluPair;
    // the channel's weight row(s) first: the longest-latency reads
    float4 wa[kChunks], wb[kChunks];
#pragma unroll
    for (int c = 0; c < kChunks; ++c) wa[c] = load4(g.w + (size_t)ch * g.k + c * 256 + lane * 4);
    if (pair) {
#pragma unroll
        for (int c = 0; c < kChunks; ++c) wb[c] = load4(g.w + (size_t)(g.n + ch) * g.k + c * 256 + lane * 4);
    }
    float4 x[kMaxRows][kChunks];
#pragma unroll
    for (int r = 0; r < kMaxRows; ++r) {
        const int rr = min(r, g.rows - 1);
#pragma unroll
        for (int c = 0; c < kChunks; ++c) x[r][c] = load4(g.x + (size_t)rr * g.ldx + c * 256 + lane * 4);
    }
    if (g.norm) {
        float4 nw[kChunks];
#pragma unroll
        for (int c = 0; c < kChunks; ++c) nw[c] = load4(g.norm + c * 256 + lane * 4);
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r) {
            float sq = 0.f;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                sq = fmaf(x[r][c].x, x[r][c].x, sq);
                sq = fmaf(x[r][c].y, x[r][c].y, sq);
                sq = fmaf(x[r][c].z, x[r][c].z, sq);
                sq = fmaf(x[r][c].w, x[r][c].w, sq);
            }
            const float scale = 1.0f / sqrtf(wave_sum(sq) / (float)g.k + 1.0e-5f);
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                x[r][c].x = x[r][c].x * scale * nw[c].x;
                x[r][c].y = x[r][c].y * scale * nw[c].y;
                x[r][c].z = x[r][c].z * scale * nw[c].z;
                x[r][c].w = x[r][c].w * scale * nw[c].w;
            }
        }
    }
    if (g.advance_position && ch == 0 && lane == 0) *g.advance_position += g.advance_by;

    auto dot_rows = [&](const float4 (&wv)[kChunks], float (&acc)[kMaxRows]) {
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r) {
            float s = 0.f;
#pragma unroll
            for (int c = 0; c < kChunks; ++c) {
                s = fmaf(wv[c].x, x[r][c].x, s);
                s = fmaf(wv[c].y, x[r][c].y, s);
                s = fmaf(wv[c].z, x[r][c].z, s);
                s = fmaf(wv[c].w, x[r][c].w, s);
            }
            acc[r] = wave_sum(s);
        }
    };
    float a[kMaxRows], b[kMaxRows] = {0.f, 0.f, 0.f, 0.f};
    dot_rows(wa, a);
    if (pair) dot_rows(wb, b);
    const int r = lane;
    if (r < g.rows) {
        float va = a[0], vb = b[0];
#pragma unroll
        for (int q = 1; q < kMaxRows; ++q)
            if (r == q) va = a[q], vb = b[q];
        float v;
        if (pair) {
            v = (va / (1.0f + q3_expf(-va))) * vb;  // CS:687-698
        } else {
            v = g.bias ? va + g.bias[ch] : va;
            if (g.epilogue == kRowsScaledResidual) v = g.residual[(size_t)r * g.ldo + ch] + v * g.scale[ch];
        }
        g.out[(size_t)r * g.ldo + ch] = v;
    }
}

// ---------------------------------------------------------------------------
// Transformer attention of one packet (CS:464-494 RoPE, CS:496-566 sliding
// attention).  One block per (head, frame).  Each block rotates the packet's
// own keys itself (so no block reads a ring slot another block writes in the
// same launch), takes older keys and values from the ring, and follows the
// reference's per-head loop: scores, max, exponentials, the sequential
// denominator and the ordered value sum.  Frame 0's block appends the
// packet's keys and values to the ring.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void codec_attention_kernel(const float* qkv, int frames,
                                                              const unsigned long long* position, float* kv_k,
                                                              float* kv_v, float* out) {
    __shared__ float q_s[64];
    __shared__ float k_s[kWindow][65];
    __shared__ float v_s[kWindow][65];
    __shared__ float p_s[kWindow];
    __shared__ float denom_s;
    const int head = blockIdx.x, f = blockIdx.y;
    const int tid = threadIdx.x;
    const unsigned long long pos = *position;
    const unsigned long long me = pos + (unsigned long long)f;
    const unsigned long long first = me + 1 > (unsigned long long)kWindow ? me + 1 - kWindow : 0ull;
    const int count = (int)(me - first + 1);
    const int old_rows = (int)(pos - first);  // window rows before the packet
    float* ring_k = kv_k + (size_t)head * kKvSlots * 64;
    float* ring_v = kv_v + (size_t)head * kKvSlots * 64;
    const int first_slot = (int)(first % kKvSlots);
    for (int idx = tid; idx < old_rows * 16; idx += 256) {  // float4 per thread
        const int j = idx >> 4, d = (idx & 15) * 4;
        int slot = first_slot + j;
        slot -= slot >= kKvSlots ? kKvSlots : 0;
        const float4 kk = load4(ring_k + slot * 64 + d), vv = load4(ring_v + slot * 64 + d);
        k_s[j][d] = kk.x, k_s[j][d + 1] = kk.y, k_s[j][d + 2] = kk.z, k_s[j][d + 3] = kk.w;
        v_s[j][d] = vv.x, v_s[j][d + 1] = vv.y, v_s[j][d + 2] = vv.z, v_s[j][d + 3] = vv.w;
    }
    if (tid < (f + 1) * 32) {  // the packet's frames 0..f, rotate-half pairs (d, d + 32)
        const int g = tid >> 5, d = tid & 31;
        const float* row = qkv + (size_t)g * 3 * 1024 + head * 64;
        const float frequency = 1.0f / powf(10000.0f, (float)(2 * d) / 64.0f);
        const float angle = (float)(pos + (unsigned long long)g) * frequency;
        const float sine = sinf(angle), cosine = cosf(angle);
        const float k1 = row[1024 + d], k2 = row[1024 + d + 32];
        const float r1 = k1 * cosine - k2 * sine, r2 = k2 * cosine + k1 * sine;
        const float v1 = row[2048 + d], v2 = row[2048 + d + 32];
        const int j = old_rows + g;
        k_s[j][d] = r1;
        k_s[j][d + 32] = r2;
        v_s[j][d] = v1;
        v_s[j][d + 32] = v2;
        if (g == f) {
            const float q1 = row[d], q2 = row[d + 32];
            q_s[d] = q1 * cosine - q2 * sine;
            q_s[d + 32] = q2 * cosine + q1 * sine;
        }
    }
    if (f == 0 && tid < frames * 32) {  // append the packet's rows to the ring
        const int g = tid >> 5, d = tid & 31;
        const float* row = qkv + (size_t)g * 3 * 1024 + head * 64;
        const float frequency = 1.0f / powf(10000.0f, (float)(2 * d) / 64.0f);
        const float angle = (float)(pos + (unsigned long long)g) * frequency;
        const float sine = sinf(angle), cosine = cosf(angle);
        const float k1 = row[1024 + d], k2 = row[1024 + d + 32];
        const int slot = (int)((pos + (unsigned long long)g) % kKvSlots);
        ring_k[slot * 64 + d] = k1 * cosine - k2 * sine;
        ring_k[slot * 64 + d + 32] = k2 * cosine + k1 * sine;
        ring_v[slot * 64 + d] = row[2048 + d];
        ring_v[slot * 64 + d + 32] = row[2048 + d + 32];
    }
    __syncthreads();
    float score = -3.402823466e+38f;
    if (tid < count) {
        float sc = 0.f;
        for (int d = 0; d < 64; ++d) sc = fmaf(q_s[d], k_s[tid][d], sc);
        score = sc * 0.125f;
    }
    // max over the window: waves, then the block
    __shared__ float wmax[4];
    float m = wave_max(score);
    if ((tid & 63) == 0) wmax[tid >> 6] = m;
    __syncthreads();
    const float maximum = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    const float e = tid < count ? q3_expf(score - maximum) : 0.f;
    if (tid < count) p_s[tid] = e;
    __syncthreads();
    if (tid == 0) {  // sequential, in window order
        float denominator = 0.f;
#pragma unroll
        for (int j = 0; j < kWindow; ++j)
            if (j < count) denominator += p_s[j];
        denom_s = denominator;
    }
    __syncthreads();
    if (tid < count) p_s[tid] = e / denom_s;  // the reference's per-term probability
    __syncthreads();
    if (tid < 64) {
        float result = 0.f;
#pragma unroll 8
        for (int j = 0; j < count; ++j) result = fmaf(p_s[j], v_s[j][tid], result);
        out[(size_t)f * 1024 + head * 64 + tid] = result;
    }
}

// ---------------------------------------------------------------------------
// Frontend codebook gather (CS:322-342) and history copies.
// ---------------------------------------------------------------------------
struct FrontendTables {
    const float* emb[kCodebooks];
    const float* usage[kCodebooks];
};

// Segment blockIdx.y, chunk `block` of `blocks`.
__device__ void copy_segment_chunk(const CopySegment* seg, int block, int blocks) {
    const CopySegment sg = seg[blockIdx.y];
    const unsigned n4 = sg.floats >> 2;
    const float4* src = reinterpret_cast<const float4*>(sg.src);
    float4* dst = reinterpret_cast<float4*>(sg.dst);
    for (unsigned i = block * 256 + threadIdx.x; i < n4; i += blocks * 256) dst[i] = src[i];
}

// blockIdx.y = segment; on segment row 0 the first `frames` blocks also
// gather frame blockIdx.x's codebook entries (all 16 lookups issued at once).
__global__ __launch_bounds__(256) void codec_frontend_kernel(const uint16_t* codes, int frames, FrontendTables t,
                                                             float* x, const CopySegment* seg) {
    if (blockIdx.y == 0 && (int)blockIdx.x < frames) {
        const int f = blockIdx.x, d = threadIdx.x;
        int code[kCodebooks];
        float usage[kCodebooks], emb[kCodebooks];
#pragma unroll
        for (int cb = 0; cb < kCodebooks; ++cb) {
            // codes beyond the 2048-entry codebooks are clamped so a corrupt
            // device frame cannot read outside the table
            code[cb] = min((int)codes[f * kCodebooks + cb], 2047);
        }
#pragma unroll
        for (int cb = 0; cb < kCodebooks; ++cb) {
            usage[cb] = t.usage[cb][code[cb]];
            emb[cb] = t.emb[cb][(size_t)code[cb] * 256 + d];
        }
        float acoustic = 0.f;
#pragma unroll
        for (int cb = 0; cb < kCodebooks; ++cb) {
            const float value = emb[cb] / fmaxf(usage[cb], 1.0e-5f);
            if (cb == 0) {
                x[f * 512 + d] = value;
            } else {
                acoustic = cb == 1 ? value : acoustic + value;
            }
        }
        x[f * 512 + 256 + d] = acoustic;
    }
    copy_segment_chunk(seg, blockIdx.x, gridDim.x);
}

__global__ __launch_bounds__(256) void copy_segments_kernel(const CopySegment* seg) {
    copy_segment_chunk(seg, blockIdx.x, gridDim.x);
}

// ---------------------------------------------------------------------------
// ConvNeXt depthwise causal convolution (CS:730-756) + LayerNorm (CS:778-808):
// one block per position, 4 channels per thread.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void dwconv_layernorm_kernel(const float* ext, const float* w, const float* b,
                                                               const float* ln_w, const float* ln_b, float* out) {
    __shared__ float red[4];
    const int p = blockIdx.x, tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float y[4];
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        float r = b[c];
#pragma unroll
        for (int k = 0; k < 7; ++k) r = fmaf(w[c * 7 + k], ext[(size_t)(p + k) * 1024 + c], r);
        y[i] = r;
        sum += r;
    }
    sum = wave_sum(sum);
    if (lane == 0) red[wave] = sum;
    __syncthreads();
    const float mean = (red[0] + red[1] + red[2] + red[3]) / 1024.0f;
    __syncthreads();
    float var = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float c = y[i] - mean;
        var = fmaf(c, c, var);
    }
    var = wave_sum(var);
    if (lane == 0) red[wave] = var;
    __syncthreads();
    const float scale = 1.0f / sqrtf((red[0] + red[1] + red[2] + red[3]) / 1024.0f + 1.0e-6f);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int c = tid + 256 * i;
        out[(size_t)p * 1024 + c] = (y[i] - mean) * scale * ln_w[c] + ln_b[c];
    }
}

// ---------------------------------------------------------------------------
// Final causal convolution 96 -> 1 (CS:1699-1782 with the im2col column order
// channel-major, tap-minor), bias, clamp (CS:1126-1131), PCM (CS:1133-1143).
// ---------------------------------------------------------------------------
// Four lanes per position, each a sequential channel-major, tap-minor fmaf
// chain over 24 of the 96 channels (float4 reads), then the four partial sums
// added in channel-group order.
__global__ __launch_bounds__(256) void final_conv_pcm_kernel(const float* ext, int positions, const float* w,
                                                             const float* b, int16_t* pcm, float* preclamp,
                                                             float* clamped) {
    __shared__ float ws[96 * 7];
    for (int i = threadIdx.x; i < 96 * 7; i += 256) ws[i] = w[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int group = lane >> 4;  // channels 24 * group .. + 23
    const int p = blockIdx.x * 64 + (threadIdx.x >> 6) * 16 + (lane & 15);
    const int pc = min(p, positions - 1);
    float4 x[7][6];
#pragma unroll
    for (int t = 0; t < 7; ++t)
#pragma unroll
        for (int q = 0; q < 6; ++q) x[t][q] = load4(ext + (size_t)(pc + t) * 96 + group * 24 + q * 4);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 6; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int c = group * 24 + q * 4 + e;
#pragma unroll
            for (int t = 0; t < 7; ++t) {
                const float xv = e == 0 ? x[t][q].x : e == 1 ? x[t][q].y : e == 2 ? x[t][q].z : x[t][q].w;
                acc = fmaf(xv, ws[c * 7 + t], acc);
            }
        }
    }
    // lanes r, r + 16, r + 32, r + 48 hold the four groups of position r
    const float g1 = __shfl(acc, (lane & 15) + 16, 64), g2 = __shfl(acc, (lane & 15) + 32, 64),
                g3 = __shfl(acc, (lane & 15) + 48, 64);
    if (group != 0 || p >= positions) return;
    const float v = ((acc + g1) + g2) + g3 + b[0];
    if (preclamp) preclamp[p] = v;
    const float c = fminf(1.0f, fmaxf(-1.0f, v));
    if (clamped) clamped[p] = c;
    const float scaled = roundf(c * 32767.0f);
    pcm[p] = (int16_t)fminf(32767.0f, fmaxf(-32768.0f, scaled));
}

// ---------------------------------------------------------------------------
// Deterministic state-machine fixture (CS:185-318, 4518-4740): integer
// stand-ins for the pre-convolution (3x + 2 h1 - h2) / 4 over the weighted code
// sum, two repeats, four transposed-convolution overlaps (3x + previous) / 4
// with carried tails, and x * 8 saturated to 16 bits.  One block; the stages
// alternate between two LDS buffers.  state: [0..1] pre-conv history,
// [2..21] the tails of strides 8, 5, 4, 3.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void fixture_packet_kernel(const uint16_t* codes, int frames, int* state,
                                                             int16_t* pcm) {
    __shared__ int buf[2][kMaxFrames * kSamplesPerFrame];
    __shared__ int tails[20];
    const int tid = threadIdx.x;
    if (tid < 20) tails[tid] = state[2 + tid];
    if (tid == 0) {
        int h1 = state[0], h2 = state[1];
        for (int f = 0; f < frames; ++f) {
            int sum = 0;
            for (int cb = 0; cb < kCodebooks; ++cb) sum += (codes[f * kCodebooks + cb] & 2047) * (cb + 1);
            const int centered = (sum & 4095) - 2048;
            const int filtered = (3 * centered + 2 * h1 - h2) / 4;
            h2 = h1;
            h1 = centered;
            for (int r = 0; r < 4; ++r) buf[0][4 * f + r] = filtered;  // repeat x2, x2
        }
        state[0] = h1;
        state[1] = h2;
    }
    __syncthreads();
    int n = 4 * frames, src = 0, tail_base = 0;
    for (int stage = 0; stage < 4; ++stage) {
        const int stride = kStride[stage];
        const int* in = buf[src];
        int* out = buf[src ^ 1];
        for (int i = tid; i < n * stride; i += 256) {
            const int ip = i / stride, phase = i - ip * stride;
            const int previous = ip == 0 ? tails[tail_base + phase] : in[ip - 1];
            out[i] = (3 * in[ip] + previous) / 4;
        }
        __syncthreads();
        if (tid < stride) tails[tail_base + tid] = in[n - 1];
        __syncthreads();
        tail_base += stride;
        n *= stride;
        src ^= 1;
    }
    for (int i = tid; i < n; i += 256) {
        const int v = buf[src][i] * 8;
        pcm[i] = (int16_t)(v > 32767 ? 32767 : (v < -32768 ? -32768 : v));
    }
    if (tid < 20) state[2 + tid] = tails[tid];
}

// ---------------------------------------------------------------------------
// load-time kernels
// ---------------------------------------------------------------------------
__global__ void bf16_to_f32_kernel(const uint16_t* src, size_t count, float* dst) {
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += (size_t)gridDim.x * 256)
        dst[i] = __uint_as_float((unsigned)src[i] << 16);
}

__global__ void repack_conv_kernel(const float* src, int out_ch, int in_ch, int taps, float* dst) {
    const size_t total = (size_t)out_ch * in_ch * taps;
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t o = i / ((size_t)taps * in_ch);
        const size_t rem = i - o * taps * in_ch;
        const size_t t = rem / in_ch, c = rem - t * in_ch;
        dst[i] = src[(o * in_ch + c) * taps + t];
    }
}

__global__ void repack_transpose_kernel(const float* src, int in_ch, int out_ch, int stride, int overlap,
                                        float* dst) {
    const int span = overlap ? 2 * stride : stride;
    const int taps = overlap ? 2 : 1;
    const size_t k = (size_t)taps * in_ch;
    const size_t total = (size_t)stride * out_ch * k;
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t row = i / k, col = i - row * k;
        const int phase = (int)(row / out_ch), o = (int)(row - (size_t)phase * out_ch);
        const int tap = (int)(col / in_ch), c = (int)(col - (size_t)tap * in_ch);
        const int kernel_index = overlap && tap == 0 ? stride + phase : phase;
        dst[i] = src[((size_t)c * out_ch + o) * span + kernel_index];
    }
}

__global__ void snake_params_kernel(float* alpha, float* beta, int channels) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c < channels) {
        alpha[c] = expf(alpha[c]);
        beta[c] = expf(beta[c]) + 1.0e-9f;
    }
}

__global__ void fill_f32_kernel(float* dst, size_t count, float value) {
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) dst[i] = value;
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
namespace {
constexpr int kTileRows[4] = {16, 32, 32, 64};
constexpr int kTileCols[4] = {64, 32, 64, 64};
}  // namespace

size_t GemmPlan::partial_floats() const {
    if (splits <= 1) return 0;
    const int s = (int)shape;
    return (size_t)splits * tiles() * kTileRows[s] * kTileCols[s];
}

GemmPlan plan_conv_gemm(int m, int n, int k, int channels_in, int cus) {
    // Blocks in flight hide the per-step load latency: weight-streaming shapes
    // (<= 16 rows) take 16x64 tiles and split K to ~2 blocks per CU; longer
    // sequences take the largest tile that still gives ~2 blocks per CU, and
    // split K (to ~1.5 blocks per CU, each slice keeping >= 4 steps) only when
    // the tiles alone do not cover the CUs: the partial round trip and the
    // reduction launch cost more than they gain above that.  (Chosen from
    // per-layer measurements on MI355X.)
    GemmPlan plan;
    // 64-float K steps (half the barriers) wherever the channels allow
    plan.k_step = channels_in % 64 == 0 ? 64 : 32;
    const long long want = 2LL * cus;
    auto tiles_for = [&](GemmShape sh) {
        const int s = (int)sh;
        return (long long)((m + kTileRows[s] - 1) / kTileRows[s]) * ((n + kTileCols[s] - 1) / kTileCols[s]);
    };
    if (m <= 16) {
        plan.shape = GemmShape::k16x64;
    } else if (tiles_for(GemmShape::k64x64) >= want) {
        plan.shape = GemmShape::k64x64;
    } else if (tiles_for(GemmShape::k32x64) >= want && n % 64 == 0) {
        plan.shape = GemmShape::k32x64;
    } else {
        plan.shape = GemmShape::k32x32;
    }
    const int s = (int)plan.shape;
    plan.tiles_m = (m + kTileRows[s] - 1) / kTileRows[s];
    plan.tiles_n = (n + kTileCols[s] - 1) / kTileCols[s];
    const long long tiles = (long long)plan.tiles_m * plan.tiles_n;
    long long splits = 1;
    if (plan.shape == GemmShape::k16x64) {
        splits = (want + tiles - 1) / tiles;
    } else if (tiles < cus) {
        splits = (3LL * cus / 2 + tiles - 1) / tiles;
    }
    splits = std::min<long long>(splits, std::max(1, (k / plan.k_step) / 4));
    plan.splits = (int)std::max<long long>(1, splits);
    return plan;
}

namespace {
template <int TM, int TN, int WM, int WN>
void launch_shape(const ConvGemmArgs& args, const GemmPlan& plan, hipStream_t stream) {
    const dim3 grid(plan.tiles_n, plan.tiles_m, plan.splits);
    if (plan.k_step == 64) {
        conv_gemm_kernel<TM, TN, WM, WN, 64><<<grid, 256, 0, stream>>>(args);
    } else {
        conv_gemm_kernel<TM, TN, WM, WN, 32><<<grid, 256, 0, stream>>>(args);
    }
    if (plan.splits > 1)
        conv_gemm_reduce_kernel<TM, TN, WM, WN>
            <<<dim3(plan.tiles_n, plan.tiles_m, 4 * TM * TN), 64, 0, stream>>>(args);
}
}  // namespace

hipError_t launch_conv_gemm(const ConvGemmArgs& args, const GemmPlan& plan, hipStream_t stream) {
    if (args.k % plan.k_step || args.channels_in % plan.k_step || args.n % 16 || args.m < 1 ||
        args.splits != plan.splits ||
        (plan.splits > 1 && !args.partial))
        return hipErrorInvalidValue;
    switch (plan.shape) {
        case GemmShape::k16x64: launch_shape<1, 1, 1, 4>(args, plan, stream); break;
        case GemmShape::k32x32: launch_shape<1, 1, 2, 2>(args, plan, stream); break;
        case GemmShape::k32x64: launch_shape<1, 2, 2, 2>(args, plan, stream); break;
        case GemmShape::k64x64: launch_shape<2, 2, 2, 2>(args, plan, stream); break;
    }
    return hipGetLastError();
}

hipError_t launch_rows_gemv(const RowsGemvArgs& g, hipStream_t stream) {
    if (g.rows < 1 || g.rows > kMaxRows || g.k % 256 || g.ldx % 4 || g.n < 1) return hipErrorInvalidValue;
    // one output channel per single-wave block: >= 512 blocks for every
    // projection of the decoder (n = 512 .. 3072)
    const unsigned blocks = (unsigned)g.n;
    switch (g.k / 256) {
        case 2: rows_gemv_kernel<2><<<blocks, 64, 0, stream>>>(g); break;
        case 4: rows_gemv_kernel<4><<<blocks, 64, 0, stream>>>(g); break;
        case 6: rows_gemv_kernel<6><<<blocks, 64, 0, stream>>>(g); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_codec_attention(const float* qkv, int frames, const unsigned long long* position, float* kv_k,
                                  float* kv_v, float* out, hipStream_t stream) {
    if (frames < 1 || frames > kMaxFrames) return hipErrorInvalidValue;
    codec_attention_kernel<<<dim3(kHeads, frames), 256, 0, stream>>>(qkv, frames, position, kv_k, kv_v, out);
    return hipGetLastError();
}

hipError_t launch_codec_frontend(const uint16_t* codes, int frames, const float* const* embeddings,
                                 const float* const* usages, float* x, const CopySegment* seg, int segments,
                                 hipStream_t stream) {
    if (frames < 1 || frames > kMaxFrames) return hipErrorInvalidValue;
    FrontendTables t;
    for (int i = 0; i < kCodebooks; ++i) {
        t.emb[i] = embeddings[i];
        t.usage[i] = usages[i];
    }
    if (segments < 1) return hipErrorInvalidValue;
    codec_frontend_kernel<<<dim3(8, segments), 256, 0, stream>>>(codes, frames, t, x, seg);
    return hipGetLastError();
}

hipError_t launch_copy_segments(const CopySegment* seg, int segments, hipStream_t stream) {
    if (segments <= 0) return hipSuccess;
    copy_segments_kernel<<<dim3(8, segments), 256, 0, stream>>>(seg);
    return hipGetLastError();
}

hipError_t launch_dwconv_layernorm(const float* ext, int positions, const float* w, const float* b,
                                   const float* ln_w, const float* ln_b, float* out, hipStream_t stream) {
    dwconv_layernorm_kernel<<<positions, 256, 0, stream>>>(ext, w, b, ln_w, ln_b, out);
    return hipGetLastError();
}

hipError_t launch_final_conv_pcm(const float* ext, int positions, const float* w, const float* b, int16_t* pcm,
                                 float* preclamp, float* clamped, hipStream_t stream) {
    final_conv_pcm_kernel<<<(positions + 63) / 64, 256, 0, stream>>>(ext, positions, w, b, pcm, preclamp, clamped);
    return hipGetLastError();
}

hipError_t launch_fixture_packet(const uint16_t* codes, int frames, int* state, int16_t* pcm, hipStream_t stream) {
    if (frames < 1 || frames > kMaxFrames) return hipErrorInvalidValue;
    fixture_packet_kernel<<<1, 256, 0, stream>>>(codes, frames, state, pcm);
    return hipGetLastError();
}

hipError_t launch_bf16_to_f32(const uint16_t* src, size_t count, float* dst, hipStream_t stream) {
    bf16_to_f32_kernel<<<blocks_for(count), 256, 0, stream>>>(src, count, dst);
    return hipGetLastError();
}

hipError_t launch_repack_conv(const float* src, int out_ch, int in_ch, int taps, float* dst, hipStream_t stream) {
    repack_conv_kernel<<<blocks_for((size_t)out_ch * in_ch * taps), 256, 0, stream>>>(src, out_ch, in_ch, taps, dst);
    return hipGetLastError();
}

hipError_t launch_repack_transpose(const float* src, int in_ch, int out_ch, int stride, bool overlap, float* dst,
                                   hipStream_t stream) {
    const size_t total = (size_t)stride * out_ch * in_ch * (overlap ? 2 : 1);
    repack_transpose_kernel<<<blocks_for(total), 256, 0, stream>>>(src, in_ch, out_ch, stride, overlap ? 1 : 0, dst);
    return hipGetLastError();
}

hipError_t launch_snake_params(float* alpha, float* beta, int channels, hipStream_t stream) {
    snake_params_kernel<<<(channels + 255) / 256, 256, 0, stream>>>(alpha, beta, channels);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float* dst, size_t count, float value, hipStream_t stream) {
    fill_f32_kernel<<<blocks_for(count), 256, 0, stream>>>(dst, count, value);
    return hipGetLastError();
}

}  // namespace q3c
