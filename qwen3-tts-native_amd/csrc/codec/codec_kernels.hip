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
// 16 x 16 (v_mfma_f32_16x16x4_f32).  K advances 32 floats per step: lane
// (row = lane & 15, group = lane >> 4) loads 8 consecutive floats at
// k + 8 * group of its A row and of its W row, and MFMA e (0..7) takes
// element e, so one MFMA's four k-slots are k + 8g + e for g = 0..3 -- the
// same k for A and W, hence a valid (reordered) dot product.  Both operands
// come straight from global memory (L1/L2): a lane's 32 bytes are contiguous
// and four lanes cover 128 contiguous bytes of a row.
//
// Split-K: slice z of Z covers a contiguous range of the 32-float steps.
// Every slice stores its partial tile; the last to arrive at the tile's
// counter sums the Z partials in slice order (deterministic), runs the
// epilogue and re-arms the counter for the next launch.
// ---------------------------------------------------------------------------
template <int TM, int TN, int WM, int WN>
__global__ __launch_bounds__(256) void conv_gemm_kernel(ConvGemmArgs g) {
    static_assert(WM * WN == 4, "4 waves");
    constexpr int BM = 16 * TM * WM, BN = 16 * TN * WN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const int row16 = lane & 15, group = lane >> 4;
    const int p_base = blockIdx.y * BM + wm * 16 * TM;
    const int col_base = blockIdx.x * BN + wn * 16 * TN;

    const float* a_row[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int p = min(p_base + i * 16 + row16, g.m - 1);
        a_row[i] = g.a + (size_t)p * g.channels_in + 8 * group;
    }
    bool n_ok[TN];
    const float* w_row[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        n_ok[j] = col_base + j * 16 < g.n;  // wave-uniform (n % 16 == 0)
        const int col = min(col_base + j * 16 + row16, g.n - 1);
        w_row[j] = g.w + (size_t)col * g.k + 8 * group;
    }

    const int steps = g.k >> 5;
    const int s0 = (int)((long long)steps * blockIdx.z / g.splits);
    const int s1 = (int)((long long)steps * (blockIdx.z + 1) / g.splits);
    // (tap, channel) of step s0, advanced incrementally (channels_in % 32 == 0)
    int tap = (s0 * 32) / g.channels_in;
    int chan = s0 * 32 - tap * g.channels_in;
    const size_t tap_stride = (size_t)g.dilation * g.channels_in;

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    float4 a_cur[TM][2], w_cur[TN][2];
    auto load_step = [&](int s, int t, int c, float4 (&av)[TM][2], float4 (&wv)[TN][2]) {
        const size_t a_off = (size_t)t * tap_stride + c;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            av[i][0] = load4(a_row[i] + a_off);
            av[i][1] = load4(a_row[i] + a_off + 4);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            if (n_ok[j]) {
                wv[j][0] = load4(w_row[j] + (size_t)s * 32);
                wv[j][1] = load4(w_row[j] + (size_t)s * 32 + 4);
            }
        }
    };
    if (s0 < s1) load_step(s0, tap, chan, a_cur, w_cur);
    for (int s = s0; s < s1; ++s) {
        float4 a_nxt[TM][2], w_nxt[TN][2];
        chan += 32;
        if (chan == g.channels_in) {
            chan = 0;
            ++tap;
        }
        const bool more = s + 1 < s1;
        if (more) load_step(s + 1, tap, chan, a_nxt, w_nxt);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const float4& a4 = a_cur[i][e >> 2];
                const float av = (e & 3) == 0 ? a4.x : (e & 3) == 1 ? a4.y : (e & 3) == 2 ? a4.z : a4.w;
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if (!n_ok[j]) continue;
                    const float4& w4 = w_cur[j][e >> 2];
                    const float wv = (e & 3) == 0 ? w4.x : (e & 3) == 1 ? w4.y : (e & 3) == 2 ? w4.z : w4.w;
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, wv, acc[i][j], 0, 0, 0);
                }
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                a_cur[i][0] = a_nxt[i][0];
                a_cur[i][1] = a_nxt[i][1];
            }
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                w_cur[j][0] = w_nxt[j][0];
                w_cur[j][1] = w_nxt[j][1];
            }
        }
    }

    if (g.splits > 1) {
        const size_t tiles = (size_t)gridDim.x * gridDim.y;
        const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
        auto slot = [&](int z, int i, int j) {
            return g.partial + ((((size_t)z * tiles + tile) * 4 + wave) * (TM * TN) + (i * TN + j)) * 256 + lane * 4;
        };
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) *reinterpret_cast<floatx4*>(slot(blockIdx.z, i, j)) = acc[i][j];
        __threadfence();
        __syncthreads();
        __shared__ int last;
        if (threadIdx.x == 0) {
            const unsigned prev = __hip_atomic_fetch_add(g.counters + tile, 1u, __ATOMIC_ACQ_REL,
                                                         __HIP_MEMORY_SCOPE_AGENT);
            last = prev == (unsigned)(g.splits - 1);
        }
        __syncthreads();
        if (!last) return;
        __threadfence();
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                floatx4 sum = *reinterpret_cast<const floatx4*>(slot(0, i, j));
                for (int z = 1; z < g.splits; ++z) sum += *reinterpret_cast<const floatx4*>(slot(z, i, j));
                acc[i][j] = sum;
            }
        if (threadIdx.x == 0)
            __hip_atomic_store(g.counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }

#pragma unroll
    for (int j = 0; j < TN; ++j) {
        if (!n_ok[j]) continue;
        const int col = col_base + j * 16 + row16;
        const int ch = col % g.channels_out;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int p = p_base + i * 16 + 4 * group + r;
                if (p < g.m) conv_epilogue(g, p, col, ch, acc[i][j][r]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Rows GEMV for 1..4 rows (transformer projections, RVQ projection, causal
// pre-convolution): the rows are staged in LDS (RMSNorm applied there when
// asked, CS:414-434), each wave computes whole output channels with float4
// weight loads along k and a butterfly sum.
// ---------------------------------------------------------------------------
constexpr int kMaxRows = 4;

template <int kCpw>
__global__ __launch_bounds__(256) void rows_gemv_kernel(RowsGemvArgs g) {
    extern __shared__ float xs[];
    __shared__ float row_scale[kMaxRows];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int total = g.rows * g.k;
    for (int idx = threadIdx.x * 4; idx < total; idx += 256 * 4) {
        const int r = idx / g.k, c = idx - r * g.k;
        *reinterpret_cast<float4*>(xs + idx) = load4(g.x + (size_t)r * g.ldx + c);
    }
    __syncthreads();
    if (g.norm) {
        if (wave < g.rows) {
            float sq = 0.f;
            for (int c = lane; c < g.k; c += 64) sq = fmaf(xs[wave * g.k + c], xs[wave * g.k + c], sq);
            sq = wave_sum(sq);
            if (lane == 0) row_scale[wave] = 1.0f / sqrtf(sq / (float)g.k + 1.0e-5f);
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < total; idx += 256) {
            const int r = idx / g.k, c = idx - r * g.k;
            xs[idx] = xs[idx] * row_scale[r] * g.norm[c];
        }
        __syncthreads();
    }
    if (g.advance_position && blockIdx.x == 0 && threadIdx.x == 0) *g.advance_position += g.advance_by;

    const bool pair = g.epilogue == kRowsSiluPair;
#pragma unroll
    for (int j = 0; j < kCpw; ++j) {
        const int ch = (blockIdx.x * 4 + wave) * kCpw + j;
        if (ch >= g.n) break;
        const float* wa = g.w + (size_t)ch * g.k;
        const float* wb = pair ? g.w + (size_t)(g.n + ch) * g.k : nullptr;
        float acc_a[kMaxRows] = {0.f, 0.f, 0.f, 0.f};
        float acc_b[kMaxRows] = {0.f, 0.f, 0.f, 0.f};
        for (int c = lane * 4; c < g.k; c += 256) {
            const float4 va = load4(wa + c);
            float4 vb = {0.f, 0.f, 0.f, 0.f};
            if (pair) vb = load4(wb + c);
#pragma unroll
            for (int r = 0; r < kMaxRows; ++r) {
                if (r >= g.rows) break;
                const float4 x = *reinterpret_cast<const float4*>(xs + r * g.k + c);
                float s = acc_a[r];
                s = fmaf(va.x, x.x, s);
                s = fmaf(va.y, x.y, s);
                s = fmaf(va.z, x.z, s);
                s = fmaf(va.w, x.w, s);
                acc_a[r] = s;
                if (pair) {
                    float t = acc_b[r];
                    t = fmaf(vb.x, x.x, t);
                    t = fmaf(vb.y, x.y, t);
                    t = fmaf(vb.z, x.z, t);
                    t = fmaf(vb.w, x.w, t);
                    acc_b[r] = t;
                }
            }
        }
#pragma unroll
        for (int r = 0; r < kMaxRows; ++r) {
            if (r >= g.rows) break;
            const float a = wave_sum(acc_a[r]);
            const float b = pair ? wave_sum(acc_b[r]) : 0.f;
            if (lane != r) continue;
            float v;
            if (pair) {
                v = (a / (1.0f + q3_expf(-a))) * b;  // CS:687-698
            } else {
                v = g.bias ? a + g.bias[ch] : a;
                if (g.epilogue == kRowsScaledResidual) v = g.residual[(size_t)r * g.ldo + ch] + v * g.scale[ch];
            }
            g.out[(size_t)r * g.ldo + ch] = v;
        }
    }
}

// ---------------------------------------------------------------------------
// Transformer attention of one packet (CS:464-494 RoPE, CS:496-566 sliding
// attention).  One block per head; the block assembles in LDS the keys and
// values of positions [first(frame 0), last frame]: older ones from the ring,
// the packet's own freshly rotated rows from registers.  Wave f attends for
// frame f.  Scores, the max, the exponentials, the sequential denominator and
// the ordered value sum follow the reference's per-head loop.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void codec_attention_kernel(const float* qkv, int frames,
                                                              const unsigned long long* position, float* kv_k,
                                                              float* kv_v, float* out) {
    constexpr int kRows = kWindow + kMaxFrames - 1;
    __shared__ float q_s[kMaxFrames][64];
    __shared__ float k_s[kRows][65];
    __shared__ float v_s[kRows][65];
    __shared__ float p_s[kMaxFrames][kWindow];
    __shared__ float denom_s[kMaxFrames];
    const int head = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const unsigned long long pos = *position;
    const unsigned long long first_all = pos + 1 > (unsigned long long)kWindow ? pos + 1 - kWindow : 0ull;
    const int old_rows = (int)(pos - first_all);
    float* ring_k = kv_k + (size_t)head * kKvSlots * 64;
    float* ring_v = kv_v + (size_t)head * kKvSlots * 64;
    for (int idx = tid; idx < old_rows * 64; idx += 256) {
        const int j = idx >> 6, d = idx & 63;
        const int slot = (int)((first_all + (unsigned long long)j) % kKvSlots);
        k_s[j][d] = ring_k[slot * 64 + d];
        v_s[j][d] = ring_v[slot * 64 + d];
    }
    if (tid < frames * 32) {
        const int f = tid >> 5, d = tid & 31;
        const float* row = qkv + (size_t)f * 3 * 1024 + head * 64;
        const float frequency = 1.0f / powf(10000.0f, (float)(2 * d) / 64.0f);
        const float angle = (float)(pos + (unsigned long long)f) * frequency;
        const float sine = sinf(angle), cosine = cosf(angle);
        const float q1 = row[d], q2 = row[d + 32];
        const float k1 = row[1024 + d], k2 = row[1024 + d + 32];
        const float v1 = row[2048 + d], v2 = row[2048 + d + 32];
        q_s[f][d] = q1 * cosine - q2 * sine;
        q_s[f][d + 32] = q2 * cosine + q1 * sine;
        const float r1 = k1 * cosine - k2 * sine, r2 = k2 * cosine + k1 * sine;
        const int j = old_rows + f;
        k_s[j][d] = r1;
        k_s[j][d + 32] = r2;
        v_s[j][d] = v1;
        v_s[j][d + 32] = v2;
        const int slot = (int)((pos + (unsigned long long)f) % kKvSlots);
        ring_k[slot * 64 + d] = r1;
        ring_k[slot * 64 + d + 32] = r2;
        ring_v[slot * 64 + d] = v1;
        ring_v[slot * 64 + d + 32] = v2;
    }
    __syncthreads();
    const int f = wave;
    const bool active = f < frames;
    const unsigned long long me = pos + (unsigned long long)f;
    const unsigned long long first = me + 1 > (unsigned long long)kWindow ? me + 1 - kWindow : 0ull;
    const int j0 = (int)(first - first_all);
    const int count = (int)(me - first + 1);
    float local_max = -3.402823466e+38f;
    if (active) {
        for (int jj = lane; jj < count; jj += 64) {
            float score = 0.f;
            for (int d = 0; d < 64; ++d) score = fmaf(q_s[f][d], k_s[j0 + jj][d], score);
            score *= 0.125f;
            p_s[f][jj] = score;
            local_max = fmaxf(local_max, score);
        }
    }
    const float maximum = wave_max(local_max);
    __syncthreads();
    if (active) {
        for (int jj = lane; jj < count; jj += 64) p_s[f][jj] = q3_expf(p_s[f][jj] - maximum);
    }
    __syncthreads();
    if (active && lane == 0) {
        float denominator = 0.f;
        for (int jj = 0; jj < count; ++jj) denominator += p_s[f][jj];
        denom_s[f] = denominator;
    }
    __syncthreads();
    if (active) {
        const float denominator = denom_s[f];
        float result = 0.f;
        for (int jj = 0; jj < count; ++jj) result = fmaf(p_s[f][jj] / denominator, v_s[j0 + jj][lane], result);
        out[(size_t)f * 1024 + head * 64 + lane] = result;
    }
}

// ---------------------------------------------------------------------------
// Frontend codebook gather (CS:322-342) and history copies.
// ---------------------------------------------------------------------------
struct FrontendTables {
    const float* emb[kCodebooks];
    const float* usage[kCodebooks];
};

__device__ void copy_segments_block(const CopySegment* seg, int segments, int block, int blocks) {
    for (int s = 0; s < segments; ++s) {
        const unsigned n4 = seg[s].floats >> 2;
        const float4* src = reinterpret_cast<const float4*>(seg[s].src);
        float4* dst = reinterpret_cast<float4*>(seg[s].dst);
        for (unsigned i = block * 256 + threadIdx.x; i < n4; i += blocks * 256) dst[i] = src[i];
    }
}

__global__ __launch_bounds__(256) void codec_frontend_kernel(const uint16_t* codes, int frames, FrontendTables t,
                                                             float* x, const CopySegment* seg, int segments) {
    if ((int)blockIdx.x < frames) {
        const int f = blockIdx.x, d = threadIdx.x;
        float acoustic = 0.f;
#pragma unroll 1
        for (int cb = 0; cb < kCodebooks; ++cb) {
            // codes beyond the 2048-entry codebooks are clamped so a corrupt
            // device frame cannot read outside the table
            const int code = min((int)codes[f * kCodebooks + cb], 2047);
            const float usage = fmaxf(t.usage[cb][code], 1.0e-5f);
            const float value = t.emb[cb][(size_t)code * 256 + d] / usage;
            if (cb == 0) {
                x[f * 512 + d] = value;
            } else {
                acoustic = cb == 1 ? value : acoustic + value;
            }
        }
        x[f * 512 + 256 + d] = acoustic;
    } else {
        copy_segments_block(seg, segments, blockIdx.x - frames, gridDim.x - frames);
    }
}

__global__ __launch_bounds__(256) void copy_segments_kernel(const CopySegment* seg, int segments) {
    copy_segments_block(seg, segments, blockIdx.x, gridDim.x);
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
__global__ __launch_bounds__(256) void final_conv_pcm_kernel(const float* ext, int positions, const float* w,
                                                             const float* b, int16_t* pcm, float* preclamp,
                                                             float* clamped) {
    __shared__ float ws[96 * 7];
    for (int i = threadIdx.x; i < 96 * 7; i += 256) ws[i] = w[i];
    __syncthreads();
    const int p = blockIdx.x * 256 + threadIdx.x;
    if (p >= positions) return;
    float acc = 0.f;
    for (int c = 0; c < 96; ++c) {
#pragma unroll
        for (int t = 0; t < 7; ++t) acc = fmaf(ext[(size_t)(p + t) * 96 + c], ws[c * 7 + t], acc);
    }
    const float v = acc + b[0];
    if (preclamp) preclamp[p] = v;
    const float c = fminf(1.0f, fmaxf(-1.0f, v));
    if (clamped) clamped[p] = c;
    const float scaled = roundf(c * 32767.0f);
    pcm[p] = (int16_t)fminf(32767.0f, fmaxf(-32768.0f, scaled));
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

__global__ void fill_u32_kernel(unsigned* dst, size_t count, unsigned value) {
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) dst[i] = value;
}

__global__ void fill_f32_kernel(float* dst, size_t count, float value) {
    for (size_t i = blockIdx.x * 256ull + threadIdx.x; i < count; i += (size_t)gridDim.x * 256) dst[i] = value;
}

}  // namespace

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
size_t GemmPlan::partial_floats() const {
    if (splits <= 1) return 0;
    const size_t tile = shape == GemmShape::kSmall ? 16 * 64 : 64 * 64;
    return (size_t)splits * tiles() * tile;
}

GemmPlan plan_conv_gemm(int m, int n, int k, int cus) {
    GemmPlan plan;
    plan.shape = m <= 16 ? GemmShape::kSmall : GemmShape::kLarge;
    const int bm = plan.shape == GemmShape::kSmall ? 16 : 64;
    plan.tiles_m = (m + bm - 1) / bm;
    plan.tiles_n = (n + 63) / 64;
    const int steps = k / 32;
    const long long tiles = (long long)plan.tiles_m * plan.tiles_n;
    // aim for two blocks per CU, each slice keeping at least 4 K-steps
    long long want = (2LL * cus + tiles - 1) / tiles;
    want = std::min<long long>(want, std::max(1, steps / 4));
    plan.splits = (int)std::max<long long>(1, want);
    return plan;
}

hipError_t launch_conv_gemm(const ConvGemmArgs& args, const GemmPlan& plan, hipStream_t stream) {
    if (args.k % 32 || args.channels_in % 32 || args.n % 16 || args.m < 1 || args.splits != plan.splits ||
        (plan.splits > 1 && (!args.partial || !args.counters)))
        return hipErrorInvalidValue;
    const dim3 grid(plan.tiles_n, plan.tiles_m, plan.splits);
    if (plan.shape == GemmShape::kSmall) {
        conv_gemm_kernel<1, 1, 1, 4><<<grid, 256, 0, stream>>>(args);
    } else {
        conv_gemm_kernel<2, 2, 2, 2><<<grid, 256, 0, stream>>>(args);
    }
    return hipGetLastError();
}

hipError_t launch_rows_gemv(const RowsGemvArgs& g, hipStream_t stream) {
    if (g.rows < 1 || g.rows > kMaxRows || g.k % 256 || g.ldx % 4 || g.n < 1) return hipErrorInvalidValue;
    const size_t lds = (size_t)g.rows * g.k * sizeof(float);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    const int cpw = g.n >= 3072 ? 2 : 1;
    const unsigned blocks = (unsigned)((g.n + 4 * cpw - 1) / (4 * cpw));
    if (cpw == 2) {
        rows_gemv_kernel<2><<<blocks, 256, lds, stream>>>(g);
    } else {
        rows_gemv_kernel<1><<<blocks, 256, lds, stream>>>(g);
    }
    return hipGetLastError();
}

hipError_t launch_codec_attention(const float* qkv, int frames, const unsigned long long* position, float* kv_k,
                                  float* kv_v, float* out, hipStream_t stream) {
    if (frames < 1 || frames > kMaxFrames) return hipErrorInvalidValue;
    codec_attention_kernel<<<kHeads, 256, 0, stream>>>(qkv, frames, position, kv_k, kv_v, out);
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
    const int copy_blocks = segments > 0 ? 64 : 0;
    codec_frontend_kernel<<<frames + copy_blocks, 256, 0, stream>>>(codes, frames, t, x, seg, segments);
    return hipGetLastError();
}

hipError_t launch_copy_segments(const CopySegment* seg, int segments, hipStream_t stream) {
    if (segments <= 0) return hipSuccess;
    copy_segments_kernel<<<64, 256, 0, stream>>>(seg, segments);
    return hipGetLastError();
}

hipError_t launch_dwconv_layernorm(const float* ext, int positions, const float* w, const float* b,
                                   const float* ln_w, const float* ln_b, float* out, hipStream_t stream) {
    dwconv_layernorm_kernel<<<positions, 256, 0, stream>>>(ext, w, b, ln_w, ln_b, out);
    return hipGetLastError();
}

hipError_t launch_final_conv_pcm(const float* ext, int positions, const float* w, const float* b, int16_t* pcm,
                                 float* preclamp, float* clamped, hipStream_t stream) {
    final_conv_pcm_kernel<<<(positions + 255) / 256, 256, 0, stream>>>(ext, positions, w, b, pcm, preclamp,
                                                                        clamped);
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

hipError_t launch_fill_u32(unsigned* dst, size_t count, unsigned value, hipStream_t stream) {
    fill_u32_kernel<<<blocks_for(count), 256, 0, stream>>>(dst, count, value);
    return hipGetLastError();
}

hipError_t launch_fill_f32(float* dst, size_t count, float value, hipStream_t stream) {
    fill_f32_kernel<<<blocks_for(count), 256, 0, stream>>>(dst, count, value);
    return hipGetLastError();
}

}  // namespace q3c
