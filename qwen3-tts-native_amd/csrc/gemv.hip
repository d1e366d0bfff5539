// int8 weight-only dequantizing GEMV / skinny GEMM for gfx950.
//
// Semantics follow native/qwen3-tts-native/native/src/int8_gemv.cu:58-293:
//   y[r][c] = scale[c] * sum_k float(W[c][k]) * float(x[r][k])
// with int8 W [out][in] row-major, bf16 x, fp32 accumulation and a per-output
// channel fp32 scale.
//
// Exact mode (rows == 1 by default) reproduces the reference's summation order
// bit-for-bit: every output channel is owned by 32 lanes (half of a wave64);
// lane l owns the 16-byte weight vectors l, l+32, l+64, ...; each vector is a
// fresh 16-term fmaf chain that is added to the lane accumulator, and the 32
// lane sums are folded by shuffle-down with offsets 16, 8, 4, 2, 1.  Because
// the lane -> k mapping does not depend on the channel, each lane keeps its
// slice of x in VGPRs for the whole kernel and the weight stream is the only
// HBM traffic: two half-waves read two 512-byte contiguous segments per
// 128-bit load instruction.  int8 -> fp32 is one SDWA sign-extending convert.
//
// Optional RMSNorm prologue (talker_kernels.cu:27-48 semantics, double bf16
// rounding): every wave recomputes inv_rms from x with the reference's
// 256-thread reduction tree emulated exactly (4 virtual threads per lane),
// then normalizes the x slice it holds.  This removes the separate RMSNorm
// launch and the normalized-activation round trip through memory.
//
// MFMA mode (rows 2..8): weights are dequantized int8 -> bf16 (exact) in
// registers and fed to v_mfma_f32_16x16x32_bf16 with the session rows padded
// to 16; the per-channel scale is applied after accumulation.
#include <type_traits>

#include "gemv_device.hpp"

namespace q3 {
namespace {

using namespace gemv_detail;

// ---------------------------------------------------------------------------
// Exact-order GEMV, one activation row, K = kVpl * 512 known at compile time.
// The grid has one half-wave per unit: one weight row (plain / residual /
// bias epilogues) or the gate row u and the up row out+u (SiLU epilogues).
// Latency order: x (and the RMSNorm gain) is requested first, then the first
// unit's weights and its epilogue operands (scales, residual, bias).  Vector
// memory completes in issue order, so x is staged into LDS, normalized once
// per block (statistic reduced by all 256 threads, each thread normalizing its
// own chunks) and each lane's x slice pulled into registers while the weights
// are still in flight; no memory round trip follows the dot product except the
// output store.
// ---------------------------------------------------------------------------
template <int kVpl, int kEpi, bool kNorm>
__global__ __launch_bounds__(kThreads) void gemv_exact_fixed(GemvArgs a) {
    if (a.input_row_index != nullptr) {
        a.input += static_cast<size_t>(*a.input_row_index) * a.in_features;
    }
    constexpr bool kSilu = (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded);
    constexpr int kRows = kSilu ? 2 : 1;
    constexpr bool kPacked = kVpl > 6;
    constexpr int kIn = kVpl * 512;
    constexpr int kChunks = kIn * 2 / 16;  // 16-byte chunks of one bf16 row
    __shared__ uint4 x_lds[kChunks];
    __shared__ float partial_lds[kNorm ? kThreads : 1];
    const int lane = threadIdx.x & 31;
    const int units = a.out_features;
    const int unit = blockIdx.x * kHalfWaves + (threadIdx.x >> 5);

    // The activation row (and RMSNorm gain) is requested first: vector memory
    // returns in issue order, so it lands while the weights are in flight and
    // the norm statistic is computed under the weight stream.
    constexpr int kPer = (kChunks + kThreads - 1) / kThreads;
    static_assert(kPer <= 3, "x staging holds at most three 16-byte chunks per thread");
    // Clamped rather than guarded (a branch here would make the compiler wait
    // for the whole weight stream before the LDS stores below); named
    // registers rather than an array, which the compiler would place in
    // scratch memory.
    auto chunk = [](int j) { return min(static_cast<int>(threadIdx.x) + j * kThreads, kChunks - 1); };
    const uint4* xin = reinterpret_cast<const uint4*>(a.input);
    const uint4* gin = reinterpret_cast<const uint4*>(a.norm_weight);
    uint4 x0{}, x1{}, x2{}, g0{}, g1{}, g2{};
    x0 = xin[chunk(0)];
    if constexpr (kNorm) g0 = gin[chunk(0)];
    if constexpr (kPer > 1) {
        x1 = xin[chunk(1)];
        if constexpr (kNorm) g1 = gin[chunk(1)];
    }
    if constexpr (kPer > 2) {
        x2 = xin[chunk(2)];
        if constexpr (kNorm) g2 = gin[chunk(2)];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the x loads ahead of the weight loads

    int4 w[kRows][kVpl];
    auto issue = [&](int u) {
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const int row = r == 0 ? u : a.out_features + u;
            const int4* base = reinterpret_cast<const int4*>(a.weight + static_cast<size_t>(row) * kIn);
#pragma unroll
            for (int i = 0; i < kVpl; ++i) w[r][i] = stream_load(base + lane + 32 * i);
        }
    };
    // Unconditional (clamped) so the x loads' wait is not merged with a path
    // that skipped the weight loads: half-waves past the end read the last
    // unit and discard it.
    const int first = unit < units ? unit : units - 1;
    issue(first);
    const EpiInputs epi = prefetch_epi<kEpi>(a, first);
    __builtin_amdgcn_sched_barrier(0);  // and the LDS stores of x behind them

    auto stage = [&](int j, const uint4& xv) {
        const int c = static_cast<int>(threadIdx.x) + j * kThreads;
        if (kChunks % kThreads == 0 || c < kChunks) x_lds[c] = xv;
    };
    stage(0, x0);
    if constexpr (kPer > 1) stage(1, x1);
    if constexpr (kPer > 2) stage(2, x2);
    __syncthreads();
    const bf16_t* xs = reinterpret_cast<const bf16_t*>(x_lds);
    if constexpr (kNorm) {
        // The block normalizes x once, in place: each thread its own chunks
        // from registers, after the statistic has been reduced.
        partial_lds[threadIdx.x] = block_partial_sq<kIn>(xs);
        __syncthreads();
        const float inverse = fold_partials256(partial_lds, kIn, a.norm_epsilon);
        stage(0, normalize_chunk(x0, g0, inverse));
        if constexpr (kPer > 1) stage(1, normalize_chunk(x1, g1, inverse));
        if constexpr (kPer > 2) stage(2, normalize_chunk(x2, g2, inverse));
        __syncthreads();
    }
    // Activation slice of this lane: vectors lane + 32*i.
    float xf[kPacked ? 1 : kVpl][16];
    uint32_t xp[kPacked ? kVpl : 1][8];
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
        float tmp[16];
        load_x16<false>(xs, nullptr, lane + 32 * i, 1.0f, tmp);
        if constexpr (kPacked) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xp[i][j] = (__float_as_uint(tmp[2 * j]) >> 16) |
                           (__float_as_uint(tmp[2 * j + 1]) & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) xf[i][j] = tmp[j];
        }
    }

    // One unit per half-wave (the grid covers every unit): no loop, so the
    // first weight vectors are consumed as soon as they land.
    float acc[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < kVpl; ++i) {
            if constexpr (kPacked) {
                acc[r] += chain16_packed(w[r][i], xp[i]);
            } else {
                acc[r] += chain16(w[r][i], xf[i]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < kRows; ++r) acc[r] = fold32(acc[r]);
    if (lane == 0 && unit < units) {
        if constexpr (kSilu) {
            finish_gate_up<kEpi>(a, unit, acc[0], acc[kRows - 1], epi);
        } else {
            finish_channel<kEpi>(a, unit, acc[0], epi);
        }
    }
}

// ---------------------------------------------------------------------------
// Exact-order rows without the RMSNorm prologue -- 2..8 (exact batched mode)
// or a whole prompt's (its text projection) -- K = 512 * kVpl known at
// compile time: the
// batch-1 kernel's layout -- one unit per half-wave, its weights (the lane's
// vectors lane + 32 i) requested first and held in registers -- against every
// input row, staged once per block in LDS.  Per row the sum is the generic
// kernel's: acc += chain16(vector i) for i in order, then fold32.
// ---------------------------------------------------------------------------
template <int kVpl, int kEpi>
__global__ __launch_bounds__(kThreads) void gemv_exact_rows_fixed(GemvArgs a) {
    constexpr bool kSilu = (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded);
    constexpr int kTiles = kSilu ? 2 : 1;
    constexpr int kIn = kVpl * 512;
    constexpr int kChunks = kIn * 2 / 16;  // 16-byte chunks of one bf16 row
    extern __shared__ __align__(16) uint4 rows_lds[];  // [rows][kChunks]
    const int lane = threadIdx.x & 31;
    const int rows = a.rows;
    const int units = a.out_features;
    const int unit = blockIdx.x * kHalfWaves + (threadIdx.x >> 5);
    const int first = unit < units ? unit : units - 1;  // clamped: see gemv_exact_fixed
    int4 w[kTiles][kVpl];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
        const int row = t == 0 ? first : a.out_features + first;
        const int4* base = reinterpret_cast<const int4*>(a.weight + static_cast<size_t>(row) * kIn);
#pragma unroll
        for (int i = 0; i < kVpl; ++i) w[t][i] = stream_load(base + lane + 32 * i);
    }
    __builtin_amdgcn_sched_barrier(0);  // the weight stream first, then the rows
    const uint4* xin = reinterpret_cast<const uint4*>(a.input);
    // rows in chunks of up to 8 through LDS (more than 8 only for a prompt's
    // rows: the weights stay in registers for all of them)
    // gridDim.y groups of rows (a long prompt's rows over more workgroups)
    const int per_group = (rows + gridDim.y - 1) / gridDim.y;
    const int r_end = min(rows, static_cast<int>(blockIdx.y + 1) * per_group);
    for (int r0 = blockIdx.y * per_group; r0 < r_end; r0 += 8) {
        const int count = min(8, r_end - r0);
        if (r0 > 0) __syncthreads();  // the previous chunk is read
        for (int c = threadIdx.x; c < count * kChunks; c += kThreads) {
            rows_lds[c] = xin[static_cast<size_t>(r0) * kChunks + c];
        }
        __syncthreads();
        for (int rr = 0; rr < count; ++rr) {
            const int r = r0 + rr;
            const bf16_t* xs = reinterpret_cast<const bf16_t*>(rows_lds + rr * kChunks);
            float acc[kTiles];
#pragma unroll
            for (int t = 0; t < kTiles; ++t) acc[t] = 0.0f;
#pragma unroll
            for (int i = 0; i < kVpl; ++i) {
                float xv[16];
                load_x16<false>(xs, nullptr, lane + 32 * i, 1.0f, xv);
#pragma unroll
                for (int t = 0; t < kTiles; ++t) acc[t] += chain16(w[t][i], xv);
            }
#pragma unroll
            for (int t = 0; t < kTiles; ++t) acc[t] = fold32(acc[t]);
            if (lane == 0 && unit < units) {
                GemvArgs row = a;
                row.out16 = a.out16 ? a.out16 + static_cast<size_t>(r) * a.out_features : nullptr;
                row.out32 = a.out32 ? a.out32 + static_cast<size_t>(r) * a.out_features : nullptr;
                if constexpr (kSilu) {
                    store_gate_up<kEpi>(row, unit, acc[0], acc[kTiles - 1]);
                } else {
                    store_channel<kEpi>(row, unit, acc[0]);
                }
            }
        }
    }
}

template <int kVpl, int kEpi>
hipError_t launch_exact_rows_fixed(const GemvArgs& a, hipStream_t s) {
    constexpr int kIn = kVpl * 512;
    static std::atomic<unsigned long long> configured{0};
    const hipError_t st = set_dynamic_lds_once(configured, reinterpret_cast<const void*>(gemv_exact_rows_fixed<kVpl, kEpi>),
                                               static_cast<int>(8 * kIn * sizeof(bf16_t)));
    if (st != hipSuccess) return st;
    const size_t lds = static_cast<size_t>(std::min(a.rows, 8)) * kIn * sizeof(bf16_t);
    // more than 8 rows: up to 4 groups of rows on their own workgroups, each
    // reading the weights again (measured: one workgroup per CU leaves the
    // per-row arithmetic's latency exposed)
    const int groups = std::min(4, (a.rows + 7) / 8);
    const dim3 grid((a.out_features + kHalfWaves - 1) / kHalfWaves, groups);
    gemv_exact_rows_fixed<kVpl, kEpi><<<grid, kThreads, lds, s>>>(a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Exact-order GEMV/GEMM for any in_features % 16 == 0 and rows 1..8.  The
// activation vectors are re-read per weight vector (they stay in L1/L2).
// ---------------------------------------------------------------------------
template <int kRows, int kEpi, bool kNorm>
__global__ __launch_bounds__(kThreads) void gemv_exact_generic(GemvArgs a) {
    if (a.input_row_index != nullptr) {
        a.input += static_cast<size_t>(*a.input_row_index) * a.in_features;
    }
    constexpr bool kSilu = (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded);
    const int lane = threadIdx.x & 31;
    const int in = a.in_features;
    const int vectors = in / 16;
    float inverse[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) {
        inverse[r] = 1.0f;
        if constexpr (kNorm) {
            inverse[r] = wave_inverse_rms(a.input + static_cast<size_t>(r) * in, in,
                                          a.norm_epsilon);
        }
    }
    const int units = kSilu ? a.out_features : a.out_features;
    const int stride = gridDim.x * kHalfWaves;
    for (int unit = blockIdx.x * kHalfWaves + (threadIdx.x >> 5); unit < units; unit += stride) {
        const int row0 = unit;
        const int row1 = kSilu ? a.out_features + unit : unit;
        const int4* w0 = reinterpret_cast<const int4*>(a.weight + static_cast<size_t>(row0) * in);
        const int4* w1 = reinterpret_cast<const int4*>(a.weight + static_cast<size_t>(row1) * in);
        float acc0[kRows];
        float acc1[kRows];
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            acc0[r] = 0.0f;
            acc1[r] = 0.0f;
        }
        for (int v = lane; v < vectors; v += 32) {
            const int4 q0 = stream_load(w0 + v);
            int4 q1 = q0;
            if constexpr (kSilu) q1 = stream_load(w1 + v);
#pragma unroll
            for (int r = 0; r < kRows; ++r) {
                float xv[16];
                load_x16<kNorm>(a.input + static_cast<size_t>(r) * in, a.norm_weight, v,
                                inverse[r], xv);
                acc0[r] += chain16(q0, xv);
                if constexpr (kSilu) acc1[r] += chain16(q1, xv);
            }
        }
#pragma unroll
        for (int r = 0; r < kRows; ++r) {
            const float g = fold32(acc0[r]);
            float u = 0.0f;
            if constexpr (kSilu) u = fold32(acc1[r]);
            if (lane == 0) {
                GemvArgs row = a;
                row.out16 = a.out16 ? a.out16 + static_cast<size_t>(r) * a.out_features : nullptr;
                row.out32 = a.out32 ? a.out32 + static_cast<size_t>(r) * a.out_features : nullptr;
                if constexpr (kSilu) {
                    store_gate_up<kEpi>(row, unit, g, u);
                } else {
                    store_channel<kEpi>(row, unit, g);
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// MFMA skinny GEMM for rows 2..8 (rows padded to 16 columns of B).
//   A (16 x 32): lane i holds W[c0 + i%16][k-group i/16]   (int8 -> bf16)
//   B (32 x 16): lane i holds x[i%16][k-group i/16]         (zero if i%16 >= rows)
//   D (16 x 16): lane i holds D[4*(i/16) + j][i%16], j < 4
// Each lane streams 16 contiguous weight bytes per step; bytes 0-7 feed the
// first MFMA and bytes 8-15 the second, with the matching activations on the
// B side, so every product pairs the right (W, x) elements.
// A block owns 16 channels (two rows for SiLU: gate tile + up tile); its four
// waves split K and fold their partial tiles through LDS.
// ---------------------------------------------------------------------------
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// int8 -> bf16 is exact; per byte one sign-extending convert to fp32 and half
// a packed fp32 -> bf16 convert (v_cvt_pk_bf16_f32 on gfx950).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ bf16x8_t bytes_to_bf16x8(uint32_t lo, uint32_t hi) {
    union {
        uint32_t u[4];
        bf16x8_t v;
    } r;
    const uint32_t w[2] = {lo, hi};
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t word = w[p >> 1];
        const int shift = 16 * (p & 1);
        const float f0 = static_cast<float>(static_cast<int>(static_cast<int8_t>((word >> shift) & 0xffu)));
        const float f1 = static_cast<float>(static_cast<int>(static_cast<int8_t>((word >> (shift + 8)) & 0xffu)));
        const bf16x2_t pair = {static_cast<__bf16>(f0), static_cast<__bf16>(f1)};
        r.u[p] = __builtin_bit_cast(uint32_t, pair);
    }
    return r.v;
}

__device__ __forceinline__ bf16x8_t load_bf16x8(const bf16_t* p) {
    union {
        uint4 q;
        bf16x8_t v;
    } r;
    r.q = *reinterpret_cast<const uint4*>(p);
    return r.v;
}

template <int kEpi, bool kNorm>
__global__ __launch_bounds__(kThreads) void gemv_mfma(GemvArgs a) {
    if (a.input_row_index != nullptr) {
        a.input += static_cast<size_t>(*a.input_row_index) * a.in_features;
    }
    constexpr bool kSilu = (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded);
    constexpr int kTiles = kSilu ? 2 : 1;
    __shared__ float fold[4][kTiles][16][16];
    __shared__ bf16_t xs_norm[kNorm ? 8 : 1][kNorm ? 6144 : 1];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int in = a.in_features;
    const int rows = a.rows;
    const int c0 = blockIdx.x * 16;
    const bf16_t* x = a.input;
    int x_stride = in;
    if constexpr (kNorm) {
        // Normalized rows staged once in LDS (in <= 6144 checked on launch).
        for (int r = wave; r < rows; r += 4) {
            const bf16_t* xr = a.input + static_cast<size_t>(r) * in;
            const float inverse = wave_inverse_rms(xr, in, a.norm_epsilon);
            for (int k = lane; k < in; k += 64) {
                xs_norm[r][k] = f2bf(normalize_one(bf2f(xr[k]), inverse, bf2f(a.norm_weight[k])));
            }
        }
        __syncthreads();
        x = &xs_norm[0][0];
        x_stride = 6144;
    }
    const int m = lane & 15;
    const int group = lane >> 4;
    const bool real_col = m < rows;
    floatx4_t acc[kTiles];
#pragma unroll
    for (int t = 0; t < kTiles; ++t) acc[t] = floatx4_t{0.f, 0.f, 0.f, 0.f};
    const int slice = in / 4;  // in % 256 == 0 checked on launch
    const int k_begin = wave * slice;
    const int k_end = k_begin + slice;
    const int channel = c0 + m;
    const bool valid_channel = channel < a.out_features;
    const int8_t* wrow[kTiles];
    wrow[0] = a.weight + static_cast<size_t>(valid_channel ? channel : 0) * in;
    if constexpr (kSilu) {
        wrow[kTiles - 1] =
            a.weight + static_cast<size_t>(a.out_features + (valid_channel ? channel : 0)) * in;
    }
    for (int k = k_begin + 16 * group; k < k_end; k += 64) {
        int4 wq[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            wq[t] = stream_load(wrow[t] + k);
        }
        bf16x8_t b0 = {};
        bf16x8_t b1 = {};
        if (real_col) {
            b0 = load_bf16x8(x + static_cast<size_t>(m) * x_stride + k);
            b1 = load_bf16x8(x + static_cast<size_t>(m) * x_stride + k + 8);
        }
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            const bf16x8_t a0 = bytes_to_bf16x8(static_cast<uint32_t>(wq[t].x), static_cast<uint32_t>(wq[t].y));
            const bf16x8_t a1 = bytes_to_bf16x8(static_cast<uint32_t>(wq[t].z), static_cast<uint32_t>(wq[t].w));
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc[t], 0, 0, 0);
            acc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[t], 0, 0, 0);
        }
    }
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            fold[wave][t][4 * group + j][m] = acc[t][j];  // [channel row][session col]
        }
    }
    __syncthreads();
    // 256 threads: thread -> (channel row, session col) of the 16x16 tile.
    const int row = threadIdx.x >> 4;
    const int col = threadIdx.x & 15;
    const int ch = c0 + row;
    if (col < rows && ch < a.out_features) {
        float value[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            value[t] = ((fold[0][t][row][col] + fold[1][t][row][col]) + fold[2][t][row][col]) +
                       fold[3][t][row][col];
        }
        GemvArgs r = a;
        r.out16 = a.out16 ? a.out16 + static_cast<size_t>(col) * a.out_features : nullptr;
        r.out32 = a.out32 ? a.out32 + static_cast<size_t>(col) * a.out_features : nullptr;
        if constexpr (kSilu) {
            store_gate_up<kEpi>(r, ch, value[0], value[kTiles - 1]);
        } else {
            store_channel<kEpi>(r, ch, value[0]);
        }
    }
}

// ---------------------------------------------------------------------------
// Batched rows (2..8 sessions) on MFMA, K = 64 * kWaves * kIters known at
// compile time.  A block owns kGroups groups of 8 output channels (as many
// gate and up rows for the SiLU epilogues); its 4 or 8 waves split K.
// Latency order: the session rows are requested first; then every weight
// vector of the wave's K slice, loaded straight in the
// v_mfma_f32_16x16x32_bf16 A operand layout and held in registers; the
// epilogue operands.  The rows are staged in LDS (and normalized there with
// the RMSNorm prologue: statistic per row by one wave with the reference's
// 256-thread tree) as the MFMA B operands, once per block for all of its
// groups: more groups per block, fewer blocks repeating that work (the
// launcher sizes the grid to one block per CU where the channel count allows).
// ---------------------------------------------------------------------------
template <int kIters, int kWaves, int kEpi, bool kNorm, int kGroups>
__global__ __launch_bounds__(64 * kWaves) void gemv_mfma_fixed(GemvArgs a) {
    constexpr int kBlock = 64 * kWaves;
    if (a.input_row_index != nullptr) {
        a.input += static_cast<size_t>(*a.input_row_index) * a.in_features;
    }
    constexpr bool kSilu = (kEpi == kEpiSiluFused || kEpi == kEpiSiluRounded);
    constexpr int kTiles = kSilu ? 2 : 1;
    constexpr int kIn = 64 * kWaves * kIters;
    constexpr int kStride = kIn + 8;  // bf16 elements per LDS row (16-byte pad)
    extern __shared__ __align__(16) bf16_t xs[];  // [rows][kStride]
    __shared__ float fold[kWaves][kTiles][kGroups][16][16];
    __shared__ float inverse_lds[8];
    __shared__ __align__(16) float statistic[kNorm ? 8 : 1][256];
    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int rows = a.rows;
    // Each group's 16x16 tile is used block-diagonally: A rows m and B
    // columns m take channel / session m % 8 over the k in the first (m < 8)
    // or second (m >= 8) 64 bytes of each 128-byte piece of the row, so
    // C[c][s] + C[c + 8][s + 8] is the sum over all of K with every weight
    // byte consumed once.  A wave's load instruction then covers 8 rows x 128
    // contiguous bytes -- whole cache lines -- where a 16-channel tile would
    // read 16 rows x 64 bytes (measured on MI355X at N = 8: gate/up
    // 12288x2048 8.1 -> 6.8 us with the rest of the kernel stripped).
    static_assert(kGroups >= 1 && kGroups <= 3, "one to three groups of 8 channels");
    static_assert(kIters % 2 == 0, "whole 128-byte pieces per wave");
    constexpr int kCh = 8 * kGroups;      // channels per block
    constexpr int kSteps = kIters / 2;    // load instructions per wave, tile and group
    const int c0 = blockIdx.x * kCh;
    const int m = lane & 15;
    const int group = lane >> 4;
    // k of this lane's 16 bytes in load step i (weights and activations alike)
    auto lane_k = [&](int i) { return wave * (kIn / kWaves) + 128 * i + 64 * (m / 8) + 16 * group; };
    constexpr int kChunks = kIn / 8;  // 16-byte chunks per row

    // 0. With the RMSNorm prologue the session rows are needed before any
    //    MFMA: request them ahead of the weights (memory returns in order).
    // The session rows (up to 8 of them) are requested ahead of the weights
    // (memory returns in order) and staged in LDS as the MFMA B operands.
    // With the RMSNorm prologue on a 256-thread block, lane l of wave w holds
    // row w + 4 (l / 32) at chunks l % 32 + 32 j (so few rows still spread
    // over the waves): its elements are exactly those of eight
    // of the reference's 256 statistic threads (elements i = v, v + 256, ...),
    // so the statistic's partial sums come straight from registers.
    constexpr bool kRowSplit = kNorm && kBlock == 256 && kChunks % 32 == 0 && kChunks / 32 <= 8;
    constexpr int kXPer = kRowSplit ? kChunks / 32 : (8 * kChunks + kBlock - 1) / kBlock;
    static_assert(kXPer <= 12, "x staging holds at most 12 chunks per thread");
    // Row-split layout: wave w holds rows w and w + 4 (lanes 0-31 and 32-63),
    // which the statistic fold below relies on (it has no block barrier).
    static_assert(!kRowSplit || kWaves == 4, "the row-split layout maps rows w and w + 4 to wave w of four");
    auto split_row = [] { return static_cast<int>(threadIdx.x >> 6) + static_cast<int>((threadIdx.x >> 3) & 4); };
    auto x_slot = [&](int j, int& r, int& c) {
        if constexpr (kRowSplit) {
            r = split_row();
            c = (threadIdx.x & 31) + 32 * j;
        } else {
            const int idx = threadIdx.x + j * kBlock;
            r = idx / kChunks;
            c = idx % kChunks;
        }
    };
    // named registers, not an array (an array here is placed in scratch)
    uint4 x0{}, x1{}, x2{}, x3{}, x4{}, x5{}, x6{}, x7{}, x8{}, x9{}, x10{}, x11{};
    // Chunk j of this thread is row (tid + j*block) / kChunks; threads past
    // the last row load nothing (a masked load issues no request).
    auto x_load = [&](int j) {
        int r, c;
        x_slot(j, r, c);
        uint4 v{};
        if (r < rows) v = *reinterpret_cast<const uint4*>(a.input + static_cast<size_t>(r) * kIn + 8 * c);
        return v;
    };
    if constexpr (kXPer > 0) x0 = x_load(0);
    if constexpr (kXPer > 1) x1 = x_load(1);
    if constexpr (kXPer > 2) x2 = x_load(2);
    if constexpr (kXPer > 3) x3 = x_load(3);
    if constexpr (kXPer > 4) x4 = x_load(4);
    if constexpr (kXPer > 5) x5 = x_load(5);
    if constexpr (kXPer > 6) x6 = x_load(6);
    if constexpr (kXPer > 7) x7 = x_load(7);
    if constexpr (kXPer > 8) x8 = x_load(8);
    if constexpr (kXPer > 9) x9 = x_load(9);
    if constexpr (kXPer > 10) x10 = x_load(10);
    if constexpr (kXPer > 11) x11 = x_load(11);
    // When kChunks divides the block, all of a thread's chunks share the
    // column c = tid % kChunks: one RMSNorm gain chunk, requested early too.
    constexpr bool kOneGain = kNorm && !kRowSplit && kBlock % kChunks == 0;
    uint4 gain_chunk{};
    if constexpr (kOneGain) gain_chunk = reinterpret_cast<const uint4*>(a.norm_weight)[threadIdx.x % kChunks];
    // row-split layout: the gain chunks of this thread's columns
    uint4 g0{}, g1{}, g2{}, g3{}, g4{}, g5{}, g6{}, g7{};
    if constexpr (kRowSplit) {
        const uint4* gain = reinterpret_cast<const uint4*>(a.norm_weight) + (threadIdx.x & 31);
        g0 = gain[0];
        if constexpr (kXPer > 1) g1 = gain[32];
        if constexpr (kXPer > 2) g2 = gain[64];
        if constexpr (kXPer > 3) g3 = gain[96];
        if constexpr (kXPer > 4) g4 = gain[128];
        if constexpr (kXPer > 5) g5 = gain[160];
        if constexpr (kXPer > 6) g6 = gain[192];
        if constexpr (kXPer > 7) g7 = gain[224];
    }
    __builtin_amdgcn_sched_barrier(0);

    // 1. weights of this wave's K slice, loaded straight in the MFMA operand
    //    layout: lane (m, g) takes 16 bytes of channel row m % kCh at
    //    lane_k(i), which feed two MFMAs (bytes 0-7 and 8-15; the activations
    //    use the same k order, so the sum covers every k once).
    //    Issued in the order the MFMA loop consumes them (memory returns in
    //    order), so the conversions and MFMAs of the first steps run while the
    //    later weights are still streaming in.
    int4 wq[kTiles][kGroups][kSteps];
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
#pragma unroll
            for (int q = 0; q < kGroups; ++q) {
                const int ch = c0 + 8 * q + m % 8;
                const int row = (t == 0 ? 0 : a.out_features) + (ch < a.out_features ? ch : 0);
                const int8_t* src = a.weight + static_cast<size_t>(row) * kIn + lane_k(i);
                wq[t][q][i] = stream_load(reinterpret_cast<const int4*>(src));
            }
        }
    }
    // epilogue operands of this thread's (channel, session) output
    static_assert(kCh <= kBlock / 8, "one thread per (channel, session) output");
    const int out_row = threadIdx.x >> 3;
    const int out_col = threadIdx.x & 7;
    const int out_ch = c0 + out_row;
    const bool writes = out_row < kCh && out_col < rows && out_ch < a.out_features;
    GemvArgs out_args = a;
    out_args.out16 = a.out16 ? a.out16 + static_cast<size_t>(writes ? out_col : 0) * a.out_features : nullptr;
    out_args.out32 = a.out32 ? a.out32 + static_cast<size_t>(writes ? out_col : 0) * a.out_features : nullptr;
    const EpiInputs epi = prefetch_epi<kEpi>(out_args, writes ? out_ch : 0);
    __builtin_amdgcn_sched_barrier(0);

    // 2. session rows into LDS
    auto x_store = [&](int j, const uint4& v) {
        int r, c;
        x_slot(j, r, c);
        if (r < rows) *reinterpret_cast<uint4*>(xs + r * kStride + 8 * c) = v;
    };
    if constexpr (kRowSplit) {
        // Statistic partials of the reference's threads v = 8 (t % 32) + e,
        // e = 0..7 (one fma chain over the thread's chunks in order), folded
        // per row in the reference's tree order by the wave that holds the
        // row; then each thread normalizes its chunks from registers.
        const int r = split_row();
        if (r < rows) {
            float part[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
            auto accumulate = [&](const uint4& v) {
                const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float lo = __uint_as_float(w[i] << 16), hi = __uint_as_float(w[i] & 0xffff0000u);
                    part[2 * i] = fmaf(lo, lo, part[2 * i]);
                    part[2 * i + 1] = fmaf(hi, hi, part[2 * i + 1]);
                }
            };
            accumulate(x0);
            if constexpr (kXPer > 1) accumulate(x1);
            if constexpr (kXPer > 2) accumulate(x2);
            if constexpr (kXPer > 3) accumulate(x3);
            if constexpr (kXPer > 4) accumulate(x4);
            if constexpr (kXPer > 5) accumulate(x5);
            if constexpr (kXPer > 6) accumulate(x6);
            if constexpr (kXPer > 7) accumulate(x7);
            float4* dst = reinterpret_cast<float4*>(&statistic[r][8 * (threadIdx.x & 31)]);
            dst[0] = make_float4(part[0], part[1], part[2], part[3]);
            dst[1] = make_float4(part[4], part[5], part[6], part[7]);
        }
        // rows w and w + 4 are held and folded by wave w alone: its LDS
        // accesses complete in order, so no block barrier is needed here
        __builtin_amdgcn_wave_barrier();
        if (wave < rows) {
            const float inverse_lo = fold_partials256(statistic[wave], kIn, a.norm_epsilon);
            const float inverse_hi = wave + 4 < rows ? fold_partials256(statistic[wave + 4], kIn, a.norm_epsilon) : 0.0f;
            const float inverse = lane < 32 ? inverse_lo : inverse_hi;
            x_store(0, normalize_chunk_hw(x0, g0, inverse));
            if constexpr (kXPer > 1) x_store(1, normalize_chunk_hw(x1, g1, inverse));
            if constexpr (kXPer > 2) x_store(2, normalize_chunk_hw(x2, g2, inverse));
            if constexpr (kXPer > 3) x_store(3, normalize_chunk_hw(x3, g3, inverse));
            if constexpr (kXPer > 4) x_store(4, normalize_chunk_hw(x4, g4, inverse));
            if constexpr (kXPer > 5) x_store(5, normalize_chunk_hw(x5, g5, inverse));
            if constexpr (kXPer > 6) x_store(6, normalize_chunk_hw(x6, g6, inverse));
            if constexpr (kXPer > 7) x_store(7, normalize_chunk_hw(x7, g7, inverse));
        }
        __syncthreads();
    } else {
        if constexpr (kXPer > 0) x_store(0, x0);
        if constexpr (kXPer > 1) x_store(1, x1);
        if constexpr (kXPer > 2) x_store(2, x2);
        if constexpr (kXPer > 3) x_store(3, x3);
        if constexpr (kXPer > 4) x_store(4, x4);
        if constexpr (kXPer > 5) x_store(5, x5);
        if constexpr (kXPer > 6) x_store(6, x6);
        if constexpr (kXPer > 7) x_store(7, x7);
        if constexpr (kXPer > 8) x_store(8, x8);
        if constexpr (kXPer > 9) x_store(9, x9);
        if constexpr (kXPer > 10) x_store(10, x10);
        if constexpr (kXPer > 11) x_store(11, x11);
        __syncthreads();
    }
    if constexpr (kNorm && !kRowSplit) {
        for (int r = wave; r < rows; r += kWaves) {
            const float inverse = wave_inverse_rms(xs + r * kStride, kIn, a.norm_epsilon);
            if (lane == 0) inverse_lds[r] = inverse;
        }
        __syncthreads();
        for (int idx = threadIdx.x; idx < rows * kChunks; idx += kBlock) {
            const int r = idx / kChunks;
            const int c = idx % kChunks;
            uint4* p = reinterpret_cast<uint4*>(xs + r * kStride + 8 * c);
            const uint4 g = kOneGain ? gain_chunk : reinterpret_cast<const uint4*>(a.norm_weight)[c];
            *p = normalize_chunk_hw(*p, g, inverse_lds[r]);
        }
        __syncthreads();
    }

    // 3. MFMAs: columns m % 8 < rows are sessions, the rest zero
    const bool real_col = m % 8 < rows;
    const bf16_t* xrow = xs + (real_col ? m % 8 : 0) * kStride;
    floatx4_t acc[kTiles][kGroups];
#pragma unroll
    for (int t = 0; t < kTiles; ++t)
#pragma unroll
        for (int q = 0; q < kGroups; ++q) acc[t][q] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < kSteps; ++i) {
        const int k = lane_k(i);
        bf16x8_t b0 = {}, b1 = {};
        if (real_col) {
            b0 = load_bf16x8(xrow + k);
            b1 = load_bf16x8(xrow + k + 8);
        }
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
#pragma unroll
            for (int q = 0; q < kGroups; ++q) {
                const int4 w = wq[t][q][i];
                const bf16x8_t a0 = bytes_to_bf16x8(static_cast<uint32_t>(w.x), static_cast<uint32_t>(w.y));
                const bf16x8_t a1 = bytes_to_bf16x8(static_cast<uint32_t>(w.z), static_cast<uint32_t>(w.w));
                acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, b0, acc[t][q], 0, 0, 0);
                acc[t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, b1, acc[t][q], 0, 0, 0);
            }
        }
    }
#pragma unroll
    for (int t = 0; t < kTiles; ++t) {
#pragma unroll
        for (int q = 0; q < kGroups; ++q) {
#pragma unroll
            for (int j = 0; j < 4; ++j) fold[wave][t][q][4 * group + j][m] = acc[t][q][j];  // [channel][session]
        }
    }
    __syncthreads();
    if (writes) {
        const int q = out_row / 8;
        const int r = out_row % 8;
        float value[kTiles];
#pragma unroll
        for (int t = 0; t < kTiles; ++t) {
            float v = fold[0][t][q][r][out_col];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) v += fold[w][t][q][r][out_col];
#pragma unroll
            for (int w = 0; w < kWaves; ++w) v += fold[w][t][q][r + 8][out_col + 8];
            value[t] = v;
        }
        if constexpr (kSilu) {
            finish_gate_up<kEpi>(out_args, out_ch, value[0], value[kTiles - 1], epi);
        } else {
            finish_channel<kEpi>(out_args, out_ch, value[0], epi);
        }
    }
}

template <int kIters, int kWaves, int kEpi, bool kNorm, int kGroups>
hipError_t launch_mfma_fixed(const GemvArgs& a, hipStream_t s) {
    constexpr int kIn = 64 * kWaves * kIters;
    constexpr int kCh = 8 * kGroups;
    const size_t lds = static_cast<size_t>(a.rows) * (kIn + 8) * sizeof(bf16_t);
    static std::atomic<unsigned long long> configured{0};
    const hipError_t st = set_dynamic_lds_once(
        configured, reinterpret_cast<const void*>(gemv_mfma_fixed<kIters, kWaves, kEpi, kNorm, kGroups>),
        static_cast<int>(8 * (kIn + 8) * sizeof(bf16_t)));
    if (st != hipSuccess) return st;
    gemv_mfma_fixed<kIters, kWaves, kEpi, kNorm, kGroups><<<(a.out_features + kCh - 1) / kCh, 64 * kWaves, lds, s>>>(a);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-row symmetric quantizer (int8_gemv.cu:20-52): absmax -> scale ->
// lrint(clamp(w / scale)).  One 256-thread block per output row.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(kThreads) void quantize_rows_kernel(const bf16_t* weight,
                                                                 int8_t* quantized, float* scales,
                                                                 int in_features) {
    __shared__ float partial[kThreads];
    const size_t offset = static_cast<size_t>(blockIdx.x) * in_features;
    const bf16_t* row = weight + offset;
    float maximum = 0.0f;
    for (int i = threadIdx.x; i < in_features; i += kThreads) {
        maximum = fmaxf(maximum, fabsf(bf2f(row[i])));
    }
    partial[threadIdx.x] = maximum;
    __syncthreads();
    for (int s = kThreads / 2; s > 0; s >>= 1) {
        if (threadIdx.x < s) partial[threadIdx.x] = fmaxf(partial[threadIdx.x], partial[threadIdx.x + s]);
        __syncthreads();
    }
    const float scale = partial[0] > 0.0f ? partial[0] / 127.0f : 1.0f;
    const float inverse = 1.0f / scale;
    if (threadIdx.x == 0) scales[blockIdx.x] = scale;
    int8_t* out = quantized + offset;
    for (int i = threadIdx.x; i < in_features; i += kThreads) {
        const float clamped = fminf(fmaxf(bf2f(row[i]) * inverse, -127.0f), 127.0f);
        out[i] = static_cast<int8_t>(__float2int_rn(clamped));
    }
}

// ---------------------------------------------------------------------------
// Dispatch
// ---------------------------------------------------------------------------
int device_cu_count() {
    static int count = [] {
        int device = 0;
        hipDeviceProp_t props{};
        if (hipGetDevice(&device) != hipSuccess || hipGetDeviceProperties(&props, device) != hipSuccess) {
            return 256;
        }
        return props.multiProcessorCount > 0 ? props.multiProcessorCount : 256;
    }();
    return count;
}

template <int kEpi, bool kNorm>
hipError_t dispatch_fixed(const GemvArgs& a, int vpl, int grid, hipStream_t s) {
    switch (vpl) {
        case 2: gemv_exact_fixed<2, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 4: gemv_exact_fixed<4, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 6: gemv_exact_fixed<6, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 12: gemv_exact_fixed<12, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int kEpi, bool kNorm>
hipError_t dispatch_generic(const GemvArgs& a, int grid, hipStream_t s) {
    switch (a.rows) {
        case 1: gemv_exact_generic<1, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 2: gemv_exact_generic<2, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 3: gemv_exact_generic<3, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 4: gemv_exact_generic<4, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 5: gemv_exact_generic<5, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 6: gemv_exact_generic<6, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 7: gemv_exact_generic<7, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        case 8: gemv_exact_generic<8, kEpi, kNorm><<<grid, kThreads, 0, s>>>(a); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int kEpi, bool kNorm>
hipError_t dispatch(const GemvArgs& a, hipStream_t s) {
    const bool mfma = a.mode == kModeMfma || (a.mode == kModeAuto && a.rows >= 2);
    if (mfma) {
        if (a.in_features % 256 != 0 || (kNorm && a.in_features > 6144)) {
            return hipErrorInvalidValue;
        }
        // Groups of 8 channels per block: as many as still leave a block for
        // three CUs in four (each block stages -- and with the RMSNorm
        // prologue normalizes -- all session rows once for its groups;
        // measured on MI355X at N = 8: talker gate/up 10.2 -> 9.2 us with 3
        // groups, QKV 6.5 -> 4.8 us and predictor gate/up 5.6 -> 5.0 us with 2).
        const int groups = (a.out_features + 7) / 8;
        const int floor_blocks = device_cu_count() * 3 / 4;
        const int per = a.out_features % 8 != 0 ? 1 : groups % 3 == 0 && groups / 3 >= floor_blocks ? 3
                                                    : groups % 2 == 0 && groups / 2 >= floor_blocks ? 2 : 1;
        auto launch = [&](auto iters, auto waves) {
            constexpr int kI = decltype(iters)::value, kW = decltype(waves)::value;
            return per == 3 ? launch_mfma_fixed<kI, kW, kEpi, kNorm, 3>(a, s)
                 : per == 2 ? launch_mfma_fixed<kI, kW, kEpi, kNorm, 2>(a, s)
                            : launch_mfma_fixed<kI, kW, kEpi, kNorm, 1>(a, s);
        };
        using I4 = std::integral_constant<int, 4>;
        using W4 = std::integral_constant<int, 4>;
        using W8 = std::integral_constant<int, 8>;
        switch (a.in_features) {
            // kIters = K / (64 * waves); 8 waves where K is long
            case 1024: return launch(I4{}, W4{});
            case 2048: return launch(std::integral_constant<int, 8>{}, W4{});
            case 3072: return launch(std::integral_constant<int, 6>{}, W8{});
            case 6144: return launch(std::integral_constant<int, 12>{}, W8{});
            default: break;
        }
        const int grid = (a.out_features + 15) / 16;
        gemv_mfma<kEpi, kNorm><<<grid, kThreads, 0, s>>>(a);
        return hipGetLastError();
    }
    if (a.rows == 1 && a.in_features % 512 == 0) {
        const int vpl = a.in_features / 512;
        if (vpl == 2 || vpl == 4 || vpl == 6 || vpl == 12) {
            const int grid = (a.out_features + kHalfWaves - 1) / kHalfWaves;
            return dispatch_fixed<kEpi, kNorm>(a, vpl, grid, s);
        }
    }
    if constexpr (!kNorm) {
        // several exact rows on a production width: weights once per unit
        if (a.rows > 1 && a.input_row_index == nullptr) {
            switch (a.in_features) {
                case 1024: return launch_exact_rows_fixed<2, kEpi>(a, s);
                case 2048: return launch_exact_rows_fixed<4, kEpi>(a, s);
                case 3072: return launch_exact_rows_fixed<6, kEpi>(a, s);
                case 6144: return launch_exact_rows_fixed<12, kEpi>(a, s);
                default: break;
            }
        }
    }
    const int generic_units = a.out_features;
    int grid = (generic_units + kHalfWaves - 1) / kHalfWaves;
    const int cap = device_cu_count() * 16;
    if (grid > cap) grid = cap;
    return dispatch_generic<kEpi, kNorm>(a, grid, s);
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

hipError_t launch_int8_gemv(const GemvArgs& a, hipStream_t stream) {
    if (a.weight == nullptr || a.scales == nullptr || a.input == nullptr) return hipErrorInvalidValue;
    if (a.in_features <= 0 || a.in_features % 16 != 0 || a.out_features <= 0) return hipErrorInvalidValue;
    if (a.rows < 1 || a.rows > 8) return hipErrorInvalidValue;
    if (!aligned16(a.weight) || !aligned16(a.input)) return hipErrorInvalidValue;
    if (a.norm_weight != nullptr && !aligned16(a.norm_weight)) return hipErrorInvalidValue;
    if (a.epilogue != kEpiStore && a.out16 == nullptr) return hipErrorInvalidValue;
    if (a.epilogue == kEpiStore && a.out16 == nullptr && a.out32 == nullptr) return hipErrorInvalidValue;
    if (a.epilogue >= kEpiBias && a.bias == nullptr) return hipErrorInvalidValue;
    if (a.input_row_index != nullptr && a.rows != 1) return hipErrorInvalidValue;
    const bool norm = a.norm_weight != nullptr;
    switch (a.epilogue) {
        case kEpiStore: return norm ? dispatch<kEpiStore, true>(a, stream) : dispatch<kEpiStore, false>(a, stream);
        case kEpiAddFma: return norm ? dispatch<kEpiAddFma, true>(a, stream) : dispatch<kEpiAddFma, false>(a, stream);
        case kEpiAddRounded: return norm ? dispatch<kEpiAddRounded, true>(a, stream) : dispatch<kEpiAddRounded, false>(a, stream);
        case kEpiSiluFused: return norm ? dispatch<kEpiSiluFused, true>(a, stream) : dispatch<kEpiSiluFused, false>(a, stream);
        case kEpiSiluRounded: return norm ? dispatch<kEpiSiluRounded, true>(a, stream) : dispatch<kEpiSiluRounded, false>(a, stream);
        case kEpiBias: return norm ? dispatch<kEpiBias, true>(a, stream) : dispatch<kEpiBias, false>(a, stream);
        case kEpiBiasSilu: return norm ? dispatch<kEpiBiasSilu, true>(a, stream) : dispatch<kEpiBiasSilu, false>(a, stream);
        case kEpiBiasAdd: return norm ? dispatch<kEpiBiasAdd, true>(a, stream) : dispatch<kEpiBiasAdd, false>(a, stream);
        default: return hipErrorInvalidValue;
    }
}

// A prompt's rows (any count) in exact order through one launch, each row's
// result the same as through launch_int8_gemv in launches of up to 8 rows
// (the per-row sum does not depend on the rows beside it).  No RMSNorm
// prologue; store and bias epilogues; K outside {1024, 2048, 3072, 6144} runs
// as launches of up to 8 rows.
hipError_t launch_int8_gemv_prompt_rows(const GemvArgs& a, hipStream_t stream) {
    if (a.weight == nullptr || a.scales == nullptr || a.input == nullptr || a.out16 == nullptr || a.rows < 1 ||
        a.out_features <= 0 || a.norm_weight != nullptr || a.input_row_index != nullptr || a.out32 != nullptr ||
        !aligned16(a.weight) || !aligned16(a.input)) {
        return hipErrorInvalidValue;
    }
    if (a.epilogue >= kEpiBias && a.bias == nullptr) return hipErrorInvalidValue;
    auto by_k = [&](auto epi) -> hipError_t {
        constexpr int kE = decltype(epi)::value;
        switch (a.in_features) {
            case 1024: return launch_exact_rows_fixed<2, kE>(a, stream);
            case 2048: return launch_exact_rows_fixed<4, kE>(a, stream);
            case 3072: return launch_exact_rows_fixed<6, kE>(a, stream);
            case 6144: return launch_exact_rows_fixed<12, kE>(a, stream);
            default: break;
        }
        // other widths: launches of up to 8 rows
        for (int r0 = 0; r0 < a.rows; r0 += 8) {
            GemvArgs part = a;
            part.rows = std::min(8, a.rows - r0);
            part.mode = kModeExact;
            part.input = a.input + static_cast<size_t>(r0) * a.in_features;
            part.out16 = a.out16 + static_cast<size_t>(r0) * a.out_features;
            const hipError_t st = launch_int8_gemv(part, stream);
            if (st != hipSuccess) return st;
        }
        return hipSuccess;
    };
    switch (a.epilogue) {
        case kEpiStore: return by_k(std::integral_constant<int, kEpiStore>{});
        case kEpiBias: return by_k(std::integral_constant<int, kEpiBias>{});
        case kEpiBiasSilu: return by_k(std::integral_constant<int, kEpiBiasSilu>{});
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_quantize_weight_rows(const bf16_t* weight, int8_t* quantized, float* scales,
                                       int in_features, int out_features, hipStream_t stream) {
    if (in_features % 16 != 0 || in_features <= 0 || out_features <= 0) return hipErrorInvalidValue;
    quantize_rows_kernel<<<out_features, kThreads, 0, stream>>>(weight, quantized, scales, in_features);
    return hipGetLastError();
}

namespace {
hipError_t reference_style(const int8_t* w, const float* s, const bf16_t* x, bf16_t* y, int in,
                           int out, int rows, int epi, hipStream_t stream) {
    if (in % 16 != 0 || rows < 1 || rows > 8) return hipErrorInvalidValue;
    GemvArgs a;
    a.weight = w;
    a.scales = s;
    a.input = x;
    a.out16 = y;
    a.in_features = in;
    a.out_features = out;
    a.rows = rows;
    a.epilogue = epi;
    a.mode = kModeExact;
    return launch_int8_gemv(a, stream);
}
}  // namespace

hipError_t launch_int8_gemm_rows(const int8_t* w, const float* s, const bf16_t* x, bf16_t* y,
                                 int in, int out, int rows, hipStream_t stream) {
    return reference_style(w, s, x, y, in, out, rows, kEpiStore, stream);
}

hipError_t launch_int8_gemm_rows_add(const int8_t* w, const float* s, const bf16_t* x, bf16_t* y,
                                     int in, int out, int rows, hipStream_t stream) {
    return reference_style(w, s, x, y, in, out, rows, kEpiAddFma, stream);
}

hipError_t launch_int8_gate_up_silu_rows(const int8_t* w, const float* s, const bf16_t* x,
                                         bf16_t* y, int in, int out, int rows, hipStream_t stream) {
    return reference_style(w, s, x, y, in, out, rows, kEpiSiluFused, stream);
}

}  // namespace q3
