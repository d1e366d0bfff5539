// Codec-token sampler and frame glue kernels, gfx950.
//
// Semantics follow native/qwen3-tts-native/native/src/sampling_kernels.cu:
//   adjusted logits (talker reserved-token mask, repetition penalty over the
//   semantic history, :30-51); greedy argmax with lower-index ties (:208-236);
//   direct categorical draw (:238-265); top-k/top-p: the top `selections`
//   tokens in the order (value desc, index asc), weights exp(double) of
//   (v/T - max/T), sequential double sums, top-p cut and one uniform draw
//   from xorshift64* (:53-69, :350-387).
//
// Design: one 1024-thread block.  The repetition penalty uses an LDS mark
// table built from the history in one pass (O(history + vocabulary)).  The
// top `selections` logits are found by an 8-bit radix select over monotone
// 32-bit keys that stops after the first pass leaving at most 128 keys at or
// above the chosen bin (bf16 logits: after two passes, up to ties); the
// survivors are ordered by rank counting (eight lanes per survivor when
// there are at most 128), which yields the exact total order.  The sampled
// token can be stored straight into the frame token array and the semantic
// history (device-resident counters), so a frame needs no host round trip.
#include "q3_common.hpp"

namespace q3 {
namespace {

constexpr int kSampleThreads = 1024;
constexpr int kMaxVocabulary = 4096;
constexpr int kCandidateCap = 1024;
// survivors ranked by eight lanes each (all 1024 threads)
constexpr int kRankParallelCap = kSampleThreads / 8;

// Build-time diagnostic: -DQ3_SAMPLE_TRACE records the wall-clock time of
// the sampler's phases (thread 0 of block 0) in q3_sample_trace.
#ifdef Q3_SAMPLE_TRACE
__device__ unsigned long long q3_sample_trace[16];
#define SAMPLE_STAMP(i)                                                         \
    do {                                                                        \
        if (blockIdx.x == 0 && threadIdx.x == 0) q3_sample_trace[i] = wall_clock64(); \
    } while (0)
#else
#define SAMPLE_STAMP(i) \
    do {                \
    } while (0)
#endif


__device__ __forceinline__ uint32_t order_key(float v) {
    uint32_t u = __float_as_uint(v);
    if (u == 0x80000000u) u = 0u;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// (order key, ~index): a larger packed key ranks earlier -- (value desc,
// index asc) for ordered values, and a total order for every bit pattern
// (NaN included), so the ranks are distinct and every token index stays in
// range.
__device__ __forceinline__ unsigned long long rank_key(float v, int index) {
    return (static_cast<unsigned long long>(order_key(v)) << 32) | static_cast<uint32_t>(~index);
}

// Inclusive prefix sum over the 64 lanes of a wave with DPP row shifts and
// row broadcasts (no LDS round trips).  Integer, so exact in any order.
__device__ __forceinline__ int wave_inclusive_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, false);  // row_shr:1
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, false);  // row_shr:2
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, false);  // row_shr:4
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, false);  // row_shr:8
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15 into rows 1, 3
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31 into rows 2, 3
    return x;
}

__device__ uint64_t next_random(uint64_t* state) {
    uint64_t value = *state;
    if (value == 0) value = 0x9e3779b97f4a7c15ULL;
    value ^= value >> 12;
    value ^= value << 25;
    value ^= value >> 27;
    *state = value;
    return value * 0x2545f4914f6cdd1dULL;
}

__device__ float uniform_random(uint64_t* state) {
    const uint64_t value = next_random(state);
    return static_cast<float>(static_cast<double>(value >> 11) * (1.0 / 9007199254740992.0));
}

// Same draw from a state value already in registers; the caller stores the
// advanced state.
__device__ float uniform_random_from(uint64_t& state) {
    const uint64_t value = next_random(&state);
    return static_cast<float>(static_cast<double>(value >> 11) * (1.0 / 9007199254740992.0));
}


__device__ __forceinline__ void sample_one(const SampleArgs& a) {
    __shared__ float values[kMaxVocabulary];
    __shared__ unsigned char marked[kMaxVocabulary];
    __shared__ double weights[kMaxVocabulary];
    __shared__ float cand_v[kCandidateCap];
    __shared__ int cand_i[kCandidateCap];
    __shared__ __align__(16) unsigned long long cand_key[kCandidateCap + 2];  // (order key, ~index): larger = earlier
    __shared__ float sorted_v[kMaxVocabulary];
    __shared__ int sorted_i[kMaxVocabulary];
    __shared__ uint32_t hist2[512];
    __shared__ float red_v[kSampleThreads / 64];
    __shared__ int red_i[kSampleThreads / 64];
    __shared__ uint32_t s_prefix;
    __shared__ int s_above;
    __shared__ int s_total;
    __shared__ int s_count;
    __shared__ int s_best;
    __shared__ double s_target;
    __shared__ double shares[72];
    __shared__ double prefix_lds[64], cumulative_lds[64];

    const int tid = threadIdx.x;
    const int V = a.vocabulary;
    const int count = a.history_count ? *a.history_count : a.history_count_fallback;
    // the generator state, requested now and used at the very end
    uint64_t random_state = (tid == 0 && a.random_state != nullptr) ? *a.random_state : 0ull;
    const bool penalize = a.suppress && a.penalty != 1.0f;
    SAMPLE_STAMP(0);

    // The logits are requested first (they do not depend on the history).
    constexpr int kPerThread = kMaxVocabulary / kSampleThreads;
    float logit[kPerThread];
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int t = tid + j * kSampleThreads;
        logit[j] = t < V ? bf2f(a.logits[t]) : 0.0f;
    }
    if (penalize) {
        for (int t = tid; t < V; t += kSampleThreads) marked[t] = 0;
        __syncthreads();
        for (int h = tid; h < count; h += kSampleThreads) {
            const int token = a.history[h];
            if (token >= 0 && token < V) marked[token] = 1;
        }
        __syncthreads();
    }
#pragma unroll
    for (int j = 0; j < kPerThread; ++j) {
        const int t = tid + j * kSampleThreads;
        if (t >= V) break;
        float value;
        if (a.suppress && t >= 2048 && t != a.eos) {
            value = -INFINITY;
        } else {
            value = logit[j];
            if (penalize && marked[t]) value = value < 0.0f ? value * a.penalty : value / a.penalty;
        }
        values[t] = value;
    }
    __syncthreads();
    SAMPLE_STAMP(1);

    const bool direct = a.do_sample != 0 && a.top_k == 0 && a.top_p >= 1.0f;
    const int selections = a.do_sample == 0 ? 1 : (a.top_k == 0 ? V : min(a.top_k, V));
    int selected = 0;

    if (a.do_sample == 0 || direct) {
        // Block argmax, lower index on ties.
        float bv = -INFINITY;
        int bi = -1;
        for (int t = tid; t < V; t += kSampleThreads) {
            const float v = values[t];
            if (bi < 0 || v > bv) {
                bv = v;
                bi = t;
            }
        }
        for (int offset = 32; offset > 0; offset >>= 1) {
            const float ov = __shfl_down(bv, offset, 64);
            const int oi = __shfl_down(bi, offset, 64);
            if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
                bv = ov;
                bi = oi;
            }
        }
        if ((tid & 63) == 0) {
            red_v[tid >> 6] = bv;
            red_i[tid >> 6] = bi;
        }
        __syncthreads();
        if (tid == 0) {
            float v = red_v[0];
            int i = red_i[0];
            for (int w = 1; w < kSampleThreads / 64; ++w) {
                if (red_i[w] >= 0 && (i < 0 || red_v[w] > v || (red_v[w] == v && red_i[w] < i))) {
                    v = red_v[w];
                    i = red_i[w];
                }
            }
            s_best = i;
        }
        __syncthreads();
        selected = s_best;
        if (direct) {
            const float maximum = values[selected] / a.temperature;
            for (int t = tid; t < V; t += kSampleThreads) {
                weights[t] = exp(static_cast<double>(values[t] / a.temperature - maximum));
            }
            __syncthreads();
            if (tid == 0) {
                double total = 0.0;
                for (int t = 0; t < V; ++t) total += weights[t];
                const double target = static_cast<double>(uniform_random(a.random_state)) * total;
                double cumulative = 0.0;
                for (int t = 0; t < V; ++t) {
                    cumulative += weights[t];
                    if (cumulative >= target) {
                        selected = t;
                        break;
                    }
                }
                s_best = selected;
            }
            __syncthreads();
            selected = s_best;
        }
    } else {
        // Radix select, most significant byte first.  After each pass the
        // count of keys at or above the chosen bin is known; once it is at
        // most kRankParallelCap the remaining passes are skipped: every key
        // whose leading bits reach the bin is a candidate, and the exact
        // rank counting below orders them (ranks past `selections` are not
        // used).  Two histogram buffers: the next pass's is cleared while
        // this pass's is scanned, two barriers per pass.
        if (tid == 0) {
            s_prefix = 0u;
            s_above = 0;
        }
        for (int b = tid; b < 512; b += kSampleThreads) hist2[b] = 0u;
        __syncthreads();
        int buffer = 0;
        for (int shift = 24; shift >= 0; shift -= 8, buffer ^= 1) {
            uint32_t* hist = hist2 + 256 * buffer;
            const uint32_t prefix = s_prefix;
            const int high = shift + 8;
            for (int t = tid; t < V; t += kSampleThreads) {
                const uint32_t key = order_key(values[t]);
                if (high >= 32 || (key >> high) == (prefix >> high)) {
                    atomicAdd(&hist[(key >> shift) & 0xffu], 1u);
                }
            }
            __syncthreads();
            if (tid < 64) {
                // Scan the bins from the top (bin 255 first) in wave 0: lane l
                // holds bins 255-4l .. 252-4l.  Integer counts, so the
                // parallel prefix equals the sequential scan.
                const int lane = tid;
                int h[4];
                int lane_total = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    h[j] = static_cast<int>(hist[255 - 4 * lane - j]);
                    lane_total += h[j];
                }
                const int inclusive = wave_inclusive_scan(lane_total);
                const int base_above = s_above;
                int before = base_above + inclusive - lane_total;
                int found = -1;
                int found_before = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (found < 0 && before + h[j] >= selections) {
                        found = j;
                        found_before = before;
                    }
                    before += h[j];
                }
                const unsigned long long hits = __ballot(found >= 0);
                const int first = hits ? __ffsll(static_cast<long long>(hits)) - 1 : -1;
                if (first < 0) {
                    if (lane == 63) {  // no bin reaches the count: chosen 0, all bins above
                        s_above = before;
                        s_prefix = prefix;
                        s_total = before;
                    }
                } else if (lane == first) {
                    s_above = found_before;
                    s_total = found_before + h[found];
                    s_prefix = prefix | (static_cast<uint32_t>(255 - 4 * lane - found) << shift);
                }
            } else if (tid >= 256 && tid < 512) {
                hist2[256 * (buffer ^ 1) + (tid - 256)] = 0u;  // next pass's buffer
            }
            __syncthreads();
            if (s_total <= kRankParallelCap) break;  // block-uniform
        }
        SAMPLE_STAMP(2);
        // keys >= threshold: the chosen bin's prefix with the unresolved
        // low bits zero
        const uint32_t threshold = s_prefix;
        if (tid == 0) s_count = 0;
        __syncthreads();
        for (int t = tid; t < V; t += kSampleThreads) {
            if (order_key(values[t]) >= threshold) {
                const int slot = atomicAdd(&s_count, 1);
                if (slot < kCandidateCap) {
                    cand_v[slot] = values[t];
                    cand_i[slot] = t;
                    cand_key[slot] = rank_key(values[t], t);
                }
            }
        }
        __syncthreads();
        const int n = s_count;
        SAMPLE_STAMP(3);
        // Rank counting over the survivors: exact total order.  The packed
        // key compares like (value desc, index asc) (order_key is monotone,
        // -0 == +0).
        if (n <= kRankParallelCap) {
            // eight lanes per survivor, each over every eighth key; the
            // integer partial ranks are added by lane swaps
            const int c = tid >> 3;
            const int part = tid & 7;
            int rank = 0;
            if (c < n) {
                const unsigned long long mine = cand_key[c];
#pragma unroll 4
                for (int j = part; j < n; j += 8) rank += static_cast<int>(cand_key[j] > mine);
            }
            rank += __shfl_xor(rank, 1, 64);
            rank += __shfl_xor(rank, 2, 64);
            rank += __shfl_xor(rank, 4, 64);
            if (c < n && part == 0) {
                sorted_v[rank] = cand_v[c];
                sorted_i[rank] = cand_i[c];
            }
        } else if (n <= kCandidateCap) {
            // a 0 pad (below every key) makes the count even, two keys per
            // LDS read
            if (tid == 0) cand_key[n] = 0ull;
            __syncthreads();
            for (int c = tid; c < n; c += kSampleThreads) {
                const unsigned long long mine = cand_key[c];
                const ulonglong2* pairs = reinterpret_cast<const ulonglong2*>(cand_key);
                int rank = 0;
                for (int j = 0; j < (n + 1) / 2; ++j) {
                    const ulonglong2 k = pairs[j];
                    rank += static_cast<int>(k.x > mine) + static_cast<int>(k.y > mine);
                }
                sorted_v[rank] = cand_v[c];
                sorted_i[rank] = cand_i[c];
            }
        } else {
            for (int t = tid; t < V; t += kSampleThreads) {
                const float v = values[t];
                const unsigned long long mine = rank_key(v, t);
                int rank = 0;
                for (int j = 0; j < V; ++j) rank += static_cast<int>(rank_key(values[j], j) > mine);
                sorted_v[rank] = v;
                sorted_i[rank] = t;
            }
        }
        __syncthreads();
        SAMPLE_STAMP(4);
        const float maximum = sorted_v[0] / a.temperature;
        // (entries selections .. 63 are 0 for the wave-0 sums below)
        const int weight_count = selections <= 64 ? 64 : selections;
        for (int r = tid; r < weight_count; r += kSampleThreads) {
            weights[r] = r < selections ? exp(static_cast<double>(sorted_v[r] / a.temperature - maximum)) : 0.0;
        }
        __syncthreads();
        SAMPLE_STAMP(5);
        if (selections <= 64) {
            // Wave 0.  Every running sum of the reference is a prefix sum in
            // rank order, so one sequential pass (all lanes, LDS broadcast
            // reads) produces them; lane r keeps prefix r, and each "first r
            // with cumulative >= x" loop becomes a ballot over the lanes.
            if (tid < 64) {
                const int lane = tid;
                // Whole steps of 8; the zero entries past `selections` leave
                // the non-negative running sums as they are.  Each prefix is
                // stored once (every lane writes the same value), so a step
                // is one add.
                const int steps = (selections + 7) & ~7;
                double running = 0.0;
                for (int r0 = 0; r0 < steps; r0 += 8) {
#pragma unroll
                    for (int u = 0; u < 8; ++u) {
                        running += weights[r0 + u];
                        prefix_lds[r0 + u] = running;
                    }
                }
                const double denominator = running;
                // The top-p cut: the first r whose running sum of shares
                // w_r / denominator reaches top_p.  With top_p >= 1 it can
                // only fall on the last candidate (and then keeps them all)
                // when the smallest weight exceeds 1e-12 of the denominator:
                // for r below the last, the tail sum w_(r+1).. >= w_last, and
                // the computed running share is at most (1 - w_last / W)(1 +
                // 130 u) with W the exact weight sum and u = 2^-53 (the
                // denominator's and the sum's rounding over <= 64 terms), which
                // stays below 1.  Otherwise the running shares are formed in
                // order as the reference does.
                int retained = selections;
                if (!(a.top_p >= 1.0f && weights[selections - 1] > 1e-12 * denominator)) {
                    shares[lane] = lane < selections ? weights[lane] / denominator : 0.0;
                    __builtin_amdgcn_wave_barrier();
                    double share_running = 0.0;
                    for (int r0 = 0; r0 < steps; r0 += 8) {
#pragma unroll
                        for (int u = 0; u < 8; ++u) {
                            share_running += shares[r0 + u];
                            cumulative_lds[r0 + u] = share_running;
                        }
                    }
                    __builtin_amdgcn_wave_barrier();
                    const double share_mine = cumulative_lds[lane];
                    const unsigned long long cut =
                        __ballot(lane < selections && share_mine >= static_cast<double>(a.top_p));
                    if (cut) retained = __ffsll(static_cast<long long>(cut));
                }
                __builtin_amdgcn_wave_barrier();
                const double prefix_mine = prefix_lds[lane];
                // sum of weights[0..retained) in order: prefix retained-1
                const double retained_total =
                    __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(prefix_mine), retained - 1),
                                     __builtin_amdgcn_readlane(__double2loint(prefix_mine), retained - 1));
                if (lane == 0) {
                    s_target = static_cast<double>(uniform_random_from(random_state)) * retained_total;
                    *a.random_state = random_state;
                }
                __builtin_amdgcn_wave_barrier();
                const double target = s_target;
                const unsigned long long hit = __ballot(lane < retained && prefix_mine >= target);
                const int r = hit ? __ffsll(static_cast<long long>(hit)) - 1 : retained - 1;
                if (lane == 0) s_best = sorted_i[r];
            }
        } else if (tid == 0) {
            double denominator = 0.0;
            for (int r = 0; r < selections; ++r) denominator += weights[r];
            double cumulative = 0.0;
            int retained = selections;
            for (int r = 0; r < selections; ++r) {
                cumulative += weights[r] / denominator;
                if (cumulative >= static_cast<double>(a.top_p)) {
                    retained = r + 1;
                    break;
                }
            }
            double retained_total = 0.0;
            for (int r = 0; r < retained; ++r) retained_total += weights[r];
            const double target = static_cast<double>(uniform_random(a.random_state)) * retained_total;
            cumulative = 0.0;
            int choice = sorted_i[retained - 1];
            for (int r = 0; r < retained; ++r) {
                cumulative += weights[r];
                if (cumulative >= target) {
                    choice = sorted_i[r];
                    break;
                }
            }
            s_best = choice;
        }
        __syncthreads();
        selected = s_best;
    }

    SAMPLE_STAMP(6);
    if (tid == 0) {
        if (a.selected) *a.selected = selected;
        if (a.store_tokens) {
            const int index = a.store_index ? *a.store_index : a.store_index_fallback;
            a.store_tokens[index] = selected;
        }
        if (a.append_history && a.append_count) {
            const int c = *a.append_count;
            a.append_history[c] = selected;
            *a.append_count = c + 1;
        }
    }
}

__global__ __launch_bounds__(kSampleThreads) void sample_kernel(SampleArgs a) { sample_one(a); }

// One block per row, each with its own arguments (the batch's sessions).
__global__ __launch_bounds__(kSampleThreads) void sample_rows_kernel(const SampleArgs* rows) {
    sample_one(rows[blockIdx.x]);
}

// bf16_argmax_kernel (runtime.cu:43-82): strided argmax + lower-index ties.
__global__ __launch_bounds__(256) void argmax_kernel(const bf16_t* logits, int vocabulary,
                                                     int* selected) {
    __shared__ float rv[4];
    __shared__ int ri[4];
    float bv = -INFINITY;
    int bi = -1;
    for (int t = threadIdx.x; t < vocabulary; t += 256) {
        const float v = bf2f(logits[t]);
        if (bi < 0 || v > bv) {
            bv = v;
            bi = t;
        }
    }
    for (int offset = 32; offset > 0; offset >>= 1) {
        const float ov = __shfl_down(bv, offset, 64);
        const int oi = __shfl_down(bi, offset, 64);
        if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) {
            bv = ov;
            bi = oi;
        }
    }
    if ((threadIdx.x & 63) == 0) {
        rv[threadIdx.x >> 6] = bv;
        ri[threadIdx.x >> 6] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            if (ri[w] >= 0 && (ri[0] < 0 || rv[w] > rv[0] || (rv[w] == rv[0] && ri[w] < ri[0]))) {
                rv[0] = rv[w];
                ri[0] = ri[w];
            }
        }
        *selected = ri[0];
    }
}

__global__ void store_token_kernel(int* tokens, int index, int value) {
    if (threadIdx.x == 0) tokens[index] = value;
}

__global__ void pack_codes_kernel(const int* tokens, uint16_t* codes, int count) {
    const int i = threadIdx.x;
    if (i < count) codes[i] = static_cast<uint16_t>(tokens[i]);
}

// One block per session of a batch: the frame's tokens into its code row.
__global__ void pack_codes_rows_kernel(const int* const* tokens, uint16_t* const* codes, int count) {
    const int i = threadIdx.x;
    if (i < count) codes[blockIdx.x][i] = static_cast<uint16_t>(tokens[blockIdx.x][i]);
}

// gather_embedding_kernel (sampling_kernels.cu:428-452): an out-of-range
// token leaves the output untouched.
__global__ void gather_embedding_kernel(const bf16_t* table, int vocabulary, int width,
                                        const int* token, bf16_t* output, bool add) {
    const int row = *token;
    if (row < 0 || row >= vocabulary) return;
    const bf16_t* src = table + static_cast<size_t>(row) * width;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += blockDim.x * gridDim.x) {
        output[i] = add ? f2bf(bf2f(output[i]) + bf2f(src[i])) : src[i];
    }
}

// One gather followed by count-1 adds, each rounded to bf16, fused.
__global__ void sum_embeddings_kernel(const bf16_t* const* tables, int count, int vocabulary0,
                                      int vocabulary, int width, const int* tokens,
                                      bf16_t* output) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width) return;
    const int first = tokens[0];
    float acc = bf2f(output[i]);
    bool have = false;
    if (first >= 0 && first < vocabulary0) {
        acc = bf2f(tables[0][static_cast<size_t>(first) * width + i]);
        have = true;
    }
    for (int r = 1; r < count; ++r) {
        const int tok = tokens[r];
        if (tok < 0 || tok >= vocabulary) continue;
        acc = round_bf(acc + bf2f(tables[r][static_cast<size_t>(tok) * width + i]));
        have = true;
    }
    if (have) output[i] = f2bf(acc);
}

// Lockstep-batch glue (talker.cu:1552-1607,1700-1770 equivalents): rows of a
// batch come from / go to per-session buffers through pointer tables.
__global__ void gather_rows_kernel(const bf16_t* const* sources, int width, bf16_t* output) {
    const bf16_t* src = sources[blockIdx.y];
    bf16_t* dst = output + static_cast<size_t>(blockIdx.y) * width;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += blockDim.x * gridDim.x) dst[i] = src[i];
}

__global__ void scatter_rows_kernel(const bf16_t* input, bf16_t* const* destinations, int width) {
    const bf16_t* src = input + static_cast<size_t>(blockIdx.y) * width;
    bf16_t* dst = destinations[blockIdx.y];
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += blockDim.x * gridDim.x) dst[i] = src[i];
}

// gather_embedding_rows_kernel semantics (talker_kernels.cu:680-709): row r
// reads token_bases[r][offset]; an out-of-range token leaves the row as is.
__global__ void gather_embedding_rows_kernel(const bf16_t* table, int vocabulary, int width,
                                             const int* const* token_bases, int offset, bf16_t* output) {
    const int token = token_bases[blockIdx.y][offset];
    if (token < 0 || token >= vocabulary) return;
    const bf16_t* src = table + static_cast<size_t>(token) * width;
    bf16_t* dst = output + static_cast<size_t>(blockIdx.y) * width;
    for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < width; i += blockDim.x * gridDim.x) dst[i] = src[i];
}

__global__ void sum_embeddings_rows_kernel(const bf16_t* const* tables, int count, int vocabulary0,
                                           int vocabulary, int width, const int* const* token_bases,
                                           bf16_t* output) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= width) return;
    const int* tokens = token_bases[blockIdx.y];
    bf16_t* out = output + static_cast<size_t>(blockIdx.y) * width;
    const int first = tokens[0];
    float acc = bf2f(out[i]);
    bool have = false;
    if (first >= 0 && first < vocabulary0) {
        acc = bf2f(tables[0][static_cast<size_t>(first) * width + i]);
        have = true;
    }
    for (int r = 1; r < count; ++r) {
        const int tok = tokens[r];
        if (tok < 0 || tok >= vocabulary) continue;
        acc = round_bf(acc + bf2f(tables[r][static_cast<size_t>(tok) * width + i]));
        have = true;
    }
    if (have) out[i] = f2bf(acc);
}

__global__ void increment_each_kernel(int* const* counters, int count) {
    const int i = threadIdx.x;
    if (i < count) *counters[i] += 1;
}

}  // namespace

hipError_t launch_gather_rows(const bf16_t* const* sources, int rows, int width, bf16_t* output,
                              hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    gather_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(sources, width, output);
    return hipGetLastError();
}

hipError_t launch_scatter_rows(const bf16_t* input, bf16_t* const* destinations, int rows, int width,
                               hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    scatter_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(input, destinations, width);
    return hipGetLastError();
}

hipError_t launch_gather_embedding_rows(const bf16_t* table, int vocabulary, int width,
                                        const int* const* token_bases, int offset, bf16_t* output,
                                        int rows, hipStream_t stream) {
    if (rows <= 0 || width <= 0) return hipErrorInvalidValue;
    gather_embedding_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(
        table, vocabulary, width, token_bases, offset, output);
    return hipGetLastError();
}

hipError_t launch_sum_embeddings_rows(const bf16_t* const* tables, int count, int vocabulary0,
                                      int vocabulary, int width, const int* const* token_bases,
                                      bf16_t* output, int rows, hipStream_t stream) {
    if (rows <= 0 || width <= 0 || count <= 0) return hipErrorInvalidValue;
    sum_embeddings_rows_kernel<<<dim3((width + 255) / 256, rows), 256, 0, stream>>>(
        tables, count, vocabulary0, vocabulary, width, token_bases, output);
    return hipGetLastError();
}

hipError_t launch_increment_each(int* const* counters, int count, hipStream_t stream) {
    if (count <= 0 || count > 64) return hipErrorInvalidValue;
    increment_each_kernel<<<1, 64, 0, stream>>>(counters, count);
    return hipGetLastError();
}

hipError_t launch_sample_logits(const bf16_t* logits, int vocabulary, bool suppress, int eos,
                                const int* history, const int* history_count,
                                int history_count_fallback, int do_sample, int top_k, float top_p,
                                float temperature, float penalty, uint64_t* random_state,
                                int* selected, int* store_tokens, const int* store_index,
                                int store_index_fallback, hipStream_t stream) {
    return launch_sample_logits_ex(logits, vocabulary, suppress, eos, history, history_count,
                                   history_count_fallback, do_sample, top_k, top_p, temperature,
                                   penalty, random_state, selected, store_tokens, store_index,
                                   store_index_fallback, nullptr, nullptr, stream);
}

hipError_t launch_sample_logits_ex(const bf16_t* logits, int vocabulary, bool suppress, int eos,
                                   const int* history, const int* history_count,
                                   int history_count_fallback, int do_sample, int top_k,
                                   float top_p, float temperature, float penalty,
                                   uint64_t* random_state, int* selected, int* store_tokens,
                                   const int* store_index, int store_index_fallback,
                                   int* append_history, int* append_count, hipStream_t stream) {
    if (vocabulary <= 0 || vocabulary > kMaxVocabulary) return hipErrorInvalidValue;
    if (top_k < 0 || !(top_p > 0.0f) || top_p > 1.0f || !(temperature > 0.0f) || !(penalty > 0.0f)) {
        return hipErrorInvalidValue;
    }
    SampleArgs a{logits, vocabulary, suppress, eos, history, history_count,
                 history_count_fallback, do_sample, top_k, top_p, temperature, penalty,
                 random_state, selected, store_tokens, store_index, store_index_fallback,
                 append_history, append_count};
    sample_kernel<<<1, kSampleThreads, 0, stream>>>(a);
    return hipGetLastError();
}

bool sample_args_valid(const SampleArgs& a) {
    return a.vocabulary > 0 && a.vocabulary <= kMaxVocabulary && a.top_k >= 0 && a.top_p > 0.0f &&
           a.top_p <= 1.0f && a.temperature > 0.0f && a.penalty > 0.0f;
}

hipError_t launch_sample_rows(const SampleArgs* device_rows, int rows, hipStream_t stream) {
    if (device_rows == nullptr || rows <= 0 || rows > 64) return hipErrorInvalidValue;
    sample_rows_kernel<<<rows, kSampleThreads, 0, stream>>>(device_rows);
    return hipGetLastError();
}

hipError_t launch_argmax_bf16(const bf16_t* logits, int vocabulary, int* selected,
                              hipStream_t stream) {
    if (vocabulary <= 0) return hipErrorInvalidValue;
    argmax_kernel<<<1, 256, 0, stream>>>(logits, vocabulary, selected);
    return hipGetLastError();
}

hipError_t launch_store_token(int* tokens, int index, int value, hipStream_t stream) {
    store_token_kernel<<<1, 64, 0, stream>>>(tokens, index, value);
    return hipGetLastError();
}

hipError_t launch_pack_frame_codes(const int* tokens, uint16_t* codes, int count,
                                   hipStream_t stream) {
    if (count <= 0 || count > 64) return hipErrorInvalidValue;
    pack_codes_kernel<<<1, 64, 0, stream>>>(tokens, codes, count);
    return hipGetLastError();
}

hipError_t launch_pack_frame_codes_rows(const int* const* tokens, uint16_t* const* codes, int count, int rows,
                                        hipStream_t stream) {
    if (count <= 0 || count > 64 || rows <= 0) return hipErrorInvalidValue;
    pack_codes_rows_kernel<<<rows, 64, 0, stream>>>(tokens, codes, count);
    return hipGetLastError();
}

hipError_t launch_gather_embedding(const bf16_t* table, int vocabulary, int width,
                                   const int* token, bf16_t* output, bool add,
                                   hipStream_t stream) {
    if (width <= 0) return hipErrorInvalidValue;
    gather_embedding_kernel<<<(width + 255) / 256, 256, 0, stream>>>(table, vocabulary, width,
                                                                     token, output, add);
    return hipGetLastError();
}

hipError_t launch_sum_embeddings(const bf16_t* const* tables, int count, int vocabulary0,
                                 int vocabulary, int width, const int* tokens, bf16_t* output,
                                 hipStream_t stream) {
    if (width <= 0 || count <= 0) return hipErrorInvalidValue;
    sum_embeddings_kernel<<<(width + 255) / 256, 256, 0, stream>>>(tables, count, vocabulary0,
                                                                   vocabulary, width, tokens,
                                                                   output);
    return hipGetLastError();
}

}  // namespace q3
