// Persistent int8 GEMV chain kernel for gfx950.
//
// One cooperative launch walks a list of dependent GEMVs (a talker decode
// step's QKV -> O -> gate/up -> down chain, 28 times) with one 256-thread
// workgroup per CU.  Between dependent GEMVs all workgroups meet at a grid
// barrier; before waiting there, every half-wave has already issued the
// 128-bit loads of its weight rows of the NEXT GEMV into registers, so HBM
// keeps streaming weights while the dependency resolves.  Per GEMV the work
// split, the reference lane order and the epilogues are those of
// gemv_exact_fixed (bit-identical results):
//   half-wave h of the grid owns units h, h + H, h + 2H, ... (H = 8 * grid);
//   a unit is one output row, or a gate row + up row pair.
// The activation vector of each GEMV (written by the previous one) is staged
// through LDS after the barrier, normalized there when the RMSNorm prologue is
// fused, and pulled into registers in the lane's slice.
#include "gemv_device.hpp"

#include "../../include/qwen3_tts_native.h"

#include <cstdio>

namespace q3 {


// Supported GEMV shapes: (vectors per lane, units per half-wave, rows per unit).
enum ChainKind : int {
    kChainK2048U2 = 0,       // 2048-wide rows, <= 2 units per half-wave
    kChainK2048U1 = 1,       // 2048-wide rows, 1 unit
    kChainK2048Pair3 = 2,    // 2048-wide gate/up pairs, <= 3 per half-wave
    kChainK6144U1 = 3,       // 6144-wide rows, 1 unit
};

namespace {

using namespace gemv_detail;

constexpr int kTileSlots = 24;  // int4 weight registers per lane
constexpr int kMaxIn = 6144;

struct ChainState {
    unsigned* barrier;             // zeroed before the launch
    int* status;                   // set to 1 if a barrier wait timed out
    unsigned long long* trace;     // optional: phase timestamps of workgroup 0
};

// Phase timestamps (100 MHz wall clock) of workgroup 0, op i, phase p.
__device__ __forceinline__ void trace_phase(const ChainState& st, int op, int phase) {
    if (st.trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0 && op < 256) {
        st.trace[op * 8 + phase] = wall_clock64();
    }
}

// Grid-wide barrier with a bounded wait.  Two levels: workgroup b arrives on
// the counter of group b % 8 (one group per XCD under round-robin dispatch);
// the last arriver of a group arrives on the global counter, which everyone
// polls.  Counters are monotone within a launch (barrier i completes at
// (i + 1) * members).  No cache fences are needed: activations travel only
// through device-coherent (agent-scope atomic) loads and stores, and
// __syncthreads orders each workgroup's stores before its arrival.  A wait
// longer than ~1 s records an error and every later barrier stops waiting,
// so the grid always drains.
constexpr int kGroups = 8;
constexpr int kLineWords = 32;  // 128-byte spacing between counters

// Split-phase barrier: arrive as soon as this workgroup's outputs are
// stored, do independent work (issue the next GEMV's weight loads), then wait.
__device__ void grid_arrive(const ChainState& st, unsigned index) {
    __syncthreads();  // every wave's stores of this op have completed
    if (threadIdx.x == 0) {
        const unsigned g = blockIdx.x % kGroups;
        const unsigned members = (gridDim.x - g + kGroups - 1) / kGroups;
        unsigned* group = st.barrier + kLineWords * (1 + g);
        const unsigned old = __hip_atomic_fetch_add(group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old + 1 == (index + 1) * members) {
            __hip_atomic_fetch_add(st.barrier, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

__device__ void grid_wait(const ChainState& st, unsigned index) {
    if (threadIdx.x == 0) {
        const unsigned groups = gridDim.x < kGroups ? gridDim.x : kGroups;
        const unsigned target = (index + 1) * groups;
        unsigned spins = 0;
        while (__hip_atomic_load(st.barrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            if ((spins & 1023u) == 0 &&
                __hip_atomic_load(st.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                break;
            }
            if (spins > (1u << 25)) {
                __hip_atomic_store(st.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    __syncthreads();
}

template <int kVpl, int kUnits, int kRowsPerUnit>
__device__ __forceinline__ void issue_tiles(const ChainOp& op, int4 (&tile)[kTileSlots]) {
    static_assert(kVpl * kUnits * kRowsPerUnit <= kTileSlots, "tile registers");
    const int lane = threadIdx.x & 31;
    const int total = gridDim.x * kHalfWaves;
    const int hw = blockIdx.x * kHalfWaves + (threadIdx.x >> 5);
    constexpr int kIn = kVpl * 512;
#pragma unroll
    for (int k = 0; k < kUnits; ++k) {
        const int unit = hw + k * total;
        if (unit < op.out_features) {
#pragma unroll
            for (int r = 0; r < kRowsPerUnit; ++r) {
                const int row = r == 0 ? unit : op.out_features + unit;
                const int4* base = reinterpret_cast<const int4*>(op.weight + static_cast<size_t>(row) * kIn);
#pragma unroll
                for (int i = 0; i < kVpl; ++i) tile[(k * kRowsPerUnit + r) * kVpl + i] = stream_load(base + lane + 32 * i);
            }
        }
    }
}

__device__ __forceinline__ void issue(const ChainOp& op, int4 (&tile)[kTileSlots]) {
    switch (op.kind) {
        case kChainK2048U2: issue_tiles<4, 2, 1>(op, tile); break;
        case kChainK2048U1: issue_tiles<4, 1, 1>(op, tile); break;
        case kChainK2048Pair3: issue_tiles<4, 3, 2>(op, tile); break;
        case kChainK6144U1: issue_tiles<12, 1, 1>(op, tile); break;
        default: break;
    }
}

template <int kEpi>
__device__ __forceinline__ GemvArgs epilogue_args(const ChainOp& op) {
    GemvArgs a;
    a.scales = op.scales;
    a.bias = op.bias;
    a.out16 = op.out16;
    a.out_features = op.out_features;
    return a;
}

template <int kVpl, int kUnits, int kRowsPerUnit, int kEpi>
__device__ void compute_tiles(const ChainOp& op, const int4 (&tile)[kTileSlots], const bf16_t* xs,
                              const bf16_t* gs, float inverse) {
    constexpr bool kPacked = kVpl > 6;
    const int lane = threadIdx.x & 31;
    const int total = gridDim.x * kHalfWaves;
    const int hw = blockIdx.x * kHalfWaves + (threadIdx.x >> 5);
    float xf[kPacked ? 1 : kVpl][16];
    uint32_t xp[kPacked ? kVpl : 1][8];
#pragma unroll
    for (int i = 0; i < kVpl; ++i) {
        float tmp[16];
        if (op.norm_weight != nullptr) {
            load_x16<true>(xs, gs, lane + 32 * i, inverse, tmp);
        } else {
            load_x16<false>(xs, gs, lane + 32 * i, inverse, tmp);
        }
        if constexpr (kPacked) {
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                xp[i][j] = (__float_as_uint(tmp[2 * j]) >> 16) | (__float_as_uint(tmp[2 * j + 1]) & 0xffff0000u);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) xf[i][j] = tmp[j];
        }
    }
    const GemvArgs a = epilogue_args<kEpi>(op);
#pragma unroll
    for (int k = 0; k < kUnits; ++k) {
        const int unit = hw + k * total;
        if (unit >= op.out_features) continue;  // uniform per half-wave
        float acc[kRowsPerUnit];
#pragma unroll
        for (int r = 0; r < kRowsPerUnit; ++r) {
            acc[r] = 0.0f;
#pragma unroll
            for (int i = 0; i < kVpl; ++i) {
                const int4 w = tile[(k * kRowsPerUnit + r) * kVpl + i];
                if constexpr (kPacked) {
                    acc[r] += chain16_packed(w, xp[i]);
                } else {
                    acc[r] += chain16(w, xf[i]);
                }
            }
            acc[r] = fold32(acc[r]);
        }
        if (lane == 0) {
            if constexpr (kRowsPerUnit == 2) {
                store_gate_up<kEpi, true>(a, unit, acc[0], acc[1]);
            } else {
                store_channel<kEpi, true>(a, unit, acc[0]);
            }
        }
    }
}

template <int kVpl, int kUnits, int kRowsPerUnit>
__device__ void compute_dispatch(const ChainOp& op, const int4 (&tile)[kTileSlots], const bf16_t* xs,
                                 const bf16_t* gs, float inverse) {
    if constexpr (kRowsPerUnit == 2) {
        if (op.epilogue == kEpiSiluFused) {
            compute_tiles<kVpl, kUnits, 2, kEpiSiluFused>(op, tile, xs, gs, inverse);
        } else {
            compute_tiles<kVpl, kUnits, 2, kEpiSiluRounded>(op, tile, xs, gs, inverse);
        }
    } else {
        switch (op.epilogue) {
            case kEpiStore: compute_tiles<kVpl, kUnits, 1, kEpiStore>(op, tile, xs, gs, inverse); break;
            case kEpiAddFma: compute_tiles<kVpl, kUnits, 1, kEpiAddFma>(op, tile, xs, gs, inverse); break;
            case kEpiAddRounded: compute_tiles<kVpl, kUnits, 1, kEpiAddRounded>(op, tile, xs, gs, inverse); break;
            case kEpiBias: compute_tiles<kVpl, kUnits, 1, kEpiBias>(op, tile, xs, gs, inverse); break;
            case kEpiBiasSilu: compute_tiles<kVpl, kUnits, 1, kEpiBiasSilu>(op, tile, xs, gs, inverse); break;
            case kEpiBiasAdd: compute_tiles<kVpl, kUnits, 1, kEpiBiasAdd>(op, tile, xs, gs, inverse); break;
            default: break;
        }
    }
}

__global__ __launch_bounds__(kThreads, 1) void persistent_chain_kernel(const ChainOp* ops, int count,
                                                                       ChainState st) {
    __shared__ uint4 x_lds[kMaxIn * 2 / 16];
    __shared__ uint4 g_lds[kMaxIn * 2 / 16];
    __shared__ float partial_lds[kThreads];
    __shared__ float inverse_lds;
    int4 tile[kTileSlots];
    if (count > 0) issue(ops[0], tile);
    for (int i = 0; i < count; ++i) {
        trace_phase(st, i, 0);
        const ChainOp op = ops[i];
        const int chunks = op.in_features * 2 / 16;
        for (int c = threadIdx.x; c < chunks; c += kThreads) {
            // the activation was written by other workgroups: device-coherent loads
            const uint32_t* src = reinterpret_cast<const uint32_t*>(op.input) + 4 * c;
            uint4 v;
            v.x = __hip_atomic_load(src + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            x_lds[c] = v;
            if (op.norm_weight != nullptr) g_lds[c] = reinterpret_cast<const uint4*>(op.norm_weight)[c];
        }
        __syncthreads();
        trace_phase(st, i, 1);
        const bf16_t* xs = reinterpret_cast<const bf16_t*>(x_lds);
        const bf16_t* gs = reinterpret_cast<const bf16_t*>(g_lds);
        if (op.norm_weight != nullptr) {
            // RMSNorm statistic with the reference's 256-thread order
            // (talker_kernels.cu:36-41): thread t sums x[t], x[t+256], ...;
            // then the block tree, folded by wave 0 exactly as wave_tree256.
            const bf16_t* xl = reinterpret_cast<const bf16_t*>(x_lds);
            float sq = 0.0f;
            for (int k = threadIdx.x; k < op.in_features; k += kThreads) {
                const float v = bf2f(xl[k]);
                sq = fmaf(v, v, sq);
            }
            partial_lds[threadIdx.x] = sq;
            __syncthreads();
            if (threadIdx.x < 64) {
                float p0 = partial_lds[threadIdx.x], p1 = partial_lds[threadIdx.x + 64];
                const float p2 = partial_lds[threadIdx.x + 128], p3 = partial_lds[threadIdx.x + 192];
                p0 += p2;
                p1 += p3;
                float value = p0 + p1;
#pragma unroll
                for (int offset = 32; offset > 0; offset >>= 1) value += __shfl_down(value, offset, 64);
                if (threadIdx.x == 0) {
                    inverse_lds = 1.0f / sqrtf(value / static_cast<float>(op.in_features) + op.norm_epsilon);
                }
            }
        }
        __syncthreads();
        trace_phase(st, i, 2);
        const float inverse = inverse_lds;
        switch (op.kind) {
            case kChainK2048U2: compute_dispatch<4, 2, 1>(op, tile, xs, gs, inverse); break;
            case kChainK2048U1: compute_dispatch<4, 1, 1>(op, tile, xs, gs, inverse); break;
            case kChainK2048Pair3: compute_dispatch<4, 3, 2>(op, tile, xs, gs, inverse); break;
            case kChainK6144U1: compute_dispatch<12, 1, 1>(op, tile, xs, gs, inverse); break;
            default: break;
        }
        trace_phase(st, i, 3);
        if (i + 1 < count) {
            grid_arrive(st, static_cast<unsigned>(i));
            issue(ops[i + 1], tile);
            trace_phase(st, i, 4);
            grid_wait(st, static_cast<unsigned>(i));
        }
        trace_phase(st, i, 5);
    }
}


// Zeroes a larger synchronization area (counters, group counters, flags).
__global__ void zero_words_kernel(unsigned* words, int count) {
    for (int i = threadIdx.x; i < count; i += blockDim.x) words[i] = 0u;
}

// Barrier cost probe: `count` barriers, no work.  variant 0: agent fences +
// relaxed atomics (the chain's barrier); 1: relaxed atomics without fences;
// 2: release add / acquire poll; 3: variant 0 polling without sleep;
// 4: variant 0 plus a 4 KB activation re-read after each barrier.
template <int kVariant>
__global__ __launch_bounds__(kThreads, 1) void barrier_probe_kernel(int count, ChainState st, const uint4* x,
                                                                    uint4* sink) {
    __shared__ uint4 lds[256];
    uint4 acc = make_uint4(0, 0, 0, 0);
    for (int i = 0; i < count; ++i) {
        __syncthreads();
        if constexpr (kVariant == 5) {
            // two-level counter: 8 groups (one per XCD under round-robin
            // dispatch), the last arriver of a group arrives globally
            if (threadIdx.x == 0) {
                unsigned* group = st.barrier + 32 * (1 + (blockIdx.x & 7));
                const unsigned members = (gridDim.x + 7 - (blockIdx.x & 7)) / 8;
                const unsigned old = __hip_atomic_fetch_add(group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (old + 1 == static_cast<unsigned>(i + 1) * members) {
                    __hip_atomic_fetch_add(st.barrier, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
                const unsigned target = static_cast<unsigned>(i + 1) * 8u;
                unsigned spins = 0;
                while (__hip_atomic_load(st.barrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > (1u << 25)) {
                        __hip_atomic_store(st.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __syncthreads();
            continue;
        }
        if constexpr (kVariant == 6) {
            // flag array: each workgroup publishes its epoch in its own slot;
            // wave 0 polls every slot in parallel
            unsigned* flags = st.barrier + 32 * 16;
            const unsigned epoch = static_cast<unsigned>(i + 1);
            if (threadIdx.x == 0) __hip_atomic_store(flags + blockIdx.x, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (threadIdx.x < 64) {
                unsigned spins = 0;
                while (true) {
                    bool ok = true;
                    for (int b = threadIdx.x; b < static_cast<int>(gridDim.x); b += 64) {
                        ok = ok && __hip_atomic_load(flags + b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= epoch;
                    }
                    if (__all(ok)) break;
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > (1u << 25)) {
                        if (threadIdx.x == 0) __hip_atomic_store(st.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __syncthreads();
            continue;
        }
        if (threadIdx.x == 0) {
            const unsigned target = static_cast<unsigned>(i + 1) * gridDim.x;
            if constexpr (kVariant == 0 || kVariant == 3 || kVariant == 4) __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
            if constexpr (kVariant == 2) {
                __hip_atomic_fetch_add(st.barrier, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                __hip_atomic_fetch_add(st.barrier, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            unsigned spins = 0;
            while (true) {
                const unsigned seen = kVariant == 2
                    ? __hip_atomic_load(st.barrier, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT)
                    : __hip_atomic_load(st.barrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (seen >= target) break;
                if constexpr (kVariant != 3) __builtin_amdgcn_s_sleep(2);
                if (++spins > (1u << 24)) {
                    __hip_atomic_store(st.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
            if constexpr (kVariant == 0 || kVariant == 3 || kVariant == 4) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        }
        __syncthreads();
        if constexpr (kVariant == 4) {
            lds[threadIdx.x] = x[threadIdx.x];
            __syncthreads();
            acc.x ^= lds[(threadIdx.x + i) & 255].x;
        }
    }
    if (acc.x == 0x12345678u) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_barrier_probe(int variant, int count, unsigned* sync, const void* x, void* sink, int workgroups,
                                hipStream_t stream) {
    zero_words_kernel<<<1, 256, 0, stream>>>(sync, 32 * 16 + 1024);
    ChainState state{sync, reinterpret_cast<int*>(sync + 1), nullptr};
    void* args[] = {&count, &state, &x, &sink};
    const void* fn = nullptr;
    switch (variant) {
        case 0: fn = reinterpret_cast<const void*>(barrier_probe_kernel<0>); break;
        case 1: fn = reinterpret_cast<const void*>(barrier_probe_kernel<1>); break;
        case 2: fn = reinterpret_cast<const void*>(barrier_probe_kernel<2>); break;
        case 3: fn = reinterpret_cast<const void*>(barrier_probe_kernel<3>); break;
        case 4: fn = reinterpret_cast<const void*>(barrier_probe_kernel<4>); break;
        case 5: fn = reinterpret_cast<const void*>(barrier_probe_kernel<5>); break;
        case 6: fn = reinterpret_cast<const void*>(barrier_probe_kernel<6>); break;
        default: return hipErrorInvalidValue;
    }
    return hipLaunchCooperativeKernel(fn, dim3(workgroups), dim3(kThreads), args, 0, stream);
}

// Picks the chain kind for a GEMV on a grid of `workgroups`; -1 if unsupported.
int chain_kind_for(int in_features, int out_features, int epilogue, int workgroups) {
    const int half_waves = workgroups * kHalfWaves;
    const bool pair = epilogue == kEpiSiluFused || epilogue == kEpiSiluRounded;
    if (in_features == 2048 && pair && out_features <= 3 * half_waves) return kChainK2048Pair3;
    if (pair) return -1;
    if (in_features == 2048 && out_features <= half_waves) return kChainK2048U1;
    if (in_features == 2048 && out_features <= 2 * half_waves) return kChainK2048U2;
    if (in_features == 6144 && out_features <= half_waves) return kChainK6144U1;
    return -1;
}

int chain_workgroups() {
    int device = 0;
    hipDeviceProp_t props{};
    if (hipGetDevice(&device) != hipSuccess || hipGetDeviceProperties(&props, device) != hipSuccess) return 0;
    return props.multiProcessorCount;
}

// ops: device array of `count` ChainOp; sync: device scratch of
// kChainSyncWords words (global counter, status, 8 group counters).
hipError_t launch_persistent_chain(const ChainOp* ops, int count, unsigned* sync, int workgroups,
                                   hipStream_t stream, unsigned long long* trace) {
    if (ops == nullptr || count <= 0 || sync == nullptr || workgroups <= 0) return hipErrorInvalidValue;
    zero_words_kernel<<<1, 256, 0, stream>>>(sync, kChainSyncWords);
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    ChainState state{sync, reinterpret_cast<int*>(sync + 1), trace};
    void* args[] = {const_cast<ChainOp**>(&ops), &count, &state};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(persistent_chain_kernel), dim3(workgroups),
                                      dim3(kThreads), args, 0, stream);
}

}  // namespace q3

using namespace q3;

// Diagnostic: microseconds per grid barrier of the persistent kernel's
// barrier variants (see barrier_probe_kernel).
extern "C" QWEN3_TTS_API int32_t qwen3_tts_benchmark_grid_barrier(int32_t device_index, int32_t variant,
                                                                  int32_t barriers, int32_t workgroups,
                                                                  double* microseconds_per_barrier,
                                                                  char* error, size_t cap) {
    auto fail = [&](const char* m) {
        if (error && cap) std::snprintf(error, cap, "%s", m);
        return QWEN3_TTS_TALKER_STATUS_CUDA;
    };
    if (microseconds_per_barrier == nullptr || barriers <= 0) return fail("invalid arguments");
    if (hipSetDevice(device_index) != hipSuccess) return fail("hipSetDevice");
    if (workgroups <= 0) workgroups = chain_workgroups();
    unsigned* sync = nullptr;
    void* x = nullptr;
    void* sink = nullptr;
    hipEvent_t a = nullptr, b = nullptr;
    hipError_t st = hipMalloc(&sync, (32 * 16 + 1024) * sizeof(unsigned));
    if (st == hipSuccess) st = hipMalloc(&x, 4096);
    if (st == hipSuccess) st = hipMalloc(&sink, 16 * static_cast<size_t>(workgroups));
    if (st == hipSuccess) st = hipMemset(x, 0, 4096);
    if (st == hipSuccess) st = hipEventCreate(&a);
    if (st == hipSuccess) st = hipEventCreate(&b);
    if (st == hipSuccess) st = launch_barrier_probe(variant, 16, sync, x, sink, workgroups, nullptr);
    if (st == hipSuccess) st = hipEventRecord(a, nullptr);
    if (st == hipSuccess) st = launch_barrier_probe(variant, barriers, sync, x, sink, workgroups, nullptr);
    if (st == hipSuccess) st = hipEventRecord(b, nullptr);
    if (st == hipSuccess) st = hipEventSynchronize(b);
    float ms = 0.0f;
    if (st == hipSuccess) st = hipEventElapsedTime(&ms, a, b);
    int status = 0;
    if (st == hipSuccess) st = hipMemcpy(&status, sync + 1, sizeof(int), hipMemcpyDeviceToHost);
    if (a) (void)hipEventDestroy(a);
    if (b) (void)hipEventDestroy(b);
    if (sync) (void)hipFree(sync);
    if (x) (void)hipFree(x);
    if (sink) (void)hipFree(sink);
    if (st != hipSuccess) return fail(hipGetErrorString(st));
    if (status != 0) return fail("barrier wait timed out");
    *microseconds_per_barrier = ms * 1000.0 / barriers;
    if (error && cap) error[0] = 0;
    return QWEN3_TTS_TALKER_STATUS_OK;
}
