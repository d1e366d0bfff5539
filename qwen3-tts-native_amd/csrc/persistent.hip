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
    unsigned* barrier;  // zeroed before the launch
    int* status;        // set to 1 if a barrier wait timed out
};

// Grid-wide barrier with a bounded wait: monotone counter, target =
// (index + 1) * gridDim.x.  Agent-scope release before arriving and acquire
// after observing the target make every workgroup's stores visible to every
// other XCD.  A wait that exceeds ~1 s records an error and lets the grid
// drain instead of hanging.
__device__ void grid_barrier(const ChainState& st, unsigned index) {
    __syncthreads();
    if (threadIdx.x == 0) {
        const unsigned target = (index + 1) * gridDim.x;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        __hip_atomic_fetch_add(st.barrier, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        unsigned spins = 0;
        while (__hip_atomic_load(st.barrier, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(2);
            ++spins;
            // after one timeout every later barrier stops waiting, so the
            // grid always drains
            if ((spins & 1023u) == 0 &&
                __hip_atomic_load(st.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
                break;
            }
            if (spins > (1u << 24)) {
                __hip_atomic_store(st.status, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
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
                store_gate_up<kEpi>(a, unit, acc[0], acc[1]);
            } else {
                store_channel<kEpi>(a, unit, acc[0]);
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
    __shared__ float inverse_lds;
    int4 tile[kTileSlots];
    if (count > 0) issue(ops[0], tile);
    for (int i = 0; i < count; ++i) {
        const ChainOp op = ops[i];
        const int chunks = op.in_features * 2 / 16;
        for (int c = threadIdx.x; c < chunks; c += kThreads) {
            x_lds[c] = reinterpret_cast<const uint4*>(op.input)[c];
            if (op.norm_weight != nullptr) g_lds[c] = reinterpret_cast<const uint4*>(op.norm_weight)[c];
        }
        __syncthreads();
        const bf16_t* xs = reinterpret_cast<const bf16_t*>(x_lds);
        const bf16_t* gs = reinterpret_cast<const bf16_t*>(g_lds);
        if (op.norm_weight != nullptr && threadIdx.x < 64) {
            const float inv = wave_inverse_rms(xs, op.in_features, op.norm_epsilon);
            if (threadIdx.x == 0) inverse_lds = inv;
        }
        __syncthreads();
        const float inverse = inverse_lds;
        switch (op.kind) {
            case kChainK2048U2: compute_dispatch<4, 2, 1>(op, tile, xs, gs, inverse); break;
            case kChainK2048U1: compute_dispatch<4, 1, 1>(op, tile, xs, gs, inverse); break;
            case kChainK2048Pair3: compute_dispatch<4, 3, 2>(op, tile, xs, gs, inverse); break;
            case kChainK6144U1: compute_dispatch<12, 1, 1>(op, tile, xs, gs, inverse); break;
            default: break;
        }
        if (i + 1 < count) issue(ops[i + 1], tile);
        grid_barrier(st, static_cast<unsigned>(i));
    }
}

__global__ void zero_sync_kernel(unsigned* barrier, int* status) {
    if (threadIdx.x == 0) {
        *barrier = 0u;
        *status = 0;
    }
}

}  // namespace

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

// ops: device array of `count` ChainOp; sync: device scratch of 2 ints.
hipError_t launch_persistent_chain(const ChainOp* ops, int count, unsigned* sync, int workgroups,
                                   hipStream_t stream) {
    if (ops == nullptr || count <= 0 || sync == nullptr || workgroups <= 0) return hipErrorInvalidValue;
    zero_sync_kernel<<<1, 64, 0, stream>>>(sync, reinterpret_cast<int*>(sync + 1));
    hipError_t st = hipGetLastError();
    if (st != hipSuccess) return st;
    ChainState state{sync, reinterpret_cast<int*>(sync + 1)};
    void* args[] = {const_cast<ChainOp**>(&ops), &count, &state};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(persistent_chain_kernel), dim3(workgroups),
                                      dim3(kThreads), args, 0, stream);
}

}  // namespace q3
