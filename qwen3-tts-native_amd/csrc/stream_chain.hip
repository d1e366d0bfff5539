// Warp-specialized persistent int8 GEMV chain for gfx950 ("stream chain").
//
// One cooperative launch runs a list of dependent GEMVs (a talker step's
// QKV -> O -> gate/up -> down, 28 times) on one 512-thread workgroup per CU:
//
//   waves 4..7 (loaders) stream this workgroup's weight rows of every GEMV,
//     in op order, into a ring of 4 x 32 KB LDS slots with global_load_lds
//     (128-bit direct-to-LDS loads: no VGPR staging).  They never wait for
//     activations, only for a free slot, so weights keep flowing from HBM
//     while the compute waves sit at a grid barrier: up to 128 KB per CU
//     (32 MB chip-wide, ~4 us of HBM time) ahead of the computation.
//   waves 0..3 (compute) per GEMV: wait for the grid barrier of the previous
//     GEMV, stage the activation vector into LDS with device-coherent loads,
//     reduce the RMSNorm statistic (reference 256-thread order), pull their
//     lane slice into registers, then consume the slots: each half-wave owns
//     whole rows and evaluates them in the reference's exact lane order
//     (lane l: 16-byte vectors l, l+32, ...; fresh 16-term fma chains; fold
//     16..1) reading the weights from LDS -- bit-identical to gemv.hip.
//
// Each workgroup owns a contiguous block of rows (pairs of gate/up rows) of
// every GEMV, so a slot is filled from one or two contiguous byte ranges.
// A chunk is at most 32 KB and at most 16 units.
//
// Synchronization: loader -> compute through per-slot fill counters in LDS,
// compute -> loader through per-slot release counters; compute waves meet
// through an LDS counter; workgroups meet through a two-level grid counter
// (per-XCD group, then global).  Every wait is bounded: a timeout raises an
// abort flag (LDS and global) that makes every other wait return, so the
// grid always drains.
#include "q3_common.hpp"
#include "gemv_device.hpp"

#include "../../include/qwen3_tts_native.h"

#include <cstdio>

namespace q3 {
namespace {

using namespace gemv_detail;

constexpr int kStreamThreads = 512;
constexpr int kComputeWaves = 4;
constexpr int kLoaderWaves = 4;
constexpr int kSlots = 4;
constexpr int kSlotBytes = 32 * 1024;
constexpr int kMaxUnitsPerChunk = 16;
constexpr int kMaxK = 6144;
constexpr int kGroupsX = 8;
constexpr int kLine = 32;  // words between global counters (128 bytes)
constexpr unsigned kSpinLimit = 1u << 24;

struct StreamState {
    unsigned* sync;  // [0] global counter, [1] status, [kLine*(1+g)] group counters
    unsigned long long* trace;
};

struct Lds {
    uint4 slot[kSlots][kSlotBytes / 16];
    uint4 x[kMaxK * 2 / 16];
    uint4 gain[kMaxK * 2 / 16];
    float partial[256];
    float inverse;
    unsigned full[kSlots];     // loader waves' completions per slot (monotone)
    unsigned freed[kSlots];    // compute waves' releases per slot (monotone)
    unsigned compute_sync;     // compute-wave barrier counter
    unsigned grid_phase;       // last grid barrier observed by compute wave 0
    unsigned abort;
};

__device__ __forceinline__ unsigned lds_load(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ void lds_add(unsigned* p, unsigned v) {
    __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ bool aborted(Lds& s, const StreamState& st) {
    return lds_load(&s.abort) != 0u;
}

__device__ void raise_abort(Lds& s, const StreamState& st) {
    __hip_atomic_store(&s.abort, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(reinterpret_cast<int*>(st.sync + 1), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Wait (whole wave) until *p >= target; false on abort / timeout.
__device__ bool wave_wait_lds(Lds& s, const StreamState& st, const unsigned* p, unsigned target) {
    unsigned spins = 0;
    while (lds_load(p) < target) {
        if (aborted(s, st)) return false;
        __builtin_amdgcn_s_sleep(1);
        if (++spins > kSpinLimit) {
            raise_abort(s, st);
            return false;
        }
    }
    return true;
}

// Work of one GEMV for workgroup b: units [u0, u1), chunked.
struct Plan {
    int u0, units, rows_per_unit, upc, chunks, k;
};

__device__ __forceinline__ Plan plan_of(const ChainOp& op) {
    Plan p;
    const bool pair = op.epilogue == kEpiSiluFused || op.epilogue == kEpiSiluRounded;
    p.rows_per_unit = pair ? 2 : 1;
    p.k = op.in_features;
    const long long total = op.out_features;
    p.u0 = static_cast<int>(total * blockIdx.x / gridDim.x);
    const int u1 = static_cast<int>(total * (blockIdx.x + 1) / gridDim.x);
    p.units = u1 - p.u0;
    int upc = kSlotBytes / (p.rows_per_unit * p.k);
    if (upc > kMaxUnitsPerChunk) upc = kMaxUnitsPerChunk;
    if (upc < 1) upc = 1;
    p.upc = upc;
    p.chunks = (p.units + upc - 1) / upc;
    return p;
}

__device__ __forceinline__ void waitcnt_vm(int n) {
    // s_waitcnt with only the vector-memory counter constrained (gfx9 encoding:
    // vmcnt[3:0] in bits 3:0, expcnt = 7 and lgkmcnt = 15 mean "no wait").
    switch (n) {
        case 0: __builtin_amdgcn_s_waitcnt(0xF70); break;
        case 1: __builtin_amdgcn_s_waitcnt(0xF71); break;
        case 2: __builtin_amdgcn_s_waitcnt(0xF72); break;
        case 3: __builtin_amdgcn_s_waitcnt(0xF73); break;
        case 4: __builtin_amdgcn_s_waitcnt(0xF74); break;
        case 5: __builtin_amdgcn_s_waitcnt(0xF75); break;
        case 6: __builtin_amdgcn_s_waitcnt(0xF76); break;
        case 7: __builtin_amdgcn_s_waitcnt(0xF77); break;
        default: __builtin_amdgcn_s_waitcnt(0xF78); break;
    }
}

// ---------------------------------------------------------------------------
// Loader waves: fill slots chunk after chunk.  A chunk of n units copies the
// gate (or only) rows [u, u+n) and, for pairs, the up rows [out+u, out+u+n);
// in the slot, row r of unit j sits at (r * n + j) * k bytes.  Wave w copies
// 1 KB blocks w, w+4, ... with one global_load_lds_dwordx4 each.  Two chunks
// stay in flight per wave; a chunk is published (fill counter += 1) once its
// loads have landed.
// ---------------------------------------------------------------------------
__device__ void loader(Lds& s, const StreamState& st, const ChainOp* ops, int count) {
    const int w = (threadIdx.x >> 6) - kComputeWaves;
    const int lane = threadIdx.x & 63;
    unsigned chunk_index = 0;
    int pending_slot = -1;
    for (int i = 0; i < count; ++i) {
        const ChainOp op = ops[i];
        const Plan p = plan_of(op);
        for (int c = 0; c < p.chunks; ++c, ++chunk_index) {
            const int slot = static_cast<int>(chunk_index % kSlots);
            const unsigned round = chunk_index / kSlots;
            if (round > 0 && !wave_wait_lds(s, st, &s.freed[slot], round * kComputeWaves)) return;
            const int ub = p.u0 + c * p.upc;
            const int n = min(p.upc, p.units - c * p.upc);
            const int range_bytes = n * p.k;            // multiple of 1 KB
            const int blocks = p.rows_per_unit * range_bytes / 1024;
            int issued = 0;
            for (int b = w; b < blocks; b += kLoaderWaves) {
                const int r = (b * 1024) / range_bytes;  // 0 = gate/only rows, 1 = up rows
                const int off = b * 1024 - r * range_bytes;
                const int row0 = r == 0 ? ub : op.out_features + ub;
                const char* src = reinterpret_cast<const char*>(op.weight) + static_cast<size_t>(row0) * p.k + off +
                                  lane * 16;
                char* dst = reinterpret_cast<char*>(&s.slot[slot][0]) + b * 1024;
                __builtin_amdgcn_global_load_lds(src, (__attribute__((address_space(3))) void*)(dst), 16,
                                                 0, 0);
                ++issued;
            }
            // the previous chunk is complete once at most `issued` loads remain
            if (pending_slot >= 0) {
                waitcnt_vm(issued);
                if (lane == 0) lds_add(&s.full[pending_slot], 1u);
            }
            pending_slot = slot;
            if (aborted(s, st)) return;
        }
    }
    if (pending_slot >= 0) {
        waitcnt_vm(0);
        if (lane == 0) lds_add(&s.full[pending_slot], 1u);
    }
}

// ---------------------------------------------------------------------------
// Compute waves
// ---------------------------------------------------------------------------
__device__ bool compute_sync(Lds& s, const StreamState& st, unsigned& epoch) {
    ++epoch;
    __builtin_amdgcn_s_waitcnt(0);  // this wave's LDS and memory traffic is complete
    if ((threadIdx.x & 63) == 0) lds_add(&s.compute_sync, 1u);
    return wave_wait_lds(s, st, &s.compute_sync, epoch * kComputeWaves);
}

__device__ void trace_at(const StreamState& st, int op, int phase) {
    if (st.trace != nullptr && blockIdx.x == 0 && threadIdx.x == 0 && op < 256) st.trace[op * 8 + phase] = wall_clock64();
}

// One half-wave evaluates one unit from the slot, reference lane order.
template <int kVpl, int kRpu, int kEpi>
__device__ __forceinline__ void unit_from_slot(const ChainOp& op, const uint4* slot, int n, int j, int unit,
                                               const float (*xf)[16], const uint32_t (*xp)[8]) {
    constexpr bool kPacked = kVpl > 6;
    constexpr int kIn = kVpl * 512;
    const int lane = threadIdx.x & 31;
    float acc[kRpu];
#pragma unroll
    for (int r = 0; r < kRpu; ++r) {
        const uint4* row = slot + static_cast<size_t>(r * n + j) * (kIn / 16);
        acc[r] = 0.0f;
#pragma unroll
        for (int i = 0; i < kVpl; ++i) {
            const uint4 q = row[lane + 32 * i];
            const int4 wv = make_int4(static_cast<int>(q.x), static_cast<int>(q.y), static_cast<int>(q.z),
                                      static_cast<int>(q.w));
            if constexpr (kPacked) {
                acc[r] += chain16_packed(wv, xp[i]);
            } else {
                acc[r] += chain16(wv, xf[i]);
            }
        }
        acc[r] = fold32(acc[r]);
    }
    if (lane == 0) {
        GemvArgs a;
        a.scales = op.scales;
        a.bias = op.bias;
        a.out16 = op.out16;
        a.out_features = op.out_features;
        if constexpr (kRpu == 2) {
            store_gate_up<kEpi, true>(a, unit, acc[0], acc[1]);
        } else {
            store_channel<kEpi, true>(a, unit, acc[0]);
        }
    }
}

template <int kVpl, int kRpu, int kEpi>
__device__ bool compute_op(Lds& s, const StreamState& st, const ChainOp& op, const Plan& p, unsigned& chunk_index,
                           float inverse) {
    constexpr bool kPacked = kVpl > 6;
    const int lane = threadIdx.x & 31;
    const int hw = threadIdx.x >> 5;  // 0..7
    const bf16_t* xs = reinterpret_cast<const bf16_t*>(s.x);
    const bf16_t* gs = reinterpret_cast<const bf16_t*>(s.gain);
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
    for (int c = 0; c < p.chunks; ++c, ++chunk_index) {
        const int slot = static_cast<int>(chunk_index % kSlots);
        const unsigned round = chunk_index / kSlots;
        if (!wave_wait_lds(s, st, &s.full[slot], (round + 1) * kLoaderWaves)) return false;
        const int n = min(p.upc, p.units - c * p.upc);
        for (int j = hw; j < n; j += 8) {
            unit_from_slot<kVpl, kRpu, kEpi>(op, s.slot[slot], n, j, p.u0 + c * p.upc + j, xf, xp);
        }
        __builtin_amdgcn_s_waitcnt(0);  // slot reads done before release
        if ((threadIdx.x & 63) == 0) lds_add(&s.freed[slot], 1u);
    }
    return true;
}

template <int kVpl>
__device__ bool compute_dispatch_epi(Lds& s, const StreamState& st, const ChainOp& op, const Plan& p,
                                     unsigned& chunk_index, float inverse) {
    switch (op.epilogue) {
        case kEpiStore: return compute_op<kVpl, 1, kEpiStore>(s, st, op, p, chunk_index, inverse);
        case kEpiAddFma: return compute_op<kVpl, 1, kEpiAddFma>(s, st, op, p, chunk_index, inverse);
        case kEpiAddRounded: return compute_op<kVpl, 1, kEpiAddRounded>(s, st, op, p, chunk_index, inverse);
        case kEpiSiluFused: return compute_op<kVpl, 2, kEpiSiluFused>(s, st, op, p, chunk_index, inverse);
        case kEpiSiluRounded: return compute_op<kVpl, 2, kEpiSiluRounded>(s, st, op, p, chunk_index, inverse);
        case kEpiBias: return compute_op<kVpl, 1, kEpiBias>(s, st, op, p, chunk_index, inverse);
        case kEpiBiasSilu: return compute_op<kVpl, 1, kEpiBiasSilu>(s, st, op, p, chunk_index, inverse);
        case kEpiBiasAdd: return compute_op<kVpl, 1, kEpiBiasAdd>(s, st, op, p, chunk_index, inverse);
        default: return false;
    }
}

// Grid barrier by compute wave 0, lane 0; the other compute waves follow
// through s.grid_phase.
__device__ void grid_arrive(const StreamState& st, unsigned index) {
    const unsigned g = blockIdx.x % kGroupsX;
    const unsigned members = (gridDim.x - g + kGroupsX - 1) / kGroupsX;
    unsigned* group = st.sync + kLine * (1 + g);
    const unsigned old = __hip_atomic_fetch_add(group, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old + 1 == (index + 1) * members) {
        __hip_atomic_fetch_add(st.sync, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

__device__ bool grid_wait(Lds& s, const StreamState& st, unsigned index) {
    if (threadIdx.x == 0) {
        const unsigned groups = gridDim.x < kGroupsX ? gridDim.x : kGroupsX;
        const unsigned target = (index + 1) * groups;
        unsigned spins = 0;
        bool ok = true;
        while (__hip_atomic_load(st.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < target) {
            __builtin_amdgcn_s_sleep(1);
            ++spins;
            if ((spins & 255u) == 0 &&
                (__hip_atomic_load(reinterpret_cast<int*>(st.sync + 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0 ||
                 aborted(s, st))) {
                ok = false;
                break;
            }
            if (spins > kSpinLimit) {
                raise_abort(s, st);
                ok = false;
                break;
            }
        }
        if (!ok) raise_abort(s, st);
        __hip_atomic_store(&s.grid_phase, index + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (threadIdx.x < 64) return !aborted(s, st);
    return wave_wait_lds(s, st, &s.grid_phase, index + 1) && !aborted(s, st);
}

__device__ void compute(Lds& s, const StreamState& st, const ChainOp* ops, int count) {
    unsigned chunk_index = 0;
    unsigned epoch = 0;
    for (int i = 0; i < count; ++i) {
        trace_at(st, i, 0);
        const ChainOp op = ops[i];
        const Plan p = plan_of(op);
        // stage x (device-coherent: written by other workgroups) and the gain
        const int chunks = op.in_features * 2 / 16;
        for (int c = threadIdx.x; c < chunks; c += kComputeWaves * 64) {
            const uint32_t* src = reinterpret_cast<const uint32_t*>(op.input) + 4 * c;
            uint4 v;
            v.x = __hip_atomic_load(src + 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.y = __hip_atomic_load(src + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.z = __hip_atomic_load(src + 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            v.w = __hip_atomic_load(src + 3, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s.x[c] = v;
            if (op.norm_weight != nullptr) s.gain[c] = reinterpret_cast<const uint4*>(op.norm_weight)[c];
        }
        if (!compute_sync(s, st, epoch)) return;
        trace_at(st, i, 1);
        float inverse = 1.0f;
        if (op.norm_weight != nullptr) {
            // RMSNorm statistic, reference 256-thread order (talker_kernels.cu:36-41)
            const bf16_t* xl = reinterpret_cast<const bf16_t*>(s.x);
            float sq = 0.0f;
            for (int k = threadIdx.x; k < op.in_features; k += 256) {
                const float v = bf2f(xl[k]);
                sq = fmaf(v, v, sq);
            }
            s.partial[threadIdx.x] = sq;
            if (!compute_sync(s, st, epoch)) return;
            if (threadIdx.x < 64) {
                float p0 = s.partial[threadIdx.x], p1 = s.partial[threadIdx.x + 64];
                const float p2 = s.partial[threadIdx.x + 128], p3 = s.partial[threadIdx.x + 192];
                p0 += p2;
                p1 += p3;
                float value = p0 + p1;
#pragma unroll
                for (int offset = 32; offset > 0; offset >>= 1) value += __shfl_down(value, offset, 64);
                if (threadIdx.x == 0) s.inverse = 1.0f / sqrtf(value / static_cast<float>(op.in_features) + op.norm_epsilon);
            }
            if (!compute_sync(s, st, epoch)) return;
            inverse = s.inverse;
        }
        trace_at(st, i, 2);
        bool ok = false;
        switch (op.in_features / 512) {
            case 2: ok = compute_dispatch_epi<2>(s, st, op, p, chunk_index, inverse); break;
            case 4: ok = compute_dispatch_epi<4>(s, st, op, p, chunk_index, inverse); break;
            case 6: ok = compute_dispatch_epi<6>(s, st, op, p, chunk_index, inverse); break;
            case 12: ok = compute_dispatch_epi<12>(s, st, op, p, chunk_index, inverse); break;
            default: break;
        }
        if (!ok) {
            raise_abort(s, st);
            return;
        }
        trace_at(st, i, 3);
        if (i + 1 < count) {
            if (!compute_sync(s, st, epoch)) return;  // all compute waves' outputs stored
            if (threadIdx.x == 0) grid_arrive(st, static_cast<unsigned>(i));
            trace_at(st, i, 4);
            if (!grid_wait(s, st, static_cast<unsigned>(i))) return;
        }
        trace_at(st, i, 5);
    }
}

__global__ __launch_bounds__(kStreamThreads, 1) void stream_chain_kernel(const ChainOp* ops, int count,
                                                                         StreamState st) {
    extern __shared__ __align__(16) unsigned char lds_raw[];
    Lds& s = *reinterpret_cast<Lds*>(lds_raw);
    if (threadIdx.x < kSlots) {
        s.full[threadIdx.x] = 0u;
        s.freed[threadIdx.x] = 0u;
    }
    if (threadIdx.x == 0) {
        s.compute_sync = 0u;
        s.grid_phase = 0u;
        s.abort = 0u;
    }
    __syncthreads();
    if (threadIdx.x < kComputeWaves * 64) {
        compute(s, st, ops, count);
    } else {
        loader(s, st, ops, count);
    }
}

__global__ void zero_stream_sync(unsigned* words, int count) {
    for (int i = threadIdx.x; i < count; i += blockDim.x) words[i] = 0u;
}

}  // namespace

bool stream_chain_supports(int in_features, int out_features, int epilogue) {
    const int vpl = in_features / 512;
    if (in_features % 512 != 0 || !(vpl == 2 || vpl == 4 || vpl == 6 || vpl == 12)) return false;
    const int rpu = (epilogue == kEpiSiluFused || epilogue == kEpiSiluRounded) ? 2 : 1;
    return out_features > 0 && rpu * in_features <= kSlotBytes;
}

size_t stream_chain_lds_bytes() { return sizeof(Lds); }

hipError_t launch_stream_chain(const ChainOp* ops, int count, unsigned* sync, int workgroups, hipStream_t stream,
                               unsigned long long* trace) {
    if (ops == nullptr || count <= 0 || sync == nullptr || workgroups <= 0) return hipErrorInvalidValue;
    static std::atomic<unsigned long long> configured{0};
    hipError_t st = set_dynamic_lds_once(configured, reinterpret_cast<const void*>(stream_chain_kernel),
                                         static_cast<int>(sizeof(Lds)));
    if (st != hipSuccess) return st;
    zero_stream_sync<<<1, 256, 0, stream>>>(sync, kChainSyncWords);
    st = hipGetLastError();
    if (st != hipSuccess) return st;
    StreamState state{sync, trace};
    void* args[] = {const_cast<ChainOp**>(&ops), &count, &state};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(stream_chain_kernel), dim3(workgroups),
                                      dim3(kStreamThreads), args, sizeof(Lds), stream);
}

}  // namespace q3
