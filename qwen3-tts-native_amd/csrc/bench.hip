// Benchmark exports of the int8 decode path, gfx950: single-GEMV bandwidth
// with rotating weight copies and the talker-step GEMV chain.  Timing uses
// hipEvents on one stream; inputs are synthetic and generated on the device.
#include "q3_common.hpp"


#include "../../include/qwen3_tts_native.h"

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

namespace q3 {
namespace {

void write_error(char* destination, size_t capacity, const char* message) {
    if (destination != nullptr && capacity != 0) std::snprintf(destination, capacity, "%s", message);
}

__device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z += 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

// int8 uniform in [-127, 127], four bytes per thread step.
__global__ void fill_int8_kernel(int8_t* out, uint64_t count, uint64_t seed) {
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        out[i] = static_cast<int8_t>(static_cast<int>(mix64(seed ^ (i * 0x9e3779b97f4a7c15ULL)) % 255u) - 127);
    }
}

__global__ void fill_scale_kernel(float* out, uint64_t count, uint64_t seed) {
    for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x; i < count;
         i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
        const float u = static_cast<float>(mix64(seed + i) >> 40) * (1.0f / 16777216.0f);
        out[i] = 1.0e-3f + u * (2.0e-2f - 1.0e-3f);
    }
}

// Plain read of `bytes` (a multiple of 16) with 16-byte nontemporal loads:
// the launch-shape ceiling of a chain of streaming kernels (no arithmetic
// beyond an xor, one conditional store).
typedef int stream_i32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void read_weights_kernel(const int8_t* weights, uint64_t bytes, int* sink) {
    const stream_i32x4* p = reinterpret_cast<const stream_i32x4*>(weights);
    const uint64_t n = bytes / 16;
    stream_i32x4 acc = {0, 0, 0, 0};
#pragma unroll 4
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += gridDim.x * 256ull) {
        acc ^= __builtin_nontemporal_load(p + i);
    }
    if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x5eed5eed) sink[0] = 1;
}

int grid_for(uint64_t n) {
    const uint64_t g = (n + 255) / 256;
    return static_cast<int>(std::min<uint64_t>(g, 65536));
}

struct Mem {
    std::vector<void*> blocks;
    ~Mem() {
        for (void* p : blocks) (void)hipFree(p);
    }
    template <typename T>
    T* get(size_t count) {
        void* p = nullptr;
        check_hip(hipMalloc(&p, count * sizeof(T)), "hipMalloc(benchmark)");
        blocks.push_back(p);
        return static_cast<T*>(p);
    }
};

}  // namespace
}  // namespace q3

using namespace q3;

extern "C" {

QWEN3_TTS_API int32_t qwen3_tts_benchmark_int8_gemv(int32_t device_index, int32_t in, int32_t out, int32_t iterations,
                                                    Qwen3TtsGemvBenchmark* output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "output benchmark pointer is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    if (in <= 0 || in % 16 != 0 || out <= 0 || iterations <= 0) {
        write_error(error, cap, "in_features must be a positive multiple of 16; out and iterations positive");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    hipEvent_t start = nullptr, stop = nullptr;
    hipStream_t stream = nullptr;
    try {
        check_hip(hipSetDevice(device_index), "hipSetDevice");
        check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        Mem mem;
        const size_t matrix = static_cast<size_t>(in) * out;
        // Enough distinct copies to exceed the 256 MB last-level cache 2.5x.
        const int copies = static_cast<int>(std::max<size_t>(2, (640ull << 20) / matrix + 1));
        int8_t* w = mem.get<int8_t>(matrix * copies);
        float* s = mem.get<float>(static_cast<size_t>(out) * copies);
        bf16_t* x = mem.get<bf16_t>(in);
        bf16_t* y = mem.get<bf16_t>(out);
        fill_int8_kernel<<<grid_for(matrix * copies), 256, 0, stream>>>(w, matrix * copies, 0x5EED0001ULL);
        fill_scale_kernel<<<grid_for(static_cast<uint64_t>(out) * copies), 256, 0, stream>>>(s, static_cast<uint64_t>(out) * copies, 0x5EED0002ULL);
        check_hip(launch_fill_bf16_normal(x, in, 0x5EED0003ULL, 0.0f, 1.0f, stream), "fill x");
        check_hip(hipEventCreate(&start), "hipEventCreate");
        check_hip(hipEventCreate(&stop), "hipEventCreate");
        GemvArgs a;
        a.scales = s;
        a.input = x;
        a.out16 = y;
        a.in_features = in;
        a.out_features = out;
        a.mode = kModeExact;
        auto launch = [&](int i) {
            const int c = i % copies;
            a.weight = w + matrix * c;
            a.scales = s + static_cast<size_t>(out) * c;
            check_hip(launch_int8_gemv(a, stream), "int8 GEMV");
        };
        float cold = 0.0f, total = 0.0f;
        check_hip(hipEventRecord(start, stream), "hipEventRecord");
        launch(0);
        check_hip(hipEventRecord(stop, stream), "hipEventRecord");
        check_hip(hipEventSynchronize(stop), "hipEventSynchronize");
        check_hip(hipEventElapsedTime(&cold, start, stop), "hipEventElapsedTime");
        for (int i = 0; i < 2 * copies; ++i) launch(i);
        check_hip(hipEventRecord(start, stream), "hipEventRecord");
        for (int i = 0; i < iterations; ++i) launch(i);
        check_hip(hipEventRecord(stop, stream), "hipEventRecord");
        check_hip(hipEventSynchronize(stop), "hipEventSynchronize");
        check_hip(hipEventElapsedTime(&total, start, stop), "hipEventElapsedTime");
        const float mean = total * 1000.0f / static_cast<float>(iterations);
        output->input_features = in;
        output->output_features = out;
        output->iterations = iterations;
        output->reserved = copies;
        output->weight_bytes = matrix;
        output->cold_launch_microseconds = cold * 1000.0f;
        output->mean_launch_microseconds = mean;
        output->tera_operations_per_second = static_cast<float>(2.0 * in * out / (mean * 1.0e-6) / 1.0e12);
        (void)hipEventDestroy(start);
        (void)hipEventDestroy(stop);
        (void)hipStreamDestroy(stream);
        write_error(error, cap, "");
        return QWEN3_TTS_TALKER_STATUS_OK;
    } catch (const std::exception& e) {
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
        if (stream) (void)hipStreamDestroy(stream);
        write_error(error, cap, e.what());
        return QWEN3_TTS_TALKER_STATUS_CUDA;
    }
}

QWEN3_TTS_API int32_t qwen3_tts_benchmark_talker_step_gemvs(int32_t device_index, Qwen3TtsStepBenchmarkV1* b,
                                                            char* error, size_t cap) {
    if (b == nullptr || b->struct_size != sizeof(Qwen3TtsStepBenchmarkV1) || b->layers <= 0 || b->hidden <= 0 ||
        b->intermediate <= 0 || b->query_width <= 0 || b->key_value_width <= 0 || b->rows < 1 || b->rows > 8 ||
        b->steps <= 0 || b->warmup < 0 || b->kernel_filter < 0 || b->kernel_filter > 4 || b->use_graph < 0 ||
        b->use_graph > 3 || (b->use_graph == 2 && b->rows != 1) ||
        (b->use_graph == 3 && (b->rows != 1 || b->kernel_filter != 0 || b->mode == kModeMfma))) {
        write_error(error, cap, "invalid step benchmark arguments");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    hipEvent_t start = nullptr, stop = nullptr;
    hipStream_t stream = nullptr;
    hipGraphExec_t exec = nullptr;
    try {
        check_hip(hipSetDevice(device_index), "hipSetDevice");
        check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        Mem mem;
        const int L = b->layers, H = b->hidden, I = b->intermediate, QW = b->query_width, KW = b->key_value_width;
        const int R = b->rows;
        const size_t qkv_rows = static_cast<size_t>(QW) + 2 * KW;
        const size_t per_layer = qkv_rows * H + static_cast<size_t>(H) * QW + 2ull * I * H + static_cast<size_t>(H) * I;
        const size_t scales_per_layer = qkv_rows + H + 2ull * I + H;
        int8_t* w = mem.get<int8_t>(per_layer * L);
        float* s = mem.get<float>(scales_per_layer * L);
        bf16_t* gains = mem.get<bf16_t>(2ull * H);
        bf16_t* hidden = mem.get<bf16_t>(static_cast<size_t>(R) * H);
        bf16_t* qkv = mem.get<bf16_t>(static_cast<size_t>(R) * qkv_rows);
        bf16_t* act = mem.get<bf16_t>(static_cast<size_t>(R) * I);
        fill_int8_kernel<<<grid_for(per_layer * L), 256, 0, stream>>>(w, per_layer * L, 0x5EED0011ULL);
        fill_scale_kernel<<<grid_for(scales_per_layer * L), 256, 0, stream>>>(s, scales_per_layer * L, 0x5EED0012ULL);
        check_hip(launch_fill_bf16_normal(gains, 2ull * H, 0x5EED0013ULL, 1.0f, 0.1f, stream), "fill gains");
        check_hip(launch_fill_bf16_normal(hidden, static_cast<uint64_t>(R) * H, 0x5EED0014ULL, 0.0f, 1.0f, stream), "fill x");
        check_hip(launch_fill_bf16_normal(qkv, static_cast<uint64_t>(R) * qkv_rows, 0x5EED0015ULL, 0.0f, 1.0f, stream), "fill q");
        check_hip(launch_fill_bf16_normal(act, static_cast<uint64_t>(R) * I, 0x5EED0016ULL, 0.0f, 1.0f, stream), "fill act");
        const int mode = b->mode;
        const int filter = b->kernel_filter;
        int* read_sink = mem.get<int>(1);
        auto launch = [&](const GemvArgs& g, const char* what) {
            if (b->use_graph == 2) {  // the same weight bytes, plain reads
                const bool pair = g.epilogue == kEpiSiluRounded || g.epilogue == kEpiSiluFused;
                const uint64_t bytes = static_cast<uint64_t>(g.in_features) * g.out_features * (pair ? 2 : 1);
                read_weights_kernel<<<1536, 256, 0, stream>>>(g.weight, bytes, read_sink);
                check_hip(hipGetLastError(), what);
                return;
            }
            check_hip(launch_int8_gemv(g, stream), what);
        };
        // QKV output has the full fused row; O reads the q part with row
        // stride qkv_rows when R == 1 (the attention output stand-in).
        auto enqueue_step = [&] {
            for (int l = 0; l < L; ++l) {
                int8_t* base = w + per_layer * l;
                float* sb = s + scales_per_layer * l;
                const int8_t* wqkv = base;
                const int8_t* wo = wqkv + qkv_rows * H;
                const int8_t* wgu = wo + static_cast<size_t>(H) * QW;
                const int8_t* wd = wgu + 2ull * I * H;
                const float* sqkv = sb;
                const float* so = sqkv + qkv_rows;
                const float* sgu = so + H;
                const float* sd = sgu + 2 * I;
                if (filter == 0 || filter == 1) {
                    GemvArgs a;
                    a.rows = R; a.mode = mode; a.norm_epsilon = 1.0e-6f;
                    a.weight = wqkv; a.scales = sqkv; a.input = hidden; a.norm_weight = gains;
                    a.in_features = H; a.out_features = static_cast<int>(qkv_rows); a.out16 = qkv;
                    a.epilogue = kEpiStore;
                    launch(a, "QKV GEMV");
                }
                if (filter == 0 || filter == 2) {
                    GemvArgs o;
                    o.rows = R; o.mode = mode;
                    o.weight = wo; o.scales = so; o.input = qkv; o.in_features = QW; o.out_features = H;
                    o.out16 = hidden; o.epilogue = R == 1 ? kEpiAddRounded : kEpiAddFma;
                    if (R > 1) o.input = act;  // rows-contiguous stand-in for attention output
                    launch(o, "O GEMV");
                }
                if (filter == 0 || filter == 3) {
                    GemvArgs g;
                    g.rows = R; g.mode = mode; g.norm_epsilon = 1.0e-6f;
                    g.weight = wgu; g.scales = sgu; g.input = hidden; g.norm_weight = gains + H;
                    g.in_features = H; g.out_features = I; g.out16 = act;
                    g.epilogue = R == 1 ? kEpiSiluRounded : kEpiSiluFused;
                    launch(g, "gate/up GEMV");
                }
                if (filter == 0 || filter == 4) {
                    GemvArgs d;
                    d.rows = R; d.mode = mode;
                    d.weight = wd; d.scales = sd; d.input = act; d.in_features = I; d.out_features = H;
                    d.out16 = hidden; d.epilogue = R == 1 ? kEpiAddRounded : kEpiAddFma;
                    launch(d, "down GEMV");
                }
            }
        };
        // use_graph 3: the whole step as one persistent launch (step_chain.hip).
        StepChainArgs chain;
        if (b->use_graph == 3) {
            bool supported = false;
            check_hip(talker_step_chain_supported(device_index, &supported), "persistent chain support query");
            if (!supported) throw DeviceFailure("persistent step chain: the device cannot hold all 256 workgroups at once");
            chain.weights = w;
            chain.scales = s;
            chain.weight_layer_stride = per_layer;
            chain.scale_layer_stride = scales_per_layer;
            chain.gain_qkv = gains;
            chain.gain_gu = gains + H;
            chain.hidden = hidden;
            chain.qkv = qkv;
            chain.act = act;
            chain.words = mem.get<unsigned long long>(talker_step_chain_words());
            chain.epoch = mem.get<unsigned>(1);
            chain.status = mem.get<int>(1);
            chain.hidden_size = H;
            chain.intermediate = I;
            chain.qkv_rows = static_cast<int>(qkv_rows);
            chain.query_width = QW;
            chain.layers = L;
            chain.epsilon = 1.0e-6f;
            check_hip(hipMemsetAsync(chain.words, 0, talker_step_chain_words() * sizeof(unsigned long long), stream),
                      "clear chain words");
            const unsigned one = 1;
            check_hip(hipMemcpyAsync(chain.epoch, &one, sizeof(one), hipMemcpyHostToDevice, stream), "chain epoch");
            check_hip(hipMemsetAsync(chain.status, 0, sizeof(int), stream), "chain status");
            check_hip(hipStreamSynchronize(stream), "chain workspace");
        }
        if (b->use_graph == 1 || b->use_graph == 2) {
            check_hip(hipStreamBeginCapture(stream, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
            enqueue_step();
            hipGraph_t graph = nullptr;
            check_hip(hipStreamEndCapture(stream, &graph), "hipStreamEndCapture");
            const hipError_t st = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
            (void)hipGraphDestroy(graph);
            check_hip(st, "hipGraphInstantiate");
        }
        auto run = [&] {
            if (b->use_graph == 3) {
                check_hip(launch_talker_step_chain(chain, stream), "persistent step chain");
            } else if (exec) {
                check_hip(hipGraphLaunch(exec, stream), "hipGraphLaunch");
            } else {
                enqueue_step();
            }
        };
        for (int i = 0; i < b->warmup; ++i) run();
        check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize(warmup)");
        check_hip(hipEventCreate(&start), "hipEventCreate");
        check_hip(hipEventCreate(&stop), "hipEventCreate");
        check_hip(hipEventRecord(start, stream), "hipEventRecord");
        for (int i = 0; i < b->steps; ++i) run();
        check_hip(hipEventRecord(stop, stream), "hipEventRecord");
        check_hip(hipEventSynchronize(stop), "hipEventSynchronize");
        float ms = 0.0f;
        check_hip(hipEventElapsedTime(&ms, start, stop), "hipEventElapsedTime");
        if (b->use_graph == 3) {
            int status = 0;
            check_hip(hipMemcpy(&status, chain.status, sizeof(int), hipMemcpyDeviceToHost), "chain status");
            if (status != 0) throw DeviceFailure("persistent step chain: a wait between GEMVs timed out");
        }
        // Algorithmic bytes of the filtered chain.
        uint64_t bytes = 0;
        auto gemv_bytes = [&](uint64_t out_rows, uint64_t in, uint64_t out, bool norm, bool rmw) {
            uint64_t v = out_rows * in + 4 * out_rows + 2ull * R * in + 2ull * R * out;
            if (norm) v += 2 * in;
            if (rmw) v += 2ull * R * out;
            return v;
        };
        if (filter == 0 || filter == 1) bytes += gemv_bytes(qkv_rows, H, qkv_rows, true, false);
        if (filter == 0 || filter == 2) bytes += gemv_bytes(H, QW, H, false, true);
        if (filter == 0 || filter == 3) bytes += gemv_bytes(2ull * I, H, I, true, false);
        if (filter == 0 || filter == 4) bytes += gemv_bytes(H, I, H, false, true);
        bytes *= static_cast<uint64_t>(L);
        uint64_t wbytes = 0;
        if (filter == 0 || filter == 1) wbytes += qkv_rows * H;
        if (filter == 0 || filter == 2) wbytes += static_cast<uint64_t>(H) * QW;
        if (filter == 0 || filter == 3) wbytes += 2ull * I * H;
        if (filter == 0 || filter == 4) wbytes += static_cast<uint64_t>(H) * I;
        b->weight_bytes = wbytes * L;
        b->algorithmic_bytes_per_step = bytes;
        b->total_milliseconds = ms;
        b->milliseconds_per_step = ms / b->steps;
        b->gemv_kernel_milliseconds_per_step = ms / b->steps;
        {
            uint64_t h = 1469598103934665603ULL;
            for (auto [ptr, count] : {std::make_pair(hidden, static_cast<size_t>(R) * H),
                                      std::make_pair(qkv, static_cast<size_t>(R) * qkv_rows),
                                      std::make_pair(act, static_cast<size_t>(R) * I)}) {
                std::vector<bf16_t> out(count);
                check_hip(hipMemcpy(out.data(), ptr, count * sizeof(bf16_t), hipMemcpyDeviceToHost), "read outputs");
                for (bf16_t v : out) {
                    h ^= v;
                    h *= 1099511628211ULL;
                }
            }
            b->output_checksum = h;
        }
        if (exec) (void)hipGraphExecDestroy(exec);
        (void)hipEventDestroy(start);
        (void)hipEventDestroy(stop);
        (void)hipStreamDestroy(stream);
        write_error(error, cap, "");
        return QWEN3_TTS_TALKER_STATUS_OK;
    } catch (const std::exception& e) {
        if (exec) (void)hipGraphExecDestroy(exec);
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
        if (stream) {
            (void)hipStreamSynchronize(stream);
            (void)hipStreamDestroy(stream);
        }
        write_error(error, cap, e.what());
        return QWEN3_TTS_TALKER_STATUS_CUDA;
    }
}

}  // extern "C"
