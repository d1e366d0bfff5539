// Diagnostics of the reference ABI (device probe, argmax / GEMV benchmarks,
// primitive self-test, weight-upload device buffers) and this build's
// additive exports (int8 GEMV entry point and benchmarks, primitive ops,
// device-memory helpers), gfx950.
//
// Reference behaviour followed: native/qwen3-tts-native/native/src/
// runtime.cu (probe :86-122, argmax benchmark :124-255), gemv.cu:88-270,
// primitive_parity.cu:115-368 and weights.cu:1-340.
#include "q3_common.hpp"

#include "../../include/qwen3_tts_native.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <limits>
#include <new>
#include <random>
#include <vector>

struct Qwen3TtsDeviceBuffer {
    int32_t device_index;
    uint8_t* device_data;
    uint8_t* pinned_staging;
    hipStream_t stream;
    uint64_t capacity_bytes;
    uint64_t staging_bytes;
    uint64_t uploaded_bytes;
    uint64_t upload_calls;
    double allocation_microseconds;
    double upload_microseconds;
    uint64_t free_before_bytes;
    uint64_t free_after_allocation_bytes;
};

namespace q3 {
namespace {

void write_error(char* destination, size_t capacity, const char* message) {
    if (destination != nullptr && capacity != 0) std::snprintf(destination, capacity, "%s", message);
}

int32_t hip_failure(hipError_t status, const char* operation, char* error, size_t capacity) {
    char message[512];
    std::snprintf(message, sizeof(message), "%s failed: %s", operation, hipGetErrorString(status));
    write_error(error, capacity, message);
    return QWEN3_TTS_TALKER_STATUS_CUDA;
}

int32_t ok(char* error, size_t capacity) {
    write_error(error, capacity, "");
    return QWEN3_TTS_TALKER_STATUS_OK;
}

int32_t launch_status(hipError_t status, const char* what, char* error, size_t capacity) {
    if (status == hipErrorInvalidValue) {
        char message[256];
        std::snprintf(message, sizeof(message), "%s: invalid arguments (shape, alignment or null pointer)", what);
        write_error(error, capacity, message);
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    if (status != hipSuccess) return hip_failure(status, what, error, capacity);
    return ok(error, capacity);
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

constexpr int kWarmupIterations = 20;

// bf16 GEMV for the bf16 benchmark export (gemv.cu:88-270 measures cuBLAS
// here).  One wave64 per output channel, 16-byte loads, fp32 accumulate.
__global__ __launch_bounds__(256) void bf16_gemv_kernel(const bf16_t* w, const bf16_t* x, bf16_t* y, int in,
                                                        int out) {
    const int lane = threadIdx.x & 63;
    const int channel = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (channel >= out) return;
    const bf16_t* row = w + static_cast<size_t>(channel) * in;
    float acc = 0.0f;
    for (int k = lane * 8; k < in; k += 512) {
        const uint4 wv = *reinterpret_cast<const uint4*>(row + k);
        const uint4 xv = *reinterpret_cast<const uint4*>(x + k);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
        const uint32_t xx[4] = {xv.x, xv.y, xv.z, xv.w};
        for (int i = 0; i < 4; ++i) {
            acc = fmaf(__uint_as_float(ww[i] << 16), __uint_as_float(xx[i] << 16), acc);
            acc = fmaf(__uint_as_float(ww[i] & 0xffff0000u), __uint_as_float(xx[i] & 0xffff0000u), acc);
        }
    }
    for (int offset = 32; offset > 0; offset >>= 1) acc += __shfl_down(acc, offset, 64);
    if (lane == 0) y[channel] = f2bf(acc);
}

}  // namespace
}  // namespace q3

using namespace q3;

extern "C" {

// ---------------------------------------------------------------------------
// Reference diagnostics
// ---------------------------------------------------------------------------
QWEN3_TTS_API int32_t qwen3_tts_probe_device(int32_t device_index, Qwen3TtsDeviceInfo* output, char* error,
                                             size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "output device-info pointer is null");
        return -1;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    hipDeviceProp_t p{};
    st = hipGetDeviceProperties(&p, device_index);
    if (st != hipSuccess) return hip_failure(st, "hipGetDeviceProperties", error, cap);
    size_t free_bytes = 0, total_bytes = 0;
    st = hipMemGetInfo(&free_bytes, &total_bytes);
    if (st != hipSuccess) return hip_failure(st, "hipMemGetInfo", error, cap);
    std::memset(output, 0, sizeof(*output));
    output->device_index = device_index;
    output->compute_major = p.major;
    output->compute_minor = p.minor;
    output->total_global_memory_bytes = p.totalGlobalMem;
    output->runtime_free_memory_bytes = free_bytes;
    output->runtime_total_memory_bytes = total_bytes;
    std::snprintf(output->device_name, sizeof(output->device_name), "%s (%s)", p.name, p.gcnArchName);
    return ok(error, cap);
}

// runtime.cu:124-255: known answer = token min(1729, V-1) set to 19.0 over a
// sin(i*0.017)*2 background.
QWEN3_TTS_API int32_t qwen3_tts_benchmark_bf16_argmax(int32_t device_index, int32_t vocabulary, int32_t iterations,
                                                      Qwen3TtsArgmaxBenchmark* output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "output benchmark pointer is null");
        return -1;
    }
    if (vocabulary <= 0 || vocabulary > 65536) {
        write_error(error, cap, "vocabulary size must be in [1, 65536]");
        return -2;
    }
    if (iterations <= 0) {
        write_error(error, cap, "iterations must be positive");
        return -3;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    const int expected = std::min(1729, vocabulary - 1);
    std::vector<bf16_t> host(static_cast<size_t>(vocabulary));
    for (int i = 0; i < vocabulary; ++i) host[i] = f2bf(std::sin(static_cast<float>(i) * 0.017f) * 2.0f);
    host[expected] = f2bf(19.0f);
    bf16_t* logits = nullptr;
    int* token = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    auto cleanup = [&] {
        if (logits) (void)hipFree(logits);
        if (token) (void)hipFree(token);
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
    };
    if ((st = hipMalloc(&logits, host.size() * 2)) != hipSuccess ||
        (st = hipMalloc(&token, sizeof(int))) != hipSuccess ||
        (st = hipMemcpy(logits, host.data(), host.size() * 2, hipMemcpyHostToDevice)) != hipSuccess ||
        (st = hipEventCreate(&start)) != hipSuccess || (st = hipEventCreate(&stop)) != hipSuccess) {
        cleanup();
        return hip_failure(st, "argmax benchmark setup", error, cap);
    }
    float cold = 0.0f, total = 0.0f;
    (void)hipEventRecord(start, nullptr);
    st = launch_argmax_bf16(logits, vocabulary, token, nullptr);
    (void)hipEventRecord(stop, nullptr);
    (void)hipEventSynchronize(stop);
    (void)hipEventElapsedTime(&cold, start, stop);
    for (int i = 0; i < kWarmupIterations && st == hipSuccess; ++i) st = launch_argmax_bf16(logits, vocabulary, token, nullptr);
    (void)hipEventRecord(start, nullptr);
    for (int i = 0; i < iterations && st == hipSuccess; ++i) st = launch_argmax_bf16(logits, vocabulary, token, nullptr);
    (void)hipEventRecord(stop, nullptr);
    (void)hipEventSynchronize(stop);
    (void)hipEventElapsedTime(&total, start, stop);
    int selected = -1;
    if (st == hipSuccess) st = hipMemcpy(&selected, token, sizeof(int), hipMemcpyDeviceToHost);
    cleanup();
    if (st != hipSuccess) return hip_failure(st, "argmax benchmark", error, cap);
    output->vocabulary_size = vocabulary;
    output->iterations = iterations;
    output->selected_token = selected;
    output->expected_token = expected;
    output->cold_launch_microseconds = cold * 1000.0f;
    output->mean_launch_microseconds = total * 1000.0f / static_cast<float>(iterations);
    if (selected != expected) {
        write_error(error, cap, "argmax known-answer check failed");
        return -5;
    }
    return ok(error, cap);
}

// gemv.cu:88-270 semantics (zeroed bf16 weights, zero-output check), measured
// on this build's own bf16 GEMV kernel.
QWEN3_TTS_API int32_t qwen3_tts_benchmark_bf16_gemv(int32_t device_index, int32_t in, int32_t out, int32_t iterations,
                                                    Qwen3TtsGemvBenchmark* output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "output benchmark pointer is null");
        return -1;
    }
    if (in <= 0 || in > 65536 || out <= 0 || out > 65536 || in % 8 != 0) {
        write_error(error, cap, "feature sizes must be in [1, 65536] (input a multiple of 8)");
        return -2;
    }
    if (iterations <= 0) {
        write_error(error, cap, "iterations must be positive");
        return -3;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    const size_t wbytes = static_cast<size_t>(in) * out * 2;
    bf16_t *w = nullptr, *x = nullptr, *y = nullptr;
    hipEvent_t start = nullptr, stop = nullptr;
    auto cleanup = [&] {
        if (w) (void)hipFree(w);
        if (x) (void)hipFree(x);
        if (y) (void)hipFree(y);
        if (start) (void)hipEventDestroy(start);
        if (stop) (void)hipEventDestroy(stop);
    };
    if ((st = hipMalloc(&w, wbytes)) != hipSuccess || (st = hipMalloc(&x, in * 2)) != hipSuccess ||
        (st = hipMalloc(&y, out * 2)) != hipSuccess || (st = hipMemset(w, 0, wbytes)) != hipSuccess ||
        (st = hipMemset(x, 0, in * 2)) != hipSuccess || (st = hipMemset(y, 0xff, out * 2)) != hipSuccess ||
        (st = hipEventCreate(&start)) != hipSuccess || (st = hipEventCreate(&stop)) != hipSuccess) {
        cleanup();
        return hip_failure(st, "bf16 GEMV benchmark setup", error, cap);
    }
    const int grid = (out + 3) / 4;
    float cold = 0.0f, total = 0.0f;
    (void)hipEventRecord(start, nullptr);
    bf16_gemv_kernel<<<grid, 256>>>(w, x, y, in, out);
    (void)hipEventRecord(stop, nullptr);
    (void)hipEventSynchronize(stop);
    (void)hipEventElapsedTime(&cold, start, stop);
    for (int i = 0; i < kWarmupIterations; ++i) bf16_gemv_kernel<<<grid, 256>>>(w, x, y, in, out);
    (void)hipEventRecord(start, nullptr);
    for (int i = 0; i < iterations; ++i) bf16_gemv_kernel<<<grid, 256>>>(w, x, y, in, out);
    (void)hipEventRecord(stop, nullptr);
    (void)hipEventSynchronize(stop);
    (void)hipEventElapsedTime(&total, start, stop);
    bf16_t first = 0xffff;
    st = hipGetLastError();
    if (st == hipSuccess) st = hipMemcpy(&first, y, 2, hipMemcpyDeviceToHost);
    cleanup();
    if (st != hipSuccess) return hip_failure(st, "bf16 GEMV benchmark", error, cap);
    if (bf2f(first) != 0.0f) {
        write_error(error, cap, "zero GEMV correctness check failed");
        return -5;
    }
    const float mean = total * 1000.0f / static_cast<float>(iterations);
    output->input_features = in;
    output->output_features = out;
    output->iterations = iterations;
    output->reserved = 0;
    output->weight_bytes = wbytes;
    output->cold_launch_microseconds = cold * 1000.0f;
    output->mean_launch_microseconds = mean;
    output->tera_operations_per_second = static_cast<float>(2.0 * in * out / (mean * 1.0e-6) / 1.0e12);
    return ok(error, cap);
}

// ---------------------------------------------------------------------------
// Weight-upload device buffer (weights.cu semantics: sequential contiguous
// uploads through a pinned staging buffer of at most 256 MiB).
// ---------------------------------------------------------------------------
static void fill_upload_metrics(const Qwen3TtsDeviceBuffer* b, Qwen3TtsWeightUploadMetrics* m) {
    if (b == nullptr || m == nullptr) return;
    std::memset(m, 0, sizeof(*m));
    m->device_index = b->device_index;
    m->allocation_bytes = b->capacity_bytes;
    m->pinned_staging_bytes = b->staging_bytes;
    m->uploaded_bytes = b->uploaded_bytes;
    m->upload_calls = b->upload_calls;
    m->free_before_bytes = b->free_before_bytes;
    m->free_after_allocation_bytes = b->free_after_allocation_bytes;
    m->allocation_microseconds = static_cast<float>(b->allocation_microseconds);
    m->upload_microseconds = static_cast<float>(b->upload_microseconds);
}

QWEN3_TTS_API void qwen3_tts_device_buffer_destroy(Qwen3TtsDeviceBuffer* b) {
    if (b == nullptr) return;
    (void)hipSetDevice(b->device_index);
    if (b->stream) (void)hipStreamSynchronize(b->stream);
    if (b->pinned_staging) (void)hipHostFree(b->pinned_staging);
    if (b->device_data) (void)hipFree(b->device_data);
    if (b->stream) (void)hipStreamDestroy(b->stream);
    delete b;
}

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_create(int32_t device_index, uint64_t capacity, uint64_t staging,
                                                     Qwen3TtsDeviceBuffer** output, Qwen3TtsWeightUploadMetrics* metrics,
                                                     char* error, size_t cap) {
    if (output == nullptr || metrics == nullptr) {
        write_error(error, cap, "output buffer or metrics pointer is null");
        return -1;
    }
    *output = nullptr;
    std::memset(metrics, 0, sizeof(*metrics));
    if (capacity == 0) {
        write_error(error, cap, "device capacity is zero or exceeds size_t");
        return -2;
    }
    if (staging == 0 || staging > 256ULL * 1024 * 1024) {
        write_error(error, cap, "staging capacity must be in [1, 256 MiB] and fit size_t");
        return -3;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    size_t free_before = 0, total = 0;
    if ((st = hipMemGetInfo(&free_before, &total)) != hipSuccess) return hip_failure(st, "hipMemGetInfo", error, cap);
    auto* b = new (std::nothrow) Qwen3TtsDeviceBuffer{};
    if (b == nullptr) {
        write_error(error, cap, "failed to allocate device-buffer metadata");
        return -4;
    }
    b->device_index = device_index;
    b->capacity_bytes = capacity;
    b->staging_bytes = staging;
    b->free_before_bytes = free_before;
    const auto t0 = std::chrono::steady_clock::now();
    if ((st = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking)) != hipSuccess ||
        (st = hipMalloc(reinterpret_cast<void**>(&b->device_data), capacity)) != hipSuccess ||
        (st = hipHostMalloc(reinterpret_cast<void**>(&b->pinned_staging), staging, hipHostMallocPortable)) != hipSuccess) {
        qwen3_tts_device_buffer_destroy(b);
        return hip_failure(st, "device buffer allocation", error, cap);
    }
    size_t free_after = 0;
    if ((st = hipMemGetInfo(&free_after, &total)) != hipSuccess) {
        qwen3_tts_device_buffer_destroy(b);
        return hip_failure(st, "hipMemGetInfo(after)", error, cap);
    }
    b->allocation_microseconds =
        std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    b->free_after_allocation_bytes = free_after;
    fill_upload_metrics(b, metrics);
    *output = b;
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_upload(Qwen3TtsDeviceBuffer* b, uint64_t offset, const void* source,
                                                     uint64_t bytes, char* error, size_t cap) {
    if (b == nullptr) {
        write_error(error, cap, "device buffer is null");
        return -1;
    }
    if (bytes != 0 && source == nullptr) {
        write_error(error, cap, "upload source is null");
        return -2;
    }
    if (offset != b->uploaded_bytes) {
        write_error(error, cap, "uploads must be contiguous and sequential");
        return -3;
    }
    if (bytes > b->capacity_bytes - offset) {
        write_error(error, cap, "upload exceeds device-buffer capacity");
        return -4;
    }
    hipError_t st = hipSetDevice(b->device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    const auto t0 = std::chrono::steady_clock::now();
    const auto* in = static_cast<const uint8_t*>(source);
    uint64_t copied = 0;
    while (copied < bytes) {
        const uint64_t chunk = std::min(b->staging_bytes, bytes - copied);
        std::memcpy(b->pinned_staging, in + copied, chunk);
        if ((st = hipMemcpyAsync(b->device_data + offset + copied, b->pinned_staging, chunk, hipMemcpyHostToDevice,
                                 b->stream)) != hipSuccess ||
            (st = hipStreamSynchronize(b->stream)) != hipSuccess) {
            return hip_failure(st, "device buffer upload", error, cap);
        }
        copied += chunk;
        b->upload_calls += 1;
    }
    b->upload_microseconds += std::chrono::duration<double, std::micro>(std::chrono::steady_clock::now() - t0).count();
    b->uploaded_bytes += bytes;
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_finish(Qwen3TtsDeviceBuffer* b, Qwen3TtsWeightUploadMetrics* metrics,
                                                     char* error, size_t cap) {
    if (b == nullptr || metrics == nullptr) {
        write_error(error, cap, "device buffer or metrics pointer is null");
        return -1;
    }
    if (b->uploaded_bytes != b->capacity_bytes) {
        write_error(error, cap, "device buffer is not completely uploaded");
        return -2;
    }
    const hipError_t st = hipStreamSynchronize(b->stream);
    if (st != hipSuccess) return hip_failure(st, "hipStreamSynchronize(finish)", error, cap);
    fill_upload_metrics(b, metrics);
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_buffer_read(Qwen3TtsDeviceBuffer* b, uint64_t offset, void* destination,
                                                   uint64_t bytes, char* error, size_t cap) {
    if (b == nullptr) {
        write_error(error, cap, "device buffer is null");
        return -1;
    }
    if (bytes != 0 && destination == nullptr) {
        write_error(error, cap, "read destination is null");
        return -2;
    }
    if (offset > b->capacity_bytes || bytes > b->capacity_bytes - offset) {
        write_error(error, cap, "read exceeds device-buffer capacity");
        return -3;
    }
    hipError_t st = hipSetDevice(b->device_index);
    if (st == hipSuccess) st = hipStreamSynchronize(b->stream);
    if (st == hipSuccess && bytes != 0) st = hipMemcpy(destination, b->device_data + offset, bytes, hipMemcpyDeviceToHost);
    if (st != hipSuccess) return hip_failure(st, "device buffer read", error, cap);
    return ok(error, cap);
}

QWEN3_TTS_API const void* qwen3_tts_device_buffer_data(const Qwen3TtsDeviceBuffer* b) {
    return b == nullptr ? nullptr : b->device_data;
}

// ---------------------------------------------------------------------------
// Primitive self-test (primitive_parity.cu:115-368 known answers; tolerance
// 0.016).  Attention runs at head_dimension 128, the only head size of the
// decode path (the reference's self-test uses 32).
// ---------------------------------------------------------------------------
QWEN3_TTS_API int32_t qwen3_tts_validate_transformer_primitives(int32_t device_index, Qwen3TtsPrimitiveParity* output,
                                                                char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "primitive parity output pointer is null");
        return -1;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st != hipSuccess) return hip_failure(st, "hipSetDevice", error, cap);
    auto to_bf = [](const std::vector<float>& v) {
        std::vector<bf16_t> r(v.size());
        for (size_t i = 0; i < v.size(); ++i) r[i] = f2bf(v[i]);
        return r;
    };
    auto from_bf = [](const std::vector<bf16_t>& v) {
        std::vector<float> r(v.size());
        for (size_t i = 0; i < v.size(); ++i) r[i] = bf2f(v[i]);
        return r;
    };
    auto max_err = [](const std::vector<float>& a, const std::vector<float>& b) {
        float m = 0.0f;
        for (size_t i = 0; i < a.size(); ++i) m = std::max(m, std::fabs(a[i] - b[i]));
        return m;
    };
    std::vector<void*> allocations;
    auto dev = [&](const void* host, size_t bytes) {
        void* p = nullptr;
        if (hipMalloc(&p, bytes) != hipSuccess) throw DeviceFailure("hipMalloc(self-test)");
        allocations.push_back(p);
        if (host && hipMemcpy(p, host, bytes, hipMemcpyHostToDevice) != hipSuccess) throw DeviceFailure("hipMemcpy(self-test)");
        return p;
    };
    auto down = [](void* p, size_t n) {
        std::vector<bf16_t> r(n);
        if (hipMemcpy(r.data(), p, n * 2, hipMemcpyDeviceToHost) != hipSuccess) throw DeviceFailure("hipMemcpy(D2H)");
        return r;
    };
    try {
        Qwen3TtsPrimitiveParity result{};
        {   // RMSNorm, width 128
            const int width = 128;
            std::vector<float> in(width), w(width);
            for (int i = 0; i < width; ++i) {
                in[i] = std::sin(i * 0.071f) * 1.7f;
                w[i] = 0.75f + std::cos(i * 0.037f) * 0.2f;
            }
            const auto inb = to_bf(in), wb = to_bf(w);
            in = from_bf(inb);
            w = from_bf(wb);
            float sq = 0.0f;
            for (float v : in) sq += v * v;
            const float inv = 1.0f / std::sqrt(sq / width + 1.0e-6f);
            std::vector<float> expected(width);
            for (int i = 0; i < width; ++i) expected[i] = round_bf(in[i] * inv * w[i]);
            void* di = dev(inb.data(), width * 2);
            void* dw = dev(wb.data(), width * 2);
            void* dout = dev(nullptr, width * 2);
            check_hip(launch_rms_norm_rows(static_cast<bf16_t*>(di), static_cast<bf16_t*>(dw), static_cast<bf16_t*>(dout), 1, width, 1.0e-6f, nullptr), "rms norm");
            result.rms_norm_max_absolute_error = max_err(from_bf(down(dout, width)), expected);
        }
        {   // RoPE, 2 heads x 128, position 37
            const int heads = 2, d = 128, half = 64, position = 37;
            std::vector<float> v(heads * d);
            for (size_t i = 0; i < v.size(); ++i) v[i] = std::sin(static_cast<float>(i) * 0.019f);
            const auto vb = to_bf(v);
            v = from_bf(vb);
            std::vector<float> expected(v.size());
            for (int h = 0; h < heads; ++h) {
                for (int i = 0; i < half; ++i) {
                    const float angle = position * std::pow(1.0e6f, -static_cast<float>(2 * i) / d);
                    const float a = v[h * d + i], b = v[h * d + i + half];
                    expected[h * d + i] = round_bf(a * std::cos(angle) - b * std::sin(angle));
                    expected[h * d + i + half] = round_bf(b * std::cos(angle) + a * std::sin(angle));
                }
            }
            void* dv = dev(vb.data(), vb.size() * 2);
            check_hip(launch_rope_rows(static_cast<bf16_t*>(dv), 1, heads, d, position, 1.0e6f, nullptr), "rope");
            result.rope_max_absolute_error = max_err(from_bf(down(dv, vb.size())), expected);
        }
        {   // attention, 4 q heads / 2 kv heads, d 128, 7 positions
            const int qh = 4, kvh = 2, d = 128, seq = 7;
            std::vector<float> q(qh * d), k(seq * kvh * d), v(seq * kvh * d);
            for (size_t i = 0; i < q.size(); ++i) q[i] = std::sin(static_cast<float>(i) * 0.031f) * 0.4f;
            for (size_t i = 0; i < k.size(); ++i) {
                k[i] = std::cos(static_cast<float>(i) * 0.023f) * 0.3f;
                v[i] = std::sin(static_cast<float>(i) * 0.017f) * 0.5f;
            }
            const auto qb = to_bf(q), kb = to_bf(k), vb = to_bf(v);
            q = from_bf(qb);
            k = from_bf(kb);
            v = from_bf(vb);
            std::vector<float> expected(q.size()), scores(seq);
            for (int h = 0; h < qh; ++h) {
                const int g = h / (qh / kvh);
                float mx = -INFINITY;
                for (int p = 0; p < seq; ++p) {
                    float dot = 0.0f;
                    for (int i = 0; i < d; ++i) dot += q[h * d + i] * k[(p * kvh + g) * d + i];
                    scores[p] = dot / std::sqrt(static_cast<float>(d));
                    mx = std::max(mx, scores[p]);
                }
                float den = 0.0f;
                for (float& s : scores) {
                    s = std::exp(s - mx);
                    den += s;
                }
                for (int i = 0; i < d; ++i) {
                    float acc = 0.0f;
                    for (int p = 0; p < seq; ++p) acc += scores[p] / den * v[(p * kvh + g) * d + i];
                    expected[h * d + i] = round_bf(acc);
                }
            }
            void* dq = dev(qb.data(), qb.size() * 2);
            void* dk = dev(kb.data(), kb.size() * 2);
            void* dvv = dev(vb.data(), vb.size() * 2);
            void* dout = dev(nullptr, qb.size() * 2);
            check_hip(launch_causal_gqa_attention(static_cast<bf16_t*>(dq), static_cast<bf16_t*>(dk), static_cast<bf16_t*>(dvv),
                                                  static_cast<bf16_t*>(dout), qh, kvh, d, seq, qh * d, nullptr),
                      "attention");
            result.attention_max_absolute_error = max_err(from_bf(down(dout, qb.size())), expected);
        }
        {   // SiLU gate, width 257
            const int width = 257;
            std::vector<float> g(width), u(width);
            for (int i = 0; i < width; ++i) {
                g[i] = std::sin(i * 0.043f) * 2.0f;
                u[i] = std::cos(i * 0.029f);
            }
            const auto gb = to_bf(g), ub = to_bf(u);
            g = from_bf(gb);
            u = from_bf(ub);
            std::vector<float> expected(width);
            for (int i = 0; i < width; ++i) expected[i] = round_bf(g[i] / (1.0f + std::exp(-g[i])) * u[i]);
            void* dg = dev(gb.data(), width * 2);
            void* du = dev(ub.data(), width * 2);
            check_hip(launch_silu_gate(static_cast<bf16_t*>(dg), static_cast<bf16_t*>(du), width, nullptr), "silu gate");
            result.silu_gate_max_absolute_error = max_err(from_bf(down(dg, width)), expected);
        }
        for (void* p : allocations) (void)hipFree(p);
        constexpr float tolerance = 0.016f;
        if (result.rms_norm_max_absolute_error > tolerance || result.rope_max_absolute_error > tolerance ||
            result.attention_max_absolute_error > tolerance || result.silu_gate_max_absolute_error > tolerance) {
            *output = result;
            write_error(error, cap, "a transformer primitive exceeded BF16 parity tolerance");
            return -2;
        }
        *output = result;
        return ok(error, cap);
    } catch (const std::exception& e) {
        for (void* p : allocations) (void)hipFree(p);
        write_error(error, cap, e.what());
        return -3;
    }
}

// ---------------------------------------------------------------------------
// Additive exports
// ---------------------------------------------------------------------------
QWEN3_TTS_API int32_t qwen3_tts_int8_gemv_v1(const Qwen3TtsInt8GemvV1* args, void* stream, char* error, size_t cap) {
    if (args == nullptr || args->struct_size != sizeof(Qwen3TtsInt8GemvV1)) {
        write_error(error, cap, "GEMV arguments are null or have the wrong struct_size");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    GemvArgs a;
    a.weight = args->weight;
    a.scales = args->scales;
    a.input = args->input;
    a.norm_weight = args->norm_weight;
    a.norm_epsilon = args->norm_epsilon;
    a.bias = args->bias;
    a.input_row_index = args->input_row_index;
    a.out16 = args->out16;
    a.out32 = args->out32;
    a.in_features = args->in_features;
    a.out_features = args->out_features;
    a.rows = args->rows;
    a.epilogue = args->epilogue;
    a.mode = args->mode;
    return launch_status(launch_int8_gemv(a, as_stream(stream)), "int8 GEMV", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_quantize_weight_rows_v1(const uint16_t* weight, int8_t* quantized, float* scales,
                                                        int32_t in, int32_t out, void* stream, char* error, size_t cap) {
    if (weight == nullptr || quantized == nullptr || scales == nullptr) {
        write_error(error, cap, "quantizer pointers are null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    return launch_status(launch_quantize_weight_rows(weight, quantized, scales, in, out, as_stream(stream)),
                         "quantize weight rows", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_rms_norm_rows(const uint16_t* input, const uint16_t* weight, uint16_t* output,
                                                 int32_t rows, int32_t width, float eps, void* stream, char* error,
                                                 size_t cap) {
    return launch_status(launch_rms_norm_rows(input, weight, output, rows, width, eps, as_stream(stream)), "rms norm",
                         error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_head_rms_norm_rows(uint16_t* values, const uint16_t* weight, int32_t rows,
                                                      int32_t heads, int32_t head_dimension, float eps, void* stream,
                                                      char* error, size_t cap) {
    return launch_status(launch_head_rms_norm_rows(values, weight, rows, heads, head_dimension, eps, as_stream(stream)),
                         "head rms norm", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_rope_rows(uint16_t* values, int32_t rows, int32_t heads, int32_t head_dimension,
                                             const int32_t* positions, float theta, void* stream, char* error,
                                             size_t cap) {
    return launch_status(launch_rope_rows_at(values, rows, heads, head_dimension, positions, theta, as_stream(stream)),
                         "rope", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_rope_table_v1(int32_t positions, int32_t head_dimension, float theta,
                                              uint16_t* host_output, char* error, size_t cap) {
    if (positions <= 0 || head_dimension <= 0 || head_dimension % 2 != 0 || host_output == nullptr) {
        write_error(error, cap, "invalid RoPE table arguments");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    const int half = head_dimension / 2;
    for (int p = 0; p < positions; ++p) {
        for (int d = 0; d < half; ++d) {
            const float exponent = static_cast<float>(2 * d) / static_cast<float>(head_dimension);
            const float angle = static_cast<float>(p) * powf(theta, -exponent);
            host_output[(static_cast<size_t>(p) * half + d) * 2] = f2bf(cosf(angle));
            host_output[(static_cast<size_t>(p) * half + d) * 2 + 1] = f2bf(sinf(angle));
        }
    }
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_qk_norm_rope_kv_append(uint16_t* qkv, const uint16_t* q_norm, const uint16_t* k_norm,
                                                          uint16_t* const* key_bases, uint16_t* const* value_bases,
                                                          const int32_t* positions, const uint16_t* rope_table,
                                                          int32_t rows, int32_t qh, int32_t kvh, int32_t hd, float eps,
                                                          void* stream, char* error, size_t cap) {
    return launch_status(launch_qk_norm_rope_kv_append(qkv, q_norm, k_norm, key_bases, value_bases, positions, rope_table,
                                                       rows, qh, kvh, hd, eps, as_stream(stream)),
                         "q/k norm + RoPE + KV append", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_attention(int32_t exact, const uint16_t* query, int32_t query_stride,
                                             uint16_t* const* key_bases, uint16_t* const* value_bases,
                                             const int32_t* positions, uint16_t* output, int32_t rows, int32_t qh,
                                             int32_t kvh, int32_t hd, int32_t max_seq, void* stream, char* error,
                                             size_t cap) {
    return launch_status(launch_attention_op(exact != 0, query, query_stride, key_bases, value_bases, positions, output,
                                             rows, qh, kvh, hd, max_seq, as_stream(stream)),
                         "attention", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_prompt_attention_v1(int32_t exact, const uint16_t* query, int32_t query_stride,
                                                      const uint16_t* key_cache, const uint16_t* value_cache,
                                                      const int32_t* positions, uint16_t* output, int32_t rows,
                                                      int32_t qh, int32_t kvh, int32_t hd, int32_t capacity,
                                                      void* stream, char* error, size_t cap) {
    return launch_status(launch_prompt_attention_op(exact != 0, query, query_stride, key_cache, value_cache, positions,
                                                    output, rows, qh, kvh, hd, capacity, as_stream(stream)),
                         "prompt attention", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_decode_attention(int32_t exact, const uint16_t* qkv, int32_t qkv_stride,
                                                    const uint16_t* q_norm, const uint16_t* k_norm,
                                                    const uint16_t* rope_table, float epsilon,
                                                    uint16_t* const* key_bases, uint16_t* const* value_bases,
                                                    const int32_t* positions, uint16_t* output, int32_t rows,
                                                    int32_t qh, int32_t kvh, int32_t hd, int32_t max_seq,
                                                    void* stream, char* error, size_t cap) {
    return launch_status(launch_decode_attention_op(exact != 0, qkv, qkv_stride, q_norm, k_norm, rope_table, epsilon,
                                                    key_bases, value_bases, positions, output, rows, qh, kvh, hd,
                                                    max_seq, as_stream(stream)),
                         "decode attention", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_decode_attention_noalloc_v1(
    int32_t exact, const uint16_t* qkv, int32_t qkv_stride, const uint16_t* q_norm, const uint16_t* k_norm,
    const uint16_t* rope_table, float epsilon, uint16_t* const* key_bases, uint16_t* const* value_bases,
    const int32_t* positions, uint16_t* output, int32_t rows, int32_t qh, int32_t kvh, int32_t hd, int32_t max_seq,
    void* stream, char* error, size_t cap) {
    if (rows > 0 && qh > 0 && kvh > 0 && hd > 0 && max_seq > 0) {
        const size_t need = decode_attention_scratch_bytes(rows, qh, kvh, hd, max_seq);
        if (need > decode_attention_scratch_limit()) {
            char message[160];
            std::snprintf(message, sizeof(message),
                          "decode attention needs %zu bytes of scratch; the allocation-free entry point holds %zu",
                          need, decode_attention_scratch_limit());
            write_error(error, cap, message);
            return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
        }
    }
    return launch_status(launch_decode_attention_op_noalloc(exact != 0, qkv, qkv_stride, q_norm, k_norm, rope_table,
                                                            epsilon, key_bases, value_bases, positions, output, rows,
                                                            qh, kvh, hd, max_seq, as_stream(stream)),
                         "decode attention (no allocation)", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_bf16_gemm_v1(const uint16_t* a, const uint16_t* b, uint16_t* c, int32_t m,
                                                int32_t n, int32_t k, int32_t lda, int32_t ldb, int32_t ldc,
                                                int32_t batch, int32_t b_group, int64_t a_batch, int64_t b_batch,
                                                int64_t c_batch, void* stream, char* error, size_t cap) {
    Bf16GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = c;
    g.m = m;
    g.n = n;
    g.k = k;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.batch = batch;
    g.b_group = b_group;
    g.a_batch = a_batch;
    g.b_batch = b_batch;
    g.c_batch = c_batch;
    return launch_status(launch_bf16_gemm(g, as_stream(stream)), "bf16 GEMM", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_bf16_gemm_split_v1(const uint16_t* a, const uint16_t* b, uint16_t* c, int32_t m,
                                                      int32_t n, int32_t k, int32_t lda, int32_t ldb, int32_t ldc,
                                                      int32_t batch, int32_t b_group, int64_t a_batch, int64_t b_batch,
                                                      int64_t c_batch, float* partial, uint64_t partial_floats,
                                                      int32_t tile, int32_t k_step, int32_t splits, int32_t epilogue,
                                                      void* stream, char* error, size_t cap) {
    if (tile < 0 || k_step < 0 || splits < 0 || (partial == nullptr && partial_floats != 0)) {
        write_error(error, cap, "bf16 GEMM: negative tile, K step or split count, or a workspace size without a workspace");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    Bf16GemmArgs g;
    g.a = a;
    g.b = b;
    g.c = c;
    g.m = m;
    g.n = n;
    g.k = k;
    g.lda = lda;
    g.ldb = ldb;
    g.ldc = ldc;
    g.batch = batch;
    g.b_group = b_group;
    g.a_batch = a_batch;
    g.b_batch = b_batch;
    g.c_batch = c_batch;
    g.partial = partial;
    g.partial_floats = static_cast<size_t>(partial_floats);
    g.force_tile = tile;
    g.force_k_step = k_step;
    g.force_splits = splits;
    g.epilogue = epilogue;
    return launch_status(launch_bf16_gemm(g, as_stream(stream)), "bf16 GEMM (split)", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_causal_softmax_v1(uint16_t* scores, int32_t heads, int32_t rows, int32_t stride,
                                                     int32_t head_dimension, void* stream, char* error, size_t cap) {
    return launch_status(launch_causal_softmax(scores, heads, rows, stride, head_dimension, as_stream(stream)),
                         "causal softmax", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_kv_scatter_rows(const uint16_t* rows_data, uint16_t* const* cache_bases,
                                                   const int32_t* positions, int32_t rows, int32_t width,
                                                   int32_t row_stride, void* stream, char* error, size_t cap) {
    return launch_status(launch_kv_scatter_rows(rows_data, cache_bases, positions, rows, width, row_stride, as_stream(stream)),
                         "kv scatter", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_elementwise(int32_t op, uint16_t* values, const uint16_t* other, int32_t rows,
                                               int32_t width, void* stream, char* error, size_t cap) {
    hipError_t st = hipErrorInvalidValue;
    switch (op) {
        case 0: st = launch_add_in_place(values, other, rows * width, as_stream(stream)); break;
        case 1: st = launch_bias_activation_rows(values, other, rows, width, false, as_stream(stream)); break;
        case 2: st = launch_bias_activation_rows(values, other, rows, width, true, as_stream(stream)); break;
        case 3: st = launch_silu_gate(values, other, rows * width, as_stream(stream)); break;
        default: break;
    }
    return launch_status(st, "elementwise op", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_sample_logits(const uint16_t* logits, int32_t vocabulary, int32_t suppress,
                                                 int32_t eos, const int32_t* history, const int32_t* history_count,
                                                 Qwen3TtsSamplingConfig s, uint64_t* random_state, int32_t* selected,
                                                 void* stream, char* error, size_t cap) {
    return launch_status(launch_sample_logits(logits, vocabulary, suppress != 0, eos, history, history_count, 0,
                                              s.do_sample, s.top_k, s.top_p, s.temperature, s.repetition_penalty,
                                              random_state, selected, nullptr, nullptr, 0, as_stream(stream)),
                         "sample logits", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_op_sum_embeddings(const uint16_t* const* tables, int32_t count, int32_t vocabulary0,
                                                  int32_t vocabulary, int32_t width, const int32_t* tokens,
                                                  uint16_t* output, void* stream, char* error, size_t cap) {
    return launch_status(launch_sum_embeddings(tables, count, vocabulary0, vocabulary, width, tokens, output, as_stream(stream)),
                         "sum embeddings", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_malloc(int32_t device_index, uint64_t bytes, void** output, char* error,
                                              size_t cap) {
    if (output == nullptr || bytes == 0) {
        write_error(error, cap, "allocation output is null or size is zero");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    hipError_t st = hipSetDevice(device_index);
    if (st == hipSuccess) st = hipMalloc(output, bytes);
    if (st != hipSuccess) return hip_failure(st, "hipMalloc", error, cap);
    return ok(error, cap);
}

QWEN3_TTS_API void qwen3_tts_device_free(void* pointer) {
    if (pointer) (void)hipFree(pointer);
}

QWEN3_TTS_API int32_t qwen3_tts_device_memcpy(void* destination, const void* source, uint64_t bytes, char* error,
                                              size_t cap) {
    const hipError_t st = hipMemcpy(destination, source, bytes, hipMemcpyDefault);
    if (st != hipSuccess) return hip_failure(st, "hipMemcpy", error, cap);
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_fill_bf16_normal(uint16_t* destination, uint64_t count, uint64_t seed, float mean,
                                                        float stddev, void* stream, char* error, size_t cap) {
    return launch_status(launch_fill_bf16_normal(destination, count, seed, mean, stddev, as_stream(stream)),
                         "fill normal", error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_device_synchronize(int32_t device_index, char* error, size_t cap) {
    hipError_t st = hipSetDevice(device_index);
    if (st == hipSuccess) st = hipDeviceSynchronize();
    if (st != hipSuccess) return hip_failure(st, "hipDeviceSynchronize", error, cap);
    return ok(error, cap);
}

QWEN3_TTS_API int32_t qwen3_tts_stream_create(int32_t device_index, void** output, char* error, size_t cap) {
    if (output == nullptr) {
        write_error(error, cap, "stream output is null");
        return QWEN3_TTS_TALKER_STATUS_INVALID_ARGUMENT;
    }
    hipStream_t s = nullptr;
    hipError_t st = hipSetDevice(device_index);
    if (st == hipSuccess) st = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    if (st != hipSuccess) return hip_failure(st, "hipStreamCreate", error, cap);
    *output = s;
    return ok(error, cap);
}

QWEN3_TTS_API void qwen3_tts_stream_destroy(void* stream) {
    if (stream) (void)hipStreamDestroy(as_stream(stream));
}

QWEN3_TTS_API int32_t qwen3_tts_stream_synchronize(void* stream, char* error, size_t cap) {
    const hipError_t st = hipStreamSynchronize(as_stream(stream));
    if (st != hipSuccess) return hip_failure(st, "hipStreamSynchronize", error, cap);
    return ok(error, cap);
}

}  // extern "C"
