"""ctypes binding of libqwen3_tts_hip.so (the MI355X int8 decode-path library).

This is the Python-side mirror of the reference's FFI caller
(native/qwen3-tts-native/src/native_talker.rs:40-140, 765-1072): the same C
structs with the same layouts (asserted like native_talker.rs:1734-1744), the
same status-code meaning, and thin wrappers over the exported entry points.
It loads only the in-tree build of this package and fails loudly when the
library is missing; there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "libqwen3_tts_hip.so"

STATUS_OK = 0
STATUS_INVALID_ARGUMENT = -1
STATUS_DEVICE = -2
STATUS_STATE = -3
STATUS_ALLOCATION = -4
STATUS_MODEL = -5

EPI_STORE, EPI_ADD_FMA, EPI_ADD_ROUNDED, EPI_SILU_FUSED, EPI_SILU_ROUNDED = 0, 1, 2, 3, 4
EPI_BIAS, EPI_BIAS_SILU, EPI_BIAS_ADD = 5, 6, 7
MODE_AUTO, MODE_EXACT, MODE_MFMA = 0, 1, 2


class Qwen3TtsError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"status {status}: {message}")
        self.status = status


# ---------------------------------------------------------------------------
# ABI structs (include/qwen3_tts_native.h)
# ---------------------------------------------------------------------------
class DeviceInfo(C.Structure):
    _fields_ = [("device_index", C.c_int32), ("compute_major", C.c_int32),
                ("compute_minor", C.c_int32), ("total_global_memory_bytes", C.c_uint64),
                ("runtime_free_memory_bytes", C.c_uint64),
                ("runtime_total_memory_bytes", C.c_uint64), ("device_name", C.c_char * 256)]


class ArgmaxBenchmark(C.Structure):
    _fields_ = [("vocabulary_size", C.c_int32), ("iterations", C.c_int32),
                ("selected_token", C.c_int32), ("expected_token", C.c_int32),
                ("cold_launch_microseconds", C.c_float), ("mean_launch_microseconds", C.c_float)]


class GemvBenchmark(C.Structure):
    _fields_ = [("input_features", C.c_int32), ("output_features", C.c_int32),
                ("iterations", C.c_int32), ("reserved", C.c_int32), ("weight_bytes", C.c_uint64),
                ("cold_launch_microseconds", C.c_float), ("mean_launch_microseconds", C.c_float),
                ("tera_operations_per_second", C.c_float)]


class WeightUploadMetrics(C.Structure):
    _fields_ = [("device_index", C.c_int32), ("reserved", C.c_int32),
                ("allocation_bytes", C.c_uint64), ("pinned_staging_bytes", C.c_uint64),
                ("uploaded_bytes", C.c_uint64), ("upload_calls", C.c_uint64),
                ("free_before_bytes", C.c_uint64), ("free_after_allocation_bytes", C.c_uint64),
                ("allocation_microseconds", C.c_float), ("upload_microseconds", C.c_float)]


class PrimitiveParity(C.Structure):
    _fields_ = [("rms_norm_max_absolute_error", C.c_float), ("rope_max_absolute_error", C.c_float),
                ("attention_max_absolute_error", C.c_float),
                ("silu_gate_max_absolute_error", C.c_float)]


class SamplingConfig(C.Structure):
    _fields_ = [("do_sample", C.c_int32), ("top_k", C.c_int32), ("top_p", C.c_float),
                ("temperature", C.c_float), ("repetition_penalty", C.c_float)]


class PrefillResult(C.Structure):
    _fields_ = [("first_semantic_token", C.c_uint16), ("reserved", C.c_uint16),
                ("prompt_tokens", C.c_uint32), ("talker_gpu_milliseconds", C.c_float)]


class CodecFrameInfo(C.Structure):
    _fields_ = [("talker_position", C.c_uint32), ("ended_by_eos", C.c_uint32),
                ("predictor_gpu_milliseconds", C.c_float), ("talker_gpu_milliseconds", C.c_float)]


class DeviceFrameViewV2(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("code_count", C.c_uint32),
                ("device_codes", C.c_void_p), ("ready_event", C.c_void_p), ("lease_id", C.c_uint64),
                ("device_index", C.c_int32), ("reserved", C.c_uint32)]


class TalkerStateInfo(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("phase", C.c_uint32),
                ("talker_position", C.c_uint32), ("semantic_history_count", C.c_uint32),
                ("frames_generated", C.c_uint64), ("device_sample_count", C.c_uint64),
                ("host_sync_count", C.c_uint64)]


class ModelMemory(C.Structure):
    _fields_ = [("shared_weight_bytes", C.c_uint64), ("tensor_count", C.c_uint32),
                ("device_index", C.c_int32)]


class SessionMemory(C.Structure):
    _fields_ = [("talker_kv_bytes", C.c_uint64), ("predictor_kv_bytes", C.c_uint64),
                ("workspace_bytes", C.c_uint64), ("max_sequence_length", C.c_uint32),
                ("reserved", C.c_uint32)]


class ModelConfigV1(C.Structure):
    _fields_ = [("struct_size", C.c_uint32)] + [
        (n, C.c_int32) for n in (
            "talker_layers", "talker_hidden", "talker_intermediate", "talker_query_heads",
            "talker_key_value_heads", "predictor_layers", "predictor_hidden",
            "predictor_intermediate", "predictor_query_heads", "predictor_key_value_heads",
            "head_dimension", "talker_vocabulary", "predictor_vocabulary", "text_vocabulary",
            "codec_eos_token")] + [("rms_epsilon", C.c_float), ("rope_theta", C.c_float)]


class Int8GemvV1(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("in_features", C.c_int32),
                ("out_features", C.c_int32), ("rows", C.c_int32), ("epilogue", C.c_int32),
                ("mode", C.c_int32), ("norm_epsilon", C.c_float), ("reserved", C.c_int32),
                ("weight", C.c_void_p), ("scales", C.c_void_p), ("input", C.c_void_p),
                ("norm_weight", C.c_void_p), ("bias", C.c_void_p),
                ("input_row_index", C.c_void_p), ("out16", C.c_void_p), ("out32", C.c_void_p)]


class StepBenchmarkV1(C.Structure):
    _fields_ = [("struct_size", C.c_uint32)] + [
        (n, C.c_int32) for n in (
            "layers", "hidden", "intermediate", "query_width", "key_value_width", "rows", "mode",
            "warmup", "steps", "use_graph", "kernel_filter")] + [
        ("weight_bytes", C.c_uint64), ("algorithmic_bytes_per_step", C.c_uint64),
        ("total_milliseconds", C.c_double), ("milliseconds_per_step", C.c_double),
        ("gemv_kernel_milliseconds_per_step", C.c_double), ("output_checksum", C.c_uint64)]


# Layouts pinned by the reference's Rust FFI test (native_talker.rs:1734-1744).
ABI_SIZES = {
    SamplingConfig: 20, PrefillResult: 12, CodecFrameInfo: 16, ModelMemory: 16,
    SessionMemory: 32, TalkerStateInfo: 40, DeviceFrameViewV2: 40,
}
for _t, _n in ABI_SIZES.items():
    assert C.sizeof(_t) == _n, (_t.__name__, C.sizeof(_t), _n)
assert C.alignment(DeviceFrameViewV2) == 8

P = C.c_void_p
I32 = C.c_int32
U64 = C.c_uint64
ERR = [C.c_char_p, C.c_size_t]

# name -> (restype, argtypes)
SIGNATURES = {
    "qwen3_tts_talker_abi_version": (C.c_uint32, []),
    "qwen3_tts_probe_device": (I32, [I32, C.POINTER(DeviceInfo)] + ERR),
    "qwen3_tts_benchmark_bf16_argmax": (I32, [I32, I32, I32, C.POINTER(ArgmaxBenchmark)] + ERR),
    "qwen3_tts_benchmark_bf16_gemv": (I32, [I32, I32, I32, I32, C.POINTER(GemvBenchmark)] + ERR),
    "qwen3_tts_device_buffer_create": (I32, [I32, U64, U64, C.POINTER(P), C.POINTER(WeightUploadMetrics)] + ERR),
    "qwen3_tts_validate_transformer_primitives": (I32, [I32, C.POINTER(PrimitiveParity)] + ERR),
    "qwen3_tts_device_buffer_upload": (I32, [P, U64, P, U64] + ERR),
    "qwen3_tts_device_buffer_finish": (I32, [P, C.POINTER(WeightUploadMetrics)] + ERR),
    "qwen3_tts_device_buffer_read": (I32, [P, U64, P, U64] + ERR),
    "qwen3_tts_device_buffer_data": (P, [P]),
    "qwen3_tts_device_buffer_destroy": (None, [P]),
    "qwen3_tts_model_create": (I32, [I32, C.POINTER(P)] + ERR),
    "qwen3_tts_model_destroy": (None, [P]),
    "qwen3_tts_model_upload_tensor": (I32, [P, C.c_char_p, P, U64, I32, C.POINTER(U64)] + ERR),
    "qwen3_tts_model_finalize": (I32, [P, C.POINTER(ModelMemory)] + ERR),
    "qwen3_tts_session_create": (I32, [P, I32, U64, C.POINTER(P), C.POINTER(SessionMemory)] + ERR),
    "qwen3_tts_session_destroy": (None, [P]),
    "qwen3_tts_session_reset": (I32, [P, U64] + ERR),
    "qwen3_tts_session_prefill": (I32, [P, C.POINTER(I32), C.POINTER(I32), I32, SamplingConfig,
                                        C.POINTER(PrefillResult)] + ERR),
    "qwen3_tts_session_next_frame": (I32, [P, C.c_uint16, I32, SamplingConfig, SamplingConfig,
                                           C.POINTER(C.c_uint16), C.c_size_t, C.POINTER(C.c_uint16),
                                           C.POINTER(CodecFrameInfo)] + ERR),
    "qwen3_tts_session_next_frame_begin_v2": (I32, [P, I32, SamplingConfig, SamplingConfig,
                                                    C.POINTER(DeviceFrameViewV2)] + ERR),
    "qwen3_tts_session_next_frame_finish_v2": (I32, [P, U64, P, C.POINTER(C.c_uint16),
                                                     C.POINTER(CodecFrameInfo)] + ERR),
    "qwen3_tts_model_batch_next_frame_begin_v2": (I32, [P, C.POINTER(P), I32, C.POINTER(I32),
                                                        C.POINTER(SamplingConfig), C.POINTER(SamplingConfig),
                                                        C.POINTER(DeviceFrameViewV2)] + ERR),
    "qwen3_tts_session_state_info": (I32, [P, C.POINTER(TalkerStateInfo)] + ERR),
    "qwen3_tts_session_read_last_hidden_v1": (I32, [P, P, U64] + ERR),
    "qwen3_tts_session_read_talker_cache_v1": (I32, [P, I32, I32, I32, P, U64] + ERR),
    # additive exports
    "qwen3_tts_model_config_default": (None, [C.POINTER(ModelConfigV1)]),
    "qwen3_tts_model_create_with_config": (I32, [I32, C.POINTER(ModelConfigV1), C.POINTER(P)] + ERR),
    "qwen3_tts_int8_gemv_v1": (I32, [C.POINTER(Int8GemvV1), P] + ERR),
    "qwen3_tts_quantize_weight_rows_v1": (I32, [P, P, P, I32, I32, P] + ERR),
    "qwen3_tts_benchmark_int8_gemv": (I32, [I32, I32, I32, I32, C.POINTER(GemvBenchmark)] + ERR),
    "qwen3_tts_op_rms_norm_rows": (I32, [P, P, P, I32, I32, C.c_float, P] + ERR),
    "qwen3_tts_op_head_rms_norm_rows": (I32, [P, P, I32, I32, I32, C.c_float, P] + ERR),
    "qwen3_tts_op_rope_rows": (I32, [P, I32, I32, I32, P, C.c_float, P] + ERR),
    "qwen3_tts_rope_table_v1": (I32, [I32, I32, C.c_float, P] + ERR),
    "qwen3_tts_op_qk_norm_rope_kv_append": (I32, [P, P, P, P, P, P, P, I32, I32, I32, I32, C.c_float, P] + ERR),
    "qwen3_tts_op_attention": (I32, [I32, P, I32, P, P, P, P, I32, I32, I32, I32, I32, P] + ERR),
    "qwen3_tts_op_prompt_attention_v1": (I32, [I32, P, I32, P, P, P, P, I32, I32, I32, I32, I32, P] + ERR),
    "qwen3_tts_op_decode_attention": (I32, [I32, P, I32, P, P, P, C.c_float, P, P, P, P, I32, I32, I32, I32, I32, P]
                                      + ERR),
    "qwen3_tts_op_decode_attention_noalloc_v1": (I32, [I32, P, I32, P, P, P, C.c_float, P, P, P, P, I32, I32, I32,
                                                        I32, I32, P] + ERR),
    "qwen3_tts_op_bf16_gemm_v1": (I32, [P, P, P, I32, I32, I32, I32, I32, I32, I32, I32, C.c_int64, C.c_int64,
                                        C.c_int64, P] + ERR),
    "qwen3_tts_op_bf16_gemm_split_v1": (I32, [P, P, P, I32, I32, I32, I32, I32, I32, I32, I32, C.c_int64,
                                              C.c_int64, C.c_int64, P, C.c_uint64, I32, I32, I32, I32, P] + ERR),
    "qwen3_tts_op_causal_softmax_v1": (I32, [P, I32, I32, I32, I32, P] + ERR),
    "qwen3_tts_op_kv_scatter_rows": (I32, [P, P, P, I32, I32, I32, P] + ERR),
    "qwen3_tts_op_elementwise": (I32, [I32, P, P, I32, I32, P] + ERR),
    "qwen3_tts_op_sample_logits": (I32, [P, I32, I32, I32, P, P, SamplingConfig, P, P, P] + ERR),
    "qwen3_tts_op_sum_embeddings": (I32, [P, I32, I32, I32, I32, P, P, P] + ERR),
    "qwen3_tts_device_malloc": (I32, [I32, U64, C.POINTER(P)] + ERR),
    "qwen3_tts_device_free": (None, [P]),
    "qwen3_tts_device_memcpy": (I32, [P, P, U64] + ERR),
    "qwen3_tts_device_fill_bf16_normal": (I32, [P, U64, U64, C.c_float, C.c_float, P] + ERR),
    "qwen3_tts_device_synchronize": (I32, [I32] + ERR),
    "qwen3_tts_stream_create": (I32, [I32, C.POINTER(P)] + ERR),
    "qwen3_tts_stream_destroy": (None, [P]),
    "qwen3_tts_stream_synchronize": (I32, [P] + ERR),
    "qwen3_tts_benchmark_talker_step_gemvs": (I32, [I32, C.POINTER(StepBenchmarkV1)] + ERR),
}

_LIB = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Load the in-tree library (raises if it has not been built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = pathlib.Path(path) if path else LIBRARY_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python qwen3-tts-native_amd/build.py` "
            "(there is no CPU fallback for the decode path)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> None:
    """Invoke a status-returning export and raise Qwen3TtsError on failure."""
    lib = load()
    err = C.create_string_buffer(512)
    status = getattr(lib, name)(*args, err, C.sizeof(err))
    if status != STATUS_OK:
        raise Qwen3TtsError(status, err.value.decode(errors="replace"))


# ---------------------------------------------------------------------------
# Device memory
# ---------------------------------------------------------------------------
class DeviceArray:
    """A device allocation holding one numpy-typed array."""

    def __init__(self, shape, dtype, device: int = 0):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        ptr = P()
        call("qwen3_tts_device_malloc", device, max(self.nbytes, 16), C.byref(ptr))
        self.ptr = ptr.value

    @classmethod
    def from_numpy(cls, array: np.ndarray, device: int = 0) -> "DeviceArray":
        a = np.ascontiguousarray(array)
        d = cls(a.shape, a.dtype, device)
        d.upload(a)
        return d

    def upload(self, array: np.ndarray) -> None:
        a = np.ascontiguousarray(array, dtype=self.dtype)
        assert a.nbytes == self.nbytes
        if self.nbytes:
            call("qwen3_tts_device_memcpy", self.ptr, a.ctypes.data, self.nbytes)

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        if self.nbytes:
            call("qwen3_tts_device_memcpy", out.ctypes.data, self.ptr, self.nbytes)
        return out

    def offset(self, elements: int) -> int:
        return self.ptr + elements * self.dtype.itemsize

    def free(self) -> None:
        if self.ptr:
            load().qwen3_tts_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def synchronize(device: int = 0) -> None:
    call("qwen3_tts_device_synchronize", device)


# ---------------------------------------------------------------------------
# bf16 helpers (round to nearest even, as the kernels)
# ---------------------------------------------------------------------------
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = 0x7FFF
    return r


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---------------------------------------------------------------------------
# Kernel-level wrappers
# ---------------------------------------------------------------------------
def int8_gemv(weight: DeviceArray, scales: DeviceArray, x: DeviceArray, in_features: int,
              out_features: int, rows: int = 1, *, out16: DeviceArray | None = None,
              out32: DeviceArray | None = None, epilogue: int = EPI_STORE, mode: int = MODE_AUTO,
              norm_weight: DeviceArray | None = None, norm_epsilon: float = 1e-6,
              bias: DeviceArray | None = None, input_row_index: DeviceArray | None = None,
              input_ptr: int | None = None, stream: int | None = None) -> None:
    a = Int8GemvV1()
    a.struct_size = C.sizeof(Int8GemvV1)
    a.in_features, a.out_features, a.rows = in_features, out_features, rows
    a.epilogue, a.mode, a.norm_epsilon = epilogue, mode, norm_epsilon
    a.weight, a.scales = weight.ptr, scales.ptr
    a.input = input_ptr if input_ptr is not None else x.ptr
    a.norm_weight = norm_weight.ptr if norm_weight is not None else None
    a.bias = bias.ptr if bias is not None else None
    a.input_row_index = input_row_index.ptr if input_row_index is not None else None
    a.out16 = out16.ptr if out16 is not None else None
    a.out32 = out32.ptr if out32 is not None else None
    call("qwen3_tts_int8_gemv_v1", C.byref(a), stream)


def quantize_weight_rows(weight: DeviceArray, quantized: DeviceArray, scales: DeviceArray,
                         in_features: int, out_features: int) -> None:
    call("qwen3_tts_quantize_weight_rows_v1", weight.ptr, quantized.ptr, scales.ptr,
         in_features, out_features, None)


def sampling(do_sample=0, top_k=0, top_p=1.0, temperature=1.0, repetition_penalty=1.0) -> SamplingConfig:
    return SamplingConfig(do_sample, top_k, top_p, temperature, repetition_penalty)


def default_config() -> ModelConfigV1:
    c = ModelConfigV1()
    load().qwen3_tts_model_config_default(C.byref(c))
    return c
