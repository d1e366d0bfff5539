"""ctypes binding of libqwen3_tts_codec_hip.so (include/qwen3_tts_codec.h).

Mirrors the reference's Rust NativeCodecLibrary
(native/qwen3-tts-native-codec/src/ffi.rs): the same structs, a weight
provider callback over named tensors, and thin model / session wrappers that
raise CodecError with the library's status and message.  There is no CPU
fallback: loading fails if the library has not been built.
"""
from __future__ import annotations

import ctypes as C
import os
import pathlib

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIBRARY_PATH = HERE / "libqwen3_tts_codec_hip.so"

CODEBOOKS = 16
MAX_PACKET_FRAMES = 4
SAMPLES_PER_FRAME = 1920
MAX_PACKET_SAMPLES = 7680
RING_SLOTS = 3
TENSOR_F32, TENSOR_BF16 = 1, 2
STATUS = {0: "ok", -1: "invalid argument", -2: "device", -3: "state", -4: "allocation", -5: "model"}


class CodecError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)} ({status}): {message}")
        self.status = status
        self.message = message


class Config(C.Structure):
    _fields_ = [("device_index", C.c_int32), ("ring_slots", C.c_int32), ("max_packet_frames", C.c_int32),
                ("reserved", C.c_int32)]


class StateInfo(C.Structure):
    _fields_ = [("frame_position", C.c_uint64), ("emitted_samples", C.c_uint64), ("device_bytes", C.c_uint64),
                ("host_pinned_bytes", C.c_uint64), ("transformer_kv_bytes", C.c_uint64),
                ("convolution_history_bytes", C.c_uint64), ("codec_ring_bytes", C.c_uint64),
                ("pcm_ring_bytes", C.c_uint64), ("kv_ring_head", C.c_uint32), ("next_ring_slot", C.c_uint32),
                ("ring_slots", C.c_uint32), ("max_packet_frames", C.c_uint32)]


class PacketResult(C.Structure):
    _fields_ = [("first_frame_position", C.c_uint64), ("first_sample_position", C.c_uint64),
                ("frame_count", C.c_uint32), ("sample_count", C.c_uint32), ("ring_slot", C.c_uint32),
                ("is_final", C.c_uint32), ("gpu_microseconds", C.c_float), ("end_to_end_microseconds", C.c_float)]


class BatchItem(C.Structure):
    _fields_ = [("context", C.c_void_p), ("codec_frames", C.c_void_p), ("frame_count", C.c_uint32),
                ("is_final", C.c_int32), ("pcm_output", C.c_void_p), ("pcm_capacity_samples", C.c_size_t),
                ("result", C.POINTER(PacketResult))]


class TensorView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("byte_length", C.c_uint64), ("shape", C.c_uint64 * 4),
                ("rank", C.c_uint32), ("dtype", C.c_uint32)]


TENSOR_AT = C.CFUNCTYPE(C.c_int32, C.c_void_p, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(TensorView),
                        C.c_char_p, C.c_size_t)


class WeightProvider(C.Structure):
    _fields_ = [("abi_version", C.c_uint32), ("reserved", C.c_uint32), ("tensor_count", C.c_uint64),
                ("user_data", C.c_void_p), ("tensor_at", TENSOR_AT)]


class ModelInfo(C.Structure):
    _fields_ = [("source_bytes", C.c_uint64), ("device_bytes", C.c_uint64), ("parameter_count", C.c_uint64),
                ("tensor_count", C.c_uint32), ("source_dtype_f32_count", C.c_uint32),
                ("source_dtype_bf16_count", C.c_uint32), ("loaded", C.c_uint32)]


class ModelMemoryInfo(C.Structure):
    _fields_ = [("source_bytes", C.c_uint64), ("shared_weight_device_bytes", C.c_uint64),
                ("parameter_count", C.c_uint64), ("transient_upload_device_bytes", C.c_uint64),
                ("tensor_count", C.c_uint32), ("warmup_completed", C.c_uint32),
                ("active_session_count", C.c_uint32), ("reserved", C.c_uint32)]


class SessionMemoryInfo(C.Structure):
    _fields_ = [("device_bytes", C.c_uint64), ("host_pinned_bytes", C.c_uint64),
                ("transformer_kv_bytes", C.c_uint64), ("convolution_history_bytes", C.c_uint64),
                ("codec_ring_bytes", C.c_uint64), ("pcm_ring_bytes", C.c_uint64),
                ("workspace_device_bytes", C.c_uint64), ("reserved", C.c_uint64)]


class DevicePacketBegin(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("reserved", C.c_uint32), ("device_codec_frames", C.c_void_p),
                ("frame_count", C.c_uint32), ("reserved_2", C.c_uint32), ("producer_ready_event", C.c_void_p),
                ("reserved_3", C.c_uint64)]


class DevicePacketBeginResult(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("reserved", C.c_uint32), ("ticket_id", C.c_uint64),
                ("codes_consumed_event", C.c_void_p), ("reserved_2", C.c_uint64)]


class DevicePacketFinish(C.Structure):
    _fields_ = [("struct_size", C.c_uint32), ("reserved", C.c_uint32), ("ticket_id", C.c_uint64),
                ("is_final", C.c_int32), ("reserved_2", C.c_uint32), ("pcm_output", C.c_void_p),
                ("pcm_capacity_samples", C.c_size_t), ("result", C.POINTER(PacketResult)),
                ("reserved_3", C.c_uint64)]


STRIDES = (8, 5, 4, 3)
STAGE_IN = (1536, 768, 384, 192)
STAGE_OUT = (768, 384, 192, 96)


def tensor_shapes() -> dict:
    """Name -> PyTorch shape of the 271 decoder tensors a provider hands over
    (the loader requires exactly 271 "decoder." tensors, CS:3281; the two RVQ
    input projections are counted but not executed)."""
    s = {}
    q = "decoder.quantizer."
    for cb in range(16):
        p = q + ("rvq_first.vq.layers.0._codebook." if cb == 0 else f"rvq_rest.vq.layers.{cb - 1}._codebook.")
        s[p + "embedding_sum"] = (2048, 256)
        s[p + "cluster_usage"] = (2048,)
    for part in ("rvq_first", "rvq_rest"):
        s[f"{q}{part}.output_proj.weight"] = (512, 256, 1)
        s[f"{q}{part}.input_proj.weight"] = (256, 512, 1)
    s["decoder.pre_conv.conv.weight"], s["decoder.pre_conv.conv.bias"] = (1024, 512, 3), (1024,)
    t = "decoder.pre_transformer."
    s[t + "input_proj.weight"], s[t + "input_proj.bias"] = (512, 1024), (512,)
    for l in range(8):
        p = f"{t}layers.{l}."
        for n, shape in (("input_layernorm.weight", (512,)), ("self_attn.q_proj.weight", (1024, 512)),
                         ("self_attn.k_proj.weight", (1024, 512)), ("self_attn.v_proj.weight", (1024, 512)),
                         ("self_attn.o_proj.weight", (512, 1024)), ("self_attn_layer_scale.scale", (512,)),
                         ("post_attention_layernorm.weight", (512,)), ("mlp.gate_proj.weight", (1024, 512)),
                         ("mlp.up_proj.weight", (1024, 512)), ("mlp.down_proj.weight", (512, 1024)),
                         ("mlp_layer_scale.scale", (512,))):
            s[p + n] = shape
    s[t + "norm.weight"], s[t + "output_proj.weight"], s[t + "output_proj.bias"] = (512,), (1024, 512), (1024,)
    for u in range(2):
        p = f"decoder.upsample.{u}."
        for n, shape in (("0.conv.weight", (1024, 1024, 2)), ("0.conv.bias", (1024,)),
                         ("1.dwconv.conv.weight", (1024, 1, 7)), ("1.dwconv.conv.bias", (1024,)),
                         ("1.norm.weight", (1024,)), ("1.norm.bias", (1024,)), ("1.pwconv1.weight", (4096, 1024)),
                         ("1.pwconv1.bias", (4096,)), ("1.pwconv2.weight", (1024, 4096)),
                         ("1.pwconv2.bias", (1024,)), ("1.gamma", (1024,))):
            s[p + n] = shape
    s["decoder.decoder.0.conv.weight"], s["decoder.decoder.0.conv.bias"] = (1536, 1024, 7), (1536,)
    for b in range(4):
        ci, co, st = STAGE_IN[b], STAGE_OUT[b], STRIDES[b]
        p = f"decoder.decoder.{b + 1}.block."
        s[p + "0.alpha"], s[p + "0.beta"] = (ci,), (ci,)
        s[p + "1.conv.weight"], s[p + "1.conv.bias"] = (ci, co, 2 * st), (co,)
        for u in range(3):
            r = f"{p}{u + 2}."
            for n, shape in (("act1.alpha", (co,)), ("act1.beta", (co,)), ("conv1.conv.weight", (co, co, 7)),
                             ("conv1.conv.bias", (co,)), ("act2.alpha", (co,)), ("act2.beta", (co,)),
                             ("conv2.conv.weight", (co, co, 1)), ("conv2.conv.bias", (co,))):
                s[r + n] = shape
    s["decoder.decoder.5.alpha"], s["decoder.decoder.5.beta"] = (96,), (96,)
    s["decoder.decoder.6.conv.weight"], s["decoder.decoder.6.conv.bias"] = (1, 96, 7), (1,)
    return s


def packet_flops(frames: int) -> int:
    """Multiply-add flops (2 per MAC) of one packet's matrix products."""
    f = frames
    t = 2 * f * (512 * 512 + 1024 * 1536 + 512 * 1024 + 8 * (3072 * 512 + 512 * 1024 + 2048 * 512 + 512 * 1024)
                 + 1024 * 512)
    up = sum(2 * (m * 2048 * 1024 + 2 * m * 4096 * 1024 * 2) for m in (f, 2 * f))
    dec = 2 * 4 * f * 1536 * 7 * 1024
    p = 4 * f
    for b in range(4):
        ci, co, st = STAGE_IN[b], STAGE_OUT[b], STRIDES[b]
        dec += 2 * p * (st * co) * (2 * ci)
        p *= st
        dec += 3 * 2 * p * co * (7 * co + co)
    dec += 2 * p * 96 * 7
    return t + up + dec


# Layouts pinned by the reference's Rust tests (ffi.rs:169-201).
ABI_SIZES = {PacketResult: 40, DevicePacketBegin: 40, DevicePacketBeginResult: 32, DevicePacketFinish: 56}

_P, _E = C.c_void_p, [C.c_char_p, C.c_size_t]
_I32, _U32 = C.c_int32, C.c_uint32
SIGNATURES = {
    "qwen3_tts_codec_abi_version_v1": (_I32, []),
    "qwen3_tts_codec_abi_version_v2": (_I32, []),
    "qwen3_tts_codec_create_v1": (_I32, [C.POINTER(Config), C.POINTER(_P)] + _E),
    "qwen3_tts_codec_destroy_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_reset_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_state_info_v1": (_I32, [_P, C.POINTER(StateInfo)] + _E),
    "qwen3_tts_codec_load_model_v1": (_I32, [_P, C.POINTER(WeightProvider), C.POINTER(ModelInfo)] + _E),
    "qwen3_tts_codec_model_info_v1": (_I32, [_P, C.POINTER(ModelInfo)] + _E),
    "qwen3_tts_codec_warmup_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_debug_frontend_packet_v1": (_I32, [_P, _P, _U32, _P, C.c_size_t, _P, C.c_size_t] + _E),
    "qwen3_tts_codec_debug_transformer_packet_v1": (_I32, [_P, _P, _U32, _P, C.c_size_t] + _E),
    "qwen3_tts_codec_debug_latent_packet_v1": (_I32, [_P, _P, _U32, _P, C.c_size_t, _P, C.c_size_t] + _E),
    "qwen3_tts_codec_debug_decoder_checkpoint_v1": (_I32, [_P, _P, _U32, _U32, _P, C.c_size_t] + _E),
    "qwen3_tts_codec_process_packet_v1": (_I32, [_P, _P, _U32, _I32, _P, C.c_size_t, C.POINTER(PacketResult)] + _E),
    "qwen3_tts_codec_process_batch_v1": (_I32, [C.POINTER(BatchItem), _U32] + _E),
    "qwen3_tts_codec_process_fixture_packet_v1": (
        _I32, [_P, _P, _U32, _I32, _P, C.c_size_t, C.POINTER(PacketResult)] + _E),
    "qwen3_tts_codec_shared_model_create_v1": (_I32, [_I32, C.POINTER(_P)] + _E),
    "qwen3_tts_codec_shared_model_destroy_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_shared_model_load_v1": (_I32, [_P, C.POINTER(WeightProvider), C.POINTER(ModelInfo)] + _E),
    "qwen3_tts_codec_shared_model_warmup_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_shared_model_info_v1": (_I32, [_P, C.POINTER(ModelInfo)] + _E),
    "qwen3_tts_codec_shared_model_memory_info_v1": (_I32, [_P, C.POINTER(ModelMemoryInfo)] + _E),
    "qwen3_tts_codec_session_create_v1": (_I32, [_P, C.POINTER(_P)] + _E),
    "qwen3_tts_codec_session_destroy_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_session_reset_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_session_cancel_v1": (_I32, [_P] + _E),
    "qwen3_tts_codec_session_state_info_v1": (_I32, [_P, C.POINTER(StateInfo)] + _E),
    "qwen3_tts_codec_session_memory_info_v1": (_I32, [_P, C.POINTER(SessionMemoryInfo)] + _E),
    "qwen3_tts_codec_session_process_packet_v1": (
        _I32, [_P, _P, _U32, _I32, _P, C.c_size_t, C.POINTER(PacketResult)] + _E),
    "qwen3_tts_codec_session_process_device_packet_begin_v2": (
        _I32, [_P, C.POINTER(DevicePacketBegin), C.POINTER(DevicePacketBeginResult)] + _E),
    "qwen3_tts_codec_session_process_device_packet_finish_v2": (_I32, [_P, C.POINTER(DevicePacketFinish)] + _E),
    "qwen3_tts_codec_session_process_batch_v1": (_I32, [C.POINTER(BatchItem), _U32] + _E),
}

_LIB = None


def load(path: os.PathLike | str | None = None) -> C.CDLL:
    """Load the in-tree codec library (raises if it has not been built)."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = pathlib.Path(path) if path else LIBRARY_PATH
    if not p.exists():
        raise FileNotFoundError(
            f"{p} is missing: build it with `python qwen3-tts-native_amd/build.py` "
            "(there is no CPU fallback for the decoder)")
    lib = C.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _LIB = lib
    return lib


def call(name: str, *args) -> None:
    err = C.create_string_buffer(512)
    status = getattr(load(), name)(*args, err, C.sizeof(err))
    if status != 0:
        raise CodecError(status, err.value.decode(errors="replace"))


def _ptr(a: np.ndarray):
    return C.c_void_p(a.ctypes.data)


class Provider:
    """Weight provider over {name: array}: fp32 arrays are passed as F32,
    arrays of dtype uint16 as raw bf16 bits."""

    def __init__(self, tensors: dict, shapes: dict | None = None):
        self.items = []
        for name, arr in tensors.items():
            arr = np.ascontiguousarray(arr)
            if arr.dtype not in (np.float32, np.uint16):
                arr = arr.astype(np.float32)
            shape = tuple(shapes[name]) if shapes and name in shapes else arr.shape
            self.items.append((name.encode(), arr, shape))
        self._names = [C.c_char_p(n) for n, _, _ in self.items]

        def tensor_at(user, index, name_out, view, err, cap):
            if index >= len(self.items):
                return -1
            name, arr, shape = self.items[index]
            name_out[0] = self._names[index]
            view.contents.data = arr.ctypes.data
            view.contents.byte_length = arr.nbytes
            for d in range(4):
                view.contents.shape[d] = shape[d] if d < len(shape) else 0
            view.contents.rank = len(shape)
            view.contents.dtype = TENSOR_BF16 if arr.dtype == np.uint16 else TENSOR_F32
            return 0

        self._callback = TENSOR_AT(tensor_at)
        self.struct = WeightProvider(1, 0, len(self.items), None, self._callback)


class SharedModel:
    def __init__(self, tensors: dict, device: int = 0, shapes: dict | None = None, warm: bool = True):
        load()
        self.handle = C.c_void_p()
        call("qwen3_tts_codec_shared_model_create_v1", device, C.byref(self.handle))
        self.info = ModelInfo()
        provider = Provider(tensors, shapes)
        call("qwen3_tts_codec_shared_model_load_v1", self.handle, C.byref(provider.struct), C.byref(self.info))
        if warm:
            call("qwen3_tts_codec_shared_model_warmup_v1", self.handle)

    def memory_info(self) -> ModelMemoryInfo:
        m = ModelMemoryInfo()
        call("qwen3_tts_codec_shared_model_memory_info_v1", self.handle, C.byref(m))
        return m

    def session(self) -> "Session":
        return Session(self)

    def close(self):
        if self.handle:
            call("qwen3_tts_codec_shared_model_destroy_v1", self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Session:
    """A decoding stream of a SharedModel (or, with model=None, a legacy
    context that owns its model)."""

    def __init__(self, model: SharedModel | None, device: int = 0):
        self.model = model
        self.handle = C.c_void_p()
        if model is not None:
            call("qwen3_tts_codec_session_create_v1", model.handle, C.byref(self.handle))
        else:
            cfg = Config(device, RING_SLOTS, MAX_PACKET_FRAMES, 0)
            call("qwen3_tts_codec_create_v1", C.byref(cfg), C.byref(self.handle))

    def packet(self, codes, is_final: bool = False):
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        pcm = np.zeros(MAX_PACKET_SAMPLES, np.int16)
        res = PacketResult()
        call("qwen3_tts_codec_session_process_packet_v1", self.handle, _ptr(codes), codes.shape[0],
             1 if is_final else 0, _ptr(pcm), pcm.size, C.byref(res))
        return pcm[: res.sample_count].copy(), res

    def fixture_packet(self, codes, is_final: bool = False):
        """The reference's weight-free state-machine fixture packet."""
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        pcm = np.zeros(MAX_PACKET_SAMPLES, np.int16)
        res = PacketResult()
        call("qwen3_tts_codec_process_fixture_packet_v1", self.handle, _ptr(codes), codes.shape[0],
             1 if is_final else 0, _ptr(pcm), pcm.size, C.byref(res))
        return pcm[: res.sample_count].copy(), res

    def state(self) -> StateInfo:
        s = StateInfo()
        call("qwen3_tts_codec_session_state_info_v1", self.handle, C.byref(s))
        return s

    def memory(self) -> SessionMemoryInfo:
        s = SessionMemoryInfo()
        call("qwen3_tts_codec_session_memory_info_v1", self.handle, C.byref(s))
        return s

    def reset(self):
        call("qwen3_tts_codec_session_reset_v1", self.handle)

    def cancel(self):
        call("qwen3_tts_codec_session_cancel_v1", self.handle)

    # -- debug hooks: outputs returned row-major [positions][channels] --------
    def debug_frontend(self, codes):
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        f = codes.shape[0]
        rvq = np.zeros(512 * f, np.float32)
        pre = np.zeros(1024 * f, np.float32)
        call("qwen3_tts_codec_debug_frontend_packet_v1", self.handle, _ptr(codes), f, _ptr(rvq), rvq.size,
             _ptr(pre), pre.size)
        return rvq.reshape(512, f).T.copy(), pre.reshape(f, 1024)

    def debug_transformer(self, codes):
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        f = codes.shape[0]
        out = np.zeros(1024 * f, np.float32)
        call("qwen3_tts_codec_debug_transformer_packet_v1", self.handle, _ptr(codes), f, _ptr(out), out.size)
        return out.reshape(f, 1024)

    def debug_latent(self, codes):
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        f = codes.shape[0]
        one = np.zeros(2 * f * 1024, np.float32)
        two = np.zeros(4 * f * 1024, np.float32)
        call("qwen3_tts_codec_debug_latent_packet_v1", self.handle, _ptr(codes), f, _ptr(one), one.size, _ptr(two),
             two.size)
        return one.reshape(1024, 2 * f).T.copy(), two.reshape(1024, 4 * f).T.copy()

    def debug_checkpoint(self, codes, checkpoint: int, positions: int, channels: int):
        codes = np.ascontiguousarray(np.atleast_2d(codes), np.uint16)
        out = np.zeros(positions * channels, np.float32)
        call("qwen3_tts_codec_debug_decoder_checkpoint_v1", self.handle, _ptr(codes), codes.shape[0], checkpoint,
             _ptr(out), out.size)
        return out.reshape(channels, positions).T.copy()

    def close(self):
        if self.handle:
            call("qwen3_tts_codec_session_destroy_v1", self.handle)
            self.handle = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def process_batch(sessions, codes_list, finals=None):
    """session_process_batch_v1 over parallel lists; returns [(pcm, result)]."""
    n = len(sessions)
    finals = finals or [False] * n
    codes = [np.ascontiguousarray(np.atleast_2d(c), np.uint16) for c in codes_list]
    pcms = [np.zeros(MAX_PACKET_SAMPLES, np.int16) for _ in range(n)]
    results = [PacketResult() for _ in range(n)]
    items = (BatchItem * n)()
    for i in range(n):
        items[i] = BatchItem(sessions[i].handle, codes[i].ctypes.data, codes[i].shape[0], 1 if finals[i] else 0,
                             pcms[i].ctypes.data, MAX_PACKET_SAMPLES, C.pointer(results[i]))
    call("qwen3_tts_codec_session_process_batch_v1", items, n)
    return [(pcms[i][: results[i].sample_count].copy(), results[i]) for i in range(n)]
