"""CPU-side checks of the drop-in boundary: the library loads, exports every
symbol declared in include/qwen3_tts_native.h, keeps the reference's struct
layouts (native/qwen3-tts-native/src/native_talker.rs:1734-1744) and rejects
invalid arguments before touching a device (int8_gemv.cu:329-331 rule:
in % 16 != 0 or rows outside [1, 8] is invalid)."""
import ctypes as C
import pathlib
import re

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "qwen3_tts_native.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"QWEN3_TTS_API\s+[\w\s\*]+?\b(qwen3_tts_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported(hip):
    lib = hip.load()
    names = declared_symbols()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding covers every declared symbol
    assert set(names) <= set(hip.SIGNATURES)


def test_reference_abi_entry_points_present(hip):
    lib = hip.load()
    reference = [
        "qwen3_tts_talker_abi_version", "qwen3_tts_probe_device", "qwen3_tts_benchmark_bf16_argmax",
        "qwen3_tts_benchmark_bf16_gemv", "qwen3_tts_device_buffer_create",
        "qwen3_tts_validate_transformer_primitives", "qwen3_tts_device_buffer_upload",
        "qwen3_tts_device_buffer_finish", "qwen3_tts_device_buffer_read", "qwen3_tts_device_buffer_data",
        "qwen3_tts_device_buffer_destroy", "qwen3_tts_model_create", "qwen3_tts_model_destroy",
        "qwen3_tts_model_upload_tensor", "qwen3_tts_model_finalize", "qwen3_tts_session_create",
        "qwen3_tts_session_destroy", "qwen3_tts_session_reset", "qwen3_tts_session_prefill",
        "qwen3_tts_session_next_frame", "qwen3_tts_session_next_frame_begin_v2",
        "qwen3_tts_session_next_frame_finish_v2", "qwen3_tts_model_batch_next_frame_begin_v2",
        "qwen3_tts_session_state_info",
    ]
    for n in reference:
        assert hasattr(lib, n), n
    assert lib.qwen3_tts_talker_abi_version() == 3


def test_struct_layouts(hip):
    for t, n in hip.ABI_SIZES.items():
        assert C.sizeof(t) == n
    assert C.alignment(hip.DeviceFrameViewV2) == 8
    assert C.sizeof(hip.GemvBenchmark) == 40


def test_default_config_is_voicedesign(hip):
    c = hip.default_config()
    assert (c.talker_layers, c.talker_hidden, c.talker_intermediate) == (28, 2048, 6144)
    assert (c.talker_query_heads, c.talker_key_value_heads, c.head_dimension) == (16, 8, 128)
    assert (c.predictor_layers, c.predictor_hidden, c.predictor_intermediate) == (5, 1024, 3072)
    assert (c.talker_vocabulary, c.predictor_vocabulary, c.text_vocabulary) == (3072, 2048, 151936)
    assert c.codec_eos_token == 2150


@pytest.mark.parametrize("in_f,rows", [(2040, 1), (2048, 0), (2048, 9)])
def test_gemv_rejects_invalid_shapes_without_device(hip, in_f, rows):
    a = hip.Int8GemvV1()
    a.struct_size = C.sizeof(hip.Int8GemvV1)
    a.in_features, a.out_features, a.rows = in_f, 64, rows
    a.weight = a.scales = a.input = a.out16 = 4096  # never dereferenced
    with pytest.raises(hip.Qwen3TtsError) as e:
        hip.call("qwen3_tts_int8_gemv_v1", C.byref(a), None)
    assert e.value.status == hip.STATUS_INVALID_ARGUMENT


def test_null_outputs_are_invalid_argument(hip):
    lib = hip.load()
    err = C.create_string_buffer(256)
    assert lib.qwen3_tts_model_create(0, None, err, 256) == hip.STATUS_INVALID_ARGUMENT
    assert b"null" in err.value
    assert lib.qwen3_tts_model_finalize(None, None, err, 256) == hip.STATUS_INVALID_ARGUMENT
    assert lib.qwen3_tts_session_state_info(None, None, err, 256) == hip.STATUS_INVALID_ARGUMENT
    view = hip.DeviceFrameViewV2()
    view.struct_size = 12  # wrong size
    assert lib.qwen3_tts_session_next_frame_begin_v2(None, 0, hip.sampling(), hip.sampling(),
                                                     C.byref(view), err, 256) == hip.STATUS_INVALID_ARGUMENT
    assert b"unsupported size" in err.value
    # session handle null -> state error path, message from the library
    info = hip.TalkerStateInfo()
    assert lib.qwen3_tts_session_state_info(None, C.byref(info), err, 256) == hip.STATUS_STATE
    assert b"session handle is null" in err.value


def test_batch_arguments_validated(hip):
    lib = hip.load()
    err = C.create_string_buffer(256)
    sessions = (C.c_void_p * 9)()
    assert lib.qwen3_tts_model_batch_next_frame_begin_v2(None, sessions, 9, None, None, None, None,
                                                         err, 256) == hip.STATUS_INVALID_ARGUMENT
