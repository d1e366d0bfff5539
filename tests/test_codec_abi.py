"""CPU-side checks of the decoder library's boundary: it loads, exports every
symbol include/qwen3_tts_codec.h declares (the reference's C ABI,
native/qwen3-tts-native-codec/native/include/qwen3_tts_codec.h), the binding
covers them, and the structs keep the layouts the reference's Rust binding
pins (native/qwen3-tts-native-codec/src/ffi.rs:169-201)."""
import ctypes as C
import pathlib
import re

import pytest

import qwen3_tts_codec_hip as codec

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "qwen3_tts_codec.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"QWEN3_TTS_CODEC_API\s+[\w\s\*]+?\b(qwen3_tts_codec_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = codec.load()
    names = declared_symbols()
    assert len(names) == 32
    assert not [n for n in names if not hasattr(lib, n)]
    assert set(names) == set(codec.SIGNATURES)
    assert lib.qwen3_tts_codec_abi_version_v1() == 1
    assert lib.qwen3_tts_codec_abi_version_v2() == 2


def test_reference_symbols_are_declared():
    """Every decoder entry point of the reference header is declared."""
    ref = pathlib.Path("/root/reference/native/qwen3-tts-native-codec/native/include/qwen3_tts_codec.h")
    if not ref.exists():
        pytest.skip("reference tree not present")
    text = re.sub(r"/\*.*?\*/", "", ref.read_text(), flags=re.S)
    theirs = set(re.findall(r"\b(qwen3_tts_codec_\w+)\s*\(", text))
    assert theirs == set(declared_symbols())


def test_struct_layouts():
    for t, n in codec.ABI_SIZES.items():
        assert C.sizeof(t) == n, t
        assert C.alignment(t) == 8
    assert C.sizeof(codec.StateInfo) == 80
    assert C.sizeof(codec.BatchItem) == 48
    assert C.sizeof(codec.TensorView) == 56
    assert C.sizeof(codec.WeightProvider) == 32
    assert C.sizeof(codec.ModelInfo) == 40


def test_invalid_arguments_rejected_without_a_device():
    lib = codec.load()
    err = C.create_string_buffer(256)
    assert lib.qwen3_tts_codec_create_v1(None, None, err, 256) == -1
    assert b"required" in err.value
    cfg = codec.Config(0, 2, 4, 0)
    out = C.c_void_p()
    assert lib.qwen3_tts_codec_create_v1(C.byref(cfg), C.byref(out), err, 256) == -1
    assert b"three ring slots" in err.value
    assert lib.qwen3_tts_codec_process_batch_v1(None, 0, err, 256) == -1
    assert lib.qwen3_tts_codec_session_create_v1(None, None, err, 256) == -1
    assert lib.qwen3_tts_codec_shared_model_create_v1(-1, C.byref(out), err, 256) == -1
