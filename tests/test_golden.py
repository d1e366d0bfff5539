"""Committed golden fixtures (tests/golden/, written by make_golden.py):
the oracle must reproduce them on the CPU, and the HIP library on the GPU."""
import ctypes as C
import hashlib
import json
import pathlib

import numpy as np
import pytest

import gen

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
SMALL = sorted(GOLDEN.glob("gemv_*.npz"))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def config1():
    import make_golden

    return make_golden.config1_inputs()


@pytest.fixture(scope="module", autouse=True)
def _golden_path():
    import sys

    sys.path.insert(0, str(GOLDEN))


def test_fixtures_present():
    assert len(SMALL) == 3
    assert (GOLDEN / "digests.json").exists() and (GOLDEN / "argmax_kat.json").exists()


@pytest.mark.parametrize("path", SMALL, ids=lambda p: p.stem)
def test_oracle_reproduces_small_fixtures(orc, path):
    f = np.load(path)
    y32, y16 = orc.int8_gemm_rows(f["w"], f["s"], f["x"])
    assert np.array_equal(y32, f["y32"]) and np.array_equal(y16, f["y16"])


def test_oracle_reproduces_config1_digest(orc):
    d = json.loads((GOLDEN / "digests.json").read_text())["config1"]
    w, s, x = config1()
    assert sha(w) + sha(s) + sha(x) == d["inputs_sha256"]
    y32, y16 = orc.int8_gemm_rows(w, s, x)
    assert sha(y32) == d["y32_sha256"] and sha(y16) == d["y16_sha256"]


def test_argmax_kat(orc):
    for k in json.loads((GOLDEN / "argmax_kat.json").read_text()):
        v = k["vocabulary_size"]
        i = np.arange(v, dtype=np.float32)
        logits = gen.bf16(np.sin(i * np.float32(0.017)) * np.float32(2.0))
        logits[k["expected_token"]] = gen.bf16(np.float32(19.0))
        assert orc.argmax_bf16(logits) == k["selected_token"]


@pytest.mark.gpu
@pytest.mark.parametrize("path", SMALL, ids=lambda p: p.stem)
def test_gpu_reproduces_small_fixtures(hip, path):
    f = np.load(path)
    rows, in_f = f["x"].shape
    out_f = f["w"].shape[0]
    w, s, x = (hip.DeviceArray.from_numpy(f[k]) for k in ("w", "s", "x"))
    y32 = hip.DeviceArray((rows, out_f), np.float32)
    y16 = hip.DeviceArray((rows, out_f), np.uint16)
    hip.int8_gemv(w, s, x, in_f, out_f, rows, out16=y16, out32=y32, mode=hip.MODE_EXACT)
    assert np.array_equal(y32.numpy(), f["y32"]) and np.array_equal(y16.numpy(), f["y16"])


@pytest.mark.gpu
def test_gpu_reproduces_config1_digest(hip):
    d = json.loads((GOLDEN / "digests.json").read_text())["config1"]
    w, s, x = config1()
    dw, ds, dx = (hip.DeviceArray.from_numpy(a) for a in (w, s, x))
    y32 = hip.DeviceArray((1, 6144), np.float32)
    y16 = hip.DeviceArray((1, 6144), np.uint16)
    hip.int8_gemv(dw, ds, dx, 2048, 6144, 1, out16=y16, out32=y32, mode=hip.MODE_EXACT)
    assert sha(y32.numpy()) == d["y32_sha256"] and sha(y16.numpy()) == d["y16_sha256"]


@pytest.mark.gpu
def test_gpu_reproduces_toy_greedy_stream(hip):
    import toy_model

    d = json.loads((GOLDEN / "digests.json").read_text())["toy_greedy_stream"]
    weights = toy_model.make_weights(toy_model.TOY, seed=3)
    model, _ = toy_model.upload(hip, toy_model.TOY, weights)
    lib = hip.load()
    s = C.c_void_p()
    mem = hip.SessionMemory()
    hip.call("qwen3_tts_session_create", model, 64, 7, C.byref(s), C.byref(mem))
    try:
        rng = np.random.default_rng(11)
        text = rng.integers(0, toy_model.TOY["text_vocabulary"], 6).astype(np.int32)
        codec = rng.integers(0, 2048, 6).astype(np.int32)
        text[1], codec[2] = -1, -1
        g = hip.SamplingConfig(0, 0, 1.0, 1.0, 1.05)
        pre = hip.PrefillResult()
        hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
                 codec.ctypes.data_as(C.POINTER(C.c_int32)), 6, g, C.byref(pre))
        assert pre.first_semantic_token == d["first"]
        sem = pre.first_semantic_token
        for f, want in enumerate(d["frames"]):
            codes = (C.c_uint16 * 16)()
            nxt = C.c_uint16()
            info = hip.CodecFrameInfo()
            hip.call("qwen3_tts_session_next_frame", s, sem, 100 + f, g, g, codes, 16, C.byref(nxt), C.byref(info))
            assert list(codes) == want["codes"] and nxt.value == want["next"]
            sem = nxt.value
    finally:
        lib.qwen3_tts_session_destroy(s)
        lib.qwen3_tts_model_destroy(model)
