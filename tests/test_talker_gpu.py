"""End-to-end parity of the talker + code-predictor frame step through the
reference C ABI (native/qwen3-tts-native/native/include/qwen3_tts_native.h)
against the oracle's restatement of TalkerContext::begin_frame
(native/qwen3-tts-native/native/src/talker.cu:1095-1262) on a reduced
geometry.  Every frame's 16 codes and the next semantic token must be
identical -- under greedy decoding and under top-k sampling from the same
seed (the sampler and the RNG are restated exactly).  Frames 1, 2 and 3+ run
eagerly, under hipGraph capture and as graph replays respectively."""
import ctypes as C
import os

import numpy as np
import pytest

import toy_model
from toy_model import TOY

pytestmark = pytest.mark.gpu

GREEDY = (0, 0, 1.0, 1.0, 1.05)
TALKER_TOPK = (1, 50, 1.0, 0.9, 1.05)
PREDICTOR_TOPK = (1, 50, 1.0, 0.9, 1.0)


@pytest.fixture(autouse=True)
def decode_step_prefill(monkeypatch):
    """These tests compare with the oracle's decode-step prefill (the bf16
    prefill has its own tests in test_prefill_gpu.py)."""
    monkeypatch.setenv("QWEN3_TTS_PREFILL", "decode")


@pytest.fixture(scope="module")
def toy(hip, orc):
    weights = toy_model.make_weights(TOY, seed=3)
    model, mem = toy_model.upload(hip, TOY, weights)
    om = toy_model.OracleModel(orc, TOY, weights)
    yield model, mem, om, weights
    hip.load().qwen3_tts_model_destroy(model)


def new_session(hip, model, max_seq=64, seed=7):
    s = C.c_void_p()
    mem = hip.SessionMemory()
    hip.call("qwen3_tts_session_create", model, max_seq, seed, C.byref(s), C.byref(mem))
    return s, mem


def prompt(rng, n):
    text = rng.integers(0, TOY["text_vocabulary"], n).astype(np.int32)
    codec = rng.integers(0, 2048, n).astype(np.int32)
    text[1] = -1  # codec-only position
    codec[2] = -1  # text-only position
    return text, codec


def gpu_prefill(hip, s, text, codec, sampling):
    out = hip.PrefillResult()
    hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
             codec.ctypes.data_as(C.POINTER(C.c_int32)), len(text), hip.SamplingConfig(*sampling), C.byref(out))
    return out


def gpu_frame(hip, s, semantic, text_token, ts, ps):
    codes = (C.c_uint16 * 16)()
    nxt = C.c_uint16()
    info = hip.CodecFrameInfo()
    hip.call("qwen3_tts_session_next_frame", s, semantic, text_token, hip.SamplingConfig(*ts),
             hip.SamplingConfig(*ps), codes, 16, C.byref(nxt), C.byref(info))
    return np.array(codes, np.uint16), nxt.value, info


@pytest.mark.parametrize("mode", ["greedy", "topk"])
def test_frames_match_oracle(hip, orc, toy, mode):
    model, _, om, _ = toy
    ts, ps = (GREEDY, GREEDY) if mode == "greedy" else (TALKER_TOPK, PREDICTOR_TOPK)
    rng = np.random.default_rng(11)
    text, codec = prompt(rng, 6)
    s, smem = new_session(hip, model, max_seq=64, seed=7)
    lib = hip.load()
    try:
        osess = toy_model.OracleSession(om, 64, 7)
        pre = gpu_prefill(hip, s, text, codec, ts)
        first = osess.prefill(text, codec, ts)
        assert pre.first_semantic_token == first
        assert pre.prompt_tokens == 6
        semantic = first
        frames = 0
        for f in range(7):
            if semantic == TOY["codec_eos_token"]:
                break
            tt = int(rng.integers(0, TOY["text_vocabulary"]))
            codes, nxt, info = gpu_frame(hip, s, semantic, tt, ts, ps)
            ocodes, onxt = osess.frame(semantic, tt, ts, ps)
            assert np.array_equal(codes, ocodes), (f, codes, ocodes)
            assert nxt == onxt, f
            assert codes[0] == semantic
            assert info.talker_position == 6 + f
            assert info.predictor_gpu_milliseconds > 0 and info.talker_gpu_milliseconds > 0
            semantic = nxt
            frames += 1
        st = hip.TalkerStateInfo()
        hip.call("qwen3_tts_session_state_info", s, C.byref(st))
        assert st.abi_version == 3
        assert st.frames_generated == frames
        assert st.talker_position == 6 + frames
        assert st.semantic_history_count == 1 + frames
        assert st.device_sample_count == 1 + 16 * frames
        assert st.host_sync_count == 1 + frames
        assert smem.max_sequence_length == 64
        tkv = TOY["talker_key_value_heads"] * 128
        assert smem.talker_kv_bytes == 2 * TOY["talker_layers"] * 64 * tkv * 2
    finally:
        lib.qwen3_tts_session_destroy(s)


def test_graphs_disabled_matches(hip, orc, toy, monkeypatch):
    """The eager enqueue (no hipGraph) gives the same frames."""
    monkeypatch.setenv("QWEN3_TTS_DISABLE_GRAPHS", "1")
    model, _, om, _ = toy
    rng = np.random.default_rng(5)
    text, codec = prompt(rng, 5)
    s, _ = new_session(hip, model, seed=99)
    try:
        osess = toy_model.OracleSession(om, 64, 99)
        semantic = gpu_prefill(hip, s, text, codec, TALKER_TOPK).first_semantic_token
        assert semantic == osess.prefill(text, codec, TALKER_TOPK)
        for f in range(4):
            if semantic == TOY["codec_eos_token"]:
                break
            codes, nxt, _ = gpu_frame(hip, s, semantic, 3 + f, TALKER_TOPK, PREDICTOR_TOPK)
            ocodes, onxt = osess.frame(semantic, 3 + f, TALKER_TOPK, PREDICTOR_TOPK)
            assert np.array_equal(codes, ocodes) and nxt == onxt
            semantic = nxt
    finally:
        hip.load().qwen3_tts_session_destroy(s)


def test_begin_finish_lease_protocol(hip, orc, toy):
    model, _, om, _ = toy
    lib = hip.load()
    rng = np.random.default_rng(21)
    text, codec = prompt(rng, 4)
    s, _ = new_session(hip, model, seed=5)
    try:
        osess = toy_model.OracleSession(om, 64, 5)
        semantic = gpu_prefill(hip, s, text, codec, GREEDY).first_semantic_token
        assert semantic == osess.prefill(text, codec, GREEDY)
        g = hip.SamplingConfig(*GREEDY)
        for f in range(3):
            view = hip.DeviceFrameViewV2()
            view.struct_size = C.sizeof(hip.DeviceFrameViewV2)
            hip.call("qwen3_tts_session_next_frame_begin_v2", s, 17 + f, g, g, C.byref(view))
            assert view.code_count == 16 and view.lease_id != 0 and view.ready_event
            # a second begin while the lease is in flight is a state error
            v2 = hip.DeviceFrameViewV2()
            v2.struct_size = C.sizeof(hip.DeviceFrameViewV2)
            with pytest.raises(hip.Qwen3TtsError) as e:
                hip.call("qwen3_tts_session_next_frame_begin_v2", s, 1, g, g, C.byref(v2))
            assert e.value.status == hip.STATUS_STATE
            nxt = C.c_uint16()
            info = hip.CodecFrameInfo()
            with pytest.raises(hip.Qwen3TtsError):  # stale lease
                hip.call("qwen3_tts_session_next_frame_finish_v2", s, view.lease_id + 1, None, C.byref(nxt), C.byref(info))
            hip.call("qwen3_tts_session_next_frame_finish_v2", s, view.lease_id, None, C.byref(nxt), C.byref(info))
            # the borrowed codes are readable once ready_event has fired; finish
            # synchronized past it and no later frame has overwritten them yet
            codes = np.zeros(16, np.uint16)
            hip.call("qwen3_tts_device_memcpy", codes.ctypes.data, view.device_codes, 32)
            ocodes, onxt = osess.frame(semantic, 17 + f, GREEDY, GREEDY)
            assert np.array_equal(codes, ocodes) and nxt.value == onxt
            semantic = nxt.value
            if semantic == TOY["codec_eos_token"]:
                break
        with pytest.raises(hip.Qwen3TtsError):  # no lease in flight
            hip.call("qwen3_tts_session_next_frame_finish_v2", s, 1, None, C.byref(nxt), C.byref(info))
    finally:
        lib.qwen3_tts_session_destroy(s)


def test_session_errors_and_reset(hip, toy):
    model, _, _, _ = toy
    lib = hip.load()
    s, _ = new_session(hip, model, max_seq=16, seed=1)
    g = hip.SamplingConfig(*GREEDY)
    codes = (C.c_uint16 * 16)()
    nxt = C.c_uint16()
    info = hip.CodecFrameInfo()
    try:
        # frame before prefill
        with pytest.raises(hip.Qwen3TtsError) as e:
            hip.call("qwen3_tts_session_next_frame", s, 0, 0, g, g, codes, 16, C.byref(nxt), C.byref(info))
        assert e.value.status == hip.STATUS_STATE and "prefilled" in str(e.value)
        # invalid sampling configuration
        bad = hip.SamplingConfig(0, -1, 1.0, 1.0, 1.0)
        text = np.arange(16, dtype=np.int32)
        codec = np.full(16, -1, np.int32)
        with pytest.raises(hip.Qwen3TtsError):
            gpu_prefill(hip, s, text, codec, (0, -1, 1.0, 1.0, 1.0))
        # prompt longer than the KV cache
        with pytest.raises(hip.Qwen3TtsError):
            gpu_prefill(hip, s, np.arange(17, dtype=np.int32), np.full(17, -1, np.int32), GREEDY)
        # a full cache refuses the next frame
        pre = gpu_prefill(hip, s, text, codec, GREEDY)
        if pre.first_semantic_token != TOY["codec_eos_token"]:
            with pytest.raises(hip.Qwen3TtsError) as e:
                hip.call("qwen3_tts_session_next_frame", s, pre.first_semantic_token, 0, g, g, codes, 16,
                         C.byref(nxt), C.byref(info))
            assert "KV cache is full" in str(e.value)
        # reset returns to READY
        hip.call("qwen3_tts_session_reset", s, 3)
        st = hip.TalkerStateInfo()
        hip.call("qwen3_tts_session_state_info", s, C.byref(st))
        assert st.phase == 1 and st.talker_position == 0 and st.frames_generated == 0
        # wrong semantic token / out-of-range text token
        pre = gpu_prefill(hip, s, text[:4], codec[:4], GREEDY)
        if pre.first_semantic_token != TOY["codec_eos_token"]:
            wrong = (pre.first_semantic_token + 1) % 2048
            with pytest.raises(hip.Qwen3TtsError) as e:
                hip.call("qwen3_tts_session_next_frame", s, wrong, 0, g, g, codes, 16, C.byref(nxt), C.byref(info))
            assert "does not match" in str(e.value)
            with pytest.raises(hip.Qwen3TtsError):
                hip.call("qwen3_tts_session_next_frame", s, pre.first_semantic_token, 10**6, g, g, codes, 16,
                         C.byref(nxt), C.byref(info))
        # undersized output buffer
        err = C.create_string_buffer(256)
        assert lib.qwen3_tts_session_next_frame(s, 0, 0, g, g, codes, 8, C.byref(nxt), C.byref(info), err,
                                                256) == hip.STATUS_INVALID_ARGUMENT
    finally:
        lib.qwen3_tts_session_destroy(s)


def test_model_contract_errors(hip):
    weights = toy_model.make_weights(TOY, seed=1)
    lib = hip.load()
    model = C.c_void_p()
    hip.call("qwen3_tts_model_create_with_config", 0, C.byref(toy_model.config_struct(hip, TOY)), C.byref(model))
    try:
        mem = hip.ModelMemory()
        with pytest.raises(hip.Qwen3TtsError) as e:  # nothing uploaded
            hip.call("qwen3_tts_model_finalize", model, C.byref(mem))
        assert e.value.status == hip.STATUS_MODEL and "tensors" in str(e.value)
        name, arr = next(iter(weights.items()))
        shape = (C.c_uint64 * arr.ndim)(*arr.shape)
        hip.call("qwen3_tts_model_upload_tensor", model, name.encode(), arr.ctypes.data, arr.nbytes, arr.ndim, shape)
        with pytest.raises(hip.Qwen3TtsError):  # duplicate
            hip.call("qwen3_tts_model_upload_tensor", model, name.encode(), arr.ctypes.data, arr.nbytes, arr.ndim, shape)
        with pytest.raises(hip.Qwen3TtsError):  # byte size mismatch
            hip.call("qwen3_tts_model_upload_tensor", model, b"x", arr.ctypes.data, arr.nbytes - 2, arr.ndim, shape)
        # a wrong shape for a required tensor is reported by finalize
        for n, a in weights.items():
            if n == name:
                continue
            if n == "talker.model.norm.weight":
                a = np.concatenate([a, a])
            shp = (C.c_uint64 * a.ndim)(*a.shape)
            hip.call("qwen3_tts_model_upload_tensor", model, n.encode(), a.ctypes.data, a.nbytes, a.ndim, shp)
        with pytest.raises(hip.Qwen3TtsError) as e:
            hip.call("qwen3_tts_model_finalize", model, C.byref(mem))
        assert "unexpected shape" in str(e.value)
        # sessions need a finalized model
        s = C.c_void_p()
        smem = hip.SessionMemory()
        with pytest.raises(hip.Qwen3TtsError):
            hip.call("qwen3_tts_session_create", model, 64, 0, C.byref(s), C.byref(smem))
    finally:
        lib.qwen3_tts_model_destroy(model)


@pytest.fixture(scope="module")
def toy_wide(hip, orc):
    c = toy_model.TOY_WIDE_PREDICTOR
    weights = toy_model.make_weights(c, seed=4)
    model, mem = toy_model.upload(hip, c, weights)
    om = toy_model.OracleModel(orc, c, weights)
    yield model, om
    hip.load().qwen3_tts_model_destroy(model)


def test_wide_predictor_frames_match_oracle(hip, orc, toy_wide):
    """The production predictor head geometry (16 query / 8 kv heads, the
    one-wave-per-head short-cache attention) gives the oracle's frames."""
    model, om = toy_wide
    rng = np.random.default_rng(21)
    text, codec = prompt(rng, 6)
    s, _ = new_session(hip, model, max_seq=64, seed=13)
    try:
        osess = toy_model.OracleSession(om, 64, 13)
        semantic = gpu_prefill(hip, s, text, codec, TALKER_TOPK).first_semantic_token
        assert semantic == osess.prefill(text, codec, TALKER_TOPK)
        for f in range(5):
            if semantic == TOY["codec_eos_token"]:
                break
            codes, nxt, _ = gpu_frame(hip, s, semantic, 7 + f, TALKER_TOPK, PREDICTOR_TOPK)
            ocodes, onxt = osess.frame(semantic, 7 + f, TALKER_TOPK, PREDICTOR_TOPK)
            assert np.array_equal(codes, ocodes), (f, codes, ocodes)
            assert nxt == onxt
            semantic = nxt
    finally:
        hip.load().qwen3_tts_session_destroy(s)
