"""End-to-end parity at the production VoiceDesign geometry (BASELINE
configs 3 and 5): talker 28 layers, hidden 2048, FFN 6144, GQA 16 query /
8 key-value heads of 128; code predictor 5 layers, hidden 1024, FFN 3072,
16 / 8 heads; codec vocabulary 3072, predictor vocabulary 2048.  The text
vocabulary is reduced to 4096 rows (it only sizes an embedding table that
one row is gathered from per position).

Weights are synthetic bf16 (see make_weights), uploaded
through the reference C ABI and quantized on the device at finalize; the
oracle quantizes the same bf16 on the host (bit-identical quantizer) and runs
the reference's layer and frame sequence (oracle/oracle.c, pinned against an
independent float64 model in test_frame_f64.py).

A 66-position prompt fills the talker cache past 64 positions, so the talker
runs the long-cache attention kernels (scores + head) and the predictor its
short-cache kernel at the real head count.  Then two greedy frames (config
3: fifteen chained greedy predictor steps feeding each next step's
embedding) and two top-k 50 / T 0.9 frames from a fixed seed (config 5) must
give identical codes and next semantic tokens, and the prefill's first token
must match.  A second session runs the same through the lockstep batch entry
point in its exact mode (batched semantics,
native/qwen3-tts-native/native/src/talker.cu:2038-2334).
"""
import ctypes as C
import os

import numpy as np
import pytest

import gen
import toy_model

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

VOICEDESIGN = dict(talker_layers=28, talker_hidden=2048, talker_intermediate=6144, talker_query_heads=16,
                   talker_key_value_heads=8, predictor_layers=5, predictor_hidden=1024,
                   predictor_intermediate=3072, predictor_query_heads=16, predictor_key_value_heads=8,
                   head_dimension=128, talker_vocabulary=3072, predictor_vocabulary=2048,
                   text_vocabulary=4096, codec_eos_token=2150, rms_epsilon=1e-6, rope_theta=1e6)

GREEDY = (0, 0, 1.0, 1.0, 1.05)
TALKER_TOPK = (1, 50, 1.0, 0.9, 1.05)
PREDICTOR_TOPK = (1, 50, 1.0, 0.9, 1.0)
PROMPT = 66


def make_weights(c, seed):
    """Decode matrices as k * 2^-12 with k uniform in [-127, 127] (exact in
    bf16; generated as int8, which keeps the 1.6 G-parameter model cheap to
    build), embeddings N(0, 1), norms ~ 1 + 0.1 N(0, 1), biases 0.02 N(0, 1)."""
    rng = np.random.default_rng(seed)
    # bf16 bits of k * 2^-12 for every int8 bit pattern k
    lut = gen.bf16(np.arange(256, dtype=np.uint8).view(np.int8).astype(np.float32) * np.float32(2.0 ** -12))
    out = {}
    for name, shape, kind in toy_model.tensor_specs(c):
        if kind == "w":
            k = rng.integers(-127, 128, size=shape, dtype=np.int8)
            out[name] = lut[k.view(np.uint8)]
            continue
        x = rng.standard_normal(shape, dtype=np.float32)
        if kind == "g":
            x = 1.0 + 0.1 * x
        elif kind == "b":
            x = 0.02 * x
        out[name] = gen.bf16(x)
    return out


@pytest.fixture(autouse=True)
def decode_step_prefill(monkeypatch):
    """These tests compare with the oracle's decode-step prefill (the bf16
    prefill has its own tests in test_prefill_gpu.py)."""
    monkeypatch.setenv("QWEN3_TTS_PREFILL", "decode")


@pytest.fixture(scope="module")
def full(hip, orc):
    print("\n[geometry] generating VoiceDesign-geometry weights", flush=True)
    weights = make_weights(VOICEDESIGN, seed=5)
    print("[geometry] uploading + finalizing on the device", flush=True)
    model, _ = toy_model.upload(hip, VOICEDESIGN, weights)
    print("[geometry] quantizing for the oracle", flush=True)
    orc.set_threads(min(16, os.cpu_count() or 1))
    om = toy_model.OracleModel(orc, VOICEDESIGN, weights)
    yield model, om
    orc.set_threads(1)
    hip.load().qwen3_tts_model_destroy(model)


def prompt(seed):
    rng = np.random.default_rng(seed)
    text = rng.integers(0, VOICEDESIGN["text_vocabulary"], PROMPT).astype(np.int32)
    codec = rng.integers(0, 2048, PROMPT).astype(np.int32)
    text[3] = -1
    codec[0] = -1
    return text, codec


def session(hip, model, seed):
    s = C.c_void_p()
    mem = hip.SessionMemory()
    hip.call("qwen3_tts_session_create", model, 128, seed, C.byref(s), C.byref(mem))
    return s


def prefill_both(hip, om, s, seed):
    text, codec = prompt(seed)
    pre = hip.PrefillResult()
    hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
             codec.ctypes.data_as(C.POINTER(C.c_int32)), PROMPT, hip.SamplingConfig(*GREEDY), C.byref(pre))
    o = toy_model.OracleSession(om, 128, seed)
    om.model.batch_semantics = 0
    first = o.prefill(text, codec, GREEDY)
    assert pre.first_semantic_token == first
    return o, first


SCHEDULE = [(GREEDY, GREEDY), (GREEDY, GREEDY), (TALKER_TOPK, PREDICTOR_TOPK), (TALKER_TOPK, PREDICTOR_TOPK)]


def test_voicedesign_geometry_frames(hip, orc, full):
    model, om = full
    s = session(hip, model, 42)
    try:
        o, sem = prefill_both(hip, om, s, 42)
        for f, (ts, ps) in enumerate(SCHEDULE):
            if sem == VOICEDESIGN["codec_eos_token"]:
                break
            print(f"[geometry] single-session frame {f}", flush=True)
            codes = (C.c_uint16 * 16)()
            nxt = C.c_uint16()
            info = hip.CodecFrameInfo()
            hip.call("qwen3_tts_session_next_frame", s, sem, 100 + f, hip.SamplingConfig(*ts),
                     hip.SamplingConfig(*ps), codes, 16, C.byref(nxt), C.byref(info))
            ocodes, onxt = o.frame(sem, 100 + f, ts, ps)
            assert list(codes) == list(ocodes), (f, list(codes), list(ocodes))
            assert nxt.value == onxt, f
            assert info.talker_position == PROMPT + f
            sem = onxt
    finally:
        hip.load().qwen3_tts_session_destroy(s)


def test_voicedesign_geometry_batched_exact(hip, orc, full, monkeypatch):
    monkeypatch.setenv("QWEN3_TTS_BATCH_GEMV", "exact")
    model, om = full
    sessions = [session(hip, model, 50 + i) for i in range(2)]
    try:
        state = [prefill_both(hip, om, s, 50 + i) for i, s in enumerate(sessions)]
        oracles, sems = [o for o, _ in state], [t for _, t in state]
        for f, (ts, ps) in enumerate(SCHEDULE[1:3]):
            live = [i for i in range(2) if sems[i] != VOICEDESIGN["codec_eos_token"]]
            if not live:
                break
            print(f"[geometry] batched frame {f} sessions {live}", flush=True)
            n = len(live)
            arr = (C.c_void_p * n)(*[sessions[i].value for i in live])
            tr = (C.c_int32 * n)(*[7 + i for i in live])
            tsa = (hip.SamplingConfig * n)(*[hip.SamplingConfig(*ts)] * n)
            psa = (hip.SamplingConfig * n)(*[hip.SamplingConfig(*ps)] * n)
            views = (hip.DeviceFrameViewV2 * n)()
            for v in views:
                v.struct_size = C.sizeof(hip.DeviceFrameViewV2)
            hip.call("qwen3_tts_model_batch_next_frame_begin_v2", model, arr, n, tr, tsa, psa, views)
            om.model.batch_semantics = 1
            for k, i in enumerate(live):
                nxt = C.c_uint16()
                info = hip.CodecFrameInfo()
                hip.call("qwen3_tts_session_next_frame_finish_v2", sessions[i], views[k].lease_id, None,
                         C.byref(nxt), C.byref(info))
                codes = np.zeros(16, np.uint16)
                hip.call("qwen3_tts_device_memcpy", codes.ctypes.data, views[k].device_codes, 32)
                ocodes, onxt = oracles[i].frame(sems[i], 7 + i, ts, ps)
                assert np.array_equal(codes, ocodes), (f, i, codes, ocodes)
                assert nxt.value == onxt
                sems[i] = onxt
    finally:
        om.model.batch_semantics = 0
        for s in sessions:
            hip.load().qwen3_tts_session_destroy(s)


def test_voicedesign_geometry_bf16_prefill(hip, orc, full, monkeypatch):
    """The bf16 prefill at full geometry (66 rows, GEMM attention) against
    the oracle's orc_prefill_bf16.  Two valid fp32 summation orders of the
    GEMMs drift apart through 28 layers (bf16 rounding flips propagate), so
    the bar is relative to that drift: for every layer's key and value cache
    and the final hidden state, the GPU's RMS distance from the oracle (fp32
    chains in k order) is at most twice the oracle's own distance to a second
    valid order (sums accumulated in double, rounded once), plus 2^-10.  At
    layer 0 both are within 2^-6 of the largest value.  First token identical
    unless the oracle's top-2 margin is below 2^-5 of the largest logit."""
    monkeypatch.delenv("QWEN3_TTS_PREFILL", raising=False)
    model, om = full
    s = session(hip, model, 77)
    try:
        text, codec = prompt(77)
        pre = hip.PrefillResult()
        hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
                 codec.ctypes.data_as(C.POINTER(C.c_int32)), PROMPT, hip.SamplingConfig(*GREEDY), C.byref(pre))
        om.model.batch_semantics = 0
        o = toy_model.OracleSession(om, 128, 77)
        first = o.prefill_bf16(text, codec, GREEDY)
        alt = toy_model.OracleSession(om, 128, 77)
        orc.set_gemm_order(1)
        try:
            alt.prefill_bf16(text, codec, GREEDY)
        finally:
            orc.set_gemm_order(0)
        kvw = VOICEDESIGN["talker_key_value_heads"] * 128
        layers = VOICEDESIGN["talker_layers"]

        def rms_rel(x, ref):
            x, ref = gen.f32(x).astype(np.float64), gen.f32(ref).astype(np.float64)
            return np.sqrt(np.mean((x - ref) ** 2)) / np.sqrt(np.mean(ref ** 2))

        def max_rel(x, ref):
            x, ref = gen.f32(x).astype(np.float64), gen.f32(ref).astype(np.float64)
            return np.max(np.abs(x - ref)) / np.max(np.abs(ref))

        report = []
        for layer in range(layers):
            for which, name in ((0, "tk"), (1, "tv")):
                got = np.zeros((PROMPT, kvw), np.uint16)
                hip.call("qwen3_tts_session_read_talker_cache_v1", s, layer, which, PROMPT, got.ctypes.data, got.nbytes)
                ref = o.bufs[name].reshape(layers, 128, kvw)[layer, :PROMPT]
                other = alt.bufs[name].reshape(layers, 128, kvw)[layer, :PROMPT]
                e_gpu, e_alt = rms_rel(got, ref), rms_rel(other, ref)
                report.append((layer, which, e_gpu, e_alt))
                assert e_gpu <= 2 * e_alt + 2 ** -10, (layer, which, e_gpu, e_alt)
                if layer == 0:
                    assert max_rel(got, ref) <= 2 ** -6 and max_rel(other, ref) <= 2 ** -6
        h = np.zeros(VOICEDESIGN["talker_hidden"], np.uint16)
        hip.call("qwen3_tts_session_read_last_hidden_v1", s, h.ctypes.data, h.nbytes)
        e_gpu, e_alt = rms_rel(h, o.bufs["last"]), rms_rel(alt.bufs["last"], o.bufs["last"])
        assert e_gpu <= 2 * e_alt + 2 ** -10, (e_gpu, e_alt)
        print(f"[geometry] bf16 prefill RMS distance from the oracle, GPU / second order: layer 27 "
              f"{report[-1][2]:.4f} / {report[-1][3]:.4f}; last hidden {e_gpu:.4f} / {e_alt:.4f}", flush=True)
        if pre.first_semantic_token != first:
            logits = gen.f32(o.bufs["logits"][:VOICEDESIGN["talker_vocabulary"]]).astype(np.float64)
            assert logits[first] - logits[pre.first_semantic_token] <= 2 ** -5 * np.max(np.abs(logits))
    finally:
        hip.load().qwen3_tts_session_destroy(s)
