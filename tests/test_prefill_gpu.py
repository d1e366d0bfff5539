"""GPU parity of the bf16 prompt prefill (native/qwen3-tts-native/native/src/
talker.cu:2750-3249) against the oracle's restatement (oracle/oracle.c
orc_prefill_bf16, pinned against the float64 model in test_frame_f64.py).

The prefill's products are fp32-accumulated bf16 GEMMs, whose summation
order the reference leaves to cuBLAS; the MFMA kernel's order differs from
the oracle's sequential one, so GEMM outputs are checked against the
float64 product (within one bf16 ulp of its rounding) and the prefill's state
-- every layer's key and value cache rows, the final hidden state -- against
the oracle within GEMM_TOL of the tensor's largest magnitude; the first
token must agree unless the oracle's top-2 margin is below LOGIT_TOL.  The
causal softmax, which sees identical inputs, is bit-exact.  Frames after a
bf16 prefill are then bit-identical to the oracle's once the oracle starts
from the GPU's prefill state (caches and last hidden state copied over)."""
import ctypes as C

import numpy as np
import pytest

import gen
import toy_model
from toy_model import TOY

pytestmark = pytest.mark.gpu

GREEDY = (0, 0, 1.0, 1.0, 1.05)
TALKER_TOPK = (1, 50, 1.0, 0.9, 1.05)
PREDICTOR_TOPK = (1, 50, 1.0, 0.9, 1.0)
# bf16 rounding flips of the GEMM outputs propagate through the layers; the
# measured worst case on these models is below 1 % of max (see test output)
GEMM_TOL = 2 ** -5
LOGIT_TOL = 2 ** -5


def dev(hip, a):
    return hip.DeviceArray.from_numpy(a)


def gemm(hip, a, b, m, n, k, lda, ldb, ldc, c_shape, batch=1, b_group=1, a_batch=0, b_batch=0, c_batch=0):
    c = hip.DeviceArray(c_shape, np.uint16)
    c.upload(np.zeros(c_shape, np.uint16))
    hip.call("qwen3_tts_op_bf16_gemm_v1", a.ptr, b.ptr, c.ptr, m, n, k, lda, ldb, ldc, batch, b_group, a_batch,
             b_batch, c_batch, None)
    return c.numpy()


def within_bound(got_bits, a_bits, b_bits):
    """The textbook bound of an fp32-accumulated dot product, |s - s_fp32| <=
    K * 2^-24 * sum |a_k b_k|, plus the bf16 rounding of the result (half an
    ulp, one ulp of slack for the double rounding)."""
    a = gen.f32(a_bits).astype(np.float64)
    b = gen.f32(b_bits).astype(np.float64)
    ref = a @ b.T
    k = a.shape[1]
    bound = np.abs(ref) * 2.0 ** -8 + k * 2.0 ** -24 * (np.abs(a) @ np.abs(b).T)
    return np.abs(gen.f32(got_bits).astype(np.float64) - ref) <= bound


# every tile size the launcher picks: 32 (all but the last two), 64, 128
@pytest.mark.parametrize("m,n,k", [(1, 3072, 2048), (66, 2048, 2048), (130, 1024, 6144), (257, 384, 1024),
                                   (5, 100, 64), (200, 136, 8), (1000, 2048, 256), (2048, 4096, 128)])
def test_bf16_gemm_matches_float64(hip, orc, m, n, k):
    rng = np.random.default_rng(m * 7 + n + k)
    a = gen.activations(rng, m, k)
    b = gen.bf16(0.05 * rng.standard_normal((n, k)).astype(np.float32))
    got = gemm(hip, dev(hip, a), dev(hip, b), m, n, k, k, k, n, (m, n))
    assert within_bound(got, a, b).all()
    # and against the oracle's fp32 order: identical except at rounding steps
    oracle = orc.bf16_gemm(a, b)
    assert np.mean(got != oracle) < 0.02


def test_bf16_gemm_batched_gqa_strides(hip, orc):
    """The prefill's score GEMM: per query head h, q_h (columns h*128.. of a
    fused row) times the keys of kv head h // 2, scores [h][rows][stride]."""
    rng = np.random.default_rng(5)
    rows, qh, kvh, d = 70, 4, 2, 128
    width = (qh + 2 * kvh) * d
    qkv = gen.activations(rng, rows, width)
    stride = 72
    got = gemm(hip, dev(hip, qkv), dev(hip, qkv[:, qh * d:].copy()), rows, rows, d, width, width - qh * d, stride,
               (qh, rows, stride), batch=qh, b_group=qh // kvh, a_batch=d, b_batch=d, c_batch=rows * stride)
    for h in range(qh):
        q = qkv[:, h * d:(h + 1) * d]
        k = qkv[:, qh * d + (h // 2) * d: qh * d + (h // 2 + 1) * d]
        assert within_bound(got[h, :, :rows], q, k).all(), h
        assert not got[h, :, rows:].any()  # columns past n untouched


def gemm_split(hip, a, b, m, n, k, tile, k_step, splits, workspace_floats=4 << 20, batch=1, b_group=1, a_batch=0,
               b_batch=0, c_batch=0, lda=None, ldb=None, ldc=None, c_shape=None, epilogue=0, c_init=None):
    c_shape = c_shape or (m, n)
    c = hip.DeviceArray(c_shape, np.uint16)
    c.upload(np.zeros(c_shape, np.uint16) if c_init is None else c_init)
    part = hip.DeviceArray(max(workspace_floats, 1), np.float32)
    hip.call("qwen3_tts_op_bf16_gemm_split_v1", a.ptr, b.ptr, c.ptr, m, n, k, lda or k, ldb or k, ldc or n, batch,
             b_group, a_batch, b_batch, c_batch, part.ptr, workspace_floats, tile, k_step, splits, epilogue, None)
    return c.numpy()


# short prompts (K split into slices added by a second launch), K not a
# multiple of the step, columns not a multiple of the tile, and the planned form
@pytest.mark.parametrize("m,n,k,tile,k_step,splits", [
    (16, 1024, 2048, 32, 256, 4), (32, 2048, 6144, 32, 256, 8), (96, 2048, 6144, 32, 128, 3),
    (5, 100, 1000, 32, 64, 5), (192, 2048, 6144, 64, 128, 4), (130, 200, 3000, 64, 64, 7),
    (40, 300, 4096, 128, 64, 16), (16, 1024, 2048, 0, 0, 0), (96, 3072, 2048, 0, 0, 0),
    (801, 1024, 6144, 0, 0, 0)])
def test_bf16_gemm_split_matches_float64(hip, orc, m, n, k, tile, k_step, splits):
    rng = np.random.default_rng(m + n + k + splits)
    a = gen.activations(rng, m, k)
    b = gen.bf16(0.05 * rng.standard_normal((n, k)).astype(np.float32))
    da, db = dev(hip, a), dev(hip, b)
    got = gemm_split(hip, da, db, m, n, k, tile, k_step, splits)
    assert within_bound(got, a, b).all()
    # no workspace: one slice, the same as the workspace-free entry point
    plain = gemm(hip, da, db, m, n, k, k, k, n, (m, n))
    if tile:
        one = gemm_split(hip, da, db, m, n, k, tile, k_step, splits, workspace_floats=0)
        assert within_bound(one, a, b).all()
    assert within_bound(plain, a, b).all()


def test_bf16_gemm_k_step_keeps_summation_order(hip, orc):
    """Without a split the MFMA chain runs over K in the same 32-element
    chunks whatever the pipeline step, so every K step gives identical bits."""
    rng = np.random.default_rng(12)
    m, n, k = 70, 160, 2056
    a = gen.activations(rng, m, k)
    b = gen.bf16(0.05 * rng.standard_normal((n, k)).astype(np.float32))
    da, db = dev(hip, a), dev(hip, b)
    for tile, steps in ((32, (64, 128, 256)), (64, (64, 128))):
        outs = [gemm_split(hip, da, db, m, n, k, tile, s, 1) for s in steps]
        for o in outs[1:]:
            assert np.array_equal(o, outs[0]), tile


def test_bf16_gemm_split_batched_gqa(hip, orc):
    """The value GEMM shape of a short prompt with K slices: per head h,
    probabilities [rows][k] times values^T of kv head h // 2."""
    rng = np.random.default_rng(13)
    heads, kvh, rows, k, d = 4, 2, 24, 512, 128
    p = gen.activations(rng, heads * rows, k).reshape(heads, rows, k)
    vt = gen.bf16(0.05 * rng.standard_normal((kvh, d, k)).astype(np.float32))
    got = gemm_split(hip, dev(hip, p), dev(hip, vt), rows, d, k, 32, 64, 4, batch=heads, b_group=heads // kvh,
                     a_batch=rows * k, b_batch=d * k, c_batch=rows * d, c_shape=(heads, rows, d))
    for h in range(heads):
        assert within_bound(got[h], p[h], vt[h // 2]).all(), h


@pytest.mark.parametrize("splits", [1, 4])
def test_bf16_gemm_epilogues_match_separate_ops(hip, orc, splits):
    """The fused residual add and SiLU gate equal the GEMM followed by the
    reference's add_in_place / silu_gate (oracle), bit for bit, with and
    without K slices."""
    rng = np.random.default_rng(40 + splits)
    m, n, k = 24, 320, 2048
    a = gen.activations(rng, m, k)
    b = gen.bf16(0.05 * rng.standard_normal((n, k)).astype(np.float32))
    other = gen.activations(rng, m, n)
    da, db = dev(hip, a), dev(hip, b)
    plain = gemm_split(hip, da, db, m, n, k, 32, 128, splits)
    added = gemm_split(hip, da, db, m, n, k, 32, 128, splits, epilogue=1, c_init=other)
    assert np.array_equal(added, orc.add_in_place(other.ravel(), plain.ravel()).reshape(m, n))
    gated = gemm_split(hip, da, db, m, n, k, 32, 128, splits, epilogue=2, c_init=other)
    assert np.array_equal(gated, orc.silu_gate(other.ravel(), plain.ravel()).reshape(m, n))


def test_bf16_gemm_split_rejects_bad_arguments(hip):
    a = hip.DeviceArray(64 * 64, np.uint16)
    with pytest.raises(hip.Qwen3TtsError):
        gemm_split(hip, a, a, 8, 8, 64, 48, 0, 0)  # no such tile
    with pytest.raises(hip.Qwen3TtsError):
        gemm_split(hip, a, a, 8, 8, 64, 64, 256, 0)  # no such K step for the tile
    with pytest.raises(hip.Qwen3TtsError):
        gemm_split(hip, a, a, 8, 8, 64, 0, 0, -1)
    with pytest.raises(hip.Qwen3TtsError):
        gemm_split(hip, a, a, 8, 8, 64, 0, 0, 0, epilogue=3)


@pytest.mark.parametrize("rows,stride", [(1, 8), (9, 16), (70, 72), (512, 512)])
def test_causal_softmax_bit_exact(hip, orc, rows, stride):
    rng = np.random.default_rng(rows)
    heads = 3
    scores = gen.bf16(3.0 * rng.standard_normal((heads, rows, stride)).astype(np.float32))
    d = dev(hip, scores)
    hip.call("qwen3_tts_op_causal_softmax_v1", d.ptr, heads, rows, stride, 128, None)
    assert np.array_equal(d.numpy(), orc.causal_softmax(scores, 128))


@pytest.fixture(scope="module")
def toy(hip, orc):
    weights = toy_model.make_weights(TOY, seed=8)
    model, _ = toy_model.upload(hip, TOY, weights)
    om = toy_model.OracleModel(orc, TOY, weights)
    yield model, om
    hip.load().qwen3_tts_model_destroy(model)


def prompt(rng, n):
    text = rng.integers(0, TOY["text_vocabulary"], n).astype(np.int32)
    codec = rng.integers(0, 2048, n).astype(np.int32)
    text[1] = -1
    codec[2 % n] = -1 if n > 2 else codec[2 % n]
    return text, codec


def gpu_prefill(hip, model, max_seq, text, codec, sampling, seed=7):
    s = C.c_void_p()
    mem = hip.SessionMemory()
    hip.call("qwen3_tts_session_create", model, max_seq, seed, C.byref(s), C.byref(mem))
    pre = hip.PrefillResult()
    hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
             codec.ctypes.data_as(C.POINTER(C.c_int32)), len(text), hip.SamplingConfig(*sampling), C.byref(pre))
    return s, pre


def read_cache(hip, s, layer, which, count):
    kvw = TOY["talker_key_value_heads"] * 128
    out = np.zeros((count, kvw), np.uint16)
    hip.call("qwen3_tts_session_read_talker_cache_v1", s, layer, which, count, out.ctypes.data, out.nbytes)
    return out


def close(got_bits, ref_bits, what):
    g, r = gen.f32(got_bits), gen.f32(ref_bits)
    err = np.max(np.abs(g - r)) / np.max(np.abs(r))
    assert err <= GEMM_TOL, f"{what}: off by {err:.4g} of max"
    return err


@pytest.mark.parametrize("rows,max_seq", [(6, 64), (70, 128), (530, 600)])
def test_bf16_prefill_matches_oracle(hip, orc, toy, monkeypatch, rows, max_seq):
    """GEMM attention (rows <= min(max_seq, 512)) and the exact per-row
    kernel (530 rows)."""
    monkeypatch.delenv("QWEN3_TTS_PREFILL", raising=False)
    model, om = toy
    rng = np.random.default_rng(rows)
    text, codec = prompt(rng, rows)
    s, pre = gpu_prefill(hip, model, max_seq, text, codec, GREEDY)
    lib = hip.load()
    try:
        o = toy_model.OracleSession(om, max_seq, 7)
        orc.set_threads(8)
        first = o.prefill_bf16(text, codec, GREEDY)
        orc.set_threads(1)
        kvw = TOY["talker_key_value_heads"] * 128
        worst = 0.0
        for layer in range(TOY["talker_layers"]):
            for which, name in ((0, "tk"), (1, "tv")):
                ref = o.bufs[name].reshape(TOY["talker_layers"], max_seq, kvw)[layer, :rows]
                worst = max(worst, close(read_cache(hip, s, layer, which, rows), ref, f"layer {layer} cache {which}"))
        h = np.zeros(TOY["talker_hidden"], np.uint16)
        hip.call("qwen3_tts_session_read_last_hidden_v1", s, h.ctypes.data, h.nbytes)
        worst = max(worst, close(h, o.bufs["last"], "last hidden"))
        if pre.first_semantic_token != first:
            logits = gen.f32(o.bufs["logits"][:TOY["talker_vocabulary"]]).astype(np.float64)
            margin = logits[first] - logits[pre.first_semantic_token]
            assert margin <= LOGIT_TOL * np.max(np.abs(logits)), (first, pre.first_semantic_token, margin)
        print(f"rows {rows}: worst cache / hidden error {worst:.3g} of max")
        st = hip.TalkerStateInfo()
        hip.call("qwen3_tts_session_state_info", s, C.byref(st))
        assert st.talker_position == rows and st.semantic_history_count == 1
    finally:
        lib.qwen3_tts_session_destroy(s)


def test_frames_after_bf16_prefill(hip, orc, toy, monkeypatch):
    """After a bf16 prefill the decode frames run on the int8 path: with the
    oracle started from the GPU's prefill state, greedy and top-k frames are
    identical."""
    monkeypatch.delenv("QWEN3_TTS_PREFILL", raising=False)
    model, om = toy
    rows, max_seq = 20, 64
    rng = np.random.default_rng(3)
    text, codec = prompt(rng, rows)
    s, pre = gpu_prefill(hip, model, max_seq, text, codec, GREEDY, seed=11)
    lib = hip.load()
    try:
        o = toy_model.OracleSession(om, max_seq, 11)
        kvw = TOY["talker_key_value_heads"] * 128
        tk = o.bufs["tk"].reshape(TOY["talker_layers"], max_seq, kvw)
        tv = o.bufs["tv"].reshape(TOY["talker_layers"], max_seq, kvw)
        for layer in range(TOY["talker_layers"]):
            tk[layer, :rows] = read_cache(hip, s, layer, 0, rows)
            tv[layer, :rows] = read_cache(hip, s, layer, 1, rows)
        hip.call("qwen3_tts_session_read_last_hidden_v1", s, o.bufs["last"].ctypes.data, o.bufs["last"].nbytes)
        o.s.position = rows
        o.bufs["history"][0] = pre.first_semantic_token
        o.s.history_count = 1
        sem = pre.first_semantic_token
        for f, (ts, ps) in enumerate([(GREEDY, GREEDY), (TALKER_TOPK, PREDICTOR_TOPK), (TALKER_TOPK, PREDICTOR_TOPK)]):
            if sem == TOY["codec_eos_token"]:
                break
            codes = (C.c_uint16 * 16)()
            nxt = C.c_uint16()
            info = hip.CodecFrameInfo()
            hip.call("qwen3_tts_session_next_frame", s, sem, 5 + f, hip.SamplingConfig(*ts), hip.SamplingConfig(*ps),
                     codes, 16, C.byref(nxt), C.byref(info))
            ocodes, onxt = o.frame(sem, 5 + f, ts, ps)
            assert list(codes) == list(ocodes), f
            assert nxt.value == onxt
            sem = onxt
    finally:
        lib.qwen3_tts_session_destroy(s)
