"""GPU parity of the decode-step primitives against the CPU oracle
(native/qwen3-tts-native/native/src/talker_kernels.cu and sampling_kernels.cu
as restated in oracle/oracle.c).  Integer/byte work and every kernel that
reproduces the reference's operation order are compared bit-for-bit."""
import ctypes as C

import numpy as np
import pytest

import gen

pytestmark = pytest.mark.gpu


# Device arrays must outlive the kernels that use them: a DeviceArray frees
# its memory when garbage-collected, so every upload is kept alive here until
# the test ends (passing `.ptr` of a temporary would hand the kernel freed
# memory).
_KEEP = []


@pytest.fixture(autouse=True)
def _release_device_arrays():
    yield
    _KEEP.clear()


def dev(hip, a):
    d = hip.DeviceArray.from_numpy(a)
    _KEEP.append(d)
    return d


def ptr_array(hip, pointers):
    return dev(hip, np.array(pointers, dtype=np.uint64))


@pytest.mark.parametrize("rows,width", [(1, 2048), (3, 1024), (1, 128), (2, 300), (2, 6144), (1, 8192), (1, 8200)])
def test_rms_norm_rows(hip, orc, rows, width):
    rng = np.random.default_rng(width + rows)
    x, g = gen.activations(rng, rows, width), gen.gains(rng, width)
    out = hip.DeviceArray((rows, width), np.uint16)
    hip.call("qwen3_tts_op_rms_norm_rows", dev(hip, x).ptr, dev(hip, g).ptr, out.ptr, rows, width,
             C.c_float(1e-6), None)
    assert np.array_equal(out.numpy(), orc.rms_norm_rows(x, g))


def test_head_rms_norm(hip, orc):
    rng = np.random.default_rng(2)
    v, g = gen.activations(rng, 2 * 16 * 128), gen.gains(rng, 128)
    d = dev(hip, v)
    hip.call("qwen3_tts_op_head_rms_norm_rows", d.ptr, dev(hip, g).ptr, 2, 16, 128, C.c_float(1e-6), None)
    assert np.array_equal(d.numpy(), orc.head_rms_norm_rows(v, g, 16, 128))


def test_rope_in_kernel_math_close(hip, orc):
    """The reference-formula RoPE op (powf/cosf/sinf on the device) agrees
    with the host libm restatement within bf16 resolution."""
    rng = np.random.default_rng(4)
    v = gen.activations(rng, 3 * 8 * 128)
    pos = np.array([0, 37, 1023], np.int32)
    d = dev(hip, v)
    hip.call("qwen3_tts_op_rope_rows", d.ptr, 3, 8, 128, dev(hip, pos).ptr, C.c_float(1e6), None)
    ref = gen.f32(orc.rope_rows(v, 8, 128, pos))
    got = gen.f32(d.numpy())
    assert np.max(np.abs(got - ref)) <= 0.016
    assert np.mean(got == ref) > 0.98


@pytest.mark.parametrize("position", [0, 5, 1023])
def test_qk_norm_rope_kv_append(hip, orc, position):
    rng = np.random.default_rng(position + 1)
    qh, kvh, d = 16, 8, 128
    qw, kw = qh * d, kvh * d
    qkv = gen.activations(rng, qw + 2 * kw)
    qn, kn = gen.gains(rng, d), gen.gains(rng, d)
    max_seq = 1024
    table = np.empty(max_seq * d, np.uint16)
    hip.call("qwen3_tts_rope_table_v1", max_seq, d, C.c_float(1e6), table.ctypes.data)
    kc = hip.DeviceArray((max_seq, kw), np.uint16)
    vc = hip.DeviceArray((max_seq, kw), np.uint16)
    kc.upload(np.zeros((max_seq, kw), np.uint16))
    vc.upload(np.zeros((max_seq, kw), np.uint16))
    dq = dev(hip, qkv)
    hip.call("qwen3_tts_op_qk_norm_rope_kv_append", dq.ptr, dev(hip, qn).ptr, dev(hip, kn).ptr,
             ptr_array(hip, [kc.ptr]).ptr, ptr_array(hip, [vc.ptr]).ptr,
             dev(hip, np.array([position], np.int32)).ptr, dev(hip, table).ptr, 1, qh, kvh, d,
             C.c_float(1e-6), None)
    q_ref = orc.rope_rows(orc.head_rms_norm_rows(qkv[:qw], qn, qh, d), qh, d, [position])
    k_ref = orc.rope_rows(orc.head_rms_norm_rows(qkv[qw:qw + kw], kn, kvh, d), kvh, d, [position])
    got = dq.numpy()
    assert np.array_equal(got[:qw], q_ref)
    assert np.array_equal(kc.numpy()[position], k_ref)
    assert np.array_equal(vc.numpy()[position], qkv[qw + kw:])
    untouched = np.delete(np.arange(max_seq), position)
    assert not kc.numpy()[untouched].any() and not vc.numpy()[untouched].any()


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("length", [1, 7, 300, 1024])
def test_attention(hip, orc, exact, length):
    rng = np.random.default_rng(length * 2 + exact)
    qh, kvh, d, max_seq = 16, 8, 128, 1024
    q = gen.activations(rng, qh * d)
    k = gen.bf16(rng.standard_normal((max_seq, kvh * d)).astype(np.float32) * 0.5)
    v = gen.activations(rng, max_seq, kvh * d)
    dk, dv = dev(hip, k), dev(hip, v)
    out = hip.DeviceArray(qh * d, np.uint16)
    pos = dev(hip, np.array([length - 1], np.int32))
    hip.call("qwen3_tts_op_attention", exact, dev(hip, q).ptr, qh * d, ptr_array(hip, [dk.ptr]).ptr,
             ptr_array(hip, [dv.ptr]).ptr, pos.ptr, out.ptr, 1, qh, kvh, d, max_seq, None)
    ref = orc.attention(q, k[:length], v[:length], qh, kvh, d, length, exact=bool(exact))
    assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("qh,kvh", [(16, 8), (8, 8), (16, 4)])
@pytest.mark.parametrize("length,max_seq", [(15, 16), (16, 16), (64, 64), (65, 65), (17, 1001), (513, 1001), (1001, 1001), (4096, 4099)])
def test_attention_groups_and_ring_edges(hip, orc, exact, qh, kvh, length, max_seq):
    """GQA group sizes 1/2/4, lengths around the value-ring and chunk edges,
    cache capacities that are not multiples of four."""
    rng = np.random.default_rng(length * 7 + qh + kvh + exact)
    d = 128
    q = gen.activations(rng, qh * d)
    k = gen.bf16(rng.standard_normal((max_seq, kvh * d)).astype(np.float32) * 0.5)
    v = gen.activations(rng, max_seq, kvh * d)
    dk, dv = dev(hip, k), dev(hip, v)
    out = hip.DeviceArray(qh * d, np.uint16)
    pos = dev(hip, np.array([length - 1], np.int32))
    hip.call("qwen3_tts_op_attention", exact, dev(hip, q).ptr, qh * d, ptr_array(hip, [dk.ptr]).ptr,
             ptr_array(hip, [dv.ptr]).ptr, pos.ptr, out.ptr, 1, qh, kvh, d, max_seq, None)
    ref = orc.attention(q, k[:length], v[:length], qh, kvh, d, length, exact=bool(exact))
    assert np.array_equal(out.numpy(), ref)


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("qh,kvh", [(16, 8), (16, 4)])
@pytest.mark.parametrize("positions,max_seq", [([0], 16), ([1], 16), ([7], 16), ([15], 16), ([5], 8),
                                               ([0, 9, 15], 16), ([63], 64), ([64], 100), ([700], 1024),
                                               ([1023], 1024), ([3, 40, 99], 100)])
def test_decode_attention_fused_matches_separate_ops(hip, orc, exact, qh, kvh, positions, max_seq):
    """The fused decode step (head norm + RoPE + KV append + attention) equals
    qk_norm_rope_kv_append followed by attention: same output, same caches."""
    rng = np.random.default_rng(sum(positions) * 3 + max_seq + qh // kvh + exact)
    d = 128
    qw, kw = qh * d, kvh * d
    rows = len(positions)
    qkv = gen.activations(rng, rows, qw + 2 * kw)
    qn, kn = gen.gains(rng, d), gen.gains(rng, d)
    table = np.empty(max_seq * d, np.uint16)
    hip.call("qwen3_tts_rope_table_v1", max_seq, d, C.c_float(1e6), table.ctypes.data)
    dtable = dev(hip, table)
    caches = [(gen.activations(rng, max_seq, kw), gen.activations(rng, max_seq, kw)) for _ in range(rows)]
    pos = dev(hip, np.array(positions, np.int32))

    def run(fused):
        kcs = [dev(hip, k.copy()) for k, _ in caches]
        vcs = [dev(hip, v.copy()) for _, v in caches]
        kb, vb = ptr_array(hip, [c.ptr for c in kcs]), ptr_array(hip, [c.ptr for c in vcs])
        dq = dev(hip, qkv.copy())
        out = hip.DeviceArray((rows, qw), np.uint16)
        if fused:
            hip.call("qwen3_tts_op_decode_attention", exact, dq.ptr, qw + 2 * kw, dev(hip, qn).ptr, dev(hip, kn).ptr,
                     dtable.ptr, C.c_float(1e-6), kb.ptr, vb.ptr, pos.ptr, out.ptr, rows, qh, kvh, d, max_seq, None)
        else:
            hip.call("qwen3_tts_op_qk_norm_rope_kv_append", dq.ptr, dev(hip, qn).ptr, dev(hip, kn).ptr, kb.ptr,
                     vb.ptr, pos.ptr, dtable.ptr, rows, qh, kvh, d, C.c_float(1e-6), None)
            hip.call("qwen3_tts_op_attention", exact, dq.ptr, qw + 2 * kw, kb.ptr, vb.ptr, pos.ptr, out.ptr, rows,
                     qh, kvh, d, max_seq, None)
        return out.numpy(), [c.numpy() for c in kcs], [c.numpy() for c in vcs], dq.numpy()

    out_f, k_f, v_f, _ = run(True)
    out_s, k_s, v_s, q_s = run(False)
    assert np.array_equal(out_f, out_s)
    for r in range(rows):
        assert np.array_equal(k_f[r], k_s[r]) and np.array_equal(v_f[r], v_s[r])
        n = positions[r] + 1
        ref = orc.attention(q_s[r][:qw], k_s[r][:n], v_s[r][:n], qh, kvh, d, n, exact=bool(exact))
        assert np.array_equal(out_f[r], ref)


@pytest.mark.parametrize("exact", [1, 0])
@pytest.mark.parametrize("qh,kvh", [(16, 8), (8, 8), (16, 4)])
@pytest.mark.parametrize("first,rows,capacity", [(0, 40, 64), (500, 24, 600), (0, 17, 17), (700, 101, 801)])
def test_prompt_attention_shared_cache(hip, orc, exact, qh, kvh, first, rows, capacity):
    """The prefill's exact attention for long prompts: consecutive prompt rows
    against one complete cache (row r attends to positions 0..first + r), in
    tiles of rows that share each key row; every row's output equals the
    oracle's causal_gqa_attention of its prefix."""
    rng = np.random.default_rng(first + rows + qh + kvh + exact)
    d = 128
    q = gen.activations(rng, rows, qh * d)
    k = gen.bf16(rng.standard_normal((capacity, kvh * d)).astype(np.float32) * 0.5)
    v = gen.activations(rng, capacity, kvh * d)
    pos = np.arange(first, first + rows, dtype=np.int32)
    out = hip.DeviceArray((rows, qh * d), np.uint16)
    hip.call("qwen3_tts_op_prompt_attention_v1", exact, dev(hip, q).ptr, qh * d, dev(hip, k).ptr, dev(hip, v).ptr,
             dev(hip, pos).ptr, out.ptr, rows, qh, kvh, d, capacity, None)
    got = out.numpy()
    for r in range(rows):
        n = first + r + 1
        ref = orc.attention(q[r], k[:n], v[:n], qh, kvh, d, n, exact=bool(exact))
        assert np.array_equal(got[r], ref), r


def test_attention_rows_with_own_caches(hip, orc):
    rng = np.random.default_rng(9)
    qh, kvh, d, max_seq, rows = 16, 8, 128, 64, 3
    lengths = [1, 17, 64]
    q = gen.activations(rng, rows, qh * d)
    ks = [gen.activations(rng, max_seq, kvh * d) for _ in range(rows)]
    vs = [gen.activations(rng, max_seq, kvh * d) for _ in range(rows)]
    dks, dvs = [dev(hip, k) for k in ks], [dev(hip, v) for v in vs]
    out = hip.DeviceArray((rows, qh * d), np.uint16)
    pos = dev(hip, np.array([n - 1 for n in lengths], np.int32))
    hip.call("qwen3_tts_op_attention", 0, dev(hip, q).ptr, qh * d, ptr_array(hip, [a.ptr for a in dks]).ptr,
             ptr_array(hip, [a.ptr for a in dvs]).ptr, pos.ptr, out.ptr, rows, qh, kvh, d, max_seq, None)
    got = out.numpy()
    for r in range(rows):
        n = lengths[r]
        assert np.array_equal(got[r], orc.attention(q[r], ks[r][:n], vs[r][:n], qh, kvh, d, n, exact=False))


def test_kv_scatter_rows(hip):
    rng = np.random.default_rng(1)
    rows, width = 3, 1024
    data = gen.activations(rng, rows, 4096)
    caches = [hip.DeviceArray((32, width), np.uint16) for _ in range(rows)]
    for c in caches:
        c.upload(np.zeros((32, width), np.uint16))
    pos = np.array([0, 9, 31], np.int32)
    hip.call("qwen3_tts_op_kv_scatter_rows", dev(hip, data).ptr, ptr_array(hip, [c.ptr for c in caches]).ptr,
             dev(hip, pos).ptr, rows, width, 4096, None)
    for r in range(rows):
        got = caches[r].numpy()
        assert np.array_equal(got[pos[r]], data[r, :width])
        assert np.count_nonzero(got) == np.count_nonzero(data[r, :width])


@pytest.mark.parametrize("op", [0, 1, 2, 3])
def test_elementwise(hip, orc, op):
    rng = np.random.default_rng(op)
    rows, width = 2, 777
    a = gen.activations(rng, rows, width)
    b = gen.activations(rng, width if op in (1, 2) else rows * width)
    d = dev(hip, a)
    hip.call("qwen3_tts_op_elementwise", op, d.ptr, dev(hip, b).ptr, rows, width, None)
    if op == 0:
        ref = orc.add_in_place(a.ravel(), b).reshape(rows, width)
    elif op in (1, 2):
        ref = orc.bias_activation(a, b, op == 2)
    else:
        ref = orc.silu_gate(a.ravel(), b).reshape(rows, width)
    assert np.array_equal(d.numpy(), ref)


def test_sum_embeddings(hip, orc):
    rng = np.random.default_rng(6)
    width, v0, v = 512, 300, 200
    tables = [gen.activations(rng, v0 if i == 0 else v, width) for i in range(16)]
    toks = np.concatenate([[250], rng.integers(0, v, 15)]).astype(np.int32)
    dts = [dev(hip, t) for t in tables]
    out = hip.DeviceArray(width, np.uint16)
    hip.call("qwen3_tts_op_sum_embeddings", ptr_array(hip, [t.ptr for t in dts]).ptr, 16, v0, v, width,
             dev(hip, toks).ptr, out.ptr, None)
    ref = tables[0][250].copy()
    for i in range(1, 16):
        ref = orc.add_in_place(ref, tables[i][toks[i]])
    assert np.array_equal(out.numpy(), ref)


def sample_gpu(hip, logits, suppress, history, cfg, state):
    d_state = dev(hip, np.array([state], np.uint64))
    tok = hip.DeviceArray(1, np.int32)
    hist = dev(hip, np.array(history if history else [0], np.int32))
    cnt = dev(hip, np.array([len(history)], np.int32))
    hip.call("qwen3_tts_op_sample_logits", dev(hip, logits).ptr, len(logits), int(suppress), 2150, hist.ptr,
             cnt.ptr, cfg, d_state.ptr, tok.ptr, None)
    return int(tok.numpy()[0]), int(d_state.numpy()[0])


@pytest.mark.parametrize("vocab", [2048, 3072])
def test_sampler_greedy_matches_oracle(hip, orc, vocab):
    rng = np.random.default_rng(vocab)
    for trial in range(6):
        logits = gen.bf16(rng.standard_normal(vocab).astype(np.float32) * 2)
        if trial == 1:  # many ties
            logits = gen.bf16(np.round(rng.standard_normal(vocab)).astype(np.float32))
        history = list(rng.integers(0, 2048, 40)) if trial % 2 else []
        for suppress in (False, True):
            cfg = hip.sampling(0, 0, 1.0, 1.0, 1.05)
            got, _ = sample_gpu(hip, logits, suppress, history, cfg, 5)
            ref, _ = orc.sample_logits(logits, suppress, 2150, history, 0, 0, 1.0, 1.0, 1.05, 5)
            assert got == ref


@pytest.mark.parametrize("top_k,top_p", [(50, 1.0), (50, 0.8), (1, 1.0), (0, 1.0), (0, 0.9), (700, 1.0), (64, 1.0)])
@pytest.mark.parametrize("vocab,suppress,penalty", [(3072, True, 1.05), (2048, False, 1.0)])
def test_sampler_topk_matches_oracle(hip, orc, top_k, top_p, vocab, suppress, penalty):
    """Same logits, same RNG state -> same token and same next state, for the
    talker's masked, penalized vocabulary and the predictor's plain one;
    every fourth trial has heavily tied logits.  (The draw compares double
    sums; exp in double on the device vs the host may differ in the last
    ulp, which only matters at an exact boundary.)"""
    rng = np.random.default_rng(top_k * 10 + int(top_p * 10) + vocab)
    state = 0x1234567
    for trial in range(12):
        raw = rng.standard_normal(vocab).astype(np.float32) * 3
        if trial % 4 == 3:
            raw = np.round(raw)
        logits = gen.bf16(raw)
        history = list(rng.integers(0, 2048, 30))
        cfg = hip.sampling(1, top_k, top_p, 0.9, penalty)
        got, gstate = sample_gpu(hip, logits, suppress, history, cfg, state)
        ref, rstate = orc.sample_logits(logits, suppress, 2150, history, 1, top_k, top_p, 0.9, penalty, state)
        assert (got, gstate) == (ref, rstate), trial
        state = rstate


@pytest.mark.parametrize("top_p", [1.0, 0.999999])
def test_sampler_topk_wide_spread_matches_oracle(hip, orc, top_p):
    """Top-k 50 whose logits span ~75 units: the smallest kept weight is
    below 1e-12 of their sum, so with top_p >= 1 the sampler cannot skip the
    running-share pass (its shortcut needs a larger smallest weight) and
    forms the shares in order; the token and the next RNG state equal the
    oracle's."""
    rng = np.random.default_rng(77)
    state = 0x2468ACE
    for trial in range(8):
        raw = rng.standard_normal(2048).astype(np.float32) - 40.0
        top = rng.choice(2048, 50, replace=False)
        raw[top] = np.linspace(30.0, -45.0, 50, dtype=np.float32) + rng.standard_normal(50).astype(np.float32) * 0.1
        logits = gen.bf16(raw)
        cfg = hip.sampling(1, 50, top_p, 0.9, 1.0)
        got, gstate = sample_gpu(hip, logits, False, [], cfg, state)
        ref, rstate = orc.sample_logits(logits, False, 2150, [], 1, 50, top_p, 0.9, 1.0, state)
        assert (got, gstate) == (ref, rstate), trial
        state = rstate


@pytest.mark.parametrize("pattern", ["all_nan", "half_nan", "nan_and_inf"])
def test_sampler_nan_logits_select_in_range(hip, pattern):
    """Logits with NaNs (a diverged model) still yield a token inside the
    vocabulary, the same one on a repeat, under every selection path: greedy,
    the direct draw, top-k (the early-stopping radix select) and top-p over
    the whole vocabulary (the all-keys rank count)."""
    vocab = 2048
    raw = np.random.default_rng(3).standard_normal(vocab).astype(np.float32)
    if pattern == "all_nan":
        raw[:] = np.nan
    elif pattern == "half_nan":
        raw[::2] = np.nan
    else:
        raw[::3] = np.nan
        raw[1::7] = np.inf
        raw[2::11] = -np.inf
    logits = gen.bf16(raw)
    for cfg in (hip.sampling(0, 0, 1.0, 1.0, 1.0), hip.sampling(1, 0, 1.0, 0.9, 1.0),
                hip.sampling(1, 50, 1.0, 0.9, 1.0), hip.sampling(1, 0, 0.9, 0.9, 1.0),
                hip.sampling(1, 700, 0.95, 0.9, 1.0)):
        first, _ = sample_gpu(hip, logits, False, [], cfg, 77)
        again, _ = sample_gpu(hip, logits, False, [], cfg, 77)
        assert 0 <= first < vocab and first == again


def test_argmax_benchmark_known_answer(hip):
    for vocab in (2048, 3072):
        out = hip.ArgmaxBenchmark()
        hip.call("qwen3_tts_benchmark_bf16_argmax", 0, vocab, 100, C.byref(out))
        assert out.selected_token == out.expected_token == 1729


def test_validate_transformer_primitives(hip):
    out = hip.PrimitiveParity()
    hip.call("qwen3_tts_validate_transformer_primitives", 0, C.byref(out))
    for f, _ in hip.PrimitiveParity._fields_:
        assert getattr(out, f) <= 0.016


def test_probe_and_bf16_gemv_benchmark(hip):
    info = hip.DeviceInfo()
    hip.call("qwen3_tts_probe_device", 0, C.byref(info))
    assert b"gfx950" in info.device_name
    assert info.total_global_memory_bytes > 200 << 30
    out = hip.GemvBenchmark()
    hip.call("qwen3_tts_benchmark_bf16_gemv", 0, 2048, 2048, 50, C.byref(out))
    assert out.mean_launch_microseconds > 0


def test_device_buffer_sequential_upload(hip):
    lib = hip.load()
    buf = C.c_void_p()
    m = hip.WeightUploadMetrics()
    hip.call("qwen3_tts_device_buffer_create", 0, 1 << 20, 1 << 16, C.byref(buf), C.byref(m))
    try:
        data = np.arange(1 << 20, dtype=np.uint8) * 7
        hip.call("qwen3_tts_device_buffer_upload", buf, 0, data.ctypes.data, 1 << 19)
        with pytest.raises(hip.Qwen3TtsError):  # not contiguous
            hip.call("qwen3_tts_device_buffer_upload", buf, 0, data.ctypes.data, 16)
        with pytest.raises(hip.Qwen3TtsError):  # not complete
            hip.call("qwen3_tts_device_buffer_finish", buf, C.byref(m))
        hip.call("qwen3_tts_device_buffer_upload", buf, 1 << 19, data[1 << 19:].ctypes.data, 1 << 19)
        hip.call("qwen3_tts_device_buffer_finish", buf, C.byref(m))
        assert m.uploaded_bytes == 1 << 20 and m.upload_calls == 16
        back = np.empty(1 << 20, np.uint8)
        hip.call("qwen3_tts_device_buffer_read", buf, 0, back.ctypes.data, 1 << 20)
        assert np.array_equal(back, data)
        assert lib.qwen3_tts_device_buffer_data(buf)
    finally:
        lib.qwen3_tts_device_buffer_destroy(buf)



def test_sampler_topk_draw_closed_form(hip):
    """The device sampler on the closed-form top-k case of the oracle tests:
    draws just below and just above every cumulative boundary pick the
    candidate the descending cumulative order gives (sampling_kernels.cu:374-386)."""
    from test_oracle import TOPK_CASE_TOKENS, _uniform, states_around, topk_case_boundaries, topk_case_logits

    logits = topk_case_logits()
    cfg = hip.sampling(1, 4, 1.0, 1.0, 1.0)
    for (i, side), seeds in states_around(topk_case_boundaries()).items():
        for st in seeds:
            _, nxt = _uniform(st)
            assert sample_gpu(hip, logits, False, [], cfg, st) == (TOPK_CASE_TOKENS[i + side], nxt), (i, side)
