"""GPU parity of the speech-tokenizer decoder library against the CPU oracle.

Everything goes through the C ABI (qwen3_tts_codec_hip).  The decoder is fp32
with reordered sums (MFMA GEMMs, block reductions) and the device's sin / exp /
erf, so the bar is comparative: at every stage the GPU's distance to the
float64 whole-utterance model must stay within 4x the oracle's own distance to
it (the fp32 rounding gap), plus 1e-7 of the stage's magnitude; PCM must agree
with the oracle within one LSB on every sample.  Paths that run the same
kernels (graph vs eager, device handoff vs host codes, batch vs one session)
must be bit-identical.
"""
import ctypes as C
import os

import numpy as np
import pytest

import codec_model as M
import oracle as O

pytestmark = pytest.mark.gpu

PACKETS = ((0, 4), (4, 5), (5, 8))
STAGES = ["rvq", "preconv", "transformer", "latent1", "latent2", 6, 7, 8, 9, 10, 11, 12, 13]


@pytest.fixture(scope="module")
def codec():
    import qwen3_tts_codec_hip

    qwen3_tts_codec_hip.load()
    return qwen3_tts_codec_hip


@pytest.fixture(scope="module")
def weights():
    return M.make_weights(0)


@pytest.fixture(scope="module")
def codes():
    return M.random_codes(8, 1)


@pytest.fixture(scope="module")
def model(codec, weights):
    return codec.SharedModel(weights)


@pytest.fixture(scope="module")
def oracle_stream(weights, codes):
    O.set_threads(16)
    orc = O.CodecOracle(weights)
    outs = [orc.packet(codes[a:b]) for a, b in PACKETS]
    return {k: np.concatenate([o[k] for o in outs]) for k in outs[0]}


@pytest.fixture(scope="module")
def whole(weights, codes):
    return M.F64Decoder(weights).run(codes)


def _err(got, ref):
    return float(np.abs(np.asarray(got, np.float64) - ref).max())


def _within(gpu, orc, ref, stage):
    e_gpu, e_orc = _err(gpu, ref), _err(orc, ref)
    bar = 4 * e_orc + 1e-7 * float(np.abs(ref).max())
    assert e_gpu <= bar, f"stage {stage}: GPU error {e_gpu:.3g} vs oracle {e_orc:.3g} (bar {bar:.3g})"
    return e_gpu, e_orc


def test_model_info(model):
    info = model.info
    assert info.loaded == 1 and info.tensor_count == 271
    assert info.parameter_count == 114_323_137
    assert info.device_bytes == 4 * 114_323_137
    assert info.source_dtype_f32_count == 271
    mem = model.memory_info()
    assert mem.warmup_completed == 1 and mem.active_session_count == 0


def test_stream_pcm_matches_oracle(model, codes, oracle_stream):
    print("codec stream 4/1/3 frames", flush=True)
    s = model.session()
    pcm = []
    for i, (a, b) in enumerate(PACKETS):
        out, res = s.packet(codes[a:b], is_final=i == len(PACKETS) - 1)
        assert res.frame_count == b - a and res.sample_count == (b - a) * 1920
        assert res.first_frame_position == a and res.first_sample_position == a * 1920
        assert res.ring_slot == i % 3
        pcm.append(out)
    pcm = np.concatenate(pcm).astype(np.int32)
    diff = np.abs(pcm - oracle_stream["pcm"])
    print(f"PCM: max diff {diff.max()}, identical {(diff == 0).mean():.4f}", flush=True)
    assert diff.max() <= 1
    assert (diff == 0).mean() > 0.85
    st = s.state()
    assert st.frame_position == 8 and st.emitted_samples == 8 * 1920 and st.next_ring_slot == 0
    assert st.kv_ring_head == 8
    # finalized: the next packet needs a reset
    with pytest.raises(Exception) as e:
        s.packet(codes[:1])
    assert e.value.status == -3


def test_stage_checkpoints_match_within_fp32_gap(model, codes, oracle_stream, whole):
    """Each debug hook runs a packet prefix on a fresh session; packets 4/1/3
    of the same stream give every stage of the oracle's stream."""
    print("codec checkpoints", flush=True)
    got = {k: [] for k in STAGES}
    sessions = {}
    for key in ["front", "trans", "latent"] + list(range(6, 14)):
        sessions[key] = model.session()
    for a, b in PACKETS:
        f = b - a
        rvq, pre = sessions["front"].debug_frontend(codes[a:b])
        got["rvq"].append(rvq)
        got["preconv"].append(pre)
        got["transformer"].append(sessions["trans"].debug_transformer(codes[a:b]))
        one, two = sessions["latent"].debug_latent(codes[a:b])
        got["latent1"].append(one)
        got["latent2"].append(two)
        for c, (per_frame, ch) in O.CODEC_CHECKPOINTS.items():
            got[c].append(sessions[c].debug_checkpoint(codes[a:b], c, per_frame * f, ch))
    for k in STAGES:
        g = np.concatenate(got[k])
        e_gpu, e_orc = _within(g, oracle_stream[k], whole[k], k)
        print(f"  {k}: GPU {e_gpu:.3g}  oracle {e_orc:.3g}  max {np.abs(whole[k]).max():.3g}", flush=True)


def test_transformer_window_83_frames(model, weights):
    """Uneven packets 4/1/3/2 across the 72-position window (the shape of the
    reference's own transformer-window fixture)."""
    print("codec transformer 83 frames", flush=True)
    codes = M.random_codes(83, 7)
    packets, a, sizes = [], 0, (4, 1, 3, 2)
    while a < 83:
        b = min(83, a + sizes[len(packets) % 4])
        packets.append((a, b))
        a = b
    s = model.session()
    orc = O.CodecOracle(weights)
    gpu = np.concatenate([s.debug_transformer(codes[a:b]) for a, b in packets])
    ref = np.concatenate([orc.packet(codes[a:b], stop_after=2)["transformer"] for a, b in packets])
    exact = M.F64Decoder(weights).run_transformer(codes)
    e_gpu, e_orc = _within(gpu, ref, exact, "transformer-83")
    print(f"  GPU {e_gpu:.3g} oracle {e_orc:.3g}", flush=True)
    assert s.state().kv_ring_head == 83 % 72


def test_graph_and_eager_are_identical(codec, model, codes):
    print("codec graph vs eager", flush=True)
    graph = model.session()
    os.environ["QWEN3_TTS_CODEC_GRAPH"] = "0"
    try:
        eager = model.session()
    finally:
        del os.environ["QWEN3_TTS_CODEC_GRAPH"]
    for a, b in PACKETS + ((0, 4), (4, 8)):
        pg, _ = graph.packet(codes[a:b])
        pe, _ = eager.packet(codes[a:b])
        np.testing.assert_array_equal(pg, pe)


def test_batch_matches_single_sessions(codec, model):
    print("codec batch of 3", flush=True)
    streams = [M.random_codes(6, 20 + i) for i in range(3)]
    single = [model.session() for _ in range(3)]
    batch = [model.session() for _ in range(3)]
    for a, b in ((0, 2), (2, 6)):
        want = [single[i].packet(streams[i][a:b])[0] for i in range(3)]
        got = codec.process_batch(batch, [streams[i][a:b] for i in range(3)])
        for i in range(3):
            np.testing.assert_array_equal(got[i][0], want[i])
            assert got[i][1].first_frame_position == a


def test_batch_with_an_invalid_item_reports_which_items_completed(codec, model):
    """An invalid item in the middle ends the batch with an error; the item
    before it completes and advances its stream (nonzero result frame_count),
    the invalid one and the one after it do not (cleared results, streams
    still at frame 0), and the completed item's PCM equals a single session's.
    Reference semantics: codec_state.cu:4474-4516 processes items in order and
    returns the first failure."""
    print("codec batch with invalid middle item", flush=True)
    streams = [M.random_codes(2, 40 + i) for i in range(3)]
    sessions = [model.session() for _ in range(3)]
    codes = [np.ascontiguousarray(c, np.uint16) for c in streams]
    pcms = [np.zeros(codec.MAX_PACKET_SAMPLES, np.int16) for _ in range(3)]
    results = [codec.PacketResult() for _ in range(3)]
    for r in results:
        r.frame_count = 99  # stale values from an earlier call
    items = (codec.BatchItem * 3)()
    for i in range(3):
        capacity = 0 if i == 1 else codec.MAX_PACKET_SAMPLES  # item 1: PCM capacity too small
        items[i] = codec.BatchItem(sessions[i].handle, codes[i].ctypes.data, 2, 0, pcms[i].ctypes.data, capacity,
                                   C.pointer(results[i]))
    with pytest.raises(codec.CodecError) as e:
        codec.call("qwen3_tts_codec_session_process_batch_v1", items, 3)
    assert e.value.status == -1
    assert [r.frame_count for r in results] == [2, 0, 0]
    assert [s.state().frame_position for s in sessions] == [2, 0, 0]
    want, _ = model.session().packet(streams[0])
    np.testing.assert_array_equal(pcms[0][: results[0].sample_count], want)
    # the streams that did not consume their packet continue from frame 0
    again = codec.process_batch(sessions[1:], streams[1:])
    assert [r.first_frame_position for _, r in again] == [0, 0]


def test_reset_restores_a_fresh_stream(model, codes):
    s = model.session()
    first, _ = s.packet(codes[:4])
    s.packet(codes[4:8], is_final=True)
    s.reset()
    again, _ = s.packet(codes[:4])
    np.testing.assert_array_equal(first, again)
    s.cancel()
    with pytest.raises(Exception) as e:
        s.packet(codes[:1])
    assert e.value.status == -3


def _hip_runtime():
    """The HIP runtime the decoder library itself links (no second runtime)."""
    hip = C.CDLL("libamdhip64.so")
    hip.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
    hip.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
    hip.hipFree.argtypes = [C.c_void_p]
    hip.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipStreamDestroy.argtypes = [C.c_void_p]
    hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
    hip.hipEventDestroy.argtypes = [C.c_void_p]
    hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]
    hip.hipMemcpyAsync.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int, C.c_void_p]
    hip.hipStreamSynchronize.argtypes = [C.c_void_p]
    return hip


def test_device_packet_handoff(codec, model, codes):
    """v2 device handoff: codes in device memory behind a producer event on
    another stream, identical PCM to host codes; stale tickets are rejected."""
    print("codec device handoff", flush=True)
    hip = _hip_runtime()
    host = model.session()
    dev = model.session()
    stream, ready, buf = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreate(C.byref(stream)) == 0
    assert hip.hipEventCreate(C.byref(ready)) == 0
    assert hip.hipMalloc(C.byref(buf), 64 * 2) == 0
    try:
        for i, (a, b) in enumerate(PACKETS):
            want, _ = host.packet(codes[a:b])
            chunk = np.ascontiguousarray(codes[a:b])
            # the producer writes the codes on its own stream and signals
            assert hip.hipMemcpyAsync(buf, chunk.ctypes.data, chunk.nbytes, 1, stream) == 0
            assert hip.hipEventRecord(ready, stream) == 0
            begin = codec.DevicePacketBegin(C.sizeof(codec.DevicePacketBegin), 0, buf.value, b - a, 0,
                                            ready.value, 0)
            out = codec.DevicePacketBeginResult(C.sizeof(codec.DevicePacketBeginResult), 0, 0, None, 0)
            codec.call("qwen3_tts_codec_session_process_device_packet_begin_v2", dev.handle, C.byref(begin),
                       C.byref(out))
            assert out.ticket_id == i + 1 and out.codes_consumed_event
            # a second begin while the ticket is pending is a state error
            with pytest.raises(codec.CodecError) as e:
                codec.call("qwen3_tts_codec_session_process_device_packet_begin_v2", dev.handle, C.byref(begin),
                           C.byref(codec.DevicePacketBeginResult(C.sizeof(codec.DevicePacketBeginResult), 0, 0,
                                                                 None, 0)))
            assert e.value.status == -3
            pcm = np.zeros(7680, np.int16)
            res = codec.PacketResult()
            bad = codec.DevicePacketFinish(C.sizeof(codec.DevicePacketFinish), 0, out.ticket_id + 7, 0, 0,
                                           pcm.ctypes.data, pcm.size, C.pointer(res), 0)
            with pytest.raises(codec.CodecError) as e:
                codec.call("qwen3_tts_codec_session_process_device_packet_finish_v2", dev.handle, C.byref(bad))
            assert e.value.status == -3
            fin = codec.DevicePacketFinish(C.sizeof(codec.DevicePacketFinish), 0, out.ticket_id, 0, 0,
                                           pcm.ctypes.data, pcm.size, C.pointer(res), 0)
            codec.call("qwen3_tts_codec_session_process_device_packet_finish_v2", dev.handle, C.byref(fin))
            np.testing.assert_array_equal(pcm[: res.sample_count], want)
            assert res.first_frame_position == a
        # host memory is not a device codec pointer
        host_codes = np.ascontiguousarray(codes[:1])
        begin = codec.DevicePacketBegin(C.sizeof(codec.DevicePacketBegin), 0, host_codes.ctypes.data, 1, 0,
                                        ready.value, 0)
        with pytest.raises(codec.CodecError) as e:
            codec.call("qwen3_tts_codec_session_process_device_packet_begin_v2", dev.handle, C.byref(begin),
                       C.byref(codec.DevicePacketBeginResult(C.sizeof(codec.DevicePacketBeginResult), 0, 0, None,
                                                             0)))
        assert e.value.status in (-1, -2)
    finally:
        hip.hipStreamSynchronize(stream)
        hip.hipFree(buf)
        hip.hipEventDestroy(ready)
        hip.hipStreamDestroy(stream)


def test_bf16_sources_and_load_errors(codec, weights):
    print("codec load contract", flush=True)
    bf = dict(weights)
    for name in ("decoder.decoder.0.conv.bias", "decoder.pre_transformer.norm.weight"):
        bf[name] = O.f32_to_bf16(weights[name])
    m = codec.SharedModel(bf, warm=False)
    assert m.info.source_dtype_bf16_count == 2 and m.info.source_dtype_f32_count == 269
    # sessions need a warmed model
    with pytest.raises(codec.CodecError) as e:
        m.session()
    assert e.value.status == -3
    m.close()
    short = dict(weights)
    short.pop("decoder.decoder.5.beta")
    with pytest.raises(codec.CodecError) as e:
        codec.SharedModel(short, warm=False)
    assert e.value.status == -5 and "271" in e.value.message
    wrong = dict(weights)
    wrong["decoder.decoder.5.beta"] = np.zeros(95, np.float32)
    with pytest.raises(codec.CodecError) as e:
        codec.SharedModel(wrong, warm=False)
    assert e.value.status == -5


def test_legacy_context_api(codec, weights, codes):
    """create_v1 + load_model_v1 + warmup_v1 (a context owning its model)."""
    s = codec.Session(None)
    info = codec.ModelInfo()
    provider = codec.Provider(weights)
    codec.call("qwen3_tts_codec_load_model_v1", s.handle, C.byref(provider.struct), C.byref(info))
    assert info.loaded == 1
    codec.call("qwen3_tts_codec_warmup_v1", s.handle)
    pcm, res = s.packet(codes[:4])
    assert res.sample_count == 7680 and res.first_frame_position == 0


def test_fixture_packets_match_reference_model(codec):
    """The weight-free fixture: 83 deterministic frames in the reference's
    1/4/2/3/4/1/3/2 packets equal its CPU model decoding them at once; after
    the final packet another is rejected; a reset restarts the stream
    (the reference's fixture parity record: 34 packets, 159,360 samples,
    max error 0, benchmarks/results/codec-incremental-fixture-parity.json)."""
    import codec_fixture as FX

    print("codec fixture", flush=True)
    frames = FX.deterministic_frames(83)
    want = FX.FixtureState().process(frames)
    s = codec.Session(None)  # a context; the fixture needs no weights
    got, positions = [], []
    plan = FX.packets(83)
    for i, (a, b) in enumerate(plan):
        pcm, res = s.fixture_packet(frames[a:b], is_final=i == len(plan) - 1)
        got.append(pcm)
        positions.append((res.first_frame_position, res.first_sample_position, res.ring_slot))
    got = np.concatenate(got)
    assert len(plan) == 34 and got.size == 159_360
    np.testing.assert_array_equal(got, want)
    assert positions[5] == (plan[5][0], plan[5][0] * 1920, 5 % 3)
    st = s.state()
    assert st.frame_position == 83 and st.emitted_samples == 159_360 and st.kv_ring_head == 83 % 72
    with pytest.raises(codec.CodecError) as e:
        s.fixture_packet(frames[:1])
    assert e.value.status == -3
    s.reset()
    again, _ = s.fixture_packet(frames[:1])
    np.testing.assert_array_equal(again, want[:1920])


def test_every_packet_size_with_bf16_sources(codec):
    """Packets of 2, 3, 1, 4, 2 frames (every graph size) from a model whose
    271 tensors arrive as bf16 (widened on the device, CS:3206-3240), against
    the oracle on the same bf16-rounded weights."""
    print("codec bf16 model, packets 2/3/1/4/2", flush=True)
    w32 = M.make_weights(5)
    bits = {k: O.f32_to_bf16(v) for k, v in w32.items()}
    rounded = {k: O.bf16_to_f32(v) for k, v in bits.items()}
    m = codec.SharedModel(bits)
    assert m.info.source_dtype_bf16_count == 271 and m.info.source_bytes == 2 * 114_323_137
    codes = M.random_codes(12, 9)
    plan = ((0, 2), (2, 5), (5, 6), (6, 10), (10, 12))
    s = m.session()
    orc = O.CodecOracle(rounded)
    got = np.concatenate([s.packet(codes[a:b])[0] for a, b in plan])
    want = np.concatenate([orc.packet(codes[a:b], trace=False)["pcm"] for a, b in plan])
    diff = np.abs(got.astype(np.int32) - want)
    print(f"  PCM vs oracle: max diff {diff.max()}, identical {(diff == 0).mean():.4f}", flush=True)
    assert got.size == 12 * 1920 and diff.max() <= 1 and (diff == 0).mean() > 0.85
    m.close()


def test_argument_and_state_errors(codec, model, codes):
    """Status codes and states of the reference's state machine
    (codec_state.cu:3984-4009, 4345-4380, 5004-5027, 5144-5330)."""
    lib = codec.load()
    err = C.create_string_buffer(256)
    s = model.session()
    pcm = np.zeros(7680, np.int16)
    res = codec.PacketResult()
    c5 = np.zeros((5, 16), np.uint16)
    # 0 or 5 frames, bad is_final, small capacity, codes out of range
    assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, c5.ctypes.data, 0, 0, pcm.ctypes.data, 7680,
                                                         C.byref(res), err, 256) == -1
    assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, c5.ctypes.data, 5, 0, pcm.ctypes.data, 7680,
                                                         C.byref(res), err, 256) == -1
    assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, c5.ctypes.data, 1, 2, pcm.ctypes.data, 7680,
                                                         C.byref(res), err, 256) == -1
    assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, c5.ctypes.data, 2, 0, pcm.ctypes.data, 1919 * 2,
                                                         C.byref(res), err, 256) == -1
    assert b"capacity" in err.value
    bad = np.full((1, 16), 2048, np.uint16)
    assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, bad.ctypes.data, 1, 0, pcm.ctypes.data, 7680,
                                                         C.byref(res), err, 256) == -1
    # none of these advanced the stream
    assert s.state().frame_position == 0
    # debug hooks: bad checkpoint id, small capacity
    out = np.zeros(16, np.float32)
    assert lib.qwen3_tts_codec_debug_decoder_checkpoint_v1(s.handle, codes.ctypes.data, 1, 14, out.ctypes.data,
                                                           out.size, err, 256) == -1
    assert lib.qwen3_tts_codec_debug_transformer_packet_v1(s.handle, codes.ctypes.data, 1, out.ctypes.data, 16,
                                                           err, 256) == -1
    # cancel while a device ticket is pending: the ticket is dropped, the
    # stream needs a reset
    hip = _hip_runtime()
    buf, ready = C.c_void_p(), C.c_void_p()
    assert hip.hipMalloc(C.byref(buf), 64) == 0 and hip.hipEventCreate(C.byref(ready)) == 0
    try:
        one = np.ascontiguousarray(codes[:1])
        assert hip.hipMemcpy(buf, one.ctypes.data, 32, 1) == 0
        assert hip.hipEventRecord(ready, None) == 0
        begin = codec.DevicePacketBegin(C.sizeof(codec.DevicePacketBegin), 0, buf.value, 1, 0, ready.value, 0)
        outb = codec.DevicePacketBeginResult(C.sizeof(codec.DevicePacketBeginResult), 0, 0, None, 0)
        codec.call("qwen3_tts_codec_session_process_device_packet_begin_v2", s.handle, C.byref(begin), C.byref(outb))
        # a host packet while the ticket is pending is a state error
        assert lib.qwen3_tts_codec_session_process_packet_v1(s.handle, one.ctypes.data, 1, 0, pcm.ctypes.data,
                                                             7680, C.byref(res), err, 256) == -3
        s.cancel()
        fin = codec.DevicePacketFinish(C.sizeof(codec.DevicePacketFinish), 0, outb.ticket_id, 0, 0,
                                       pcm.ctypes.data, pcm.size, C.pointer(res), 0)
        assert lib.qwen3_tts_codec_session_process_device_packet_finish_v2(s.handle, C.byref(fin), err, 256) == -3
        # a wrong struct size is rejected before anything runs
        s.reset()
        begin.struct_size = 8
        assert lib.qwen3_tts_codec_session_process_device_packet_begin_v2(s.handle, C.byref(begin), C.byref(outb),
                                                                           err, 256) == -1
        # after the reset the stream decodes from the start again
        first, r = s.packet(codes[:1])
        assert r.first_frame_position == 0 and first.size == 1920
    finally:
        hip.hipFree(buf)
        hip.hipEventDestroy(ready)
    mem = s.memory()
    st = s.state()
    assert mem.device_bytes == st.device_bytes > mem.transformer_kv_bytes > 0
    assert mem.codec_ring_bytes == 3 * 4 * 16 * 2 and mem.pcm_ring_bytes == 3 * 7680 * 2
