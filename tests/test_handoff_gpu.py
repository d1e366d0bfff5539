"""The talker-to-decoder device handoff, end to end on one GPU.

The talker library leases each frame's 16 codes in device memory behind a
ready event (qwen3_tts_session_next_frame_begin_v2); the decoder library takes
that pointer and event directly (qwen3_tts_codec_session_process_device_packet_begin_v2,
no host copy) and returns a consumed event, which the talker waits on before
it may overwrite the codes (next_frame_finish_v2's consumer_done_event) --
the reference's "device-to-device codec handoff" (native/qwen3-tts-native/
native/include/qwen3_tts_native.h:112-128,313-343; native/qwen3-tts-native-codec/
native/src/codec_state.cu:5144-5262).  The PCM must equal the decoder library's
host-code path bit for bit, and the CPU oracle decoding the oracle talker's
codes within one LSB.
"""
import ctypes as C

import numpy as np
import pytest

import codec_model as CM
import oracle as O
import toy_model
from toy_model import TOY

pytestmark = pytest.mark.gpu

TALKER_TOPK = (1, 50, 1.0, 0.9, 1.05)
PREDICTOR_TOPK = (1, 50, 1.0, 0.9, 1.0)


@pytest.fixture(autouse=True)
def decode_step_prefill(monkeypatch):
    monkeypatch.setenv("QWEN3_TTS_PREFILL", "decode")


def test_talker_codes_decode_through_device_handoff(hip, orc):
    import qwen3_tts_codec_hip as codec

    print("talker -> codec device handoff", flush=True)
    weights = toy_model.make_weights(TOY, seed=3)
    model, _ = toy_model.upload(hip, TOY, weights)
    om = toy_model.OracleModel(orc, TOY, weights)
    cweights = CM.make_weights(0)
    cmodel = codec.SharedModel(cweights)
    lib = hip.load()
    s = C.c_void_p()
    mem = hip.SessionMemory()
    hip.call("qwen3_tts_session_create", model, 64, 11, C.byref(s), C.byref(mem))
    try:
        rng = np.random.default_rng(4)
        text = rng.integers(0, TOY["text_vocabulary"], 5).astype(np.int32)
        cprompt = rng.integers(0, 2048, 5).astype(np.int32)
        pre = hip.PrefillResult()
        hip.call("qwen3_tts_session_prefill", s, text.ctypes.data_as(C.POINTER(C.c_int32)),
                 cprompt.ctypes.data_as(C.POINTER(C.c_int32)), 5, hip.SamplingConfig(*TALKER_TOPK), C.byref(pre))
        osess = toy_model.OracleSession(om, 64, 11)
        semantic = osess.prefill(text, cprompt, TALKER_TOPK)
        assert semantic == pre.first_semantic_token
        dev = cmodel.session()
        host = cmodel.session()
        corc = O.CodecOracle(cweights)
        got, want, ref = [], [], []
        for f in range(6):
            if semantic == TOY["codec_eos_token"]:
                break
            view = hip.DeviceFrameViewV2()
            view.struct_size = C.sizeof(hip.DeviceFrameViewV2)
            hip.call("qwen3_tts_session_next_frame_begin_v2", s, 3 + f, hip.SamplingConfig(*TALKER_TOPK),
                     hip.SamplingConfig(*PREDICTOR_TOPK), C.byref(view))
            begin = codec.DevicePacketBegin(C.sizeof(codec.DevicePacketBegin), 0, view.device_codes, 1, 0,
                                            view.ready_event, 0)
            out = codec.DevicePacketBeginResult(C.sizeof(codec.DevicePacketBeginResult), 0, 0, None, 0)
            codec.call("qwen3_tts_codec_session_process_device_packet_begin_v2", dev.handle, C.byref(begin),
                       C.byref(out))
            nxt = C.c_uint16()
            info = hip.CodecFrameInfo()
            # the talker may overwrite the leased codes only after the decoder consumed them
            hip.call("qwen3_tts_session_next_frame_finish_v2", s, view.lease_id, out.codes_consumed_event,
                     C.byref(nxt), C.byref(info))
            pcm = np.zeros(1920, np.int16)
            res = codec.PacketResult()
            fin = codec.DevicePacketFinish(C.sizeof(codec.DevicePacketFinish), 0, out.ticket_id, 0, 0,
                                           pcm.ctypes.data, pcm.size, C.pointer(res), 0)
            codec.call("qwen3_tts_codec_session_process_device_packet_finish_v2", dev.handle, C.byref(fin))
            ocodes, onxt = osess.frame(semantic, 3 + f, TALKER_TOPK, PREDICTOR_TOPK)
            assert nxt.value == onxt
            got.append(pcm)
            want.append(host.packet(ocodes)[0])  # same codes through host memory
            ref.append(corc.packet(ocodes, trace=False)["pcm"])
            semantic = nxt.value
        assert len(got) >= 2
        got, want, ref = (np.concatenate(x) for x in (got, want, ref))
        np.testing.assert_array_equal(got, want)
        diff = np.abs(got.astype(np.int32) - ref)
        print(f"  {len(got) // 1920} frames, PCM vs oracle: max diff {diff.max()}, "
              f"identical {(diff == 0).mean():.4f}", flush=True)
        assert diff.max() <= 1 and (diff == 0).mean() > 0.85
    finally:
        lib.qwen3_tts_session_destroy(s)
        lib.qwen3_tts_model_destroy(model)
        cmodel.close()
