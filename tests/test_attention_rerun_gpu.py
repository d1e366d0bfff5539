"""The exact decode attention's rerun path (csrc/attention.hip,
attention_group_kernel): the value chains run on provisional probabilities
and are rerun from the first 64-position block whose exact probability
differs.  With QWEN3_TTS_ATTENTION_SKEW_PROVISIONAL=1 the provisional
normalizer is off by 2^-7, so nearly every probability differs and the rerun
covers almost the whole chain; the result must still equal the oracle's
exact attention (causal_gqa_attention_kernel, talker_kernels.cu:287-357)
bit for bit.  The switch is read once per process, so the cases run in a
child process."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [(16, 8, 65, 65), (16, 8, 1001, 1001), (8, 8, 700, 1024), (16, 4, 513, 1001), (16, 8, 129, 1024)]


def run_cases(hip, orc):
    import gen

    d = 128
    for qh, kvh, length, max_seq in CASES:
        rng = np.random.default_rng(length + 17 * qh + kvh)
        q = gen.activations(rng, qh * d)
        k = gen.bf16(rng.standard_normal((max_seq, kvh * d)).astype(np.float32) * 0.5)
        v = gen.activations(rng, max_seq, kvh * d)
        keep = [hip.DeviceArray.from_numpy(x) for x in (q, k, v, np.array([length - 1], np.int32))]
        dq, dk, dv, pos = keep
        kb = hip.DeviceArray.from_numpy(np.array([dk.ptr], np.uint64))
        vb = hip.DeviceArray.from_numpy(np.array([dv.ptr], np.uint64))
        out = hip.DeviceArray(qh * d, np.uint16)
        print("case", qh, kvh, length, max_seq, flush=True)
        hip.call("qwen3_tts_op_attention", 1, dq.ptr, qh * d, kb.ptr, vb.ptr, pos.ptr, out.ptr, 1, qh, kvh, d,
                 max_seq, None)
        ref = orc.attention(q, k[:length], v[:length], qh, kvh, d, length, exact=True)
        assert np.array_equal(out.numpy(), ref), (qh, kvh, length, max_seq)


def test_rerun_path_matches_the_oracle():
    env = dict(os.environ, QWEN3_TTS_ATTENTION_SKEW_PROVISIONAL="1")
    res = subprocess.run([sys.executable, __file__, "--child"], capture_output=True, text=True, timeout=110, env=env)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "rerun ok" in res.stdout


if __name__ == "__main__" and "--child" in sys.argv:
    import pathlib

    root = pathlib.Path(__file__).resolve().parents[1]
    sys.path[:0] = [str(root / "qwen3-tts-native_amd"), str(root / "oracle"), str(root / "tests")]
    import oracle
    import qwen3_tts_hip

    qwen3_tts_hip.load()
    oracle.lib()
    run_cases(qwen3_tts_hip, oracle)
    print("rerun ok", flush=True)
