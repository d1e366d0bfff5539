"""The allocation-free decode attention entry point
(qwen3_tts_op_decode_attention_noalloc_v1) against the allocating one
(qwen3_tts_op_decode_attention): identical outputs and caches, bit for bit,
on two calls in a row on the shared static scratch (the second smaller, so
stale scratch contents of the first call must not leak into it), plus the
size limit's error."""
import ctypes as C

import numpy as np
import pytest

import gen

pytestmark = pytest.mark.gpu

D = 128


def dev(hip, a):
    return hip.DeviceArray.from_numpy(a)


def ptr_array(hip, ptrs):
    return dev(hip, np.array(ptrs, np.uint64))


def run_case(hip, entry, exact, qh, kvh, positions, max_seq, seed):
    rng = np.random.default_rng(seed)
    qw, kw = qh * D, kvh * D
    rows = len(positions)
    qkv = gen.activations(rng, rows, qw + 2 * kw)
    qn, kn = gen.gains(rng, D), gen.gains(rng, D)
    table = np.empty(max_seq * D, np.uint16)
    hip.call("qwen3_tts_rope_table_v1", max_seq, D, C.c_float(1e6), table.ctypes.data)
    caches = [(gen.activations(rng, max_seq, kw), gen.activations(rng, max_seq, kw)) for _ in range(rows)]
    kcs = [dev(hip, k) for k, _ in caches]
    vcs = [dev(hip, v) for _, v in caches]
    kb, vb = ptr_array(hip, [c.ptr for c in kcs]), ptr_array(hip, [c.ptr for c in vcs])
    out = hip.DeviceArray((rows, qw), np.uint16)
    keep = [dev(hip, qkv), dev(hip, qn), dev(hip, kn), dev(hip, table), dev(hip, np.array(positions, np.int32))]
    dq, dqn, dkn, dt, pos = keep
    hip.call(entry, exact, dq.ptr, qw + 2 * kw, dqn.ptr, dkn.ptr, dt.ptr, C.c_float(1e-6), kb.ptr, vb.ptr, pos.ptr,
             out.ptr, rows, qh, kvh, D, max_seq, None)
    return out.numpy(), [c.numpy() for c in kcs], [c.numpy() for c in vcs]


@pytest.mark.parametrize("exact", [1, 0])
def test_noalloc_matches_allocating_entry_point(hip, exact):
    cases = [(16, 8, [700, 5, 1023], 1024, 11), (16, 8, [3], 64, 12)]  # second call smaller
    for qh, kvh, positions, max_seq, seed in cases:
        ref = run_case(hip, "qwen3_tts_op_decode_attention", exact, qh, kvh, positions, max_seq, seed)
        got = run_case(hip, "qwen3_tts_op_decode_attention_noalloc_v1", exact, qh, kvh, positions, max_seq, seed)
        assert np.array_equal(got[0], ref[0]), (positions, max_seq)
        for r in range(len(positions)):
            assert np.array_equal(got[1][r], ref[1][r]) and np.array_equal(got[2][r], ref[2][r])


def test_noalloc_rejects_sizes_beyond_its_scratch(hip):
    null = C.c_void_p()
    with pytest.raises(hip.Qwen3TtsError) as e:
        # 8 rows at 8192 positions need ~140 MB of scratch
        hip.call("qwen3_tts_op_decode_attention_noalloc_v1", 1, null, 4096, null, null, null, C.c_float(1e-6), null,
                 null, null, null, 8, 16, 8, D, 8192, None)
    assert e.value.status == hip.STATUS_INVALID_ARGUMENT
    assert "scratch" in str(e.value)
