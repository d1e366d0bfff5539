"""The allocation-free decode attention entry point
(qwen3_tts_op_decode_attention_noalloc_v1) against the allocating one
(qwen3_tts_op_decode_attention): identical outputs and caches, bit for bit,
on two calls in a row on the shared static scratch (the second smaller, so
stale scratch contents of the first call must not leak into it), on two
streams back to back (the entry point orders them), captured into a hipGraph
and replayed (also as the first call of a fresh process), plus the size
limit's error."""
import ctypes as C
import subprocess
import sys

import numpy as np
import pytest

import gen

pytestmark = pytest.mark.gpu

D = 128


def dev(hip, a):
    return hip.DeviceArray.from_numpy(a)


def ptr_array(hip, ptrs):
    return dev(hip, np.array(ptrs, np.uint64))


def prepare(hip, exact, qh, kvh, positions, max_seq, seed):
    """Device inputs of one call; returns (launch(entry, stream), read())."""
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
    dq, dqn, dkn, dt = dev(hip, qkv), dev(hip, qn), dev(hip, kn), dev(hip, table)
    pos = dev(hip, np.array(positions, np.int32))
    keep = [kcs, vcs, kb, vb, out, dq, dqn, dkn, dt, pos]

    def launch(entry, stream):
        hip.call(entry, exact, dq.ptr, qw + 2 * kw, dqn.ptr, dkn.ptr, dt.ptr, C.c_float(1e-6), kb.ptr, vb.ptr,
                 pos.ptr, out.ptr, rows, qh, kvh, D, max_seq, stream)

    def read():
        return out.numpy(), [c.numpy() for c in kcs], [c.numpy() for c in vcs]

    launch.keep = keep
    return launch, read


def same(got, ref):
    return (np.array_equal(got[0], ref[0]) and all(np.array_equal(a, b) for a, b in zip(got[1], ref[1]))
            and all(np.array_equal(a, b) for a, b in zip(got[2], ref[2])))


def reference(hip, case):
    launch, read = prepare(hip, *case)
    launch("qwen3_tts_op_decode_attention", None)
    hip.synchronize()
    return read()


class Runtime:
    """The few HIP runtime calls the tests need for streams and graphs."""

    def __init__(self, hip):
        self.hip = hip
        self.rt = C.CDLL("libamdhip64.so")
        for name in ("hipStreamBeginCapture", "hipStreamEndCapture", "hipGraphInstantiate", "hipGraphLaunch",
                     "hipStreamSynchronize", "hipGraphExecDestroy", "hipGraphDestroy"):
            getattr(self.rt, name).restype = C.c_int

    def stream(self):
        s = C.c_void_p()
        self.hip.call("qwen3_tts_stream_create", 0, C.byref(s))
        return s

    def check(self, status, what):
        assert status == 0, f"{what} failed: {status}"

    def sync(self, s):
        self.check(self.rt.hipStreamSynchronize(s), "hipStreamSynchronize")

    def capture(self, s, body):
        self.check(self.rt.hipStreamBeginCapture(s, 1), "hipStreamBeginCapture")  # thread-local mode
        body()
        graph = C.c_void_p()
        self.check(self.rt.hipStreamEndCapture(s, C.byref(graph)), "hipStreamEndCapture")
        exe = C.c_void_p()
        self.check(self.rt.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)), "hipGraphInstantiate")
        return graph, exe

    def launch(self, exe, s):
        self.check(self.rt.hipGraphLaunch(exe, s), "hipGraphLaunch")

    def destroy(self, graph, exe):
        self.rt.hipGraphExecDestroy(exe)
        self.rt.hipGraphDestroy(graph)


CASE_A = (1, 16, 8, [700, 5, 1023], 1024, 21)
CASE_B = (1, 16, 8, [300, 900], 1024, 22)


def test_noalloc_calls_on_two_streams_are_ordered(hip):
    """Back-to-back calls on two streams without a host wait: the second
    waits for the first call's kernels instead of overwriting its scratch."""
    rt = Runtime(hip)
    ref_a, ref_b = reference(hip, CASE_A), reference(hip, CASE_B)
    s1, s2 = rt.stream(), rt.stream()
    try:
        for _ in range(3):
            la, ra = prepare(hip, *CASE_A)
            lb, rb = prepare(hip, *CASE_B)
            la("qwen3_tts_op_decode_attention_noalloc_v1", s1)
            lb("qwen3_tts_op_decode_attention_noalloc_v1", s2)
            rt.sync(s1)
            rt.sync(s2)
            assert same(ra(), ref_a) and same(rb(), ref_b)
    finally:
        hip.load().qwen3_tts_stream_destroy(s1)
        hip.load().qwen3_tts_stream_destroy(s2)


def capture_and_replay(hip, rt, replays=3):
    """Capture one no-allocation call on a non-default stream, replay it
    several times with eager work of the same entry point between the
    replays, and check every replay against the allocating entry point."""
    ref_a, ref_b = reference(hip, CASE_A), reference(hip, CASE_B)
    s, other = rt.stream(), rt.stream()
    la, ra = prepare(hip, *CASE_A)
    graph, exe = rt.capture(s, lambda: la("qwen3_tts_op_decode_attention_noalloc_v1", s))
    try:
        for _ in range(replays):
            rt.launch(exe, s)
            rt.sync(s)
            assert same(ra(), ref_a)
            lb, rb = prepare(hip, *CASE_B)
            lb("qwen3_tts_op_decode_attention_noalloc_v1", other)
            rt.sync(other)
            assert same(rb(), ref_b)
    finally:
        rt.destroy(graph, exe)
        hip.load().qwen3_tts_stream_destroy(s)
        hip.load().qwen3_tts_stream_destroy(other)


def test_noalloc_under_graph_capture(hip):
    capture_and_replay(hip, Runtime(hip))


def test_noalloc_first_call_of_a_process_under_capture():
    """The per-device scratch address is looked up on the first call; here
    that first call happens while a stream is being captured."""
    res = subprocess.run([sys.executable, __file__, "--fresh-capture"], capture_output=True, text=True, timeout=110)
    assert res.returncode == 0, res.stdout + res.stderr
    assert "fresh capture ok" in res.stdout


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


if __name__ == "__main__" and "--fresh-capture" in sys.argv:
    import pathlib

    root = pathlib.Path(__file__).resolve().parents[1]
    sys.path[:0] = [str(root / "qwen3-tts-native_amd"), str(root / "tests")]
    import qwen3_tts_hip

    qwen3_tts_hip.load()
    rt = Runtime(qwen3_tts_hip)
    s = rt.stream()
    la, ra = prepare(qwen3_tts_hip, *CASE_A)
    graph, exe = rt.capture(s, lambda: la("qwen3_tts_op_decode_attention_noalloc_v1", s))  # first call
    rt.launch(exe, s)
    rt.sync(s)
    got = ra()
    rt.destroy(graph, exe)
    assert same(got, reference(qwen3_tts_hip, CASE_A))
    print("fresh capture ok", flush=True)
