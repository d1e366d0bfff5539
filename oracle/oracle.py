"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The shipped library never uses
it.  Each wrapper calls the C restatement in oracle.c, which cites the
reference file:line it follows.
"""
from __future__ import annotations

import ctypes as C
import pathlib
import subprocess

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(LIB_PATH))
    return _lib


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_bf16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def bf16_to_f32(x):
    x = _c(x, np.uint16)
    out = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def quantize_weight_rows(weight_bf16):
    w = _c(weight_bf16, np.uint16)
    out_f, in_f = w.shape
    q = np.empty((out_f, in_f), np.int8)
    s = np.empty(out_f, np.float32)
    lib().orc_quantize_weight_rows(_p(w), _p(q), _p(s), in_f, out_f)
    return q, s


def int8_gemm_rows(weight, scales, x_bf16):
    """Returns (y32, y16) with the reference's exact summation order."""
    w = _c(weight, np.int8)
    s = _c(scales, np.float32)
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    rows, in_f = x.shape
    out_f = w.shape[0]
    y32 = np.empty((rows, out_f), np.float32)
    y16 = np.empty((rows, out_f), np.uint16)
    lib().orc_int8_gemm_rows(_p(w), _p(s), _p(x), in_f, out_f, rows, _p(y32), _p(y16))
    return y32, y16


def int8_gemm_rows_mt(weight, scales, x_bf16, threads):
    w = _c(weight, np.int8)
    s = _c(scales, np.float32)
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    rows, in_f = x.shape
    out_f = w.shape[0]
    y32 = np.empty((rows, out_f), np.float32)
    lib().orc_int8_gemm_rows_mt(_p(w), _p(s), _p(x), in_f, out_f, rows, _p(y32), None, threads)
    return y32


def int8_gemm_rows_f64(weight, scales, x_bf16):
    w = _c(weight, np.int8)
    s = _c(scales, np.float32)
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    rows, in_f = x.shape
    out_f = w.shape[0]
    y = np.empty((rows, out_f), np.float64)
    lib().orc_int8_gemm_rows_f64(_p(w), _p(s), _p(x), in_f, out_f, rows, _p(y))
    return y


def int8_gemm_rows_add(weight, scales, x_bf16, inout_bf16):
    w = _c(weight, np.int8)
    s = _c(scales, np.float32)
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    io = _c(np.atleast_2d(inout_bf16), np.uint16).copy()
    rows, in_f = x.shape
    lib().orc_int8_gemm_rows_add(_p(w), _p(s), _p(x), _p(io), in_f, w.shape[0], rows)
    return io


def int8_gate_up_silu_rows(weight, scales, x_bf16):
    w = _c(weight, np.int8)
    s = _c(scales, np.float32)
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    rows, in_f = x.shape
    out_f = w.shape[0] // 2
    y = np.empty((rows, out_f), np.uint16)
    lib().orc_int8_gate_up_silu_rows(_p(w), _p(s), _p(x), _p(y), in_f, out_f, rows)
    return y


def rms_norm_rows(x_bf16, weight_bf16, eps=1e-6):
    x = _c(np.atleast_2d(x_bf16), np.uint16)
    g = _c(weight_bf16, np.uint16)
    out = np.empty_like(x)
    lib().orc_rms_norm_rows(_p(x), _p(g), _p(out), x.shape[0], x.shape[1], C.c_float(eps))
    return out


def head_rms_norm_rows(values_bf16, weight_bf16, heads, head_dim, eps=1e-6):
    v = _c(values_bf16, np.uint16).copy()
    g = _c(weight_bf16, np.uint16)
    rows = v.size // (heads * head_dim)
    lib().orc_head_rms_norm_rows(_p(v), _p(g), rows, heads, head_dim, C.c_float(eps))
    return v


def rope_rows(values_bf16, heads, head_dim, positions, theta=1e6):
    v = _c(values_bf16, np.uint16).copy()
    pos = _c(positions, np.int32)
    lib().orc_rope_rows(_p(v), len(pos), heads, head_dim, _p(pos), C.c_float(theta))
    return v


def attention(query, key_cache, value_cache, query_heads, kv_heads, head_dim, length, exact=True):
    q = _c(query, np.uint16)
    k = _c(key_cache, np.uint16)
    v = _c(value_cache, np.uint16)
    out = np.empty(query_heads * head_dim, np.uint16)
    fn = lib().orc_causal_gqa_attention if exact else lib().orc_causal_gqa_attention_fast
    fn(_p(q), _p(k), _p(v), _p(out), query_heads, kv_heads, head_dim, length)
    return out


def add_in_place(dst, src):
    d = _c(dst, np.uint16).copy()
    s = _c(src, np.uint16)
    lib().orc_add_in_place(_p(d), _p(s), d.size)
    return d


def bias_activation(values, bias, silu):
    v = _c(np.atleast_2d(values), np.uint16).copy()
    b = _c(bias, np.uint16)
    lib().orc_bias_activation(_p(v), _p(b), v.shape[0], v.shape[1], int(silu))
    return v


def silu_gate(gate, up):
    g = _c(gate, np.uint16).copy()
    u = _c(up, np.uint16)
    lib().orc_silu_gate(_p(g), _p(u), g.size)
    return g


def argmax_bf16(logits):
    x = _c(logits, np.uint16)
    return lib().orc_argmax_bf16(_p(x), x.size)


def sample_logits(logits, suppress, eos, history, do_sample, top_k, top_p, temperature,
                  penalty, state):
    """Returns (token, new_state)."""
    x = _c(logits, np.uint16)
    h = _c(history, np.int32) if len(history) else np.zeros(1, np.int32)
    st = C.c_uint64(state)
    L = lib()
    L.orc_sample_logits.restype = C.c_int
    L.orc_sample_logits.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_int,
                                    C.c_int, C.c_int, C.c_float, C.c_float, C.c_float,
                                    C.POINTER(C.c_uint64)]
    tok = L.orc_sample_logits(_p(x), x.size, int(suppress), eos, _p(h), len(history), do_sample,
                              top_k, top_p, temperature, penalty, C.byref(st))
    return tok, st.value


def expf_array(x):
    x = _c(x, np.float32)
    out = np.empty_like(x)
    lib().orc_expf_array(_p(x), _p(out), C.c_size_t(x.size))
    return out


def set_threads(threads: int) -> None:
    """Threads for the model-level GEMVs of large matrices (bit-identical
    results for any count)."""
    lib().orc_set_threads(int(threads))


def set_gemv_double_sum(on: bool) -> None:
    """Test switch: every int8 GEMV sums in double and rounds once -- a
    second valid summation order (not the reference's), for measuring the
    drift between two valid orders."""
    lib().orc_set_gemv_double_sum(int(bool(on)))


def bf16_gemm(a_bits, b_bits):
    """c = bf16(a @ b^T) with the oracle's fp32 accumulation (k order)."""
    a = _c(np.atleast_2d(a_bits), np.uint16)
    b = _c(np.atleast_2d(b_bits), np.uint16)
    m, k = a.shape
    n = b.shape[0]
    c = np.empty((m, n), np.uint16)
    lib().orc_bf16_gemm(_p(a), _p(b), _p(c), m, n, k, k, k, n)
    return c


def causal_softmax(scores_bits, head_dimension):
    """causal_softmax_kernel on [heads][rows][stride] bf16 scores (copy)."""
    s = _c(scores_bits, np.uint16).copy()
    heads, rows, stride = s.shape
    lib().orc_causal_softmax(_p(s), heads, rows, stride, head_dimension)
    return s


def set_gemm_order(order: int) -> None:
    """0: the bf16 GEMM's fp32 chain in k order (default); 1: accumulated in
    double and rounded once."""
    lib().orc_set_gemm_order(int(order))


# ---- speech-tokenizer decoder (codec_oracle.c) ----------------------------
CODEC_TENSORS = 269


class _CodecTrace(C.Structure):
    _fields_ = [("rvq", C.c_void_p), ("preconv", C.c_void_p), ("transformer", C.c_void_p),
                ("latent1", C.c_void_p), ("latent2", C.c_void_p), ("checkpoints", C.c_void_p * 14),
                ("stop_after", C.c_int)]


def codec_tensor_table():
    """[(name, float elements)] in the order orc_codec_packet takes them."""
    L = lib()
    L.orc_codec_tensor_name.restype = C.c_char_p
    L.orc_codec_tensor_elements.restype = C.c_uint64
    return [(L.orc_codec_tensor_name(i).decode(), int(L.orc_codec_tensor_elements(i)))
            for i in range(CODEC_TENSORS)]


# Decoder checkpoint -> (positions per frame, channels), CS:2066-2274.
CODEC_CHECKPOINTS = {6: (4, 1536), 7: (32, 768), 8: (160, 384), 9: (640, 192), 10: (1920, 96),
                     11: (1920, 96), 12: (1920, 1), 13: (1920, 1)}


class CodecOracle:
    """One decoding stream of the CPU decoder over fp32 weights given in
    codec_tensor_table() order (a dict name -> array, or a list)."""

    def __init__(self, weights):
        table = codec_tensor_table()
        if isinstance(weights, dict):
            weights = [weights[name] for name, _ in table]
        self._weights = [np.ascontiguousarray(w, np.float32).reshape(-1) for w in weights]
        for (name, count), w in zip(table, self._weights):
            if w.size != count:
                raise ValueError(f"{name}: {w.size} elements, expected {count}")
        self._ptrs = (C.c_void_p * CODEC_TENSORS)(*[w.ctypes.data for w in self._weights])
        L = lib()
        L.orc_codec_state_create.restype = C.c_void_p
        L.orc_codec_state_destroy.argtypes = [C.c_void_p]
        L.orc_codec_state_reset.argtypes = [C.c_void_p]
        L.orc_codec_packet.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                       C.POINTER(_CodecTrace)]
        self._state = L.orc_codec_state_create()

    def __del__(self):
        if getattr(self, "_state", None):
            lib().orc_codec_state_destroy(self._state)
            self._state = None

    def reset(self):
        lib().orc_codec_state_reset(self._state)

    def packet(self, codes, stop_after=0, trace=True):
        """Decodes one packet; returns a dict with 'pcm' (int16, empty for a
        stopped packet) and, with trace, the row-major stage outputs (names
        and decoder checkpoint numbers 6..13; zeros past a stop)."""
        codes = _c(np.atleast_2d(codes), np.uint16)
        frames = codes.shape[0]
        out = {"pcm": np.zeros(frames * 1920, np.int16)}
        tr = _CodecTrace()
        if trace:
            for name, shape in (("rvq", (frames, 512)), ("preconv", (frames, 1024)),
                                ("transformer", (frames, 1024)), ("latent1", (2 * frames, 1024)),
                                ("latent2", (4 * frames, 1024))):
                out[name] = np.zeros(shape, np.float32)
                setattr(tr, name, out[name].ctypes.data)
            for c, (per_frame, channels) in CODEC_CHECKPOINTS.items():
                out[c] = np.zeros((per_frame * frames, channels), np.float32)
                tr.checkpoints[c] = out[c].ctypes.data
        tr.stop_after = stop_after
        n = lib().orc_codec_packet(self._ptrs, self._state, codes.ctypes.data, frames,
                                   out["pcm"].ctypes.data, C.byref(tr))
        if n < 0:
            raise ValueError("packet must hold 1-4 frames")
        if n == 0:
            out["pcm"] = out["pcm"][:0]
        return out
