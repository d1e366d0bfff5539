"""Pins the CPU oracle (oracle/oracle.c) before it is trusted as the checker.

Each check is independent of the oracle's own code: fp64 closed forms, exact
rational brute force on tiny inputs, the reference's own known-answer tests
(native/qwen3-tts-native/native/src/primitive_parity.cu:115-368,
runtime.cu:153-159 and benchmarks/results/bf16-argmax-vocab{2048,3072}.json),
invariants, and a sensitivity check that a plausible mistake (wrong
summation order) is detected.
"""
import math
from fractions import Fraction

import numpy as np
import pytest

import gen


# ---------------------------------------------------------------------------
# exact float32 arithmetic on rationals (brute force)
# ---------------------------------------------------------------------------
def f32_round(x: Fraction) -> float:
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.frexp(float(a))[1] - 1  # 2^e <= a < 2^(e+1), adjusted below
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** max(e - 23, -149)
    q = a / ulp
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return float(np.float32(sign * n * ulp))


def fma32(a, b, c):
    return f32_round(Fraction(a) * Fraction(b) + Fraction(c))


def add32(a, b):
    return f32_round(Fraction(a) + Fraction(b))


def brute_dot_reference_order(w_row, x_row):
    """int8_gemv.cu:67-125 evaluated in exact rational arithmetic with one
    rounding per operation: 32 lanes, strided 16-element vectors, fresh fma
    chains, shuffle-down fold 16..1."""
    acc = [0.0] * 32
    vectors = len(w_row) // 16
    for lane in range(32):
        for v in range(lane, vectors, 32):
            s = 0.0
            for j in range(16):
                s = fma32(float(w_row[16 * v + j]), float(x_row[16 * v + j]), s)
            acc[lane] = add32(acc[lane], s)
    off = 16
    while off:
        for lane in range(off):
            acc[lane] = add32(acc[lane], acc[lane + off])
        off //= 2
    return acc[0]


def test_gemv_matches_exact_rational_brute_force(orc, rng):
    in_f, out_f = 1024, 3
    w = gen.weights(rng, out_f, in_f)
    # wide dynamic range so that the summation order changes the result
    x32 = (rng.standard_normal(in_f) * np.exp2(rng.integers(-6, 7, in_f))).astype(np.float32)
    x = gen.bf16(x32)
    s = np.ones(out_f, np.float32)
    y32, _ = orc.int8_gemm_rows(w, s, x)
    xf = gen.f32(x)
    for c in range(out_f):
        assert y32[0, c] == brute_dot_reference_order(w[c], xf)


def test_summation_order_is_observable(orc, rng):
    """A sequential (wrong-order) fp32 dot differs from the reference order on
    adversarial inputs, so the bit-exact GPU tests can detect an order bug."""
    in_f, out_f = 2048, 64
    w = gen.weights(rng, out_f, in_f)
    x = gen.bf16((rng.standard_normal(in_f) * np.exp2(rng.integers(-8, 9, in_f))).astype(np.float32))
    s = np.ones(out_f, np.float32)
    y32, _ = orc.int8_gemm_rows(w, s, x)
    xf = gen.f32(x)
    seq = np.zeros(out_f, np.float32)
    for c in range(out_f):
        acc = np.float32(0)
        for k in range(in_f):
            acc = np.float32(acc + np.float32(w[c, k]) * xf[k])
        seq[c] = acc
    assert np.any(seq != y32[0])


@pytest.mark.parametrize("out_f,in_f,rows", [(64, 256, 1), (130, 512, 3), (64, 256, 8), (6144, 2048, 1)])
def test_gemv_close_to_fp64(orc, rng, out_f, in_f, rows):
    w = gen.weights(rng, out_f, in_f)
    s = gen.scales(rng, out_f)
    x = gen.activations(rng, rows, in_f)
    y32, y16 = orc.int8_gemm_rows(w, s, x)
    y64 = orc.int8_gemm_rows_f64(w, s, x)
    assert np.allclose(y32, y64, rtol=1e-5, atol=1e-4)
    assert np.array_equal(y16, gen.bf16(y32))


def test_gemv_special_cases(orc, rng):
    in_f, out_f = 512, 48
    w = gen.weights(rng, out_f, in_f)
    # W = 0 -> y = 0 (the reference's zero check, gemv.cu:247-250)
    y, _ = orc.int8_gemm_rows(np.zeros_like(w), gen.scales(rng, out_f), gen.activations(rng, 1, in_f))
    assert np.all(y == 0)
    # one-hot x -> scaled column, exactly
    k = 77
    x = np.zeros((1, in_f), np.float32)
    x[0, k] = 1.5
    s = gen.scales(rng, out_f)
    y, _ = orc.int8_gemm_rows(w, s, gen.bf16(x))
    assert np.array_equal(y[0], (w[:, k].astype(np.float32) * np.float32(1.5)) * s)
    # scale = 1 and small-integer x -> exact integer dot products
    xi = rng.integers(-3, 4, size=(2, in_f)).astype(np.float32)
    y, _ = orc.int8_gemm_rows(w, np.ones(out_f, np.float32), gen.bf16(xi))
    assert np.array_equal(y, (xi.astype(np.int64) @ w.astype(np.int64).T).astype(np.float32))


def test_gemm_add_and_gate_up_closed_forms(orc, rng):
    in_f, out_f = 512, 96
    w = gen.weights(rng, out_f, in_f)
    s = gen.scales(rng, out_f)
    x = gen.activations(rng, 2, in_f)
    base = gen.activations(rng, 2, out_f)
    out = orc.int8_gemm_rows_add(w, s, x, base)
    ref = gen.f32(base).astype(np.float64) + orc.int8_gemm_rows_f64(w, s, x)
    assert np.allclose(gen.f32(out), ref, rtol=2 ** -7, atol=1e-3)
    # rows with different residuals: the epilogue reads its own row
    assert not np.array_equal(out[0], out[1])
    wgu = gen.weights(rng, 2 * out_f, in_f)
    sgu = gen.scales(rng, 2 * out_f)
    y = orc.int8_gate_up_silu_rows(wgu, sgu, x)
    g = orc.int8_gemm_rows_f64(wgu[:out_f], sgu[:out_f], x)
    u = orc.int8_gemm_rows_f64(wgu[out_f:], sgu[out_f:], x)
    ref = g / (1.0 + np.exp(-g)) * u
    assert np.allclose(gen.f32(y), ref, rtol=2 ** -7, atol=1e-3)


def test_quantizer_invariants(orc, rng):
    w = gen.bf16(rng.standard_normal((40, 512)).astype(np.float32) * 0.02)
    w[3] = 0  # zero row -> scale 1
    q, s = orc.quantize_weight_rows(w)
    wf = gen.f32(w)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert s[3] == 1.0 and np.all(q[3] == 0)
    nz = [r for r in range(40) if r != 3]
    amax = np.abs(wf[nz]).max(axis=1)
    assert np.array_equal(s[nz], (amax / np.float32(127)).astype(np.float32))
    # the row maximum maps to +-127
    assert np.all(np.abs(q[nz]).max(axis=1) == 127)
    # dequantization error is within half a step (plus fp32 slack)
    err = np.abs(q[nz].astype(np.float32) * s[nz, None] - wf[nz])
    assert np.all(err <= s[nz, None] * 0.5 * (1 + 1e-5))
    # ties round to even (lrintf): 0.5 and 1.5 steps
    w2 = gen.bf16(np.array([[127.0, 0.5, 1.5, -0.5, -2.5] + [0.0] * 11], np.float32))
    q2, s2 = orc.quantize_weight_rows(w2)
    assert s2[0] == 1.0 and list(q2[0, :5]) == [127, 0, 2, 0, -2]


# ---------------------------------------------------------------------------
# primitives: the reference's own known-answer tests (primitive_parity.cu)
# ---------------------------------------------------------------------------
def _bfr(x):
    return gen.f32(gen.bf16(np.asarray(x, np.float32)))


def test_rms_norm_known_answer(orc):
    i = np.arange(128, dtype=np.float32)
    x = gen.bf16(np.sin(i * np.float32(0.071)) * np.float32(1.7))
    g = gen.bf16(np.float32(0.75) + np.cos(i * np.float32(0.037)) * np.float32(0.2))
    xf, gf = gen.f32(x), gen.f32(g)
    inv = 1.0 / np.sqrt(np.sum(xf.astype(np.float64) ** 2) / 128 + 1e-6)
    expected = _bfr(xf * inv * gf)
    got = gen.f32(orc.rms_norm_rows(x, g))[0]
    assert np.max(np.abs(got - expected)) <= 0.016
    # double rounding is visible: bf16(bf16(x*inv)*g) vs bf16(x*inv*g)
    assert np.max(np.abs(got - expected)) <= 2 * np.max(np.abs(expected)) * 2 ** -8


def test_rope_known_answer(orc):
    heads, d, pos = 2, 128, 37
    v = gen.bf16(np.sin(np.arange(heads * d, dtype=np.float32) * np.float32(0.019)))
    vf = gen.f32(v).reshape(heads, d)
    half = d // 2
    expected = np.empty_like(vf)
    for i in range(half):
        ang = pos * 1e6 ** (-(2 * i) / d)
        a, b = vf[:, i], vf[:, i + half]
        expected[:, i] = a * np.cos(ang) - b * np.sin(ang)
        expected[:, i + half] = b * np.cos(ang) + a * np.sin(ang)
    got = gen.f32(orc.rope_rows(v, heads, d, [pos])).reshape(heads, d)
    assert np.max(np.abs(got - _bfr(expected))) <= 0.016
    # position 0 is the identity
    assert np.array_equal(orc.rope_rows(v, heads, d, [0]), v)


@pytest.mark.parametrize("exact", [True, False])
def test_attention_known_answer(orc, exact):
    qh, kvh, d, seq = 4, 2, 32, 7
    q = gen.bf16(np.sin(np.arange(qh * d, dtype=np.float32) * np.float32(0.031)) * np.float32(0.4))
    kk = np.arange(seq * kvh * d, dtype=np.float32)
    k = gen.bf16(np.cos(kk * np.float32(0.023)) * np.float32(0.3))
    v = gen.bf16(np.sin(kk * np.float32(0.017)) * np.float32(0.5))
    qf, kf, vf = gen.f32(q).reshape(qh, d), gen.f32(k).reshape(seq, kvh, d), gen.f32(v).reshape(seq, kvh, d)
    expected = np.empty((qh, d), np.float64)
    for h in range(qh):
        g = h // (qh // kvh)
        sc = kf[:, g, :].astype(np.float64) @ qf[h] / np.sqrt(d)
        p = np.exp(sc - sc.max())
        p /= p.sum()
        expected[h] = p @ vf[:, g, :]
    got = gen.f32(orc.attention(q, k, v, qh, kvh, d, seq, exact=exact)).reshape(qh, d)
    assert np.max(np.abs(got - expected)) <= 0.016
    # a single position returns that position's value row (softmax of one = 1)
    one = gen.f32(orc.attention(q, k, v, qh, kvh, d, 1, exact=exact)).reshape(qh, d)
    for h in range(qh):
        assert np.array_equal(one[h], vf[0, h // 2])


def test_silu_gate_known_answer(orc):
    i = np.arange(257, dtype=np.float32)
    g = gen.bf16(np.sin(i * np.float32(0.043)) * 2)
    u = gen.bf16(np.cos(i * np.float32(0.029)))
    gf, uf = gen.f32(g).astype(np.float64), gen.f32(u).astype(np.float64)
    expected = gf / (1 + np.exp(-gf)) * uf
    got = gen.f32(orc.silu_gate(g, u))
    assert np.max(np.abs(got - expected)) <= 0.016


def test_bias_activation_closed_form(orc, rng):
    x = gen.activations(rng, 2, 300)
    b = gen.activations(rng, 300)
    plain = gen.f32(orc.bias_activation(x, b, False))
    assert np.array_equal(plain, _bfr(gen.f32(x) + gen.f32(b)))
    act = gen.f32(orc.bias_activation(x, b, True)).astype(np.float64)
    z = (gen.f32(x) + gen.f32(b)).astype(np.float64)
    assert np.allclose(act, z / (1 + np.exp(-z)), rtol=2 ** -7, atol=1e-6)


def test_expf_within_one_ulp(orc):
    x = np.concatenate([np.linspace(-103.9, 88.7, 400001, dtype=np.float32),
                        np.array([0.0, -0.0, 1e-30, -1e-30, 88.72, -87.33], np.float32)])
    got = orc.expf_array(x)
    ref = np.exp(x.astype(np.float64)).astype(np.float32)
    gi = got.view(np.int32).astype(np.int64)
    ri = ref.view(np.int32).astype(np.int64)
    assert np.max(np.abs(gi - ri)) <= 1
    assert orc.expf_array(np.array([np.inf, -np.inf, 100.0, -200.0], np.float32)).tolist() == [np.inf, 0.0, np.inf, 0.0]


# ---------------------------------------------------------------------------
# sampler
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("vocab", [2048, 3072])
def test_argmax_known_answer(orc, vocab):
    """runtime.cu:153-159 and benchmarks/results/bf16-argmax-vocab{2048,3072}.json
    (selected_token == expected_token == 1729)."""
    i = np.arange(vocab, dtype=np.float32)
    logits = gen.bf16(np.sin(i * np.float32(0.017)) * np.float32(2.0))
    logits[1729] = gen.bf16(np.float32(19.0))
    assert orc.argmax_bf16(logits) == 1729
    tok, _ = orc.sample_logits(logits, False, 2150, [], 0, 0, 1.0, 1.0, 1.0, 7)
    assert tok == 1729


def test_greedy_ties_lower_index_and_talker_mask(orc):
    logits = gen.bf16(np.zeros(3072, np.float32))
    logits[[5, 9, 2500]] = gen.bf16(np.float32(3.0))
    tok, _ = orc.sample_logits(logits, False, 2150, [], 0, 0, 1.0, 1.0, 1.0, 1)
    assert tok == 5
    # talker mask: >= 2048 except EOS is -inf
    logits2 = gen.bf16(np.zeros(3072, np.float32))
    logits2[2500] = gen.bf16(np.float32(9.0))
    logits2[2150] = gen.bf16(np.float32(5.0))
    tok, _ = orc.sample_logits(logits2, True, 2150, [], 0, 0, 1.0, 1.0, 1.0, 1)
    assert tok == 2150
    # repetition penalty divides positive logits of history tokens
    logits3 = gen.bf16(np.zeros(3072, np.float32))
    logits3[10] = gen.bf16(np.float32(2.0))
    logits3[11] = gen.bf16(np.float32(1.9))
    tok, _ = orc.sample_logits(logits3, True, 2150, [10], 0, 0, 1.0, 1.0, 1.5, 1)
    assert tok == 11


def test_topk_one_is_argmax_and_draws_follow_softmax(orc, rng):
    logits = gen.activations(rng, 2048)
    best = orc.argmax_bf16(logits)
    state = 12345
    for _ in range(20):
        tok, state = orc.sample_logits(logits, False, 2150, [], 1, 1, 1.0, 0.9, 1.0, state)
        assert tok == best
    # top-k = 4 draws follow softmax(v / T) over the 4 largest
    lg = np.full(2048, -5.0, np.float32)
    lg[[100, 200, 300, 400]] = [2.0, 1.5, 1.0, 0.5]
    lb = gen.bf16(lg)
    counts = {}
    state = 99
    n = 4000
    for _ in range(n):
        tok, state = orc.sample_logits(lb, False, 2150, [], 1, 4, 1.0, 0.9, 1.0, state)
        counts[tok] = counts.get(tok, 0) + 1
    assert set(counts) <= {100, 200, 300, 400}
    w = np.exp(np.array([2.0, 1.5, 1.0, 0.5]) / 0.9)
    w /= w.sum()
    for t, p in zip([100, 200, 300, 400], w):
        assert abs(counts.get(t, 0) / n - p) < 4 * np.sqrt(p * (1 - p) / n) + 1e-3
    # top-p below the first weight keeps only the argmax
    for _ in range(20):
        tok, state = orc.sample_logits(lb, False, 2150, [], 1, 4, 0.05, 0.9, 1.0, state)
        assert tok == 100


def test_xorshift_zero_state_reseeds(orc):
    import ctypes as C
    lib = orc.lib()
    lib.orc_xorshift64star.restype = C.c_uint64
    s0, s1 = C.c_uint64(0), C.c_uint64(0x9E3779B97F4A7C15)
    assert lib.orc_xorshift64star(C.byref(s0)) == lib.orc_xorshift64star(C.byref(s1))
    # published xorshift64* step (Vigna 2016): shifts 12, 25, 27, multiplier 0x2545F4914F6CDD1D
    x = 0x9E3779B97F4A7C15
    x ^= x >> 12
    x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
    x ^= x >> 27
    assert s0.value == x


def _xorshift64star(state):
    """Published xorshift64* step (Vigna 2016) with the reference's zero-state
    reseed (sampling_kernels.cu:53-63): returns (output, next state)."""
    m = (1 << 64) - 1
    x = state or 0x9E3779B97F4A7C15
    x ^= x >> 12
    x ^= (x << 25) & m
    x ^= x >> 27
    return (x * 0x2545F4914F6CDD1D) & m, x


def _uniform(state):
    out, nxt = _xorshift64star(state)
    return float(np.float32((out >> 11) * 2.0 ** -53)), nxt


TOPK_CASE_TOKENS = [400, 100, 300, 200]          # descending logit order
TOPK_CASE_LOGITS = [2.0, 1.25, 0.5, -0.75]       # exact in bf16


def topk_case_boundaries(temperature=1.0):
    """Cumulative weights of the retained candidates in descending order,
    normalized: the u values where the draw moves to the next candidate
    (target = u * total; candidate r is the first with cumulative >= target,
    sampling_kernels.cu:374-386)."""
    w = [math.exp(v / temperature - TOPK_CASE_LOGITS[0] / temperature) for v in TOPK_CASE_LOGITS]
    c = np.cumsum(w)
    return list(c[:-1] / c[-1])


def states_around(boundaries, margin=2e-3, count=1):
    """RNG states whose draw u lies just below / just above each boundary."""
    want = {(i, side): [] for i in range(len(boundaries)) for side in (0, 1)}
    seed = 1
    while any(len(v) < count for v in want.values()):
        u, _ = _uniform(seed)
        for i, b in enumerate(boundaries):
            if b - margin < u < b and len(want[(i, 0)]) < count:
                want[(i, 0)].append(seed)
            if b < u < b + margin and len(want[(i, 1)]) < count:
                want[(i, 1)].append(seed)
        seed += 1
    return want


def topk_case_logits():
    lg = np.full(2048, -8.0, np.float32)
    lg[TOPK_CASE_TOKENS] = TOPK_CASE_LOGITS
    return gen.bf16(lg)


def test_topk_draw_maps_u_through_the_descending_cumulative_order(orc):
    """Closed form: four candidates with known weights exp(v - max), a draw
    u from a known xorshift64* state, and the token is the first candidate
    in DESCENDING logit order whose cumulative weight reaches u * total --
    checked just below and just above every boundary (a reversed or
    ascending order, or an off-by-one at the boundary, fails here)."""
    bounds = topk_case_boundaries()
    logits = topk_case_logits()
    for (i, side), seeds in states_around(bounds).items():
        for st in seeds:
            u, nxt = _uniform(st)
            expected = TOPK_CASE_TOKENS[i + side]
            tok, state = orc.sample_logits(logits, False, 2150, [], 1, 4, 1.0, 1.0, 1.0, st)
            assert (tok, state) == (expected, nxt), (i, side, u)


@pytest.mark.parametrize("d", [64, 128])
def test_attention_scale_is_correctly_rounded(d):
    """The attention scale 1.0f/sqrtf(d) (oracle, decode attention and the
    prefill's causal softmax; the reference's rsqrtf at talker_kernels.cu:136,
    247, 303, 443, 527) is the float32 nearest to 1/sqrt(d): the exact squares
    of the midpoints to its neighbours bracket 1/d."""
    f = np.float32(1.0) / np.sqrt(np.float32(d))
    lo = Fraction(float(np.nextafter(f, np.float32(0))))
    hi = Fraction(float(np.nextafter(f, np.float32(1))))
    x = Fraction(float(f))
    assert ((lo + x) / 2) ** 2 * d < 1 < ((x + hi) / 2) ** 2 * d
    if d == 128:
        assert float(f).hex() == "0x1.6a09e60000000p-4"
