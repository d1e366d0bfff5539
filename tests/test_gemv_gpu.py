"""GPU parity of the int8 GEMV family against the CPU oracle.

Exact mode must be bit-identical to the reference's summation order
(native/qwen3-tts-native/native/src/int8_gemv.cu:58-293 as restated in
oracle/oracle.c); MFMA mode (rows >= 2) must satisfy the north-star tolerance
|y - y_ref| <= 1e-2 + 1e-3 |y_ref| on fp32 outputs.
"""
import numpy as np
import pytest

import gen

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-2


def dev(hip, a):
    return hip.DeviceArray.from_numpy(a)


# every matrix shape of the decode path (talker, predictor, heads, text
# projection, small_to_mtp) plus small/odd shapes the generic path handles
SHAPES = [
    (64, 256), (130, 512), (6144, 2048), (4096, 2048), (2048, 2048), (2048, 6144),
    (4096, 1024), (1024, 2048), (1024, 3072), (2048, 1024), (3072, 2048), (6, 48),
]


@pytest.mark.parametrize("out_f,in_f", SHAPES)
def test_exact_rows1_bit_identical(hip, orc, out_f, in_f):
    rng = np.random.default_rng(out_f * 7 + in_f)
    w, s, x = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, 1, in_f)
    ref32, ref16 = orc.int8_gemm_rows(w, s, x)
    dw, ds, dx = dev(hip, w), dev(hip, s), dev(hip, x)
    y32 = hip.DeviceArray((1, out_f), np.float32)
    y16 = hip.DeviceArray((1, out_f), np.uint16)
    hip.int8_gemv(dw, ds, dx, in_f, out_f, 1, out16=y16, out32=y32, mode=hip.MODE_EXACT)
    got32 = y32.numpy()
    assert np.array_equal(got32.view(np.uint32), ref32.view(np.uint32)), \
        f"{np.count_nonzero(got32 != ref32)} of {out_f} differ"
    assert np.array_equal(y16.numpy(), ref16)


# toy widths take the generic kernel; 1024/2048/3072/6144 the fixed-K rows kernel
@pytest.mark.parametrize("rows", [1, 2, 3, 5, 8])
@pytest.mark.parametrize("out_f,in_f", [(64, 256), (130, 512), (1000, 1024), (2048, 2048), (301, 3072), (2048, 6144)])
def test_exact_rows_bit_identical(hip, orc, rows, out_f, in_f):
    rng = np.random.default_rng(rows * 1000 + out_f)
    w, s, x = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, rows, in_f)
    ref32, ref16 = orc.int8_gemm_rows(w, s, x)
    y32 = hip.DeviceArray((rows, out_f), np.float32)
    y16 = hip.DeviceArray((rows, out_f), np.uint16)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y16, out32=y32,
                  mode=hip.MODE_EXACT)
    assert np.array_equal(y32.numpy(), ref32)
    assert np.array_equal(y16.numpy(), ref16)


@pytest.mark.parametrize("rows", [2, 4, 8])
@pytest.mark.parametrize("out_f,in_f", [(12288, 2048), (2048, 6144), (1028, 2048), (1024, 3072), (2052, 1024), (4096, 2048),
                                        (3072, 1024), (64, 256), (130, 512)])
def test_mfma_rows_within_tolerance(hip, orc, rows, out_f, in_f):
    rng = np.random.default_rng(rows + out_f + in_f)
    w, s, x = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, rows, in_f)
    ref32, _ = orc.int8_gemm_rows(w, s, x)
    y32 = hip.DeviceArray((rows, out_f), np.float32)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out32=y32, mode=hip.MODE_MFMA)
    got = y32.numpy()
    err = np.abs(got - ref32)
    assert np.all(err <= ATOL + RTOL * np.abs(ref32)), f"max err {err.max()}"
    # and it is really a different (MFMA) summation, not a copy of the exact path
    ref64 = orc.int8_gemm_rows_f64(w, s, x)
    assert np.allclose(got, ref64, rtol=1e-5, atol=1e-4)


@pytest.mark.parametrize("mode,rows", [("exact", 1), ("exact", 4), ("mfma", 2), ("mfma", 4)])
def test_epilogues(hip, orc, mode, rows):
    rng = np.random.default_rng(7 + rows)
    in_f, out_f = 1024, 384
    m = hip.MODE_EXACT if mode == "exact" else hip.MODE_MFMA
    w, s, x = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, rows, in_f)
    base = gen.activations(rng, rows, out_f)
    # add (fma epilogue, int8_gemv.cu:192-196)
    y = dev(hip, base)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_ADD_FMA, mode=m)
    ref = orc.int8_gemm_rows_add(w, s, x, base)
    check(mode, y.numpy(), ref)
    # add rounded (GEMV bf16 then add_in_place)
    y = dev(hip, base)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_ADD_ROUNDED, mode=m)
    _, p16 = orc.int8_gemm_rows(w, s, x)
    ref = np.stack([orc.add_in_place(base[r], p16[r]) for r in range(rows)])
    check(mode, y.numpy(), ref)
    # gate/up fused SiLU (int8_gemv.cu:283-289) and rounded (silu_gate kernel)
    wgu, sgu = gen.weights(rng, 2 * out_f, in_f), gen.scales(rng, 2 * out_f)
    y = hip.DeviceArray((rows, out_f), np.uint16)
    hip.int8_gemv(dev(hip, wgu), dev(hip, sgu), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_SILU_FUSED, mode=m)
    check(mode, y.numpy(), orc.int8_gate_up_silu_rows(wgu, sgu, x))
    y = hip.DeviceArray((rows, out_f), np.uint16)
    hip.int8_gemv(dev(hip, wgu), dev(hip, sgu), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_SILU_ROUNDED, mode=m)
    _, g16 = orc.int8_gemm_rows(wgu[:out_f], sgu[:out_f], x)
    _, u16 = orc.int8_gemm_rows(wgu[out_f:], sgu[out_f:], x)
    ref = np.stack([orc.silu_gate(g16[r], u16[r]) for r in range(rows)])
    check(mode, y.numpy(), ref)
    # bias epilogues (GEMV + bias_activation), and bias + residual add
    b = gen.activations(rng, out_f)
    for epi, silu in ((hip.EPI_BIAS, False), (hip.EPI_BIAS_SILU, True)):
        y = hip.DeviceArray((rows, out_f), np.uint16)
        hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y, epilogue=epi,
                      bias=dev(hip, b), mode=m)
        check(mode, y.numpy(), orc.bias_activation(p16, b, silu))
    y = dev(hip, base)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_BIAS_ADD, bias=dev(hip, b), mode=m)
    pb = orc.bias_activation(p16, b, False)
    ref = np.stack([orc.add_in_place(base[r], pb[r]) for r in range(rows)])
    check(mode, y.numpy(), ref)


def check(mode, got16, ref16):
    if mode == "exact":
        assert np.array_equal(got16, ref16), f"{np.count_nonzero(got16 != ref16)} differ"
    else:
        g, r = gen.f32(got16), gen.f32(ref16)
        assert np.all(np.abs(g - r) <= ATOL + 8e-3 * np.abs(r)), np.abs(g - r).max()


@pytest.mark.parametrize("in_f,out_f", [(2048, 4096), (1024, 4096), (2048, 12288 // 2), (512, 64)])
def test_rmsnorm_prologue_bit_identical(hip, orc, in_f, out_f):
    """GEMV with the RMSNorm fused as prologue == rms_norm then GEMV."""
    rng = np.random.default_rng(in_f + out_f)
    w, s, x, g = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, 1, in_f), gen.gains(rng, in_f)
    xn = orc.rms_norm_rows(x, g)
    ref32, ref16 = orc.int8_gemm_rows(w, s, xn)
    y32 = hip.DeviceArray((1, out_f), np.float32)
    y16 = hip.DeviceArray((1, out_f), np.uint16)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, 1, out16=y16, out32=y32,
                  norm_weight=dev(hip, g), mode=hip.MODE_EXACT)
    assert np.array_equal(y32.numpy(), ref32)
    assert np.array_equal(y16.numpy(), ref16)


@pytest.mark.parametrize("rows", [2, 3, 8])
@pytest.mark.parametrize("in_f", [1024, 2048, 3072])
@pytest.mark.parametrize("out_f", [1024, 1004])
def test_rmsnorm_prologue_mfma_rows(hip, orc, rows, in_f, out_f):
    """Batched RMSNorm prologue (both block shapes: 16 channels, and 8
    channels over two K halves for the fused gate/up at K >= 2048), ragged
    channel counts included."""
    rng = np.random.default_rng(5 + rows + in_f + out_f)
    w, s, x, g = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, rows, in_f), gen.gains(rng, in_f)
    xn = orc.rms_norm_rows(x, g)
    ref32, _ = orc.int8_gemm_rows(w, s, xn)
    y32 = hip.DeviceArray((rows, out_f), np.float32)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out32=y32,
                  norm_weight=dev(hip, g), mode=hip.MODE_MFMA)
    got = y32.numpy()
    assert np.all(np.abs(got - ref32) <= ATOL + RTOL * np.abs(ref32))
    wgu, sgu = gen.weights(rng, 2 * out_f, in_f), gen.scales(rng, 2 * out_f)
    y = hip.DeviceArray((rows, out_f), np.uint16)
    hip.int8_gemv(dev(hip, wgu), dev(hip, sgu), dev(hip, x), in_f, out_f, rows, out16=y,
                  epilogue=hip.EPI_SILU_FUSED, norm_weight=dev(hip, g), mode=hip.MODE_MFMA)
    check("mfma", y.numpy(), orc.int8_gate_up_silu_rows(wgu, sgu, xn))


def test_input_row_index(hip, orc):
    """The GEMV reads its activation row from a table through a device index."""
    rng = np.random.default_rng(11)
    in_f, out_f, vocab = 1024, 256, 50
    table = gen.activations(rng, vocab, in_f)
    w, s = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f)
    idx = dev(hip, np.array([37], np.int32))
    y = hip.DeviceArray((1, out_f), np.uint16)
    dtable = dev(hip, table)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dtable, in_f, out_f, 1, out16=y, input_row_index=idx,
                  mode=hip.MODE_EXACT)
    _, ref = orc.int8_gemm_rows(w, s, table[37])
    assert np.array_equal(y.numpy(), ref)


def test_quantizer_matches_oracle(hip, orc):
    rng = np.random.default_rng(3)
    w = gen.bf16(rng.standard_normal((300, 1024)).astype(np.float32) * 0.05)
    w[7] = 0
    q = hip.DeviceArray((300, 1024), np.int8)
    s = hip.DeviceArray(300, np.float32)
    hip.quantize_weight_rows(dev(hip, w), q, s, 1024, 300)
    rq, rs = orc.quantize_weight_rows(w)
    assert np.array_equal(q.numpy(), rq)
    assert np.array_equal(s.numpy(), rs)


def test_int8_gemv_benchmark_runs(hip):
    import ctypes as C
    out = hip.GemvBenchmark()
    hip.call("qwen3_tts_benchmark_int8_gemv", 0, 2048, 6144, 200, C.byref(out))
    assert out.mean_launch_microseconds > 0
    assert out.reserved >= 48  # rotating copies exceed the last-level cache
