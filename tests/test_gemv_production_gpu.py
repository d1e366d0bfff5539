"""Bit-exact parity of the production GEMV instantiations at full decode shape.

The talker and predictor frames, and the bench's step chain, run the
batch-1 fixed-K kernel at K = 1024 / 2048 / 3072 / 6144 (512-byte vectors per
lane: 2 / 4 / 6 / 12) with one epilogue each and, for the projections that
follow an RMSNorm, the fused norm prologue.  Every (K, epilogue, norm)
combination is compared here, bit for bit, with the oracle's restatement of
native/qwen3-tts-native/native/src/int8_gemv.cu:58-293 (plain, residual and
gate/up-SiLU kernels), talker_kernels.cu:27-48 (RMSNorm) and the
GEMV-then-elementwise sequences of talker.cu:3251-3456, at the real output
widths of the model:

  talker: QKV 4096x2048 (+norm), O 2048x2048 (+residual), gate/up
          12288x2048 (+norm, SiLU), down 2048x6144 (+residual),
          codec head 3072x2048 (+final norm), text fc1/fc2 2048x2048 (+bias)
  predictor: QKV 4096x1024 (+norm), O 1024x2048, gate/up 6144x1024
          (+norm, SiLU), down 1024x3072, heads 2048x1024 (+final norm),
          small_to_mtp 1024x2048 (+bias)

and a two-layer talker GEMV chain (the bench's step at its real shapes) is
compared with the oracle's chain of the same four projections.
"""
import numpy as np
import pytest

import gen

pytestmark = pytest.mark.gpu

# (out width of the kernel's output, in_features) per K; SiLU epilogues read
# 2*out weight rows.
OUT_FOR_K = {1024: 3072, 2048: 6144, 3072: 1024, 6144: 2048}
EPILOGUES = ["store", "add_fma", "add_rounded", "silu_fused", "silu_rounded", "bias", "bias_silu", "bias_add"]


def dev(hip, a):
    return hip.DeviceArray.from_numpy(a)


def oracle_epilogue(orc, name, w, s, xn, base, bias):
    """The oracle's output for one epilogue on normalized (or raw) input xn."""
    out_f = base.shape[-1]
    if name == "store":
        return orc.int8_gemm_rows(w, s, xn)[1]
    if name == "add_fma":
        return orc.int8_gemm_rows_add(w, s, xn, base)
    if name == "add_rounded":
        return orc.add_in_place(base, orc.int8_gemm_rows(w, s, xn)[1])
    if name == "silu_fused":
        return orc.int8_gate_up_silu_rows(w, s, xn)
    if name == "silu_rounded":
        g16 = orc.int8_gemm_rows(w[:out_f], s[:out_f], xn)[1]
        u16 = orc.int8_gemm_rows(w[out_f:], s[out_f:], xn)[1]
        return orc.silu_gate(g16, u16)
    p16 = orc.int8_gemm_rows(w, s, xn)[1]
    if name == "bias":
        return orc.bias_activation(p16, bias, False)
    if name == "bias_silu":
        return orc.bias_activation(p16, bias, True)
    if name == "bias_add":
        return orc.add_in_place(base, orc.bias_activation(p16, bias, False))
    raise ValueError(name)


@pytest.mark.parametrize("norm", [False, True])
@pytest.mark.parametrize("epilogue", EPILOGUES)
@pytest.mark.parametrize("in_f", sorted(OUT_FOR_K))
def test_fixed_k_instantiation_bit_exact(hip, orc, in_f, epilogue, norm):
    out_f = OUT_FOR_K[in_f]
    silu = epilogue.startswith("silu")
    rng = np.random.default_rng(in_f * 31 + EPILOGUES.index(epilogue) * 7 + int(norm))
    w_rows = 2 * out_f if silu else out_f
    w, s = gen.weights(rng, w_rows, in_f), gen.scales(rng, w_rows)
    x, g = gen.activations(rng, 1, in_f), gen.gains(rng, in_f)
    base = gen.activations(rng, 1, out_f)
    bias = gen.activations(rng, out_f)
    xn = orc.rms_norm_rows(x, g) if norm else x
    ref = oracle_epilogue(orc, epilogue, w, s, xn, base, bias)

    y = dev(hip, base) if epilogue in ("add_fma", "add_rounded", "bias_add") else hip.DeviceArray((1, out_f), np.uint16)
    epi = getattr(hip, "EPI_" + epilogue.upper())
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, 1, out16=y, epilogue=epi,
                  norm_weight=dev(hip, g) if norm else None,
                  bias=dev(hip, bias) if epilogue.startswith("bias") else None, mode=hip.MODE_EXACT)
    got = y.numpy()
    assert np.array_equal(got, ref), f"{np.count_nonzero(got != ref)} of {out_f} differ"


@pytest.mark.parametrize("in_f", sorted(OUT_FOR_K))
def test_fixed_k_fp32_output_with_norm(hip, orc, in_f):
    """The fp32 output (the value just before the bf16 store,
    int8_gemv.cu:123-124) of the normed fixed-K kernel."""
    out_f = OUT_FOR_K[in_f]
    rng = np.random.default_rng(in_f + 99)
    w, s = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f)
    x, g = gen.activations(rng, 1, in_f), gen.gains(rng, in_f)
    ref32, ref16 = orc.int8_gemm_rows(w, s, orc.rms_norm_rows(x, g))
    y32 = hip.DeviceArray((1, out_f), np.float32)
    y16 = hip.DeviceArray((1, out_f), np.uint16)
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, 1, out16=y16, out32=y32,
                  norm_weight=dev(hip, g), mode=hip.MODE_EXACT)
    assert np.array_equal(y32.numpy().view(np.uint32), ref32.view(np.uint32))
    assert np.array_equal(y16.numpy(), ref16)


def test_talker_step_chain_two_layers(hip, orc):
    """Two talker layers of the bench's GEMV chain (QKV+norm, O+residual,
    gate/up+norm+SiLU, down+residual at hidden 2048, q width 2048, kv width
    1024, intermediate 6144), chained on the device exactly as the step
    benchmark chains them, against the oracle's chain.  The O projection
    reads the q part of the QKV output (the attention output's stand-in)."""
    H, QW, KW, I = 2048, 2048, 1024, 6144
    qkv_rows = QW + 2 * KW
    rng = np.random.default_rng(2026)
    hidden = gen.activations(rng, 1, H)
    g_in, g_post = gen.gains(rng, H), gen.gains(rng, H)
    dh = dev(hip, hidden)
    qkv = hip.DeviceArray((1, qkv_rows), np.uint16)
    act = hip.DeviceArray((1, I), np.uint16)
    dg_in, dg_post = dev(hip, g_in), dev(hip, g_post)
    ref = hidden.copy()
    for layer in range(2):
        wqkv, sqkv = gen.weights(rng, qkv_rows, H), gen.scales(rng, qkv_rows)
        wo, so = gen.weights(rng, H, QW), gen.scales(rng, H)
        wgu, sgu = gen.weights(rng, 2 * I, H), gen.scales(rng, 2 * I)
        wd, sd = gen.weights(rng, H, I), gen.scales(rng, H)
        hip.int8_gemv(dev(hip, wqkv), dev(hip, sqkv), dh, H, qkv_rows, 1, out16=qkv,
                      norm_weight=dg_in, mode=hip.MODE_EXACT)
        hip.int8_gemv(dev(hip, wo), dev(hip, so), qkv, QW, H, 1, out16=dh,
                      epilogue=hip.EPI_ADD_ROUNDED, mode=hip.MODE_EXACT)
        hip.int8_gemv(dev(hip, wgu), dev(hip, sgu), dh, H, I, 1, out16=act,
                      epilogue=hip.EPI_SILU_ROUNDED, norm_weight=dg_post, mode=hip.MODE_EXACT)
        hip.int8_gemv(dev(hip, wd), dev(hip, sd), act, I, H, 1, out16=dh,
                      epilogue=hip.EPI_ADD_ROUNDED, mode=hip.MODE_EXACT)

        q16 = orc.int8_gemm_rows(wqkv, sqkv, orc.rms_norm_rows(ref, g_in))[1]
        ref = orc.add_in_place(ref, orc.int8_gemm_rows(wo, so, q16[:, :QW])[1])
        xn = orc.rms_norm_rows(ref, g_post)
        a16 = orc.silu_gate(orc.int8_gemm_rows(wgu[:I], sgu[:I], xn)[1], orc.int8_gemm_rows(wgu[I:], sgu[I:], xn)[1])
        ref = orc.add_in_place(ref, orc.int8_gemm_rows(wd, sd, a16)[1])
        got = dh.numpy()
        assert np.array_equal(got, ref), f"layer {layer}: {np.count_nonzero(got != ref)} of {H} differ"
        assert np.array_equal(qkv.numpy(), q16)
        assert np.array_equal(act.numpy(), a16)


# MFMA mode (rows 2..8) at the production widths.  The launcher packs 1, 2 or
# 3 groups of 8 channels per block by width (talker gate/up 3, QKV 2, O and
# down 1; predictor QKV and gate/up 2), so these shapes run every group count
# with the norm prologue and the SiLU / residual epilogues.  The summation
# order is MFMA's: bf16 outputs within one bf16 rounding step (2^-7 of the
# value, the result of the sum rounding either way) plus ATOL of the oracle's
# exact-order result; fp32 outputs within the north-star bar 1e-2 + 1e-3|y|.
MFMA_SHAPES = [  # (kernel output width, in_features, epilogue, norm)
    (4096, 2048, "store", True), (2048, 2048, "add_fma", False), (6144, 2048, "silu_fused", True),
    (2048, 6144, "add_fma", False), (4096, 1024, "store", True), (1024, 2048, "add_fma", False),
    (3072, 1024, "silu_fused", True), (1024, 3072, "add_fma", False)]


@pytest.mark.parametrize("rows", [2, 8])
@pytest.mark.parametrize("out_f,in_f,epilogue,norm", MFMA_SHAPES)
def test_mfma_production_widths(hip, orc, rows, out_f, in_f, epilogue, norm):
    silu = epilogue.startswith("silu")
    rng = np.random.default_rng(out_f + 3 * in_f + rows)
    w_rows = 2 * out_f if silu else out_f
    w, s = gen.weights(rng, w_rows, in_f), gen.scales(rng, w_rows)
    x, g = gen.activations(rng, rows, in_f), gen.gains(rng, in_f)
    base = gen.activations(rng, rows, out_f)
    xn = orc.rms_norm_rows(x, g) if norm else x
    ref = oracle_epilogue(orc, epilogue, w, s, xn, base, None)
    y = dev(hip, base) if epilogue == "add_fma" else hip.DeviceArray((rows, out_f), np.uint16)
    y32 = hip.DeviceArray((rows, out_f), np.float32) if epilogue == "store" else None
    hip.int8_gemv(dev(hip, w), dev(hip, s), dev(hip, x), in_f, out_f, rows, out16=y, out32=y32,
                  epilogue=getattr(hip, "EPI_" + epilogue.upper()), norm_weight=dev(hip, g) if norm else None,
                  mode=hip.MODE_MFMA)
    got, want = gen.f32(y.numpy()), gen.f32(ref)
    assert np.all(np.abs(got - want) <= 1e-2 + 2.0 ** -7 * np.abs(want)), np.max(np.abs(got - want))
    if y32 is not None:
        ref32 = orc.int8_gemm_rows(w, s, xn)[0]
        err = np.abs(y32.numpy() - ref32)
        assert np.all(err <= 1e-2 + 1e-3 * np.abs(ref32)), err.max()
