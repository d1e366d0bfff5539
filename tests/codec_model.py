"""Synthetic speech-tokenizer decoder weights and an independent float64 model.

The float64 model restates the decoder from its module structure (the
PyTorch speech-tokenizer decoder whose tensors the reference loads by name,
native/qwen3-tts-native-codec/native/src/codec_state.cu:3281-3298): it runs a
WHOLE utterance at once, with zero left padding for the causal convolutions,
full transposed convolutions trimmed on the right, and a causal attention mask
limited to a 72-position window.  The streaming decoders (the C oracle and the
HIP library) carry the same computation across packets in histories, overlap
tails and a KV ring; agreeing with this model pins that state handling, the
layer order and the parameter semantics without sharing any code with them.
"""
from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

STRIDES = (8, 5, 4, 3)
STAGE_IN = (1536, 768, 384, 192)
STAGE_OUT = (768, 384, 192, 96)
DILATIONS = (1, 3, 9)
WINDOW = 72


def tensor_shapes():
    """Shapes of the 271 decoder tensors (PyTorch layouts): the 269 the
    decoder executes plus the two encoder-side RVQ input projections that a
    checkpoint carries and the loader counts but never reads."""
    s = {}
    q = "decoder.quantizer"
    s[f"{q}.rvq_first.vq.layers.0._codebook.embedding_sum"] = (2048, 256)
    s[f"{q}.rvq_first.vq.layers.0._codebook.cluster_usage"] = (2048,)
    for c in range(15):
        s[f"{q}.rvq_rest.vq.layers.{c}._codebook.embedding_sum"] = (2048, 256)
        s[f"{q}.rvq_rest.vq.layers.{c}._codebook.cluster_usage"] = (2048,)
    for part in ("rvq_first", "rvq_rest"):
        s[f"{q}.{part}.output_proj.weight"] = (512, 256, 1)
        s[f"{q}.{part}.input_proj.weight"] = (256, 512, 1)
    s["decoder.pre_conv.conv.weight"] = (1024, 512, 3)
    s["decoder.pre_conv.conv.bias"] = (1024,)
    t = "decoder.pre_transformer"
    s[f"{t}.input_proj.weight"] = (512, 1024)
    s[f"{t}.input_proj.bias"] = (512,)
    for l in range(8):
        p = f"{t}.layers.{l}"
        s[f"{p}.input_layernorm.weight"] = (512,)
        for n in ("q", "k", "v"):
            s[f"{p}.self_attn.{n}_proj.weight"] = (1024, 512)
        s[f"{p}.self_attn.o_proj.weight"] = (512, 1024)
        s[f"{p}.self_attn_layer_scale.scale"] = (512,)
        s[f"{p}.post_attention_layernorm.weight"] = (512,)
        s[f"{p}.mlp.gate_proj.weight"] = (1024, 512)
        s[f"{p}.mlp.up_proj.weight"] = (1024, 512)
        s[f"{p}.mlp.down_proj.weight"] = (512, 1024)
        s[f"{p}.mlp_layer_scale.scale"] = (512,)
    s[f"{t}.norm.weight"] = (512,)
    s[f"{t}.output_proj.weight"] = (1024, 512)
    s[f"{t}.output_proj.bias"] = (1024,)
    for u in range(2):
        p = f"decoder.upsample.{u}"
        s[f"{p}.0.conv.weight"] = (1024, 1024, 2)
        s[f"{p}.0.conv.bias"] = (1024,)
        s[f"{p}.1.dwconv.conv.weight"] = (1024, 1, 7)
        s[f"{p}.1.dwconv.conv.bias"] = (1024,)
        s[f"{p}.1.norm.weight"] = (1024,)
        s[f"{p}.1.norm.bias"] = (1024,)
        s[f"{p}.1.pwconv1.weight"] = (4096, 1024)
        s[f"{p}.1.pwconv1.bias"] = (4096,)
        s[f"{p}.1.pwconv2.weight"] = (1024, 4096)
        s[f"{p}.1.pwconv2.bias"] = (1024,)
        s[f"{p}.1.gamma"] = (1024,)
    s["decoder.decoder.0.conv.weight"] = (1536, 1024, 7)
    s["decoder.decoder.0.conv.bias"] = (1536,)
    for b in range(4):
        ci, co, st = STAGE_IN[b], STAGE_OUT[b], STRIDES[b]
        p = f"decoder.decoder.{b + 1}.block"
        s[f"{p}.0.alpha"] = (ci,)
        s[f"{p}.0.beta"] = (ci,)
        s[f"{p}.1.conv.weight"] = (ci, co, 2 * st)
        s[f"{p}.1.conv.bias"] = (co,)
        for u in range(3):
            r = f"{p}.{u + 2}"
            s[f"{r}.act1.alpha"] = (co,)
            s[f"{r}.act1.beta"] = (co,)
            s[f"{r}.conv1.conv.weight"] = (co, co, 7)
            s[f"{r}.conv1.conv.bias"] = (co,)
            s[f"{r}.act2.alpha"] = (co,)
            s[f"{r}.act2.beta"] = (co,)
            s[f"{r}.conv2.conv.weight"] = (co, co, 1)
            s[f"{r}.conv2.conv.bias"] = (co,)
    s["decoder.decoder.5.alpha"] = (96,)
    s["decoder.decoder.5.beta"] = (96,)
    s["decoder.decoder.6.conv.weight"] = (1, 96, 7)
    s["decoder.decoder.6.conv.bias"] = (1,)
    return s


TINY_USAGE_CODE = 7  # a codebook entry whose cluster usage sits below the 1e-5 clamp


def make_weights(seed=0):
    """fp32 weights with O(1) activations through every stage."""
    rng = np.random.default_rng(seed)
    w = {}

    def normal(shape, std):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    for name, shape in tensor_shapes().items():
        fan_in = int(np.prod(shape[1:])) if len(shape) > 1 else 1
        if name.endswith("embedding_sum"):
            usage_name = name.replace("embedding_sum", "cluster_usage")
            usage = rng.uniform(0.5, 2.0, shape[0]).astype(np.float32)
            usage[TINY_USAGE_CODE] = 1e-7
            w[usage_name] = usage
            emb = rng.standard_normal(shape) * usage[:, None]
            emb[TINY_USAGE_CODE] *= 1e-5 / 1e-7
            w[name] = emb.astype(np.float32)
        elif name.endswith("cluster_usage"):
            continue
        elif name.endswith("rvq_rest.output_proj.weight"):
            w[name] = normal(shape, 1.0 / math.sqrt(256 * 15))
        elif name.endswith(("alpha", "beta")):
            w[name] = normal(shape, 0.3)
        elif name.endswith(("layer_scale.scale", "gamma")):
            w[name] = rng.uniform(0.05, 0.2, shape).astype(np.float32)
        elif name.endswith(("layernorm.weight", "norm.weight")):
            w[name] = (1.0 + normal(shape, 0.1)).astype(np.float32)
        elif name.endswith("bias"):
            w[name] = normal(shape, 0.05)
        elif ".block.1.conv.weight" in name or name.startswith("decoder.upsample") and name.endswith("0.conv.weight"):
            # transposed convolutions [in][out][k]: each output sums 2 taps x in
            w[name] = normal(shape, 1.0 / math.sqrt(2 * shape[0]))
        elif name == "decoder.decoder.6.conv.weight":
            w[name] = normal(shape, 0.25 / math.sqrt(fan_in))
        elif ".conv1.conv.weight" in name or ".conv2.conv.weight" in name:
            w[name] = normal(shape, 0.5 / math.sqrt(fan_in))
        else:
            w[name] = normal(shape, 1.0 / math.sqrt(fan_in))
    return w


def random_codes(frames, seed=1):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 2048, (frames, 16), dtype=np.uint16)
    codes[::3, 0] = TINY_USAGE_CODE
    codes[1::4, 5] = TINY_USAGE_CODE
    return codes


# ---------------------------------------------------------------------------
class F64Decoder:
    """Whole-utterance float64 decoder.  Every method takes and returns
    [time][channels] arrays."""

    window = WINDOW
    layer_norm_eps = 1e-6
    rms_eps = 1e-5
    usage_floor = 1e-5

    def __init__(self, weights):
        self.w = {k: np.asarray(v, np.float64) for k, v in weights.items()}

    # -- building blocks ---------------------------------------------------
    def conv(self, x, weight, bias, dilation=1):
        """Causal Conv1d: weight [out][in][k], zero left padding (k-1)*d."""
        k = weight.shape[2]
        pad = (k - 1) * dilation
        xp = np.concatenate([np.zeros((pad, x.shape[1])), x])
        y = np.zeros((x.shape[0], weight.shape[0]))
        for j in range(k):
            y += xp[j * dilation: j * dilation + x.shape[0]] @ np.ascontiguousarray(weight[:, :, j].T)
        return y + (0.0 if bias is None else bias)

    def conv_transpose(self, x, weight, bias, stride):
        """ConvTranspose1d (weight [in][out][k]) trimmed to T * stride."""
        k = weight.shape[2]
        t = x.shape[0]
        y = np.zeros((t * stride + k - stride, weight.shape[1]))
        for j in range(k):
            y[j: j + stride * t: stride] += x @ np.ascontiguousarray(weight[:, :, j])
        return y[: t * stride] + bias

    def snake(self, x, alpha, beta):
        a, b = np.exp(alpha), np.exp(beta)
        return x + np.sin(x * a) ** 2 / (b + 1e-9)

    def rms_norm(self, x, weight):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.rms_eps) * weight

    def layer_norm(self, x, weight, bias):
        mean = x.mean(axis=-1, keepdims=True)
        var = ((x - mean) ** 2).mean(axis=-1, keepdims=True)
        return (x - mean) / np.sqrt(var + self.layer_norm_eps) * weight + bias

    def gelu(self, x):
        return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))

    def rope(self, x, positions):
        """rotate_half RoPE, base 10000, on [time][heads][64]."""
        inv = 1.0 / 10000.0 ** (np.arange(0, 64, 2) / 64.0)
        ang = positions[:, None] * inv[None, :]
        cos = np.concatenate([np.cos(ang)] * 2, axis=-1)[:, None, :]
        sin = np.concatenate([np.sin(ang)] * 2, axis=-1)[:, None, :]
        half = np.concatenate([-x[..., 32:], x[..., :32]], axis=-1)
        return x * cos + half * sin

    # -- stages ------------------------------------------------------------
    def rvq(self, codes):
        q = "decoder.quantizer"
        out = []
        for part, books in (("rvq_first", [0]), ("rvq_rest", range(1, 16))):
            acc = 0.0
            for j, cb in enumerate(books):
                p = f"{q}.{part}.vq.layers.{j}._codebook"
                emb = self.w[f"{p}.embedding_sum"] / np.maximum(self.w[f"{p}.cluster_usage"], self.usage_floor)[:, None]
                acc = acc + emb[codes[:, cb].astype(np.int64)]
            out.append(acc @ self.w[f"{q}.{part}.output_proj.weight"][:, :, 0].T)
        return out[0] + out[1]

    def preconv(self, rvq):
        return self.conv(rvq, self.w["decoder.pre_conv.conv.weight"], self.w["decoder.pre_conv.conv.bias"])

    def attention_mask(self, t):
        i = np.arange(t)[:, None]
        j = np.arange(t)[None, :]
        return (j <= i) & (j > i - self.window)

    def transformer(self, x):
        w = self.w
        t = "decoder.pre_transformer"
        h = x @ w[f"{t}.input_proj.weight"].T + w[f"{t}.input_proj.bias"]
        n = h.shape[0]
        pos = np.arange(n, dtype=np.float64)
        mask = self.attention_mask(n)
        for l in range(8):
            p = f"{t}.layers.{l}"
            a = self.rms_norm(h, w[f"{p}.input_layernorm.weight"])
            q = (a @ w[f"{p}.self_attn.q_proj.weight"].T).reshape(n, 16, 64)
            k = (a @ w[f"{p}.self_attn.k_proj.weight"].T).reshape(n, 16, 64)
            v = (a @ w[f"{p}.self_attn.v_proj.weight"].T).reshape(n, 16, 64)
            q, k = self.rope(q, pos), self.rope(k, pos)
            scores = np.einsum("ihd,jhd->hij", q, k) / 8.0
            scores = np.where(mask[None], scores, -np.inf)
            scores = np.exp(scores - scores.max(axis=-1, keepdims=True))
            probs = scores / scores.sum(axis=-1, keepdims=True)
            att = np.einsum("hij,jhd->ihd", probs, v).reshape(n, 1024)
            h = h + (att @ w[f"{p}.self_attn.o_proj.weight"].T) * w[f"{p}.self_attn_layer_scale.scale"]
            m = self.rms_norm(h, w[f"{p}.post_attention_layernorm.weight"])
            g = m @ w[f"{p}.mlp.gate_proj.weight"].T
            u = m @ w[f"{p}.mlp.up_proj.weight"].T
            act = g / (1.0 + np.exp(-g)) * u
            h = h + (act @ w[f"{p}.mlp.down_proj.weight"].T) * w[f"{p}.mlp_layer_scale.scale"]
        h = self.rms_norm(h, w[f"{t}.norm.weight"])
        return h @ w[f"{t}.output_proj.weight"].T + w[f"{t}.output_proj.bias"]

    def upsample(self, x, stage):
        w = self.w
        p = f"decoder.upsample.{stage}"
        y = self.conv_transpose(x, w[f"{p}.0.conv.weight"], w[f"{p}.0.conv.bias"], 2)
        d = w[f"{p}.1.dwconv.conv.weight"]  # [C][1][7], depthwise
        yp = np.concatenate([np.zeros((6, y.shape[1])), y])
        z = sum(yp[j: j + y.shape[0]] * d[:, 0, j] for j in range(7)) + w[f"{p}.1.dwconv.conv.bias"]
        z = self.layer_norm(z, w[f"{p}.1.norm.weight"], w[f"{p}.1.norm.bias"])
        z = self.gelu(z @ w[f"{p}.1.pwconv1.weight"].T + w[f"{p}.1.pwconv1.bias"])
        z = z @ w[f"{p}.1.pwconv2.weight"].T + w[f"{p}.1.pwconv2.bias"]
        return y + z * w[f"{p}.1.gamma"]

    def residual_unit(self, x, prefix, dilation):
        w = self.w
        y = self.snake(x, w[f"{prefix}.act1.alpha"], w[f"{prefix}.act1.beta"])
        y = self.conv(y, w[f"{prefix}.conv1.conv.weight"], w[f"{prefix}.conv1.conv.bias"], dilation)
        y = self.snake(y, w[f"{prefix}.act2.alpha"], w[f"{prefix}.act2.beta"])
        y = self.conv(y, w[f"{prefix}.conv2.conv.weight"], w[f"{prefix}.conv2.conv.bias"])
        return x + y

    def stage(self, x, b):
        w = self.w
        p = f"decoder.decoder.{b + 1}.block"
        y = self.snake(x, w[f"{p}.0.alpha"], w[f"{p}.0.beta"])
        y = self.conv_transpose(y, w[f"{p}.1.conv.weight"], w[f"{p}.1.conv.bias"], STRIDES[b])
        for u in range(3):
            y = self.residual_unit(y, f"{p}.{u + 2}", DILATIONS[u])
        return y

    def run(self, codes):
        """All stage outputs of one utterance of codes [frames][16]."""
        w = self.w
        out = {}
        out["rvq"] = self.rvq(codes)
        out["preconv"] = self.preconv(out["rvq"])
        out["transformer"] = self.transformer(out["preconv"])
        out["latent1"] = self.upsample(out["transformer"], 0)
        out["latent2"] = self.upsample(out["latent1"], 1)
        x = self.conv(out["latent2"], w["decoder.decoder.0.conv.weight"], w["decoder.decoder.0.conv.bias"])
        out[6] = x
        for b in range(4):
            x = self.stage(x, b)
            out[7 + b] = x
        x = self.snake(x, w["decoder.decoder.5.alpha"], w["decoder.decoder.5.beta"])
        out[11] = x
        x = self.conv(x, w["decoder.decoder.6.conv.weight"], w["decoder.decoder.6.conv.bias"])
        out[12] = x
        out[13] = np.clip(x, -1.0, 1.0)
        out["pcm"] = np.clip(np.round(out[13][:, 0] * 32767.0), -32768, 32767).astype(np.int16)
        return out

    def run_transformer(self, codes):
        return self.transformer(self.preconv(self.rvq(codes)))


# ---- structural mutants: each is a plausible mistake the check must catch --
class SwappedTransposeTaps(F64Decoder):
    def conv_transpose(self, x, weight, bias, stride):
        k = weight.shape[2]
        flipped = np.concatenate([weight[:, :, stride:], weight[:, :, :stride]], axis=2) if k == 2 * stride else weight
        return super().conv_transpose(x, flipped, bias, stride)


class NoDilation(F64Decoder):
    def conv(self, x, weight, bias, dilation=1):
        return super().conv(x, weight, bias, 1)


class InterleavedRope(F64Decoder):
    def rope(self, x, positions):
        inv = 1.0 / 10000.0 ** (np.arange(0, 64, 2) / 64.0)
        ang = positions[:, None] * inv[None, :]
        cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        even, odd = x[..., 0::2], x[..., 1::2]
        out = np.empty_like(x)
        out[..., 0::2] = even * cos - odd * sin
        out[..., 1::2] = odd * cos + even * sin
        return out


class Window71(F64Decoder):
    window = 71


class LinearSnake(F64Decoder):
    def snake(self, x, alpha, beta):
        return x + np.sin(x * alpha) ** 2 / (beta + 1e-9)


class RmsInConvNext(F64Decoder):
    """ConvNeXt normalised like the transformer (no mean removal)."""

    def layer_norm(self, x, weight, bias):
        return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.layer_norm_eps) * weight + bias


class NoUsageClamp(F64Decoder):
    usage_floor = 0.0
