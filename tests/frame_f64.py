"""An independent float64 NumPy model of the reference's talker + code
predictor frame, used to pin the oracle's layer and frame sequence.

TEST INFRASTRUCTURE ONLY.  It is written from the reference's CUDA sources,
not from oracle/oracle.c, with whole-vector float64 arithmetic (matrix
products, vectorised norms and softmax) instead of the reference's fp32
accumulation orders.  Values are rounded to bf16 only where the reference
stores a bf16 tensor, so the model agrees with the oracle up to the rounding
differences of the accumulation order, while any difference in *structure* --
the order of the layer's operations, residual placement, which hidden state
seeds predictor position 0, which embedding table and LM head a codebook
uses, the RoPE positions, the text projection, the sampler's mask and
repetition penalty -- shows as an error far above that level.

Sources restated (K = native/qwen3-tts-native/native/src):
  decoder layer, single session     K/talker.cu:3251-3456
  decoder layer, lockstep batch row K/talker.cu:2038-2334 (fused gate/up SiLU
                                    K/int8_gemv.cu:206-293, residual GEMM
                                    K/int8_gemv.cu:132-199, fast attention
                                    K/talker_kernels.cu:506-595)
  RMSNorm, head RMSNorm, RoPE       K/talker_kernels.cu:27-114
  exact attention                   K/talker_kernels.cu:287-357
  add / bias / SiLU-gate            K/talker_kernels.cu:359-421
  talker step + codec head          K/talker.cu:3458-3495
  predictor position                K/talker.cu:3497-3544
  generated embedding               K/talker.cu:3546-3581
  text projection                   K/talker.cu:2676-2719
  prompt embedding                  K/talker.cu:2721-2748
  frame sequence                    K/talker.cu:1095-1244
  sampler mask and penalty          K/sampling_kernels.cu:30-51
  quantizer (absmax / 127)          K/int8_gemv.cu:20-52
  bf16 prefill (bf16 weights, GEMM  K/talker.cu:2750-3249,
  attention, causal softmax)        K/talker_kernels.cu:115-191,232-260
"""
from __future__ import annotations

import numpy as np

CODEBOOKS = 16


def bf(x):
    """Round float64 values to bf16 (returned as float64)."""
    a = np.asarray(x, dtype=np.float64).astype(np.float32)
    u = a.reshape(-1).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).reshape(a.shape).astype(np.float64)


def from_bits(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dequantize(w_bits):
    """Per-row absmax int8 quantization of a bf16 matrix, returned as the
    float64 matrix q * s it stands for."""
    w = from_bits(w_bits).astype(np.float32)
    amax = np.max(np.abs(w), axis=1)
    s = np.where(amax > 0, amax / np.float32(127.0), np.float32(1.0)).astype(np.float32)
    q = np.clip(np.rint(w * (np.float32(1.0) / s)[:, None]), -127, 127)
    return q.astype(np.float64) * s.astype(np.float64)[:, None]


def silu(x):
    return x / (1.0 + np.exp(-x))


class Dims:
    def __init__(self, c, part):
        self.hidden = c[f"{part}_hidden"]
        self.intermediate = c[f"{part}_intermediate"]
        self.qh = c[f"{part}_query_heads"]
        self.kvh = c[f"{part}_key_value_heads"]
        self.d = c["head_dimension"]
        self.layers = c[f"{part}_layers"]


class F64Model:
    def __init__(self, c: dict, weights: dict, batch_semantics: bool = False):
        self.c, self.batch = c, batch_semantics
        self.eps, self.theta = c["rms_epsilon"], c["rope_theta"]
        self.eos = c["codec_eos_token"]
        self.pv = c["predictor_vocabulary"]
        g = lambda n: from_bits(weights[n])  # noqa: E731
        self.talker = Dims(c, "talker")
        self.predictor = Dims(c, "predictor")
        self.layers = {}
        for part, prefix in (("talker", "talker.model.layers"), ("predictor", "talker.code_predictor.model.layers")):
            out = []
            for l in range(c[f"{part}_layers"]):
                p = f"{prefix}.{l}."
                out.append(dict(
                    in_norm=g(p + "input_layernorm.weight"), post_norm=g(p + "post_attention_layernorm.weight"),
                    q_norm=g(p + "self_attn.q_norm.weight"), k_norm=g(p + "self_attn.k_norm.weight"),
                    q=dequantize(weights[p + "self_attn.q_proj.weight"]),
                    k=dequantize(weights[p + "self_attn.k_proj.weight"]),
                    v=dequantize(weights[p + "self_attn.v_proj.weight"]),
                    o=dequantize(weights[p + "self_attn.o_proj.weight"]),
                    gate=dequantize(weights[p + "mlp.gate_proj.weight"]),
                    up=dequantize(weights[p + "mlp.up_proj.weight"]),
                    down=dequantize(weights[p + "mlp.down_proj.weight"]),
                    w16={n: from_bits(weights[p + n + ".weight"]) for n in (
                        "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                        "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj")}))
            self.layers[part] = out
        self.codec_embedding = g("talker.model.codec_embedding.weight")
        self.text_embedding = g("talker.model.text_embedding.weight")
        self.fc1 = dequantize(weights["talker.text_projection.linear_fc1.weight"])
        self.fc1_b = g("talker.text_projection.linear_fc1.bias")
        self.fc2 = dequantize(weights["talker.text_projection.linear_fc2.weight"])
        self.fc2_b = g("talker.text_projection.linear_fc2.bias")
        self.talker_norm = g("talker.model.norm.weight")
        self.codec_head = dequantize(weights["talker.codec_head.weight"])
        self.codec_head16 = from_bits(weights["talker.codec_head.weight"])
        self.s2m = dequantize(weights["talker.code_predictor.small_to_mtp_projection.weight"])
        self.s2m_b = g("talker.code_predictor.small_to_mtp_projection.bias")
        self.predictor_norm = g("talker.code_predictor.model.norm.weight")
        self.pred_emb = [g(f"talker.code_predictor.model.codec_embedding.{i}.weight") for i in range(15)]
        self.heads = [dequantize(weights[f"talker.code_predictor.lm_head.{i}.weight"]) for i in range(15)]

    # -- primitives -------------------------------------------------------
    def rms_norm(self, x, gain):
        inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.eps)
        return bf(bf(x * inv) * gain)

    def rope(self, x, position, d):
        """x: [heads, d]; rotate-half pairs (i, i + d/2) with bf16 cos/sin
        and a bf16 rounding of each product (talker_kernels.cu:72-114)."""
        half = d // 2
        angle = position * self.theta ** (-(2.0 * np.arange(half)) / d)
        cos, sin = bf(np.cos(angle)), bf(np.sin(angle))
        a, b = x[:, :half], x[:, half:]
        return np.concatenate([bf(bf(a * cos) - bf(b * sin)), bf(bf(b * cos) + bf(a * sin))], axis=1)

    def attention(self, q, keys, values, dims):
        """q [qh, d]; keys/values [length, kvh, d]."""
        group = dims.qh // dims.kvh
        out = np.empty_like(q)
        for h in range(dims.qh):
            k = keys[:, h // group, :]
            v = values[:, h // group, :]
            if self.batch:
                scores = (k @ q[h]) / np.sqrt(dims.d)
                p = np.exp(scores - scores.max())
                out[h] = bf((p @ v) / p.sum())
            else:
                scores = bf(bf(k @ q[h]) / np.sqrt(dims.d))
                p = np.exp(scores - scores.max())
                p = bf(p / p.sum())
                out[h] = bf(p @ v)
        return out

    # -- decoder ----------------------------------------------------------
    def decoder(self, part, h, cache, position):
        dims = getattr(self, part)
        for l, L in enumerate(self.layers[part]):
            x = self.rms_norm(h, L["in_norm"])
            q = bf(L["q"] @ x).reshape(dims.qh, dims.d)
            k = bf(L["k"] @ x).reshape(dims.kvh, dims.d)
            v = bf(L["v"] @ x).reshape(dims.kvh, dims.d)
            q = self.rope(self.rms_norm(q, L["q_norm"]), position, dims.d)
            k = self.rope(self.rms_norm(k, L["k_norm"]), position, dims.d)
            cache["k"][l][position] = k
            cache["v"][l][position] = v
            a = self.attention(q, cache["k"][l][:position + 1], cache["v"][l][:position + 1], dims).reshape(-1)
            if self.batch:
                h = bf(h + L["o"] @ a)
                x = self.rms_norm(h, L["post_norm"])
                act = bf(silu(L["gate"] @ x) * (L["up"] @ x))
                h = bf(h + L["down"] @ act)
            else:
                h = bf(h + bf(L["o"] @ a))
                x = self.rms_norm(h, L["post_norm"])
                act = bf(bf(silu(bf(L["gate"] @ x))) * bf(L["up"] @ x))
                h = bf(h + bf(L["down"] @ act))
        return h

    def new_cache(self, part, rows):
        dims = getattr(self, part)
        shape = (dims.layers, rows, dims.kvh, dims.d)
        return {"k": np.zeros(shape), "v": np.zeros(shape)}

    def project_text(self, token):
        t = bf(self.fc1 @ self.text_embedding[token])
        t = bf(silu(t + self.fc1_b))
        return bf(bf(self.fc2 @ t) + self.fc2_b)

    def talker_step(self, state, x):
        """One talker position: returns (final normalized hidden, logits)."""
        h = self.decoder("talker", x, state["talker"], state["position"])
        last = self.rms_norm(h, self.talker_norm)
        state["last_hidden"] = last
        state["position"] += 1
        return last, bf(self.codec_head @ last)

    def predictor_position(self, state, x, position, head):
        h = bf(bf(self.s2m @ x) + self.s2m_b)
        h = self.decoder("predictor", h, state["predictor"], position)
        if head < 0:
            return None
        return bf(self.heads[head] @ self.rms_norm(h, self.predictor_norm))

    def talker_scores(self, logits, history, penalty):
        """Greedy score of every talker token: reserved ids >= the predictor
        vocabulary (except EOS) masked, repetition penalty over history."""
        s = logits.copy()
        mask = np.arange(len(s)) >= self.pv
        mask[self.eos] = False
        s[mask] = -np.inf
        if penalty != 1.0 and len(history):
            idx = np.unique(np.asarray(history))
            s[idx] = np.where(s[idx] < 0, s[idx] * penalty, s[idx] / penalty)
        return s

    # -- session ----------------------------------------------------------
    def new_session(self, max_seq):
        return {"talker": self.new_cache("talker", max_seq), "predictor": self.new_cache("predictor", CODEBOOKS),
                "position": 0, "history": [], "last_hidden": None}

    def prompt_embedding(self, text_token, codec_token):
        x = self.project_text(text_token) if text_token >= 0 else np.zeros(self.talker.hidden)
        if codec_token >= 0:
            x = bf(x + self.codec_embedding[codec_token])
        return x

    def frame_logits(self, state, codes, trailing_text):
        """Runs one frame with the given 16 codes (teacher forcing) and
        returns the 15 predictor logit vectors (codebooks 1..15, each
        computed before its token is known) and the talker's logits."""
        pred_logits = []
        self.predictor_position(state, state["last_hidden"], 0, -1)
        x = self.codec_embedding[codes[0]]
        pred_logits.append(self.predictor_position(state, x, 1, 0))
        for r in range(1, CODEBOOKS - 1):
            x = self.pred_emb[r - 1][codes[r]]
            pred_logits.append(self.predictor_position(state, x, r + 1, r))
        x = self.codec_embedding[codes[0]]
        for r in range(CODEBOOKS - 1):
            x = bf(x + self.pred_emb[r][codes[r + 1]])
        x = bf(x + self.project_text(trailing_text))
        _, logits = self.talker_step(state, x)
        return pred_logits, logits

    # -- bf16 prefill -----------------------------------------------------
    def score_scale(self, d):
        return 1.0 / np.sqrt(d)

    def prefill_bf16(self, state, text, codec, gemm_capacity):
        """The reference's prompt prefill: bf16 weights, every product a
        GEMM rounded to bf16; attention by materialized scores and the causal
        softmax when the prompt fits gemm_capacity, else the exact per-row
        kernel.  Returns the logits; fills the talker caches and last hidden."""
        dims = self.talker
        rows = len(text)
        h = np.stack([self.prompt_embedding(int(t), int(c)) for t, c in zip(text, codec)])
        scale = self.score_scale(dims.d)
        group = dims.qh // dims.kvh
        for l, L in enumerate(self.layers["talker"]):
            w = L["w16"]
            x = self.rms_norm(h, L["in_norm"])
            q = bf(x @ w["self_attn.q_proj"].T).reshape(rows, dims.qh, dims.d)
            k = bf(x @ w["self_attn.k_proj"].T).reshape(rows, dims.kvh, dims.d)
            v = bf(x @ w["self_attn.v_proj"].T).reshape(rows, dims.kvh, dims.d)
            q = self.rms_norm(q, L["q_norm"])
            k = self.rms_norm(k, L["k_norm"])
            q = np.stack([self.rope(q[r], r, dims.d) for r in range(rows)])
            k = np.stack([self.rope(k[r], r, dims.d) for r in range(rows)])
            state["talker"]["k"][l][:rows] = k
            state["talker"]["v"][l][:rows] = v
            attn = np.empty((rows, dims.qh, dims.d))
            if rows <= gemm_capacity:
                causal = np.tril(np.ones((rows, rows), bool))
                for hh in range(dims.qh):
                    s = bf(bf(q[:, hh] @ k[:, hh // group].T) * scale)
                    s = np.where(causal, s, -np.inf)
                    e = np.exp(s - s.max(axis=1, keepdims=True))
                    p = bf(e / e.sum(axis=1, keepdims=True))
                    attn[:, hh] = bf(p @ v[:, hh // group])
            else:
                for r in range(rows):
                    attn[r] = self.attention(q[r], k[:r + 1], v[:r + 1], dims)
            h = bf(h + bf(attn.reshape(rows, -1) @ w["self_attn.o_proj"].T))
            x = self.rms_norm(h, L["post_norm"])
            act = bf(bf(silu(bf(x @ w["mlp.gate_proj"].T))) * bf(x @ w["mlp.up_proj"].T))
            h = bf(h + bf(act @ w["mlp.down_proj"].T))
        last = self.rms_norm(h[-1], self.talker_norm)
        state["last_hidden"] = last
        state["position"] = rows
        return bf(self.codec_head16 @ last)
