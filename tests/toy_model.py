"""A reduced-geometry VoiceDesign checkpoint for end-to-end tests.

Tensor names and shapes follow the reference's contract
(native/qwen3-tts-native/native/src/talker.cu:488-562,693-747) with smaller
dimensions.  The same bf16 weights are uploaded to the HIP library through the
reference C ABI and quantized on the host by the oracle's quantizer (which the
GPU quantizer matches bit-for-bit), then wired into the oracle's model
structs, so a frame on the GPU and a frame in the oracle start from identical
state.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

import gen

TOY = dict(talker_layers=2, talker_hidden=512, talker_intermediate=1024, talker_query_heads=4,
           talker_key_value_heads=2, predictor_layers=2, predictor_hidden=256,
           predictor_intermediate=512, predictor_query_heads=4, predictor_key_value_heads=2,
           head_dimension=128, talker_vocabulary=3072, predictor_vocabulary=2048,
           text_vocabulary=1000, codec_eos_token=2150, rms_epsilon=1e-6, rope_theta=1e6)

# The same, with the production predictor's head geometry (16 query / 8 kv
# heads).
TOY_WIDE_PREDICTOR = dict(TOY, predictor_query_heads=16, predictor_key_value_heads=8)


def tensor_specs(c: dict):
    """(name, shape, kind) for every tensor of the checkpoint."""
    H = c["talker_hidden"]
    specs = [("talker.model.codec_embedding.weight", (c["talker_vocabulary"], H), "emb"),
             ("talker.model.text_embedding.weight", (c["text_vocabulary"], H), "emb"),
             ("talker.text_projection.linear_fc1.weight", (H, H), "w"),
             ("talker.text_projection.linear_fc1.bias", (H,), "b"),
             ("talker.text_projection.linear_fc2.weight", (H, H), "w"),
             ("talker.text_projection.linear_fc2.bias", (H,), "b"),
             ("talker.model.norm.weight", (H,), "g"),
             ("talker.codec_head.weight", (c["talker_vocabulary"], H), "w"),
             ("talker.code_predictor.small_to_mtp_projection.weight", (c["predictor_hidden"], H), "w"),
             ("talker.code_predictor.small_to_mtp_projection.bias", (c["predictor_hidden"],), "b"),
             ("talker.code_predictor.model.norm.weight", (c["predictor_hidden"],), "g")]
    for part, prefix in (("talker", "talker.model.layers"), ("predictor", "talker.code_predictor.model.layers")):
        h, i = c[f"{part}_hidden"], c[f"{part}_intermediate"]
        qw = c[f"{part}_query_heads"] * c["head_dimension"]
        kw = c[f"{part}_key_value_heads"] * c["head_dimension"]
        d = c["head_dimension"]
        for l in range(c[f"{part}_layers"]):
            p = f"{prefix}.{l}"
            specs += [(f"{p}.input_layernorm.weight", (h,), "g"), (f"{p}.self_attn.q_proj.weight", (qw, h), "w"),
                      (f"{p}.self_attn.k_proj.weight", (kw, h), "w"), (f"{p}.self_attn.v_proj.weight", (kw, h), "w"),
                      (f"{p}.self_attn.o_proj.weight", (h, qw), "w"), (f"{p}.self_attn.q_norm.weight", (d,), "g"),
                      (f"{p}.self_attn.k_norm.weight", (d,), "g"),
                      (f"{p}.post_attention_layernorm.weight", (h,), "g"),
                      (f"{p}.mlp.gate_proj.weight", (i, h), "w"), (f"{p}.mlp.up_proj.weight", (i, h), "w"),
                      (f"{p}.mlp.down_proj.weight", (h, i), "w")]
    for g in range(15):
        specs += [(f"talker.code_predictor.model.codec_embedding.{g}.weight", (c["predictor_vocabulary"], H), "emb"),
                  (f"talker.code_predictor.lm_head.{g}.weight", (c["predictor_vocabulary"], c["predictor_hidden"]), "w")]
    return specs


def make_weights(c: dict, seed: int = 0, weight_std: float = 0.05):
    rng = np.random.default_rng(seed)
    out = {}
    for name, shape, kind in tensor_specs(c):
        if kind == "g":
            x = 1.0 + 0.1 * rng.standard_normal(shape)
        elif kind == "b":
            x = 0.02 * rng.standard_normal(shape)
        elif kind == "emb":
            x = rng.standard_normal(shape)
        else:
            x = weight_std * rng.standard_normal(shape)
        out[name] = gen.bf16(x.astype(np.float32))
    return out


def config_struct(hip, c: dict):
    s = hip.ModelConfigV1()
    s.struct_size = C.sizeof(hip.ModelConfigV1)
    for k, v in c.items():
        setattr(s, k, v)
    return s


def upload(hip, c: dict, weights: dict, device: int = 0):
    """Create + upload + finalize through the C ABI; returns the model handle."""
    model = C.c_void_p()
    hip.call("qwen3_tts_model_create_with_config", device, C.byref(config_struct(hip, c)), C.byref(model))
    for name, arr in weights.items():
        shape = (C.c_uint64 * arr.ndim)(*arr.shape)
        hip.call("qwen3_tts_model_upload_tensor", model, name.encode(), arr.ctypes.data, arr.nbytes, arr.ndim, shape)
    mem = hip.ModelMemory()
    hip.call("qwen3_tts_model_finalize", model, C.byref(mem))
    return model, mem


# ---------------------------------------------------------------------------
# oracle model structs (oracle/oracle.h)
# ---------------------------------------------------------------------------
class OrcDims(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("hidden", "intermediate", "query_heads", "key_value_heads",
                                        "head_dimension", "layers")]


class OrcLayer(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in ("input_norm", "q_norm", "k_norm", "post_norm", "q", "k", "v", "o",
                                           "gate_up", "down", "q_s", "k_s", "v_s", "o_s", "gate_up_s", "down_s",
                                           "q16", "k16", "v16", "o16", "gate16", "up16", "down16")]


class OrcModel(C.Structure):
    _fields_ = [("talker", OrcDims), ("predictor", OrcDims), ("talker_vocab", C.c_int),
                ("predictor_vocab", C.c_int), ("text_vocab", C.c_int), ("codebooks", C.c_int),
                ("codec_eos", C.c_int), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
                ("talker_layers", C.c_void_p), ("predictor_layers", C.c_void_p),
                ("codec_embedding", C.c_void_p), ("text_embedding", C.c_void_p),
                ("text_fc1", C.c_void_p), ("text_fc2", C.c_void_p), ("text_fc1_s", C.c_void_p),
                ("text_fc2_s", C.c_void_p), ("text_fc1_bias", C.c_void_p), ("text_fc2_bias", C.c_void_p),
                ("talker_norm", C.c_void_p), ("codec_head", C.c_void_p), ("codec_head_s", C.c_void_p),
                ("small_to_mtp", C.c_void_p), ("small_to_mtp_s", C.c_void_p),
                ("small_to_mtp_bias", C.c_void_p), ("predictor_norm", C.c_void_p),
                ("predictor_embeddings", C.c_void_p), ("predictor_heads", C.c_void_p),
                ("predictor_heads_s", C.c_void_p), ("batch_semantics", C.c_int), ("codec_head16", C.c_void_p)]


class OrcSession(C.Structure):
    _fields_ = [("max_seq", C.c_int), ("position", C.c_int), ("history_count", C.c_int),
                ("history", C.c_void_p), ("random_state", C.c_uint64), ("talker_k", C.c_void_p),
                ("talker_v", C.c_void_p), ("pred_k", C.c_void_p), ("pred_v", C.c_void_p),
                ("last_hidden", C.c_void_p), ("logits", C.c_void_p), ("trace_logits", C.c_void_p)]


class OrcSampling(C.Structure):
    _fields_ = [("do_sample", C.c_int), ("top_k", C.c_int), ("top_p", C.c_float),
                ("temperature", C.c_float), ("repetition_penalty", C.c_float)]


def _ptr(a):
    return a.ctypes.data


class OracleModel:
    """Host-side int8 model for the oracle (keeps every buffer alive)."""

    def __init__(self, orc, c: dict, weights: dict, batch_semantics: bool = False):
        self.orc, self.c, self.keep = orc, c, []
        q = {}

        def quant(*names):
            w = np.concatenate([weights[n] for n in names], axis=0)
            qq, ss = orc.quantize_weight_rows(w)
            self.keep += [qq, ss]
            return qq, ss

        def layers(part, prefix):
            arr = (OrcLayer * c[f"{part}_layers"])()
            for l in range(c[f"{part}_layers"]):
                p = f"{prefix}.{l}"
                L = arr[l]
                L.input_norm = _ptr(weights[f"{p}.input_layernorm.weight"])
                L.post_norm = _ptr(weights[f"{p}.post_attention_layernorm.weight"])
                L.q_norm = _ptr(weights[f"{p}.self_attn.q_norm.weight"])
                L.k_norm = _ptr(weights[f"{p}.self_attn.k_norm.weight"])
                for fld, names in (("q", ["self_attn.q_proj"]), ("k", ["self_attn.k_proj"]),
                                   ("v", ["self_attn.v_proj"]), ("o", ["self_attn.o_proj"]),
                                   ("gate_up", ["mlp.gate_proj", "mlp.up_proj"]), ("down", ["mlp.down_proj"])):
                    qq, ss = quant(*[f"{p}.{n}.weight" for n in names])
                    setattr(L, fld, _ptr(qq))
                    setattr(L, fld + "_s", _ptr(ss))
                for fld, name in (("q16", "self_attn.q_proj"), ("k16", "self_attn.k_proj"), ("v16", "self_attn.v_proj"),
                                  ("o16", "self_attn.o_proj"), ("gate16", "mlp.gate_proj"), ("up16", "mlp.up_proj"),
                                  ("down16", "mlp.down_proj")):
                    setattr(L, fld, _ptr(weights[f"{p}.{name}.weight"]))
            self.keep.append(arr)
            return arr

        m = OrcModel()
        for part in ("talker", "predictor"):
            d = getattr(m, part)
            d.hidden, d.intermediate = c[f"{part}_hidden"], c[f"{part}_intermediate"]
            d.query_heads, d.key_value_heads = c[f"{part}_query_heads"], c[f"{part}_key_value_heads"]
            d.head_dimension, d.layers = c["head_dimension"], c[f"{part}_layers"]
        m.talker_vocab, m.predictor_vocab = c["talker_vocabulary"], c["predictor_vocabulary"]
        m.text_vocab, m.codebooks, m.codec_eos = c["text_vocabulary"], 16, c["codec_eos_token"]
        m.rms_eps, m.rope_theta = c["rms_epsilon"], c["rope_theta"]
        tl = layers("talker", "talker.model.layers")
        pl = layers("predictor", "talker.code_predictor.model.layers")
        m.talker_layers, m.predictor_layers = C.addressof(tl), C.addressof(pl)
        m.codec_embedding = _ptr(weights["talker.model.codec_embedding.weight"])
        m.text_embedding = _ptr(weights["talker.model.text_embedding.weight"])
        for fld, name in (("text_fc1", "talker.text_projection.linear_fc1.weight"),
                          ("text_fc2", "talker.text_projection.linear_fc2.weight"),
                          ("codec_head", "talker.codec_head.weight"),
                          ("small_to_mtp", "talker.code_predictor.small_to_mtp_projection.weight")):
            qq, ss = quant(name)
            setattr(m, fld, _ptr(qq))
            setattr(m, fld + "_s", _ptr(ss))
        m.text_fc1_bias = _ptr(weights["talker.text_projection.linear_fc1.bias"])
        m.text_fc2_bias = _ptr(weights["talker.text_projection.linear_fc2.bias"])
        m.talker_norm = _ptr(weights["talker.model.norm.weight"])
        m.small_to_mtp_bias = _ptr(weights["talker.code_predictor.small_to_mtp_projection.bias"])
        m.predictor_norm = _ptr(weights["talker.code_predictor.model.norm.weight"])
        embs = (C.c_void_p * 15)(*[_ptr(weights[f"talker.code_predictor.model.codec_embedding.{g}.weight"])
                                   for g in range(15)])
        heads, heads_s = (C.c_void_p * 15)(), (C.c_void_p * 15)()
        for g in range(15):
            qq, ss = quant(f"talker.code_predictor.lm_head.{g}.weight")
            heads[g], heads_s[g] = _ptr(qq), _ptr(ss)
        self.keep += [embs, heads, heads_s, weights]
        m.predictor_embeddings, m.predictor_heads, m.predictor_heads_s = (
            C.addressof(embs), C.addressof(heads), C.addressof(heads_s))
        m.batch_semantics = int(batch_semantics)
        m.codec_head16 = _ptr(weights["talker.codec_head.weight"])
        self.model = m
        lib = orc.lib()
        lib.orc_frame_step.restype = C.c_int
        lib.orc_prefill.restype = C.c_int


class OracleSession:
    def __init__(self, om: OracleModel, max_seq: int, seed: int):
        c = om.c
        self.om, self.lib = om, om.orc.lib()
        tkv = c["talker_key_value_heads"] * c["head_dimension"]
        pkv = c["predictor_key_value_heads"] * c["head_dimension"]
        self.bufs = dict(
            history=np.zeros(max_seq, np.int32),
            tk=np.zeros(c["talker_layers"] * max_seq * tkv, np.uint16),
            tv=np.zeros(c["talker_layers"] * max_seq * tkv, np.uint16),
            pk=np.zeros(c["predictor_layers"] * 16 * pkv, np.uint16),
            pv=np.zeros(c["predictor_layers"] * 16 * pkv, np.uint16),
            last=np.zeros(c["talker_hidden"], np.uint16),
            logits=np.zeros(max(c["talker_vocabulary"], c["predictor_vocabulary"]), np.uint16),
            trace=np.zeros((16, max(c["talker_vocabulary"], c["predictor_vocabulary"])), np.uint16))
        s = OrcSession()
        s.max_seq, s.position, s.history_count = max_seq, 0, 0
        s.random_state = seed if seed != 0 else 0x9E3779B97F4A7C15
        b = self.bufs
        s.history, s.talker_k, s.talker_v = _ptr(b["history"]), _ptr(b["tk"]), _ptr(b["tv"])
        s.pred_k, s.pred_v, s.last_hidden, s.logits = _ptr(b["pk"]), _ptr(b["pv"]), _ptr(b["last"]), _ptr(b["logits"])
        s.trace_logits = _ptr(b["trace"])
        self.s = s

    def prefill(self, text, codec, sampling):
        """Prefill as consecutive int8 decode steps (the library's decode-step
        prefill mode)."""
        t = np.ascontiguousarray(text, np.int32)
        cd = np.ascontiguousarray(codec, np.int32)
        return self.lib.orc_prefill(C.byref(self.om.model), C.byref(self.s), t.ctypes.data_as(C.c_void_p),
                                    cd.ctypes.data_as(C.c_void_p), len(t), C.byref(OrcSampling(*sampling)))

    def prefill_bf16(self, text, codec, sampling):
        """The reference's bf16 prefill (GEMM attention up to
        min(max_seq, 512) positions, the exact kernel beyond)."""
        t = np.ascontiguousarray(text, np.int32)
        cd = np.ascontiguousarray(codec, np.int32)
        cap = min(self.s.max_seq, 512)
        return self.lib.orc_prefill_bf16(C.byref(self.om.model), C.byref(self.s), t.ctypes.data_as(C.c_void_p),
                                         cd.ctypes.data_as(C.c_void_p), len(t), C.byref(OrcSampling(*sampling)), cap)

    def frame(self, semantic, text_token, talker_sampling, predictor_sampling):
        codes = np.zeros(16, np.uint16)
        nxt = self.lib.orc_frame_step(C.byref(self.om.model), C.byref(self.s), semantic, text_token,
                                      C.byref(OrcSampling(*talker_sampling)),
                                      C.byref(OrcSampling(*predictor_sampling)), codes.ctypes.data_as(C.c_void_p))
        return codes, nxt
