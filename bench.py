"""Headline benchmark of the MI355X int8 weight-only decode path.

Workload: one talker decode step's GEMV chain at
batch 1 -- 28 layers, hidden 2048, each layer = fused QKV 2048->4096 with the
input RMSNorm fused as prologue, O 2048->2048 + residual, gate+up 2048->12288
with the post-attention RMSNorm prologue and SiLU-gate epilogue, down
6144->2048 + residual -- on synthetic int8 weights (uniform [-127,127],
per-row scales uniform [1e-3,2e-2]) distinct per layer (1.41 GB, far above the
256 MB last-level cache), x ~ N(0,1).  A step is one pass of the chain,
replayed as a hipGraph; inputs are resident in HBM before timing.

value = algorithmic bytes per step / time per step (GB/s).  The JSON line
also carries the roofline of the dominant kernel (the gate/up GEMV, timed
alone over its 28 per-layer launches with hipEvents on the launching
stream), the CPU baseline (the oracle's multithreaded exact-order GEMV on
this host), and the full codec frame step (talker + 15-step code predictor,
config 5) through the C ABI as frames/s and real-time factor.
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "qwen3-tts-native_amd"))

HBM_PEAK_GBS = 8000.0
LAYERS, HIDDEN, INTER, QW, KW = 28, 2048, 6144, 2048, 1024


def step_benchmark(hip, steps, warmup, kernel_filter=0, use_graph=1, rows=1, mode=1):
    b = hip.StepBenchmarkV1()
    b.struct_size = C.sizeof(hip.StepBenchmarkV1)
    b.layers, b.hidden, b.intermediate, b.query_width, b.key_value_width = LAYERS, HIDDEN, INTER, QW, KW
    b.rows, b.mode, b.warmup, b.steps, b.use_graph, b.kernel_filter = rows, mode, warmup, steps, use_graph, kernel_filter
    hip.call("qwen3_tts_benchmark_talker_step_gemvs", 0, C.byref(b))
    return b


def pmc_traffic():
    """HBM bytes per launch of the dominant kernel from the two rocprofv3 PMC
    passes (FETCH_SIZE, WRITE_SIZE, calibrated on a 256 MiB copy) recorded in
    profiles/gemv_gate_up_hbm_traffic_pmc.md; None if that record is absent."""
    path = ROOT / "profiles" / "gemv_gate_up_hbm_traffic_pmc.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    except OSError:
        pass
    return None


def single_gemv(hip, iterations: int = 2000):
    """Config 1: one 6144x2048 int8 GEMV at batch 1 (bf16 y), rotating weight
    copies so every launch streams from HBM; mean launch time over
    `iterations` back-to-back launches (hipEvents on the launching stream)."""
    out = hip.GemvBenchmark()
    hip.call("qwen3_tts_benchmark_int8_gemv", 0, 2048, 6144, iterations, C.byref(out))
    bytes_ = 6144 * 2048 + 4 * 6144 + 2 * 2048 + 2 * 6144
    return {"shape": "6144x2048", "rows": 1, "us_per_launch": round(out.mean_launch_microseconds, 3),
            "achieved_gbs": round(bytes_ / (out.mean_launch_microseconds * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(bytes_ / (out.mean_launch_microseconds * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def batched(hip, steps: int, warmup: int):
    """Config 4: N concurrent sessions as a skinny GEMM on MFMA, for the two
    shapes of the config (gate+up 12288x2048 with its RMSNorm prologue and
    fused SiLU; down 2048x6144 with the residual epilogue), 28 distinct
    layers so the weights stream from HBM."""
    result = {}
    for n in (2, 4, 8):
        for name, filt, out_f, in_f in (("gate_up_12288x2048", 3, 2 * INTER, HIDDEN), ("down_2048x6144", 4, HIDDEN, INTER)):
            b = step_benchmark(hip, steps, warmup, kernel_filter=filt, rows=n, mode=2)
            us = b.milliseconds_per_step * 1000.0 / LAYERS
            bytes_ = b.algorithmic_bytes_per_step / LAYERS
            flops = 2.0 * n * out_f * in_f
            result[f"n{n}_{name}"] = {"us_per_launch": round(us, 3),
                                      "achieved_gbs": round(bytes_ / (us * 1e-6) / 1e9, 1),
                                      "tflops": round(flops / (us * 1e-6) / 1e12, 2)}
    return result


def cpu_baseline(seconds: float = 8.0):
    """Oracle exact-order int8 GEMV chain on the host cores (bounded sample):
    once on every core this process may run on (its CPU affinity set, the
    box's share of the host), once on one thread."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    rng = np.random.default_rng(0)
    sample_layers = 2
    mats = []
    for _ in range(sample_layers):
        for out_f, in_f in ((QW + 2 * KW, HIDDEN), (HIDDEN, QW), (2 * INTER, HIDDEN), (HIDDEN, INTER)):
            w = rng.integers(-127, 128, size=(out_f, in_f), dtype=np.int8)
            s = rng.uniform(1e-3, 2e-2, out_f).astype(np.float32)
            x = oracle.f32_to_bf16(rng.standard_normal(in_f).astype(np.float32))
            mats.append((w, s, x))
    per_layer = sum(w.nbytes + 4 * w.shape[0] + 2 * w.shape[1] + 2 * w.shape[0] for w, _, _ in mats) / sample_layers

    def timed(n_threads, budget):
        t0 = time.perf_counter()
        layers_done = 0
        while True:
            for w, s, x in mats:
                oracle.int8_gemm_rows_mt(w, s, x, n_threads)
            layers_done += sample_layers
            if time.perf_counter() - t0 >= budget:
                break
        dt = time.perf_counter() - t0
        return per_layer * layers_done / dt / 1e9, layers_done, dt

    gbs, layers_done, dt = timed(threads, seconds)
    gbs1, layers1, dt1 = timed(1, seconds)
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{layers_done} talker-layer GEMV chains (QKV, O, gate+up, down; {sample_layers} distinct "
                  f"layers cycled) in {dt:.1f} s with the oracle's exact-order int8 GEMV on {threads} threads "
                  f"(every core of this process's CPU affinity set; the host reports {os.cpu_count()})",
        "one_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                       "sample": f"{layers1} talker-layer GEMV chains in {dt1:.1f} s on one thread"},
    }


# Config 3's algorithmic bytes: 15 steps x (5 predictor layers + the
# 2048x1024 LM head), weights + scales + activations.
PREDICTOR_CHAIN_BYTES = 1_218_232_320


def predictor_chain_entry(ms):
    """Median predictor GPU time of the greedy frames, as config 3's
    effective bandwidth (its unique weights stay in the 256 MB Infinity
    Cache across the 15 steps)."""
    if not ms:
        return None
    med = sorted(ms)[len(ms) // 2]
    return {"frames": len(ms), "sampling": "greedy argmax", "passes": 16,
            "gpu_ms_median": round(med, 4),
            "effective_gbs": round(PREDICTOR_CHAIN_BYTES / (med * 1e6), 1)}


def build_model(hip):
    """The VoiceDesign-geometry model of config 5 with synthetic bf16 weights
    (quantized to int8 at finalize), uploaded through the C ABI.  Returns the
    model handle and the config; the caller destroys the model."""
    import numpy as np

    cfg = hip.default_config()
    model = C.c_void_p()
    hip.call("qwen3_tts_model_create", 0, C.byref(model))
    scratch = []
    try:
        T, P = (cfg.talker_hidden, cfg.talker_intermediate, cfg.talker_query_heads * 128,
                cfg.talker_key_value_heads * 128), \
               (cfg.predictor_hidden, cfg.predictor_intermediate, cfg.predictor_query_heads * 128,
                cfg.predictor_key_value_heads * 128)
        tensors = []

        def layer(prefix, d):
            h, i, qw, kw = d
            return [(f"{prefix}.input_layernorm.weight", (h,), 1.0), (f"{prefix}.self_attn.q_proj.weight", (qw, h), 0),
                    (f"{prefix}.self_attn.k_proj.weight", (kw, h), 0), (f"{prefix}.self_attn.v_proj.weight", (kw, h), 0),
                    (f"{prefix}.self_attn.o_proj.weight", (h, qw), 0), (f"{prefix}.self_attn.q_norm.weight", (128,), 1.0),
                    (f"{prefix}.self_attn.k_norm.weight", (128,), 1.0),
                    (f"{prefix}.post_attention_layernorm.weight", (h,), 1.0),
                    (f"{prefix}.mlp.gate_proj.weight", (i, h), 0), (f"{prefix}.mlp.up_proj.weight", (i, h), 0),
                    (f"{prefix}.mlp.down_proj.weight", (h, i), 0)]

        H = T[0]
        tensors += [("talker.model.codec_embedding.weight", (cfg.talker_vocabulary, H), 0),
                    ("talker.model.text_embedding.weight", (cfg.text_vocabulary, H), 0),
                    ("talker.text_projection.linear_fc1.weight", (H, H), 0),
                    ("talker.text_projection.linear_fc1.bias", (H,), 0),
                    ("talker.text_projection.linear_fc2.weight", (H, H), 0),
                    ("talker.text_projection.linear_fc2.bias", (H,), 0),
                    ("talker.model.norm.weight", (H,), 1.0),
                    ("talker.codec_head.weight", (cfg.talker_vocabulary, H), 0),
                    ("talker.code_predictor.small_to_mtp_projection.weight", (P[0], H), 0),
                    ("talker.code_predictor.small_to_mtp_projection.bias", (P[0],), 0),
                    ("talker.code_predictor.model.norm.weight", (P[0],), 1.0)]
        for l in range(cfg.talker_layers):
            tensors += layer(f"talker.model.layers.{l}", T)
        for l in range(cfg.predictor_layers):
            tensors += layer(f"talker.code_predictor.model.layers.{l}", P)
        for g in range(15):
            tensors += [(f"talker.code_predictor.model.codec_embedding.{g}.weight", (cfg.predictor_vocabulary, H), 0),
                        (f"talker.code_predictor.lm_head.{g}.weight", (cfg.predictor_vocabulary, P[0]), 0)]
        biggest = max(int(np.prod(s)) for _, s, _ in tensors)
        buf = hip.DeviceArray(biggest, np.uint16)
        scratch.append(buf)
        for seed, (name, shape, mean) in enumerate(tensors):
            n = int(np.prod(shape))
            std = 0.05 if mean else (1.0 if "embedding" in name else 0.02)
            hip.call("qwen3_tts_device_fill_bf16_normal", buf.ptr, n, 1000 + seed, C.c_float(mean), C.c_float(std), None)
            hip.synchronize()
            shp = (C.c_uint64 * len(shape))(*shape)
            hip.call("qwen3_tts_model_upload_tensor", model, name.encode(), buf.ptr, 2 * n, len(shape), shp)
        mem = hip.ModelMemory()
        hip.call("qwen3_tts_model_finalize", model, C.byref(mem))
    except Exception:
        hip.load().qwen3_tts_model_destroy(model)
        raise
    finally:
        for b in scratch:
            b.free()
    return model, cfg


def frame_benchmark(hip, frames: int = 200, max_seq: int = 1024, warm: int = 3, greedy: int = 20):
    """Config 5 through the reference C ABI: VoiceDesign geometry, synthetic
    bf16 weights quantized to int8 at finalize, prompt of `prompt` tokens,
    then `frames` codec frames with top-k 50 / T 0.9 from a fixed seed.  The
    prompt fills the KV cache so that the timed frames run at context
    max_seq - frames .. max_seq (attention reads up to 1024 positions).
    An end token sampled on the way (random weights) ends the session: it is
    reset and prefilled again outside the timing with as many prompt tokens
    as the session had positions when it ended, so the frames after it run at
    the same context as without the restart and every run times the same
    number of frames over the same context range (each frame is timed on the
    host: the call returns its codes).
    Before the timed frames, `greedy` frames run the code predictor with
    greedy argmax (config 3: the 15-step predictor chain); its GPU time per
    frame is reported separately (it covers 16 passes through the 5 layers:
    the chain's 15 steps plus the pass that seeds it from the talker)."""
    import numpy as np

    prompt = max_seq - frames - warm - greedy
    lib = hip.load()
    model, cfg = build_model(hip)
    try:
        session = C.c_void_p()
        smem = hip.SessionMemory()
        hip.call("qwen3_tts_session_create", model, max_seq, 42, C.byref(session), C.byref(smem))
        try:
            rng = np.random.default_rng(1)
            # prompt tokens for the longest re-prefill (a restart just before
            # the last frame); the first prefill takes the first `prompt`
            text = rng.integers(0, cfg.text_vocabulary, max_seq).astype(np.int32)
            codec = rng.integers(0, 2048, max_seq).astype(np.int32)
            ts = hip.sampling(1, 50, 1.0, 0.9, 1.05)
            ps = hip.sampling(1, 50, 1.0, 0.9, 1.0)
            pre = hip.PrefillResult()
            t0 = time.perf_counter()
            hip.call("qwen3_tts_session_prefill", session, text.ctypes.data_as(C.POINTER(C.c_int32)),
                     codec.ctypes.data_as(C.POINTER(C.c_int32)), prompt, ts, C.byref(pre))
            prefill_s = time.perf_counter() - t0
            semantic = C.c_uint16(pre.first_semantic_token)
            codes = (C.c_uint16 * 16)()
            info = hip.CodecFrameInfo()
            nxt = C.c_uint16()
            trailing = rng.integers(0, cfg.text_vocabulary, frames + warm + greedy + 8).astype(np.int32)
            done = 0
            pred_ms = talk_ms = 0.0
            greedy_ms = []
            eos = 0
            greedy_ps = hip.sampling(0, 0, 1.0, 1.0, 1.0)
            timed = 0.0
            seeds = iter(range(100, 1000))

            def restart(context):
                # random weights: the end token can come up and end the
                # session; it is reset and prefilled again outside the timing
                # up to the context the ended session had reached
                hip.call("qwen3_tts_session_reset", session, next(seeds))
                again = hip.PrefillResult()
                hip.call("qwen3_tts_session_prefill", session, text.ctypes.data_as(C.POINTER(C.c_int32)),
                         codec.ctypes.data_as(C.POINTER(C.c_int32)), context, ts, C.byref(again))
                hip.synchronize()
                return C.c_uint16(again.first_semantic_token)

            context_range = [None, None]
            for f in range(frames + warm + greedy):
                while semantic.value == cfg.codec_eos_token:
                    eos += 1
                    semantic = restart(prompt + f)
                if f == warm + greedy:
                    context_range[0] = prompt + f
                context_range[1] = prompt + f + 1
                chain = warm <= f < warm + greedy
                t0 = time.perf_counter()
                hip.call("qwen3_tts_session_next_frame", session, semantic, int(trailing[f]), ts,
                         greedy_ps if chain else ps, codes, 16, C.byref(nxt), C.byref(info))
                dt = time.perf_counter() - t0  # the frame returns its codes on the host: synchronous
                semantic = C.c_uint16(nxt.value)
                if chain:
                    greedy_ms.append(info.predictor_gpu_milliseconds)
                if f >= warm + greedy:
                    timed += dt
                    done += 1
                    pred_ms += info.predictor_gpu_milliseconds
                    talk_ms += info.talker_gpu_milliseconds
            frame_ms = timed * 1000.0 / max(done, 1)
            return {
                "frames": done, "prompt_tokens": prompt, "max_sequence_length": max_seq,
                "frames_per_second": round(1000.0 / frame_ms, 2),
                "ms_per_frame": round(frame_ms, 3),
                "rtf": round(frame_ms / 80.0, 4),
                "predictor_gpu_ms_per_frame": round(pred_ms / max(done, 1), 3),
                "talker_gpu_ms_per_frame": round(talk_ms / max(done, 1), 3),
                "prefill_seconds": round(prefill_s, 3),
                "sessions_restarted_after_end_token": eos,
                "timed_context_positions": context_range,
                "sampling": "talker top-k 50 T 0.9 rep 1.05; predictor top-k 50 T 0.9; seed 42",
                "predictor_chain_config3": predictor_chain_entry(greedy_ms),
            }
        finally:
            lib.qwen3_tts_session_destroy(session)
    finally:
        lib.qwen3_tts_model_destroy(model)


# bf16 GEMM flops of one prompt row through the talker (q, k, v, o, gate, up,
# down at hidden 2048, q width 2048, kv width 1024, FFN 6144), without attention.
PREFILL_FLOPS_PER_ROW = 2 * 28 * (2048 * 2048 + 2 * 1024 * 2048 + 2048 * 2048 + 3 * 6144 * 2048)


def prefill_benchmark(hip, rows_list=(96, 512, 801), repeats: int = 5, max_seq: int = 1024):
    """The bf16 prompt prefill through the C ABI at VoiceDesign geometry:
    prompts of `rows_list` positions (96: a short voice-design prompt, whose
    GEMMs split K; 512: GEMM attention, the largest the reference's GEMM path
    takes; 801: the exact per-row attention), the
    median of `repeats` prefills each (qwen3_tts_session_prefill's own GPU
    time), as prompt positions per second and the GEMMs' TFLOP/s."""
    import numpy as np

    lib = hip.load()
    model, cfg = build_model(hip)
    out = {}
    try:
        session = C.c_void_p()
        smem = hip.SessionMemory()
        hip.call("qwen3_tts_session_create", model, max_seq, 5, C.byref(session), C.byref(smem))
        try:
            rng = np.random.default_rng(3)
            for rows in rows_list:
                times = []
                for _ in range(repeats + 1):
                    text = rng.integers(0, cfg.text_vocabulary, rows).astype(np.int32)
                    codec = rng.integers(0, 2048, rows).astype(np.int32)
                    pre = hip.PrefillResult()
                    hip.call("qwen3_tts_session_prefill", session, text.ctypes.data_as(C.POINTER(C.c_int32)),
                             codec.ctypes.data_as(C.POINTER(C.c_int32)), rows, hip.sampling(0, 0, 1.0, 1.0, 1.0),
                             C.byref(pre))
                    times.append(pre.talker_gpu_milliseconds)
                ms = sorted(times[1:])[len(times[1:]) // 2]
                out[f"rows{rows}"] = {"gpu_ms": round(ms, 3), "positions_per_second": round(rows / (ms * 1e-3), 1),
                                      "gemm_tflops": round(rows * PREFILL_FLOPS_PER_ROW / (ms * 1e-3) / 1e12, 2),
                                      "attention": "GEMM" if rows <= 512 else "exact per-row kernel"}
        finally:
            lib.qwen3_tts_session_destroy(session)
    finally:
        lib.qwen3_tts_model_destroy(model)
    return out


def batched_frames(hip, ns=(2, 4, 8), frames: int = 30, warm: int = 2, max_seq: int = 1024):
    """Multi-session serving through the batch entry point
    (qwen3_tts_model_batch_next_frame_begin_v2, the reference's lockstep
    batch: batched GEMVs on MFMA, batched attention): max(ns) sessions are
    prefilled once, then for each N the first N sessions step `warm` untimed
    and `frames` timed batched frames (talker top-k 50 / T 0.9 / rep 1.05,
    predictor top-k 50 / T 0.9).  The runs share the sessions, so contexts
    grow from ~870 to ~1010 positions over the three runs.  A session that
    samples the end token (random weights) is reset and prefilled again
    outside the timed region, so every batch keeps N sessions (counted)."""
    import numpy as np

    lib = hip.load()
    model, cfg = build_model(hip)
    sessions = []
    try:
        nmax = max(ns)
        prompt = max_seq - len(ns) * (frames + warm) - 8
        rng = np.random.default_rng(7)
        ts = hip.sampling(1, 50, 1.0, 0.9, 1.05)
        ps = hip.sampling(1, 50, 1.0, 0.9, 1.0)
        semantic = [0] * nmax
        restarts = 0

        def start(i, seed):
            # prefill session i (again after an end token) until its first
            # token is not the end token
            nonlocal restarts
            for attempt in range(8):
                hip.call("qwen3_tts_session_reset", sessions[i], seed + 1000 * attempt)
                text = rng.integers(0, cfg.text_vocabulary, prompt).astype(np.int32)
                codec = rng.integers(0, 2048, prompt).astype(np.int32)
                pre = hip.PrefillResult()
                hip.call("qwen3_tts_session_prefill", sessions[i], text.ctypes.data_as(C.POINTER(C.c_int32)),
                         codec.ctypes.data_as(C.POINTER(C.c_int32)), prompt, ts, C.byref(pre))
                if pre.first_semantic_token != cfg.codec_eos_token:
                    semantic[i] = pre.first_semantic_token
                    return
                restarts += 1
            raise RuntimeError("prefill keeps sampling the end token")

        for i in range(nmax):
            s = C.c_void_p()
            mem = hip.SessionMemory()
            hip.call("qwen3_tts_session_create", model, max_seq, 100 + i, C.byref(s), C.byref(mem))
            sessions.append(s)
            start(i, 100 + i)
        results = {"prompt_tokens": prompt, "frames": frames,
                   "sampling": "talker top-k 50 T 0.9 rep 1.05; predictor top-k 50 T 0.9"}
        for n in ns:
            timed_frames = 0
            timed_batches = 0
            t_total = 0.0
            for f in range(warm + frames):
                live = list(range(n))
                k = n
                arr = (C.c_void_p * k)(*[sessions[i].value for i in live])
                tr = (C.c_int32 * k)(*[int(x) for x in rng.integers(0, cfg.text_vocabulary, k)])
                tsa = (hip.SamplingConfig * k)(*[ts] * k)
                psa = (hip.SamplingConfig * k)(*[ps] * k)
                views = (hip.DeviceFrameViewV2 * k)()
                for v in views:
                    v.struct_size = C.sizeof(hip.DeviceFrameViewV2)
                t0 = time.perf_counter()
                hip.call("qwen3_tts_model_batch_next_frame_begin_v2", model, arr, k, tr, tsa, psa, views)
                for j, i in enumerate(live):
                    nxt = C.c_uint16()
                    info = hip.CodecFrameInfo()
                    hip.call("qwen3_tts_session_next_frame_finish_v2", sessions[i], views[j].lease_id, None,
                             C.byref(nxt), C.byref(info))
                    semantic[i] = nxt.value
                dt = time.perf_counter() - t0
                for i in live:
                    if semantic[i] == cfg.codec_eos_token:  # outside the timed region
                        restarts += 1
                        start(i, 500 + 17 * restarts)
                if f >= warm:
                    timed_frames += k
                    timed_batches += 1
                    t_total += dt
            ms = 1000.0 * t_total / max(1, timed_batches)
            results[f"n{n}"] = {"ms_per_batched_frame": round(ms, 3),
                                "session_frames_per_second": round(timed_frames / max(t_total, 1e-9), 1),
                                "aggregate_rtf": round(t_total / max(timed_frames, 1) / 0.080, 4),
                                "session_frames": timed_frames}
        results["sessions_restarted_after_end_token"] = restarts
        return results
    finally:
        for s in sessions:
            lib.qwen3_tts_session_destroy(s)
        lib.qwen3_tts_model_destroy(model)


def codec_cpu_baseline(weights, packets: int = 2):
    """The CPU oracle of the decoder (oracle/codec_oracle.c) decoding
    `packets` 4-frame packets of one stream on every core of this process's
    affinity set (bounded sample: a few seconds)."""
    import numpy as np

    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    oracle.set_threads(threads)
    orc = oracle.CodecOracle(weights)
    rng = np.random.default_rng(7)
    t0 = time.perf_counter()
    for _ in range(packets):
        orc.packet(rng.integers(0, 2048, (4, 16), dtype=np.uint16), trace=False)
    dt = (time.perf_counter() - t0) / packets
    return {"value": round(dt * 1e3, 1), "unit": "ms per 4-frame packet", "rtf": round(dt / 0.32, 3),
            "cores": threads, "kind": "port",
            "sample": f"{packets} packets of 4 frames, one stream, the oracle's fp32 decoder on {threads} threads"}


FP32_MFMA_PEAK_TFLOPS = 157.3


def codec_weights(seed: int = 0):
    """Random fp32 decoder weights of the real geometry (271 tensors,
    114,323,137 parameters): N(0, 1/fan_in) matrices, unit norms, small
    scales, cluster usage U[0.5, 2]."""
    import numpy as np
    import qwen3_tts_codec_hip as codec

    rng = np.random.default_rng(seed)
    out = {}
    for name, shape in codec.tensor_shapes().items():
        fan_in = int(np.prod(shape[1:])) if len(shape) > 1 else 1
        if name.endswith("cluster_usage"):
            w = rng.uniform(0.5, 2.0, shape)
        elif name.endswith(("scale", "gamma")):
            w = np.full(shape, 0.1)
        elif name.endswith(("norm.weight", "layernorm.weight")):
            w = np.ones(shape)
        elif len(shape) == 1:
            w = rng.standard_normal(shape) * 0.05
        else:
            w = rng.standard_normal(shape) / np.sqrt(fan_in)
        out[name] = w.astype(np.float32)
    return out


def codec_benchmark(packets: int = 200, warm: int = 20, streams: int = 6, sizes=(1, 4), cpu: bool = True):
    """The speech-tokenizer decoder through its C ABI: a continuous stream of
    `packets` packets per size (1 and 4 frames = 80 / 320 ms of audio) on one
    session, each packet's own GPU time and end-to-end latency (median); then
    `streams` concurrent sessions through qwen3_tts_codec_session_process_batch_v1
    (aggregate audio seconds per wall second).  The reference's published
    numbers (GB10): 11.65 ms per 1-frame packet, 62.09 ms per 4-frame packet
    (benchmarks/results/native-codec-decoder-bf16.json, p50)."""
    import numpy as np
    import qwen3_tts_codec_hip as codec

    weights = codec_weights()
    model = codec.SharedModel(weights)
    rng = np.random.default_rng(5)
    out = {"weights": "synthetic fp32, real geometry (114,323,137 parameters)"}
    try:
        for frames in sizes:
            s = model.session()
            gpu, e2e = [], []
            for i in range(warm + packets):
                if i and i % 500 == 0:
                    s.reset()
                codes = rng.integers(0, 2048, (frames, 16), dtype=np.uint16)
                _, res = s.packet(codes)
                if i >= warm:
                    gpu.append(res.gpu_microseconds)
                    e2e.append(res.end_to_end_microseconds)
            s.close()
            g, e = float(np.median(gpu)), float(np.median(e2e))
            audio_us = frames * 80_000.0
            flops = codec.packet_flops(frames)
            out[f"frames{frames}"] = {
                "gpu_us_p50": round(g, 1), "end_to_end_us_p50": round(e, 1),
                "end_to_end_us_p99": round(float(np.percentile(e2e, 99)), 1),
                "rtf_p50": round(e / audio_us, 5), "packet_gflop": round(flops / 1e9, 3),
                "tflops": round(flops / (g * 1e-6) / 1e12, 2),
                "frac_of_fp32_mfma_peak": round(flops / (g * 1e-6) / 1e12 / FP32_MFMA_PEAK_TFLOPS, 4),
                "weight_gbs": round(4 * 114_323_137 / (g * 1e-6) / 1e9, 1),
                "vs_reference_gb10_p50": round((11_651.3 if frames == 1 else 62_086.3) / e, 1)}
        sessions = [model.session() for _ in range(streams)]
        t0, audio = time.perf_counter(), 0.0
        for i in range(warm + packets // 2 if streams else 0):
            if i == warm:
                t0 = time.perf_counter()
            codes = [rng.integers(0, 2048, (4, 16), dtype=np.uint16) for _ in range(streams)]
            codec.process_batch(sessions, codes)
            if i >= warm:
                audio += streams * 0.32
        wall = time.perf_counter() - t0
        if streams:
            out[f"batch{streams}_4frame"] = {"audio_seconds_per_second": round(audio / wall, 1),
                                             "aggregate_rtf": round(wall / audio, 5)}
        for s in sessions:
            s.close()
    finally:
        model.close()
    if cpu:
        out["cpu_baseline"] = codec_cpu_baseline(weights)
    return out


def streaming_benchmark(hip, requests: int = 6, prompt: int = 96, frames: int = 100, packet_frames: int = 4):
    """One voice-design request after another on one warm talker session and
    one decoder session, both libraries in this process, as a serving loop
    would run them (the reference's qwen3-tts-bench defaults: 4-frame
    packets; session_bench.rs measures TTFA from request start to the first
    frame's codes).  Each request: session reset, prefill of a `prompt`-token
    prompt (bf16 path), then `frames` frames (top-k 50 / T 0.9), every
    `packet_frames` frames decoded to PCM through the host-code packet API;
    talker and decoder run one after the other on this thread (no overlap).
    Reports the median TTFA to the first frame's codes and to the first PCM
    packet, and the end-to-end RTF (wall time over audio time).  Random
    weights: the reference's published figures (0.287-0.47 RTF, TTFA p50
    55-60 ms on a DGX Spark) are for its real checkpoint and
    prompts, so the comparison is of work per frame, not of audio."""
    import numpy as np
    import qwen3_tts_codec_hip as codec

    lib = hip.load()
    model, cfg = build_model(hip)
    cmodel = codec.SharedModel(codec_weights())
    try:
        session = C.c_void_p()
        smem = hip.SessionMemory()
        hip.call("qwen3_tts_session_create", model, 1024, 9, C.byref(session), C.byref(smem))
        dec = cmodel.session()
        try:
            rng = np.random.default_rng(11)
            ts = hip.sampling(1, 50, 1.0, 0.9, 1.05)
            ps = hip.sampling(1, 50, 1.0, 0.9, 1.0)
            codes = (C.c_uint16 * 16)()
            info = hip.CodecFrameInfo()
            nxt = C.c_uint16()
            ttfa_codes, ttfa_pcm, rtf, done_frames, eos = [], [], [], 0, 0
            for r in range(requests + 1):  # the first request warms up
                text = rng.integers(0, cfg.text_vocabulary, prompt).astype(np.int32)
                cprompt = rng.integers(0, 2048, prompt).astype(np.int32)
                trailing = rng.integers(0, cfg.text_vocabulary, frames).astype(np.int32)
                hip.synchronize()
                t0 = time.perf_counter()
                hip.call("qwen3_tts_session_reset", session, 100 + r)
                dec.reset()
                pre = hip.PrefillResult()
                hip.call("qwen3_tts_session_prefill", session, text.ctypes.data_as(C.POINTER(C.c_int32)),
                         cprompt.ctypes.data_as(C.POINTER(C.c_int32)), prompt, ts, C.byref(pre))
                semantic = C.c_uint16(pre.first_semantic_token)
                pending, first_codes, first_pcm, n = [], None, None, 0
                for f in range(frames):
                    if semantic.value == cfg.codec_eos_token:
                        eos += 1
                        break
                    hip.call("qwen3_tts_session_next_frame", session, semantic, int(trailing[f]), ts, ps, codes, 16,
                             C.byref(nxt), C.byref(info))
                    if first_codes is None:
                        first_codes = time.perf_counter() - t0
                    pending.append(np.frombuffer(codes, np.uint16).copy())
                    semantic = C.c_uint16(nxt.value)
                    n += 1
                    if len(pending) == packet_frames:
                        dec.packet(np.stack(pending))
                        pending = []
                        if first_pcm is None:
                            first_pcm = time.perf_counter() - t0
                if pending:
                    dec.packet(np.stack(pending), is_final=True)
                wall = time.perf_counter() - t0
                if r and n >= packet_frames:
                    ttfa_codes.append(first_codes * 1e3)
                    ttfa_pcm.append(first_pcm * 1e3)
                    rtf.append(wall / (n * 0.08))
                    done_frames += n
            if not rtf:
                raise RuntimeError("every timed request ended by the end token before its first packet")
            return {"requests": len(rtf), "prompt_tokens": prompt, "frames_per_request": frames,
                    "frames_decoded": done_frames, "packet_frames": packet_frames,
                    "ttfa_codes_ms_p50": round(float(np.median(ttfa_codes)), 2),
                    "ttfa_pcm_ms_p50": round(float(np.median(ttfa_pcm)), 2),
                    "rtf_end_to_end_p50": round(float(np.median(rtf)), 4),
                    "requests_ended_by_eos": eos,
                    "reference_dgx_spark": {"rtf": "0.287-0.47", "ttfa_p50_ms": "55-60"}}
        finally:
            dec.close()
            lib.qwen3_tts_session_destroy(session)
    finally:
        cmodel.close()
        lib.qwen3_tts_model_destroy(model)


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--frames", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-frames", action="store_true")
    ap.add_argument("--only-dominant", action="store_true",
                    help="run only the dominant kernel's workload (the 28 gate/up GEMVs of a step) and a "
                         "256 MiB device-to-device copy that calibrates the HBM byte counters; for rocprofv3 --pmc")
    ap.add_argument("--only-batched-gemv", action="store_true",
                    help="run only config 4's MFMA GEMVs (N = 2, 4, 8; gate+up and down, 28 distinct layers); "
                         "for rocprofv3 --pmc")
    ap.add_argument("--only-prefill", action="store_true",
                    help="run only the bf16 prompt prefill at VoiceDesign geometry (prompts of 512 and 801 "
                         "positions, 5 each); for rocprofv3 kernel statistics")
    ap.add_argument("--only-codec", action="store_true",
                    help="run only the speech-tokenizer decoder benchmark (packets of 1 and 4 frames, 6 batched "
                         "streams); for rocprofv3 kernel statistics")
    ap.add_argument("--codec-frames", type=int, default=0,
                    help="with --only-codec: one packet size only (1..4) and no batched streams (a clean "
                         "per-layer kernel trace)")
    ap.add_argument("--only-streaming", action="store_true",
                    help="run only the end-to-end streaming requests (talker prefill and frames, 4-frame "
                         "decoder packets; TTFA and RTF)")
    ap.add_argument("--only-batched-frames", action="store_true",
                    help="run only the batched-frame workload (N = 8 sessions through the batch entry point); "
                         "for rocprofv3 kernel statistics")
    ap.add_argument("--only-frames", action="store_true",
                    help="run only config 5's frame step (prompt, greedy predictor-chain frames, timed top-k "
                         "frames; no decoder); for rocprofv3 kernel statistics")
    ap.add_argument("--only-chain", action="store_true",
                    help="run only config 2's chain three ways (the per-GEMV hipGraph, the launch-shape ceiling "
                         "of plain reads, the persistent launch); for rocprofv3 kernel traces")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build runs the decode path on a single MI355X "
              f"(--gpus {args.gpus} is not supported)", file=sys.stderr)
        return 2
    import qwen3_tts_hip as hip

    hip.load()
    if args.only_batched_gemv:
        import numpy as np

        out = {"batched_config4": batched(hip, args.steps, args.warmup)}
        size = 256 << 20  # calibrates the HBM byte counters
        src = hip.DeviceArray(size, np.uint8)
        dst = hip.DeviceArray(size, np.uint8)
        hip.call("qwen3_tts_device_memcpy", dst.ptr, src.ptr, size)
        hip.synchronize()
        out["copy_bytes"] = size
        print(json.dumps(out), flush=True)
        return 0
    if args.only_prefill:
        print(json.dumps({"prefill": prefill_benchmark(hip)}), flush=True)
        return 0
    if args.only_codec:
        if args.codec_frames:
            out = codec_benchmark(packets=50, warm=5, streams=0, sizes=(args.codec_frames,), cpu=False)
        else:
            out = codec_benchmark(cpu=not args.no_cpu)
        print(json.dumps({"codec": out}), flush=True)
        return 0
    if args.only_streaming:
        print(json.dumps({"streaming": streaming_benchmark(hip)}), flush=True)
        return 0
    if args.only_frames:
        print(json.dumps({"frame_step": frame_benchmark(hip, frames=args.frames)}), flush=True)
        return 0
    if args.only_chain:
        out = {}
        for name, graph in (("graph", 1), ("ceiling", 2), ("persistent", 3)):
            b = step_benchmark(hip, args.steps, args.warmup, use_graph=graph)
            out[name] = {"ms_per_step": round(b.milliseconds_per_step, 4),
                         "weight_gbs": round(b.weight_bytes / (b.milliseconds_per_step * 1e-3) / 1e9, 1),
                         "checksum": f"{b.output_checksum:016x}"}
        print(json.dumps(out), flush=True)
        return 0
    if args.only_batched_frames:
        print(json.dumps({"batched_frames": batched_frames(hip, ns=(8,))}), flush=True)
        return 0
    if args.only_dominant:
        import numpy as np

        step_benchmark(hip, args.steps, args.warmup, kernel_filter=3)
        size = 256 << 20
        src = hip.DeviceArray(size, np.uint8)
        dst = hip.DeviceArray(size, np.uint8)
        hip.call("qwen3_tts_device_memcpy", dst.ptr, src.ptr, size)
        hip.synchronize()
        print(json.dumps({"dominant_kernel_launches": 28 * (args.steps + args.warmup), "copy_bytes": size}))
        return 0
    main_run = step_benchmark(hip, args.steps, args.warmup)
    ms = main_run.milliseconds_per_step
    value = main_run.algorithmic_bytes_per_step / (ms * 1e-3) / 1e9
    # dominant kernel: the gate/up GEMV (25.2 MB int8 per launch), alone
    dom = step_benchmark(hip, args.steps, args.warmup, kernel_filter=3)
    launch_us = dom.milliseconds_per_step * 1000.0 / LAYERS
    launch_bytes = dom.algorithmic_bytes_per_step / LAYERS
    achieved = launch_bytes / (launch_us * 1e-6) / 1e9
    line = {
        "metric": "int8 GEMV achieved HBM GB/s (talker decode step, batch 1)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8xbf16->fp32",
        "data": "synthetic int8 weights U[-127,127], scales U[1e-3,2e-2], x ~ N(0,1); distinct weights per layer",
        "config": {"workload": "talker decode step GEMVs, batch 1, 28 layers, hidden 2048 (configs[1])",
                   "layers": LAYERS, "hidden": HIDDEN, "intermediate": INTER, "qkv_out": QW + 2 * KW,
                   "rows": 1, "graph": True,
                   "algorithmic_bytes_per_step": int(main_run.algorithmic_bytes_per_step),
                   "weight_bytes_per_step": int(main_run.weight_bytes)},
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": pmc_traffic(),
                     "traffic_source": "recorded rocprofv3 PMC passes of this kernel "
                                       "(profiles/gemv_gate_up_hbm_traffic_pmc.md), not measured in this run",
                     "kernel": "gemv_exact_fixed<4, SiluRounded, norm> (gate+up 12288x2048)",
                     "bytes_per_launch": int(launch_bytes), "us_per_launch": round(launch_us, 3)},
    }
    # The launch-shape ceiling: the same 112 launches (same weight bytes,
    # same graph) as plain 16-byte reads with no GEMV arithmetic.
    ceiling = step_benchmark(hip, args.steps, args.warmup, use_graph=2)
    ceiling_gbs = main_run.weight_bytes / (ceiling.milliseconds_per_step * 1e-3) / 1e9
    gemv_weight_gbs = main_run.weight_bytes / (ms * 1e-3) / 1e9
    line["launch_ceiling"] = {"what": "the step's 112 launches as plain reads of the same weights (one hipGraph)",
                              "ms_per_step": round(ceiling.milliseconds_per_step, 4),
                              "weight_gbs": round(ceiling_gbs, 1),
                              "gemv_weight_gbs": round(gemv_weight_gbs, 1),
                              "gemv_fraction_of_ceiling": round(gemv_weight_gbs / ceiling_gbs, 4)}
    # The same chain as one persistent launch per step (step_chain.hip): the
    # GEMVs hand their outputs over through tagged words instead of kernel
    # boundaries; bit-identical outputs on the same inputs.
    try:
        chain = step_benchmark(hip, args.steps, args.warmup, use_graph=3)
        line["persistent_chain"] = {
            "what": "the step's 112 GEMVs in one persistent launch (tagged-word hand-off between GEMVs)",
            "ms_per_step": round(chain.milliseconds_per_step, 4),
            "achieved_gbs": round(chain.algorithmic_bytes_per_step / (chain.milliseconds_per_step * 1e-3) / 1e9, 1),
            "bit_identical_to_graph": bool(chain.output_checksum == main_run.output_checksum)}
    except Exception as e:  # report, never hide
        line["persistent_chain"] = {"error": str(e)}
    line["single_gemv_config1"] = single_gemv(hip)
    line["batched_config4"] = batched(hip, max(args.steps // 4, 5), max(args.warmup // 2, 2))
    if not args.no_frames:
        try:
            line["frame_step"] = frame_benchmark(hip, frames=args.frames)
        except Exception as e:  # report, never hide
            line["frame_step"] = {"error": str(e)}
        try:
            line["prefill"] = prefill_benchmark(hip)
        except Exception as e:  # report, never hide
            line["prefill"] = {"error": str(e)}
        try:
            line["batched_frames"] = batched_frames(hip)
        except Exception as e:  # report, never hide
            line["batched_frames"] = {"error": str(e)}
        try:
            line["streaming"] = streaming_benchmark(hip)
        except Exception as e:  # report, never hide
            line["streaming"] = {"error": str(e)}
        try:
            line["codec"] = codec_benchmark(cpu=not args.no_cpu)
        except Exception as e:  # report, never hide
            line["codec"] = {"error": str(e)}
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
