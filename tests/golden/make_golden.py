"""Writes the committed golden fixtures of tests/golden/ from the CPU oracle.

Fixtures (inputs and expected outputs; regenerate with
`python tests/golden/make_golden.py`):
  gemv_<out>x<in>_r<rows>.npz   int8 W, fp32 scales, bf16 x, fp32 y, bf16 y
                                (exact reference order) for small shapes
  digests.json                  SHA-256 of the oracle's fp32 and bf16 outputs
                                for BASELINE config 1 (W 6144x2048 uniform
                                [-127,127], scales U[1e-3,2e-2], x ~ N(0,1)
                                from numpy default_rng(20261201)), and the
                                greedy token stream of the toy model (seed 3,
                                prompt seed 11, 4 frames)
  argmax_kat.json               the reference's argmax known-answer results
                                (benchmarks/results/bf16-argmax-vocab*.json):
                                vocabulary, selected and expected token
"""
import hashlib
import json
import pathlib
import sys

import numpy as np

HERE = pathlib.Path(__file__).resolve().parent
ROOT = HERE.parents[1]
for p in (ROOT / "oracle", ROOT / "tests"):
    sys.path.insert(0, str(p))

import gen  # noqa: E402
import oracle  # noqa: E402

SMALL = [(64, 256, 1), (130, 512, 3), (64, 256, 8)]
CONFIG1_SEED = 20261201


def config1_inputs():
    rng = np.random.default_rng(CONFIG1_SEED)
    w = gen.weights(rng, 6144, 2048)
    s = gen.scales(rng, 6144)
    x = gen.activations(rng, 1, 2048)
    return w, s, x


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def toy_greedy_stream(frames=4):
    import toy_model

    weights = toy_model.make_weights(toy_model.TOY, seed=3)
    om = toy_model.OracleModel(oracle, toy_model.TOY, weights)
    sess = toy_model.OracleSession(om, 64, 7)
    rng = np.random.default_rng(11)
    text = rng.integers(0, toy_model.TOY["text_vocabulary"], 6).astype(np.int32)
    codec = rng.integers(0, 2048, 6).astype(np.int32)
    text[1], codec[2] = -1, -1
    greedy = (0, 0, 1.0, 1.0, 1.05)
    sem = sess.prefill(text, codec, greedy)
    stream = {"first": int(sem), "frames": []}
    for f in range(frames):
        codes, nxt = sess.frame(sem, 100 + f, greedy, greedy)
        stream["frames"].append({"codes": [int(c) for c in codes], "next": int(nxt)})
        sem = nxt
    return stream


def main():
    for out_f, in_f, rows in SMALL:
        rng = np.random.default_rng(out_f * 1000 + in_f + rows)
        w, s, x = gen.weights(rng, out_f, in_f), gen.scales(rng, out_f), gen.activations(rng, rows, in_f)
        y32, y16 = oracle.int8_gemm_rows(w, s, x)
        np.savez_compressed(HERE / f"gemv_{out_f}x{in_f}_r{rows}.npz", w=w, s=s, x=x, y32=y32, y16=y16)
    w, s, x = config1_inputs()
    y32, y16 = oracle.int8_gemm_rows(w, s, x)
    digests = {"config1": {"seed": CONFIG1_SEED, "inputs_sha256": sha(w) + sha(s) + sha(x),
                           "y32_sha256": sha(y32), "y16_sha256": sha(y16)},
               "toy_greedy_stream": toy_greedy_stream()}
    (HERE / "digests.json").write_text(json.dumps(digests, indent=1) + "\n")
    kat = [{"vocabulary_size": 2048, "selected_token": 1729, "expected_token": 1729,
            "source": "benchmarks/results/bf16-argmax-vocab2048.json"},
           {"vocabulary_size": 3072, "selected_token": 1729, "expected_token": 1729,
            "source": "benchmarks/results/bf16-argmax-vocab3072.json"}]
    (HERE / "argmax_kat.json").write_text(json.dumps(kat, indent=1) + "\n")


if __name__ == "__main__":
    main()
