"""Stage timeline of the persistent predictor pass (csrc/pred_chain.hip).

Builds a diagnostic copy of the library with -DQ3_PRED_TRACE into
_build_trace/ next to this file (the library build has no stamps), runs the
frame benchmark's frames through it (graph replay, the product path) and
prints, for workgroup 0 of the last pass, the wall-clock time at which each
stage's input was staged and its outputs published.

    python3 qwen3-tts-native_amd/pred_trace.py [frames]
"""
import concurrent.futures
import ctypes as C
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
sys.path[:0] = [str(HERE), str(HERE.parent)]

import build as B  # noqa: E402


def build_traced() -> pathlib.Path:
    out = HERE / "_build_trace"
    out.mkdir(exist_ok=True)
    sources = sorted((HERE / "csrc").glob("*.hip"))

    def compile_one(src):
        obj = out / (src.stem + ".o")
        r = subprocess.run([B.HIPCC, *B.FLAGS, "-DQ3_PRED_TRACE", "-c", str(src), "-o", str(obj)],
                           capture_output=True, text=True)
        if r.returncode:
            raise RuntimeError(r.stderr[-3000:])
        return obj

    with concurrent.futures.ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(compile_one, sources))
    lib = out / "libqwen3_tts_hip.so"
    r = subprocess.run([B.HIPCC, f"--offload-arch={B.ARCH}", "-shared", "-fPIC", "-o", str(lib), *map(str, objs)],
                       capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(r.stderr)
    for o in objs:
        o.unlink()
    return lib


def main(frames: int = 40) -> None:
    import qwen3_tts_hip as hip
    import bench

    hip.LIBRARY_PATH = build_traced()
    hip._LIB = None
    lib = hip.load()
    res = bench.frame_benchmark(hip, frames=frames, greedy=4)
    print({k: res[k] for k in ("ms_per_frame", "predictor_gpu_ms_per_frame", "talker_gpu_ms_per_frame")})
    t = (C.c_ulonglong * 128)()
    lib.qwen3_tts_debug_pred_trace.argtypes = [C.c_void_p]
    if lib.qwen3_tts_debug_pred_trace(C.cast(t, C.c_void_p)) != 0:
        raise RuntimeError("reading the stamps failed")
    us = lambda i: (t[i] - t[0]) / 100.0  # noqa: E731  (100 MHz clock)
    print("small_to_mtp published %.2f us" % us(1))
    print("layer | QKV in | QKV out | attention rows in | O in | O out | gate/up in | gate/up out | down in | down out")
    for layer in range(5):
        o = 10 * layer
        print("%d | " % layer + " | ".join("%.2f" % us(i + o) for i in range(2, 11)))
    print("head in %.2f, logits written %.2f us" % (us(52), us(53)))
    print("attention of head 0 | start | operands staged | norm + RoPE | scores | probabilities | published")
    for layer in range(5):
        o = 64 + 8 * layer
        print("%d | " % layer + " | ".join("%.2f" % us(o + k) for k in range(6)))


if __name__ == "__main__":
    main(int(sys.argv[1]) if len(sys.argv) > 1 else 40)
