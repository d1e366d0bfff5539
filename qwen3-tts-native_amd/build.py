"""Builds the two gfx950 libraries with hipcc, next to this file:

- libqwen3_tts_hip.so from csrc/*.hip: the talker / code-predictor decode
  path (include/qwen3_tts_native.h);
- libqwen3_tts_codec_hip.so from csrc/codec/*.hip: the speech-tokenizer
  decoder (include/qwen3_tts_codec.h), a separate library as in the reference.

Each source compiles to an object under _build/ in parallel.  Always rebuilds
(no staleness checks): the build is a few seconds per file.
"""
import concurrent.futures
import os
import pathlib
import subprocess
import sys

HERE = pathlib.Path(__file__).resolve().parent
LIBRARIES = {
    HERE / "libqwen3_tts_hip.so": sorted((HERE / "csrc").glob("*.hip")),
    HERE / "libqwen3_tts_codec_hip.so": sorted((HERE / "csrc" / "codec").glob("*.hip")),
}
OUT = HERE / "libqwen3_tts_hip.so"
CODEC_OUT = HERE / "libqwen3_tts_codec_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("PYTORCH_ROCM_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    # Exact operation order: no implicit a*b+c contraction anywhere.
    "-ffp-contract=off",
    # Packed fp32 VALU ops are disabled on purpose for this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def _compile(src: pathlib.Path) -> pathlib.Path:
    obj = HERE / "_build" / (src.parent.name + "_" + src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = ("packed-fp32-ops", "is not a recognized feature")
    err = "\n".join(l for l in res.stderr.splitlines() if not any(n in l for n in noise))
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build() -> pathlib.Path:
    (HERE / "_build").mkdir(exist_ok=True)
    sources = [src for srcs in LIBRARIES.values() for src in srcs]
    jobs = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = dict(zip(sources, pool.map(_compile, sources)))
    for out, srcs in LIBRARIES.items():
        tmp = out.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *(str(objs[s]) for s in srcs)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"link of {out.name} failed:\n{res.stderr}")
        os.replace(tmp, out)
    return OUT


if __name__ == "__main__":
    print(build())
