"""Persistent talker-step GEMV chain (csrc/step_chain.hip, step benchmark
use_graph = 3) against the per-GEMV exact kernels (use_graph = 1).

Both runs start from the same device-generated inputs (the step benchmark's
seeded fills) and run the same number of steps; the FNV-1a checksum of the
final hidden, QKV and activation rows must be identical, i.e. every bf16
output of the chain is bit-identical to the per-GEMV path, which the
production tests pin to the oracle GEMV by GEMV
(tests/test_gemv_production_gpu.py).  The layer sequence follows
native/qwen3-tts-native/native/src/talker.cu:3251-3456 without the attention
(the O projection reads the query part of the QKV output, as in the step
benchmark).
"""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu

HIDDEN, INTER, QW, KW = 2048, 6144, 2048, 1024


def _step(hip, layers, steps, warmup, use_graph, rows=1, mode=1):
    b = hip.StepBenchmarkV1()
    b.struct_size = C.sizeof(hip.StepBenchmarkV1)
    b.layers, b.hidden, b.intermediate, b.query_width, b.key_value_width = layers, HIDDEN, INTER, QW, KW
    b.rows, b.mode, b.warmup, b.steps, b.use_graph, b.kernel_filter = rows, mode, warmup, steps, use_graph, 0
    hip.call("qwen3_tts_benchmark_talker_step_gemvs", 0, C.byref(b))
    return b


@pytest.mark.parametrize("layers,steps,warmup", [(1, 1, 0), (2, 3, 1), (28, 1, 0), (28, 6, 2)])
def test_persistent_chain_bit_identical_to_per_gemv_kernels(hip, layers, steps, warmup):
    graph = _step(hip, layers, steps, warmup, use_graph=1)
    chain = _step(hip, layers, steps, warmup, use_graph=3)
    assert chain.output_checksum == graph.output_checksum
    assert chain.algorithmic_bytes_per_step == graph.algorithmic_bytes_per_step
    assert chain.milliseconds_per_step > 0.0


def test_persistent_chain_steps_chain_state(hip):
    """The chain carries the hidden row from one launch to the next (the
    epoch tags advance per launch): 4 steps differ from 3 steps."""
    three = _step(hip, 2, 3, 0, use_graph=3)
    four = _step(hip, 2, 4, 0, use_graph=3)
    assert three.output_checksum != four.output_checksum
    assert four.output_checksum == _step(hip, 2, 4, 0, use_graph=1).output_checksum


@pytest.mark.parametrize("rows,mode", [(2, 1), (1, 2)])
def test_persistent_chain_rejects_unsupported_shapes(hip, rows, mode):
    with pytest.raises(hip.Qwen3TtsError) as info:
        _step(hip, 2, 1, 0, use_graph=3, rows=rows, mode=mode)
    assert info.value.status == -1
