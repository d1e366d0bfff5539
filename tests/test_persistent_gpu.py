"""The persistent GEMV chain kernel (one cooperative launch per talker step,
grid barriers between dependent GEMVs, next-GEMV weights prefetched before
each barrier) must produce bit-identical hidden states to the same chain run
as one kernel launch per GEMV.  Variant 2 is the tile-prefetching chain,
variant 3 the warp-specialized chain (loader waves stream weights through an
LDS ring with direct-to-LDS loads), variants 4 and 5 the linked per-GEMV
launches on two streams (4: one graph per stream, 5: eager), ordered by
their link counters only."""
import ctypes as C

import pytest

pytestmark = pytest.mark.gpu


def run(hip, use_graph, layers, steps=1, warmup=0, kernel_filter=0):
    b = hip.StepBenchmarkV1()
    b.struct_size = C.sizeof(hip.StepBenchmarkV1)
    b.layers, b.hidden, b.intermediate, b.query_width, b.key_value_width = layers, 2048, 6144, 2048, 1024
    b.rows, b.mode, b.warmup, b.steps, b.use_graph, b.kernel_filter = 1, 1, warmup, steps, use_graph, kernel_filter
    hip.call("qwen3_tts_benchmark_talker_step_gemvs", 0, C.byref(b))
    return b


@pytest.mark.parametrize("variant", [2, 3, 4, 5])
@pytest.mark.parametrize("layers,steps", [(1, 1), (2, 1), (28, 2)])
def test_persistent_chain_bit_identical(hip, layers, steps, variant):
    eager = run(hip, 0, layers, steps=steps)
    persistent = run(hip, variant, layers, steps=steps)
    assert persistent.output_checksum == eager.output_checksum
    assert persistent.algorithmic_bytes_per_step == eager.algorithmic_bytes_per_step


@pytest.mark.parametrize("variant", [2, 3])
@pytest.mark.parametrize("kernel_filter", [1, 2, 3, 4])
def test_persistent_single_kind_chains(hip, kernel_filter, variant):
    eager = run(hip, 0, 3, kernel_filter=kernel_filter)
    persistent = run(hip, variant, 3, kernel_filter=kernel_filter)
    assert persistent.output_checksum == eager.output_checksum


@pytest.mark.parametrize("variant", [4, 5])
@pytest.mark.parametrize("kernel_filter", [1, 2, 4])
def test_linked_single_kind_chains(hip, kernel_filter, variant):
    """Consecutive launches of one kind (two gate/up launches do not fit the
    device together, so that kind is refused)."""
    eager = run(hip, 0, 3, steps=3, kernel_filter=kernel_filter)
    linked = run(hip, variant, 3, steps=3, kernel_filter=kernel_filter)
    assert linked.output_checksum == eager.output_checksum


def test_linked_refuses_launches_that_do_not_fit(hip):
    with pytest.raises(hip.Qwen3TtsError, match="do not fit"):
        run(hip, 4, 2, kernel_filter=3)
