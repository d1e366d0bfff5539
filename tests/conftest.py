import os
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
for p in (ROOT / "qwen3-tts-native_amd", ROOT / "oracle", ROOT / "tests"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP library)")


@pytest.fixture
def rng():
    return np.random.default_rng(1234)


@pytest.fixture(scope="session")
def hip():
    import qwen3_tts_hip

    qwen3_tts_hip.load()
    return qwen3_tts_hip


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle
