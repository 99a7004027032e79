"""Shared test setup.

Markers: ``gpu`` tests need an MI355X (run with ``-m gpu``); everything else
runs on the CPU. Synthetic GGUF models are generated once per session into a
temporary directory from fixed seeds (the golden fixtures record the SHA-256
of the bytes they were made from).
"""

from __future__ import annotations

import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD GPU (MI355X) and the built libhipllm.so")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def model_dir(tmp_path_factory):
    return tmp_path_factory.mktemp("models")


@pytest.fixture(scope="session")
def golden_model(model_dir):
    """Returns fn(case) -> (gguf path, golden dict) for a golden case."""
    sys.path.insert(0, str(GOLDEN))
    import make_golden  # noqa: E402
    from myllm_amd import synth

    cache = {}

    def get(case: str):
        if case not in cache:
            path = make_golden.model_path(case, model_dir)
            golden = dict(np.load(GOLDEN / f"{case}_golden.npz"))
            sha = synth.file_sha256(path)
            assert sha == str(golden["gguf_sha256"]), f"{case}: regenerated GGUF differs from the golden input"
            cache[case] = (path, golden)
        return cache[case]

    return get


@pytest.fixture(scope="session")
def cuda():
    if not gpu_available():
        pytest.fail("GPU test selected but no GPU is visible")
    import torch
    return torch.device("cuda:0")
