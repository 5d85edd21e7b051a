import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libq4dec.so")
    config.addinivalue_line("markers", "slow: long-running (full 28-layer model)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    def load(name):
        return dict(np.load(GOLDEN / f"{name}.npz", allow_pickle=False))
    return load


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no GPU is visible")
    return torch.device("cuda:0")


def pytest_collection_modifyitems(config, items):
    # GPU tests never silently pass on a CPU box: they fail in `dev` instead.
    # This hook only keeps the CPU suite quick by skipping them when no GPU
    # exists and the user did not ask for them explicitly with -m gpu.
    markexpr = config.getoption("-m") or ""
    if "gpu" in markexpr and "not gpu" not in markexpr:
        return
    if gpu_available() or os.environ.get("Q4D_FORCE_GPU_TESTS"):
        return
    skip = pytest.mark.skip(reason="no GPU visible (run with -m gpu on an MI355X)")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def qwen3_full():
    """The full 28-layer Qwen3-0.6B shapes with seeded random Q4 weights (seed 0):
    (config, host weights, fp32 oracle model), built once per session."""
    import oracle as o
    from llm_accelerator_amd.model import Qwen3Config, random_host_weights
    cfg = Qwen3Config()
    host = random_host_weights(cfg, seed=0)
    om = o.OracleModel.from_q4(o.OracleConfig(), host["layers"], *host["embed_tokens"], host["norm"])
    return cfg, host, om
