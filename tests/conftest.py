"""Shared test setup: repository root on sys.path, the `gpu` marker, fixtures."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (ROCm device) and the built HIP library")


def load_golden(name: str):
    """Committed fixture arrays (data only, no pickles)."""
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def golden():
    return {n: load_golden(n + ".npz") for n in ("codebooks", "rotations", "quantize", "attention")}


@pytest.fixture(scope="session")
def device():
    import torch

    assert torch.cuda.is_available(), "GPU tests need a visible ROCm device"
    print(f"[gpu] {torch.cuda.get_device_name(0)}", flush=True)
    return torch.device("cuda", 0)


def pytest_sessionfinish(session, exitstatus):
    """Write the attention parity margins (max-abs, mean-rel per checked
    output) as JSON lines to $TQ_MARGINS_OUT, when set."""
    path = os.environ.get("TQ_MARGINS_OUT")
    mod = sys.modules.get("tests.test_attention_gpu")
    if not path or mod is None:
        return
    import json

    with open(path, "w") as f:
        for m in mod.MARGINS:
            f.write(json.dumps(m) + "\n")
