import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "plamo3-0.8b-runtime_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")
    config.addinivalue_line("markers", "slow: long-running")


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def model_dir():
    """Synthetic seed-0 model directory (config, config-mlx, safetensors, packed .p12)."""
    from plamo_hip import synth
    d, sha = synth.ensure_model(packed=True)
    return d, sha


@pytest.fixture(scope="session")
def oracle_weights(model_dir):
    from oracle.model import Weights
    return Weights(model_dir[0])


@pytest.fixture(scope="session")
def golden():
    import json
    with open(os.path.join(ROOT, "tests", "golden", "manifest.json")) as f:
        return json.load(f)
