import os
import sys
import tempfile

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("dinov3-loom_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def has_gpu() -> bool:
    return os.path.exists("/dev/kfd")


@pytest.fixture(scope="session")
def gpu():
    if not has_gpu():
        pytest.skip("no GPU (/dev/kfd absent)")
    return True


@pytest.fixture(scope="session")
def weights_dir():
    with tempfile.TemporaryDirectory(prefix="dinov3_w_") as d:
        yield d


@pytest.fixture(scope="session")
def weight_file(weights_dir):
    """Seeded random-init safetensors files: preset 0 (BASELINE) and 1 (stress)."""
    import dinov3_hrx

    cache = {}

    def get(preset: int, seed: int = 0) -> str:
        key = (preset, seed)
        if key not in cache:
            path = os.path.join(weights_dir, f"w_p{preset}_s{seed}.safetensors")
            dinov3_hrx.write_random_weights(path, seed=seed, preset=preset)
            cache[key] = path
        return cache[key]

    return get


@pytest.fixture(scope="session")
def oracle_weights(weight_file):
    import oracle

    cache = {}

    def get(preset: int, seed: int = 0):
        key = (preset, seed)
        if key not in cache:
            cache[key] = oracle.Weights.from_file(weight_file(preset, seed))
        return cache[key]

    return get


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / np.sqrt((a @ a) * (b @ b)))
