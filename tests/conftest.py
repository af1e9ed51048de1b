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


def to_frag(a):
    """Row-major [rows][k] -> fragment order (rows padded to 32 with zeros):
    32-row x 16-column blocks of 64 lanes x 8 values, lane hi*32 + l holding
    row l, columns 8hi .. 8hi+7 of the block; blocks row-block-major."""
    a = np.asarray(a)
    rows, k = a.shape
    rp = (rows + 31) // 32 * 32
    p = np.zeros((rp, k), a.dtype)
    p[:rows] = a
    return np.ascontiguousarray(p.reshape(rp // 32, 32, k // 16, 2, 8).transpose(0, 2, 3, 1, 4))


def from_frag(f, rows, k):
    """Inverse of to_frag (padding rows dropped)."""
    rp = (rows + 31) // 32 * 32
    return np.asarray(f).reshape(rp // 32, k // 16, 2, 32, 8).transpose(0, 3, 1, 2, 4).reshape(rp, k)[:rows]
