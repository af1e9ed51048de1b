"""Whole-forward parity and API behaviour on the GPU (tests/model.rs:61-99
restated on seeded random-init weights, plus the configs of BASELINE.json).

Parity bar: all-token and CLS cosine against the float64 oracle > 0.9999
(tests/model.rs:85-86) and max-abs error within a per-preset ceiling
(MAX_ABS below); batched vs single-image
cosine > 0.99999 (tests/model.rs:87-93); bitwise determinism of a repeated
batched forward (tests/model.rs:95)."""
import os

import numpy as np
import pytest

import dinov3_hrx as d
import oracle

from conftest import cosine

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _threads(gpu):
    oracle.set_threads(min(16, os.cpu_count() or 1))


@pytest.fixture(scope="module")
def models(weight_file):
    cache = {}

    def get(preset=0, max_batch=4, image_size=224):
        key = (preset, max_batch, image_size)
        if key not in cache:
            cache[key] = d.DINOv3.load(weight_file(preset), d.Options(0, max_batch, image_size))
        return cache[key]

    yield get
    for m in cache.values():
        m.close()


# Max-abs ceilings against the float64 oracle, per weight preset. Measured
# on the MI355X: about 1.8e-3 on the BASELINE preset (0) and 0.0106-0.0137 on
# the stress preset (1) over every image size and batch tested; the ceilings
# leave about 1.5-3x of margin, so an accuracy regression that keeps the
# cosine above 0.9999 (tests/model.rs:79-86) still fails here.
MAX_ABS = {0: 0.005, 1: 0.02}


def compare(got, want, what, preset):
    """All-token and CLS cosine > 0.9999 and max-abs within the preset's
    ceiling; prints the three figures."""
    got = np.asarray(got, np.float64)
    err = float(np.abs(got - want).max())
    c_all, c_cls = cosine(got, want), cosine(got[0], want[0])
    print(f"{what}: all-token cos {c_all:.7f}  CLS cos {c_cls:.7f}  max-abs {err:.4g} (ceiling {MAX_ABS[preset]})")
    assert c_all > 0.9999 and c_cls > 0.9999, what
    assert err <= MAX_ABS[preset], f"{what}: max-abs {err:.4g} above {MAX_ABS[preset]}"
    return c_all, c_cls, err


@pytest.mark.parametrize("preset", [0, 1])
def test_forward_matches_oracle(models, oracle_weights, preset):
    m = models(preset)
    px = d.random_pixels(1, 2)
    out = m.forward(px)
    assert out.shape == (2, 201, 384) and out.dtype == np.float32
    for i in range(2):
        want = oracle.forward(oracle_weights(preset), px[i], 14)
        compare(out[i], want, f"preset {preset} image {i}", preset)


def test_acceptance_pattern_and_changing_batch(models, oracle_weights):
    # tests/model.rs:61-99 with its input sin(0.037 i) * 0.6 over 4 images.
    m = models(1)
    images = (np.sin(np.arange(4 * d.IMAGE_ELEMENTS, dtype=np.float64) * 0.037) * 0.6).astype(np.float32)
    batched = m.forward(images)
    for i in range(4):
        img = images[i * d.IMAGE_ELEMENTS:(i + 1) * d.IMAGE_ELEMENTS]
        got = m.forward(img)[0]
        want = oracle.forward(oracle_weights(1), img, 14)
        compare(got, want, f"acceptance image {i}", 1)
        assert cosine(batched[i], got) > 0.99999
    assert np.array_equal(m.forward(images), batched)  # bitwise determinism
    with pytest.raises(d.DINOv3Error, match="complete 3×224×224 images"):
        m.forward(np.zeros(3, np.float32))
    with pytest.raises(d.DINOv3Error, match="finite"):
        m.forward(np.full(d.IMAGE_ELEMENTS, np.nan, np.float32))


def test_chunking_and_empty(models):
    m = models(1, max_batch=4)
    px = d.random_pixels(3, 10)
    out = m.forward(px)
    assert out.shape == (10, 201, 384)
    # chunks are [0..4), [4..8), [8..10); the last chunk equals a batch of 2
    assert np.array_equal(out[8:], m.forward(px[8:]))
    assert np.array_equal(out[4:8], m.forward(px[4:8]))
    assert m.forward(np.zeros(0, np.float32)).shape == (0, 201, 384)


def test_pipelined_chunks_equal_single_chunks(models):
    # 9 chunks of 4 (the last of 2) alternate the two transfer slots with
    # uploads, graphs and readbacks of neighbouring chunks overlapping; each
    # chunk's rows equal the same images run alone.
    m = models(1, max_batch=4)
    px = d.random_pixels(12, 34)
    out = m.forward(px)
    assert out.shape == (34, 201, 384)
    for first in (0, 4, 16, 28, 32):
        n = min(4, 34 - first)
        assert np.array_equal(out[first:first + n], m.forward(px[first:first + n])), first


def test_cls_and_patch_mean(models):
    m = models(1)
    px = d.random_pixels(4, 3)
    out = m.forward(px)
    assert np.array_equal(m.cls(px), out[:, 0])
    pm = m.patch_mean(px)
    want = np.zeros((3, 384), np.float32)
    for t in range(5, 201):  # lib.rs:139-144: float32 += v / 196 in token order
        want += out[:, t] / np.float32(196)
    assert np.array_equal(pm, want)


def test_full_batch_64_rows_independent_of_batch(models, oracle_weights):
    # Config 3 (b = 64, 12,864 token rows): every row's arithmetic is the same
    # whatever the batch, so the first and last images of the b = 64 forward
    # equal bitwise the same images run as a batch of 2.
    m = models(0, max_batch=64)
    px = d.random_pixels(1, 64)
    out = m.forward(px)
    assert np.all(np.isfinite(out))
    assert np.array_equal(out[:2], m.forward(px[:2]))
    assert np.array_equal(out[62:], m.forward(px[62:]))
    for i in (0, 63):
        compare(out[i], oracle.forward(oracle_weights(0), px[i], 14), f"b64 image {i}", 0)


def test_batch_32_stress_matches_oracle(models, oracle_weights):
    # Config 2: the reference's default resident capacity (lib.rs:20-27),
    # b = 32 (6,432 token rows, two image groups of 16 images), on the
    # stress preset; the first and last image of each group against the
    # oracle, and the batch's first and last images bitwise equal to the same
    # images run as a batch of 2.
    m = models(1, max_batch=32)
    px = d.random_pixels(21, 32)
    out = m.forward(px)
    assert out.shape == (32, 201, 384) and np.all(np.isfinite(out))
    for i in (0, 15, 16, 31):
        compare(out[i], oracle.forward(oracle_weights(1), px[i], 14), f"b32 stress image {i}", 1)
    assert np.array_equal(out[:2], m.forward(px[:2]))
    assert np.array_equal(out[30:], m.forward(px[30:]))


def test_batch_64_stress_every_grouping(models, oracle_weights):
    # Config 3 (the headline, b = 64) on the stress preset: one image of each
    # of three image groups (and the last image) against the
    # oracle; all 64 outputs bitwise equal for every grouping bench.py may
    # pick (1-4 concurrent groups) and to the same images run as batches of 16.
    m = models(1, max_batch=64)
    px = d.random_pixels(22, 64)
    m.set_branches(3)
    out = m.forward(px)
    assert out.shape == (64, 201, 384) and np.all(np.isfinite(out))
    for i in (0, 21, 42, 63):
        compare(out[i], oracle.forward(oracle_weights(1), px[i], 14), f"b64 stress image {i}", 1)
    try:
        for n in (1, 2, 4):
            m.set_branches(n)
            assert np.array_equal(m.forward(px), out), f"{n} groups"
    finally:
        m.set_branches(2)
    for first in range(0, 64, 16):
        assert np.array_equal(m.forward(px[first:first + 16]), out[first:first + 16]), first


def test_512_batch_8_grouped_plan(models, oracle_weights):
    # Config 5 as bench.py runs it: 512x512 (1029 tokens), b = 8 in two
    # concurrent image groups of 4. One image per group against the oracle;
    # the batch bitwise equal to one group, to batches of 2 and, for those
    # two images, to batches of 1 (the default plan uses the residual GEMM
    # at every batch size, so an image's bits do not depend on the batch).
    m = models(1, max_batch=8, image_size=512)
    px = d.random_pixels(23, 8, 512)
    out = m.forward(px)
    assert out.shape == (8, 1029, 384) and np.all(np.isfinite(out))
    for i in (0, 7):
        compare(out[i], oracle.forward(oracle_weights(1), px[i], 32), f"512 b8 image {i}", 1)
    try:
        m.set_branches(1)
        assert np.array_equal(m.forward(px), out)
    finally:
        m.set_branches(2)
    assert np.array_equal(m.forward(px[:2]), out[:2])
    assert np.array_equal(m.forward(px[6:]), out[6:])
    assert np.array_equal(m.forward(px[:1]), out[:1])
    assert np.array_equal(m.forward(px[7:]), out[7:])


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_half_precision_checkpoints(models, tmp_path, weight_file, dtype):
    # weights.rs:30-45: F16 and BF16 tensors are widened to float32 before
    # packing. The stress weights stored as F16 / BF16 must give (a) the
    # oracle's forward on the widened values and (b) bitwise the forward of
    # an F32 file holding those widened values (widening is exact, so the
    # packed bytes are the same).
    import torch
    from safetensors.numpy import load_file, save_file
    from safetensors.torch import save_file as save_torch

    src = load_file(weight_file(1))
    tdt = torch.float16 if dtype == "F16" else torch.bfloat16
    half = {k: torch.from_numpy(v).to(tdt) for k, v in src.items()}
    widened = {k: v.to(torch.float32).numpy() for k, v in half.items()}
    assert any(not np.array_equal(widened[k], src[k]) for k in src)  # the rounding is real
    hpath, fpath = str(tmp_path / "half.safetensors"), str(tmp_path / "widened.safetensors")
    save_torch(half, hpath)
    save_file(widened, fpath)
    px = d.random_pixels(24, 2)
    with d.DINOv3.load(hpath, d.Options(0, 2)) as mh, d.DINOv3.load(fpath, d.Options(0, 2)) as mf:
        got = mh.forward(px)
        assert np.array_equal(got, mf.forward(px))
    ow = oracle.Weights(widened)
    for i in range(2):
        compare(got[i], oracle.forward(ow, px[i], 14), f"{dtype} checkpoint image {i}", 1)


@pytest.mark.parametrize("preset", [0, 1])
def test_layernorm_fusion_matches_unfused_plan(models, oracle_weights, preset):
    m = models(preset, max_batch=8)
    px = d.random_pixels(6, 8)
    fused = m.forward(px)
    m.set_layernorm_fusion(False)
    try:
        plain = m.forward(px)
    finally:
        m.set_layernorm_fusion(True)
    for i in range(8):
        assert cosine(fused[i], plain[i]) > 0.99999
    want = oracle.forward(oracle_weights(preset), px[0], 14)
    compare(plain[0], want, f"unfused plan preset {preset}", preset)
    compare(fused[0], want, f"fused plan preset {preset}", preset)


def test_branches_are_bitwise_identical(models):
    # Image groups recorded as concurrent graph branches: every grouping gives
    # the same bits (a row's arithmetic never depends on its group), in both
    # graph replay and the direct-dispatch path used by benchmark().
    m = models(1, max_batch=16)
    px = d.random_pixels(8, 16)
    m.set_branches(1)
    try:
        base = m.forward(px)
        for n in (2, 3, 4):
            m.set_branches(n)
            assert np.array_equal(m.forward(px), base), f"{n} branches"
            assert np.array_equal(m.forward(px[:9]), base[:9]), f"{n} branches, 9 images"
        t = m.benchmark(px, 10)
        assert t.samples == 10
        assert np.array_equal(m.forward(px), base)
        with pytest.raises(d.DINOv3Error, match="branches must be 1..4"):
            m.set_branches(5)
    finally:
        m.set_branches(2)


def test_splitk_variant(models):
    # Both down-projection variants at batch 8 and at batch 1 (the
    # reference's split-K case, lib.rs:218-225): the same result to f16
    # rounding; switching back restores the residual plan's bits.
    m = models(1, max_batch=8)
    px = d.random_pixels(5, 8)
    base = m.forward(px)
    m.set_splitk(1)
    try:
        split = m.forward(px)
        split1 = m.forward(px[:1])
    finally:
        m.set_splitk(0)
    for i in range(8):
        assert cosine(split[i], base[i]) > 0.99999
    assert np.array_equal(split1, split[:1])
    assert np.array_equal(m.forward(px), base)
    assert np.array_equal(m.forward(px[:1]), base[:1])


@pytest.mark.parametrize("preset", [0, 1])
def test_512_high_resolution(models, oracle_weights, preset):
    # Config 5: 512x512, 1024 patches + 5 = 1029 tokens, RoPE on the 32x32 grid.
    m = models(preset, max_batch=2, image_size=512)
    assert m.tokens == 1029
    px = d.random_pixels(1, 1, 512)
    out = m.forward(px)
    assert out.shape == (1, 1029, 384)
    compare(out[0], oracle.forward(oracle_weights(preset), px[0], 32), f"512 preset {preset}", preset)


@pytest.mark.parametrize("size", [16, 64, 256, 384])
def test_other_image_sizes(models, oracle_weights, size):
    # Image sizes other than 224 and 512 (any multiple of 16 is accepted):
    # 6 (the smallest: one patch), 21, 261 and 581 tokens run the attention
    # kernel with a run-time count of 64-key blocks, and the RoPE tables and
    # patch gather of 1x1, 4x4, 16x16 and 24x24 grids. Stress preset against the oracle; each image of the
    # batch of two equals it alone, bitwise.
    G = size // 16
    m = models(1, max_batch=2, image_size=size)
    assert m.tokens == G * G + 5
    px = d.random_pixels(size, 2, size)
    out = m.forward(px)
    assert out.shape == (2, G * G + 5, 384)
    for i in range(2):
        compare(out[i], oracle.forward(oracle_weights(1), px[i], G), f"{size}x{size} image {i}", 1)
    assert np.array_equal(m.forward(px[1:]), out[1:])


def test_largest_image_size(models, oracle_weights):
    # The largest accepted image, 1024x1024: 4096 patches + 5 = 4101 tokens
    # (65 run-time key blocks per head, RoPE on the 64x64 grid).
    m = models(1, max_batch=1, image_size=1024)
    assert m.tokens == 4101
    px = d.random_pixels(1024, 1, 1024)
    out = m.forward(px)
    compare(out[0], oracle.forward(oracle_weights(1), px[0], 64), "1024x1024", 1)


def test_benchmark(models):
    m = models(0)
    px = d.random_pixels(1, 4)
    t = m.benchmark(px, 10)
    assert t.samples == 10 and 0 < t.graph.median_ms <= t.graph.p95_ms and 0 < t.direct.median_ms
    with pytest.raises(d.DINOv3Error, match="at least ten"):
        m.benchmark(px, 9)
    with pytest.raises(d.DINOv3Error, match="one nonempty batch"):
        m.benchmark(d.random_pixels(1, 5), 10)
    with pytest.raises(d.DINOv3Error, match="one nonempty batch"):
        m.benchmark(np.zeros(0, np.float32), 10)


def test_gpu_failure_poisons_session(weight_file):
    m = d.DINOv3.load(weight_file(0), d.Options(0, 2))
    px = d.random_pixels(1, 1)
    m.forward(px)
    m._fail_next_gpu_call()
    with pytest.raises(d.DINOv3Error):
        m.forward(px)
    with pytest.raises(d.DINOv3Error, match="session is unusable after a GPU failure"):
        m.forward(px)
    m.close()
