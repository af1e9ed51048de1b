"""Pins the float64 CPU oracle (oracle/dinov3_oracle.c) without retyping it:
the reference's own known-answer tests, an independent IEEE float16
implementation (numpy), closed forms and special cases, brute force on tiny
inputs, and golden vectors of transformers' float64 DINOv3ViTModel."""
import glob
import os

import numpy as np
import pytest

import oracle

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def test_patchify_kat():
    # lib.rs:307-327: ramp input, every destination checked against its source.
    img = np.arange(3 * 224 * 224, dtype=np.float32)
    out = oracle.patchify(img, 14).reshape(14, 14, 3, 16, 16)
    src = img.reshape(3, 14, 16, 14, 16)  # c, gy, dy, gx, dx
    assert np.array_equal(out, src.transpose(1, 3, 0, 2, 4))


def test_f16_packing_kat():
    # weights.rs:152-169: values at the float16 limits, including -0.
    v = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65519.0, -65519.0], np.float32)
    back = oracle.f16_bits_to_f32(oracle.f32_to_f16_bits(v))
    assert back.tolist() == [0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65504.0, -65504.0]
    assert np.signbit(back[1])


def test_f16_matches_numpy_on_random_bit_patterns():
    rng = np.random.default_rng(7)
    v = rng.integers(0, 2**32, size=1 << 20, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([65520.0, -65520.0, 2.0**-25, 2.0**-24, 1.5 * 2.0**-24, 2.0**-14 - 2.0**-25, np.inf, -np.inf],
                       np.float32)
    v = np.concatenate([v, special])
    ours = oracle.f32_to_f16_bits(v)
    with np.errstate(over="ignore"):
        ref = v.astype(np.float16).view(np.uint16)
    nan = np.isnan(v)
    assert np.array_equal(ours[~nan], ref[~nan])
    assert np.all(np.isnan(oracle.f16_bits_to_f32(ours[nan])))
    # and back: every f16 bit pattern widens exactly
    allbits = np.arange(1 << 16, dtype=np.uint16)
    w = oracle.f16_bits_to_f32(allbits)
    ok = ~np.isnan(w)
    assert np.array_equal(w[ok], allbits.view(np.float16).astype(np.float32)[ok])


@pytest.mark.parametrize("grid", [14, 32])
def test_rope_tables_match_transformers(grid):
    # transformers' get_patches_center_coordinates / inv_freq / tile layout,
    # evaluated in float64 by tests/golden/make_golden.py.
    ref = np.load(os.path.join(GOLDEN, f"rope_g{grid}.npz"))
    c, s = oracle.rope_tables(grid)
    assert np.abs(c - ref["cos"]).max() < 1e-7
    assert np.abs(s - ref["sin"]).max() < 1e-7


def test_rope_table_closed_form_points():
    c, s = oracle.rope_tables(14)
    # patch (0,0), channel 0: angle = 2*pi*(2*0.5/14 - 1) = 2*pi*(-13/14)
    a = 2 * np.pi * (-13 / 14)
    assert abs(c[0, 0] - np.cos(a)) < 1e-7 and abs(s[0, 0] - np.sin(a)) < 1e-7
    # last frequency j = 15: divisor 100^(15/16); x-axis entries at 16..31 of patch (0, 13)
    a = 2 * np.pi * (2 * 13.5 / 14 - 1) / 100 ** (15 / 16)
    assert abs(c[13, 31] - np.cos(a)) < 1e-7
    # the second half repeats the first
    assert np.array_equal(c[:, :32], c[:, 32:]) and np.array_equal(s[:, :32], s[:, 32:])


def test_linear_brute_force():
    rng = np.random.default_rng(1)
    for m, k, n in [(1, 1, 1), (3, 5, 2), (7, 13, 9), (5, 384, 3)]:
        x, w, b = rng.normal(size=(m, k)), rng.normal(size=(n, k)), rng.normal(size=n)
        want = np.array([[sum(x[i, t] * w[j, t] for t in range(k)) + b[j] for j in range(n)] for i in range(m)])
        assert np.allclose(oracle.linear(x, w, b), want, rtol=1e-12, atol=1e-12)
        assert np.allclose(oracle.linear(x, w), want - b, rtol=1e-12, atol=1e-12)


def test_layernorm_closed_forms():
    rng = np.random.default_rng(2)
    g, b = rng.normal(size=384), rng.normal(size=384)
    # a constant row normalises to beta
    assert np.allclose(oracle.layernorm(np.full((1, 384), 3.25), g, b), b[None], atol=1e-12)
    # +-1 alternating row: mean 0, variance 1 -> x / sqrt(1 + 1e-5)
    x = np.tile([1.0, -1.0], 192)[None]
    assert np.allclose(oracle.layernorm(x, np.ones(384), np.zeros(384)), x / np.sqrt(1 + 1e-5), atol=1e-14)
    # shift invariance, and a scale by s equals eps divided by s^2: with
    # eps 1e-5 against a row variance of 1e6, the result is LN without eps
    x = rng.normal(size=(4, 384))
    assert np.allclose(oracle.layernorm(x + 7, g, b), oracle.layernorm(x, g, b), atol=1e-12)
    z = (x - x.mean(1, keepdims=True)) / x.std(1, keepdims=True)
    assert np.allclose(oracle.layernorm(x * 1000, g, b), z * g + b, atol=1e-9)


def test_attention_special_cases():
    rng = np.random.default_rng(3)
    T = 9
    k, v = rng.normal(size=(T, 384)), rng.normal(size=(T, 384))
    # q = 0 gives uniform weights: every row is the mean of V
    out = oracle.attention(np.zeros((T, 384)), k, v)
    assert np.allclose(out, np.broadcast_to(v.mean(0), (T, 384)), atol=1e-12)
    # a single key gives V
    out = oracle.attention(rng.normal(size=(1, 384)), k[:1], v[:1])
    assert np.allclose(out, v[:1], atol=1e-12)
    # brute force per head against an explicit softmax for a tiny case
    q = rng.normal(size=(T, 384))
    want = np.zeros((T, 384))
    for h in range(6):
        sl = slice(64 * h, 64 * h + 64)
        s = q[:, sl] @ k[:, sl].T * 0.125
        p = np.exp(s - s.max(1, keepdims=True))
        want[:, sl] = (p / p.sum(1, keepdims=True)) @ v[:, sl]
    assert np.allclose(oracle.attention(q, k, v), want, atol=1e-12)


def test_rope_special_cases():
    rng = np.random.default_rng(4)
    G = 3
    T = G * G + 5
    x = rng.normal(size=(T, 384))
    y = oracle.rope(x, G)
    # prefix tokens are untouched; rotations preserve each (c, c+32) pair's norm
    assert np.array_equal(y[:5], x[:5])
    xs = x[5:].reshape(-1, 6, 2, 32)
    ys = y[5:].reshape(-1, 6, 2, 32)
    assert np.allclose(np.hypot(xs[:, :, 0], xs[:, :, 1]), np.hypot(ys[:, :, 0], ys[:, :, 1]), atol=1e-12)
    # channel 0 of patch 4 (row 1, col 1): angle from the y coordinate
    a = 2 * np.pi * (2 * 1.5 / G - 1)
    assert abs(y[5 + 4, 0] - (x[9, 0] * np.cos(a) - x[9, 32] * np.sin(a))) < 1e-12


def test_swiglu_closed_form():
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0])
    u = np.array([2.0, 1.0, 1.0, 1.0, 1.0])
    want = g / (1 + np.exp(-g)) * u
    assert np.allclose(oracle.swiglu(g, u), want, atol=1e-15)
    assert oracle.swiglu(np.array([0.0]), np.array([5.0]))[0] == 0.0


def _golden_cases():
    return sorted(os.path.basename(p)[:-4] for p in glob.glob(os.path.join(GOLDEN, "g*_*.npz")))


@pytest.mark.parametrize("name", _golden_cases())
def test_forward_matches_transformers_golden(name, oracle_weights):
    import dinov3_hrx

    f = np.load(os.path.join(GOLDEN, name + ".npz"))
    grid, preset = int(f["grid"]), int(f["preset"])
    w = oracle_weights(preset)
    # the weights and pixels are the ones the fixture was made from
    assert np.allclose([a.sum() for a in w.arrays], f["weight_sums"], rtol=0, atol=1e-9)
    px = dinov3_hrx.random_pixels(int(f["pixel_seed"]), 1, 16 * grid)
    assert abs(px.astype(np.float64).sum() - float(f["pixel_sum"])) < 1e-6
    if grid == 32:
        oracle.set_threads(min(16, os.cpu_count() or 1))
    out = oracle.forward(w, px[0], grid)
    got = out if "out" in f else out[f["rows"]]
    want = f["out"] if "out" in f else f["row_values"]
    assert np.abs(got - want).max() < 1e-10
    assert np.abs(np.linalg.norm(out, axis=1) - f["norms"]).max() < 1e-10
