"""The command-line front end (dinov3-loom_amd/csrc/cli.cpp), mirroring the
reference binary src/main.rs:6-88: argument checks and their order, raw
float32 in/out, and the two benchmark JSON lines."""
import json
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLI = os.path.join(ROOT, "dinov3-loom_amd", "lib", "dinov3-hrx")


def run(*args, **kw):
    if not os.path.exists(CLI):
        pytest.fail(f"{CLI} is not built (python dinov3-loom_amd/build.py)")
    return subprocess.run([CLI, *map(str, args)], capture_output=True, timeout=kw.pop("timeout", 120), **kw)


def error_text(p) -> str:
    assert p.returncode == 1, p
    return p.stderr.decode().strip()


def test_max_batch_checked_first(tmp_path):
    # main.rs:28-31: before the input file is even opened.
    for mb in (0, 65):
        p = run("--input", tmp_path / "missing.f32", "--max-batch", mb)
        assert error_text(p) == "Error: max_batch must be 1..=64"


def test_input_required_and_read(tmp_path):
    assert "--input" in error_text(run())
    assert "missing.f32" in error_text(run("--input", tmp_path / "missing.f32"))


def test_input_must_be_whole_floats(tmp_path, weight_file):
    # main.rs:37-40, checked before the model is loaded.
    px = tmp_path / "px.f32"
    px.write_bytes(b"\0" * 6)
    p = run("--input", px, "--model", weight_file(0))
    assert error_text(p) == "Error: input must be little-endian float32 NCHW RGB"


def test_missing_model_file(tmp_path):
    px = tmp_path / "px.f32"
    px.write_bytes(b"")
    p = run("--input", px, "--model", tmp_path / "none.safetensors")
    assert "none.safetensors" in error_text(p)


def test_bad_flag_value(tmp_path):
    assert "--device" in error_text(run("--input", tmp_path / "x", "--device", "zero"))
    assert "--bogus" in error_text(run("--input", tmp_path / "x", "--bogus"))


@pytest.mark.gpu
def test_cli_matches_forward(gpu, tmp_path, weight_file):
    import dinov3_hrx as d

    path = weight_file(1)
    px = d.random_pixels(7, 3)
    (tmp_path / "px.f32").write_bytes(px.astype("<f4").tobytes())
    p = run("--input", tmp_path / "px.f32", "--model", path, "--max-batch", 2, "--output", tmp_path / "out.f32")
    assert p.returncode == 0, p.stderr.decode()
    got = np.frombuffer((tmp_path / "out.f32").read_bytes(), "<f4").reshape(3, 201, 384)
    with d.DINOv3.load(path, d.Options(device=0, max_batch=2)) as m:
        want = m.forward(px)
    assert np.array_equal(got, want)
    # Without --output and --benchmark the tokens go to stdout.
    p = run("--input", tmp_path / "px.f32", "--model", path, "--max-batch", 2)
    assert p.returncode == 0, p.stderr.decode()
    assert np.array_equal(np.frombuffer(p.stdout, "<f4").reshape(3, 201, 384), want)


@pytest.mark.gpu
def test_cli_benchmark_lines(gpu, tmp_path, weight_file):
    import dinov3_hrx as d

    (tmp_path / "px.f32").write_bytes(d.random_pixels(3, 2).astype("<f4").tobytes())
    p = run("--input", tmp_path / "px.f32", "--model", weight_file(0), "--max-batch", 2, "--benchmark", 12)
    assert p.returncode == 0, p.stderr.decode()
    resident = json.loads(p.stderr.decode().strip().splitlines()[-1])
    assert resident["samples"] == 12 and set(resident) == {"samples", "graph", "direct"}
    assert 0 < resident["graph"]["median_ms"] <= resident["graph"]["p95_ms"]
    warm = json.loads(p.stdout.decode().strip())
    assert warm["scope"] == "warm end-to-end, including transfers" and warm["samples"] == 12
    assert 0 < warm["median_ms"] <= warm["p95_ms"] and warm["setup_ms"] > 0
    # Fewer than 10 iterations: the resident benchmark refuses first
    # (engine.rs:131), before main.rs:67's own check is reached.
    p = run("--input", tmp_path / "px.f32", "--model", weight_file(0), "--max-batch", 2, "--benchmark", 5)
    assert error_text(p).endswith("Error: use at least ten timing samples")
