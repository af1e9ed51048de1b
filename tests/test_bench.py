"""bench.py's output contract: one JSON line with the metric, the roofline of
the dominant kernel and the CPU baseline; algorithmic work per launch from
closed forms; one GPU only."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def test_more_than_one_gpu_is_refused():
    for args, env in ((["--gpus", "2"], {}), (["--gpus", "1"], {"WORLD_SIZE": "2"})):
        p = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), *args], capture_output=True, text=True,
                           timeout=120, env={**os.environ, **env})
        assert p.returncode == 2 and p.stdout == ""
        assert "one GPU" in p.stderr


def test_forward_flops_per_image():
    # Per image at 224x224 (T = 201, 14 x 14 patches), written out term by
    # term: patch embedding 2*196*768*384; per block QKV 2*201*384*1152,
    # attention 4*6*201^2*64 (QK^T and PV), o-projection 2*201*384^2,
    # gate/up 2*201*384*3072, down 2*201*1536*384.
    expect = {"patch_embed": 115_605_504, "qkv_rope": 177_831_936, "attention": 62_055_936,
              "resid_384": 59_277_312, "swiglu": 474_218_496, "resid_1536": 237_109_248}
    for name, flops in expect.items():
        assert bench.kernel_work(name, 1, 201, 14)[0] == flops, name
    total = expect["patch_embed"] + 12 * sum(v for k, v in expect.items() if k != "patch_embed")
    assert total == 12_241_520_640
    assert abs(total / 1e9 - bench.GFLOP_PER_IMAGE) < 1e-4
    # Work scales with the batch; split-K does the down projection's FLOPs.
    assert bench.kernel_work("swiglu", 64, 201, 14)[0] == 64 * expect["swiglu"]
    assert bench.kernel_work("splitk", 1, 201, 14)[0] == expect["resid_1536"]


def test_algorithmic_bytes_closed_forms():
    r = 64 * 201
    # The residual GEMMs read A and W and read and write the f16 residual stream.
    assert bench.kernel_work("resid_1536", 64, 201, 14)[1] == r * 1536 * 2 + 1536 * 384 * 2 + 2 * r * 384 * 2
    # Final LayerNorm: f16 in, f32 out.
    assert bench.kernel_work("layernorm_f32", 64, 201, 14)[1] == r * 384 * 6
    # Attention reads q, k, v and writes the output, all f16 [r][384].
    assert bench.kernel_work("attention", 64, 201, 14)[1] == 4 * r * 384 * 2


def test_committed_traffic_covers_the_forward_kernels():
    # The HBM traffic figures bench.py reports come from the committed
    # rocprofv3 summary; each is at least close to the algorithmic bytes (the
    # caches cannot remove compulsory traffic of tensors this large) and not
    # wildly above them.
    for name in ("patch_embed", "qkv_rope", "attention", "resid_384", "swiglu", "resid_1536"):
        t = bench.measured_traffic(name)
        assert isinstance(t, int), name
        alg = bench.kernel_work(name, 64, 201, 14)[1]
        assert 0.9 * alg <= t <= 3 * alg, (name, t, alg)


@pytest.mark.gpu
def test_bench_json_line(gpu):
    p = subprocess.run([sys.executable, "-u", os.path.join(ROOT, "bench.py"), "--steps", "5", "--warmup", "2",
                        "--branches", "2", "--cpu-seconds", "2"], capture_output=True, text=True, timeout=600,
                       cwd=ROOT)
    assert p.returncode == 0, p.stderr[-2000:]
    lines = p.stdout.strip().splitlines()
    assert len(lines) == 1
    d = json.loads(lines[0])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in d, key
    assert d["n_gpus"] == 1 and d["steps"] == 5 and d["warmup"] == 2 and d["higher_is_better"] is True
    assert d["unit"] == "images/s" and d["value"] > 0
    assert abs(d["value"] - 64 / (d["ms_per_step"] * 1e-3)) <= 1e-3 * d["value"]
    assert d["config"]["batch"] == 64 and d["config"]["branches"] == 2 and "workload" in d["config"]
    roof = d["roofline"]
    assert roof["bound"] in ("mfma", "hbm") and roof["unit"] in ("TFLOP/s", "GB/s")
    assert roof["peak"] == (2500.0 if roof["bound"] == "mfma" else 8000.0)
    assert abs(roof["frac"] - roof["achieved"] / roof["peak"]) < 1e-3 and 0 < roof["frac"] < 1
    assert roof["traffic"] == bench.measured_traffic(roof["kernel"])
    # achieved = algorithmic work per launch / average launch time
    flops, nbytes = bench.kernel_work(roof["kernel"], 64, 201, 14)
    work = flops / 1e12 if roof["bound"] == "mfma" else nbytes / 1e9
    assert abs(roof["achieved"] - work / (roof["avg_us"] * 1e-6)) <= 0.01 * roof["achieved"]
    cpu = d["cpu_baseline"]
    assert cpu["kind"] == "port" and cpu["cores"] == 1 and cpu["value"] > 0 and cpu["sample"]
    assert cpu["all_cores"]["nproc"] >= cpu["all_cores"]["usable_cpus"] >= cpu["all_cores"]["cores"] >= 1
    # what `value` and `sync_replay` each time
    assert "back-to-back" in d["value_scope"] and "engine.rs:130-190" in d["sync_replay"]["what"]


def test_sync_replay_statistics(monkeypatch):
    # engine.rs:130-190: median = t[n/2], p95 = t[ceil(0.95 n) - 1] of the
    # sorted samples. Replays of 1..100 ms in shuffled order.
    import random

    order = list(range(1, 101))
    random.Random(4).shuffle(order)
    clock = []
    for ms in order:
        clock += [0.0, ms / 1e3]
    it = iter(clock)
    monkeypatch.setattr(bench.time, "perf_counter", lambda: next(it))

    class Fake:
        def synchronize(self):
            pass

        def replay(self, b):
            pass

    s = bench.sync_stats(Fake(), 64, 100)
    assert s["median_ms"] == 51.0 and s["p95_ms"] == 95.0 and s["samples"] == 100
    assert s["images_per_s_at_median"] == round(64 / 0.051, 1)
    assert bench.cpu_model()
