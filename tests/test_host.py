"""CPU tests of the library's host side through its C ABI: exported symbols,
option and input validation, weight validation before GPU initialisation,
safetensors parsing, float16 packing, patchify, the seeded generators and the
Hugging Face cache resolver. No test here launches GPU work."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

import dinov3_hrx as d
from dinov3_hrx import ceilings
import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions(headers=("dinov3.h", "dinov3_engine.h")):
    names = []
    for h in headers:
        text = open(os.path.join(ROOT, "include", h)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        names += re.findall(r"\b((?:dinov3|dhx)_[a-z0-9_]+)\s*\(", text)
    return sorted(set(names))


def test_library_exports_every_declared_function():
    lib = ctypes.CDLL(d.LIB_PATH)
    names = declared_functions()
    assert len(names) > 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # The machine-ceiling probes live in their own measurement library.
    probe_names = declared_functions(("dinov3_probe.h",))
    assert probe_names == ["dhx_probe"]
    assert not hasattr(lib, "dhx_probe")
    probe_lib = ctypes.CDLL(ceilings.PROBE_LIB_PATH)
    assert all(hasattr(probe_lib, n) for n in probe_names)


def test_binding_structs_match_header(tmp_path):
    text = open(os.path.join(ROOT, "include", "dinov3_engine.h")).read()
    consts = dict(re.findall(r"#define (DHX_MAX_\w+) (\d+)", text))
    assert int(consts["DHX_MAX_SCALARS"]) == d.MAX_SCALARS and int(consts["DHX_MAX_BINDINGS"]) == d.MAX_BINDINGS
    assert int(consts["DHX_MAX_BRANCHES"]) == d.MAX_BRANCHES
    enum = dict((n, int(v)) for n, v in re.findall(r"(DHX_K_\w+) = (\d+)", text))
    assert [n[6:].lower() for n, _ in sorted(enum.items(), key=lambda kv: kv[1])] == d.KERNELS
    # the struct layouts the C compiler gives the header
    src = tmp_path / "layout.c"
    src.write_text('#include <stdio.h>\n#include <stddef.h>\n#include "dinov3.h"\nint main(void) {'
                   'printf("%zu %zu %zu %zu %zu\\n", sizeof(dhx_region), sizeof(dhx_launch), '
                   'offsetof(dhx_launch, bindings), sizeof(dinov3_options), sizeof(dhx_timings)); return 0; }\n')
    exe = tmp_path / "layout"
    subprocess.check_call(["gcc", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)])
    sizes = [int(v) for v in subprocess.check_output([str(exe)]).split()]
    assert sizes == [ctypes.sizeof(d.Region), ctypes.sizeof(d.Launch), d.Launch.bindings.offset,
                     ctypes.sizeof(d._Options), ctypes.sizeof(d._Timings)]


def test_probe_rejects_unsupported_arguments():
    # Checked before any HIP call, so this runs without a GPU.
    for kind, param in (("valu", 3), ("exp2", 0), ("loads_l2", 5), ("mfma_random", 1), ("chains", 3), ("chains", 0)):
        with pytest.raises(d.DINOv3Error, match="unsupported probe"):
            ceilings.probe(kind, param)


def test_constants_match_reference():
    assert d.IMAGE_ELEMENTS == 3 * 224 * 224 and d.TOKENS == 201 and d.HIDDEN == 384


def test_rejects_options_before_loading():
    # tests/model.rs:5-27: max_batch 0 and 65 fail before any file I/O.
    for mb in (0, 65):
        with pytest.raises(d.DINOv3Error, match=r"max_batch must be 1\.\.=64"):
            d.DINOv3.load("/nonexistent", d.Options(max_batch=mb))
        with pytest.raises(d.DINOv3Error, match=r"max_batch must be 1\.\.=64"):
            d.DINOv3.from_pretrained(d.Options(max_batch=mb))


def test_missing_file_error():
    with pytest.raises(d.DINOv3Error, match=r"read /nonexistent"):
        d.DINOv3.load("/nonexistent", d.Options(max_batch=4))


@pytest.mark.parametrize("dtype", ["F32", "BF16"])
@pytest.mark.parametrize("value", [100_000.0, -100_000.0])
def test_rejects_overflowing_weights_before_gpu_initialization(tmp_path, dtype, value):
    # tests/model.rs:29-59: a one-tensor file whose first value overflows
    # float16 fails while packing patch_w, before any other tensor is read
    # and before the device is opened (there is no GPU here, so reaching the
    # device would fail with a different message).
    import torch
    from safetensors.torch import save_file

    t = torch.zeros((384, 3, 16, 16), dtype=torch.float32 if dtype == "F32" else torch.bfloat16)
    t.view(-1)[0] = value
    path = tmp_path / "model.safetensors"
    save_file({"embeddings.patch_embeddings.weight": t}, str(path))
    with pytest.raises(d.DINOv3Error) as e:
        d.DINOv3.load(str(path), d.Options())
    assert "patch_w[0]" in str(e.value) and "finite float16" in str(e.value)


def test_weight_validation_errors(tmp_path):
    from safetensors.numpy import save_file

    path = str(tmp_path / "m.safetensors")
    save_file({"embeddings.patch_embeddings.weight": np.zeros((384, 3, 16, 8), np.float32)}, path)
    with pytest.raises(d.DINOv3Error, match=r"embeddings.patch_embeddings.weight: expected \[384, 3, 16, 16\], "
                                             r"found \[384, 3, 16, 8\]"):
        d.DINOv3.load(path, d.Options())
    save_file({"embeddings.patch_embeddings.weight": np.zeros((384, 3, 16, 16), np.float32)}, path)
    with pytest.raises(d.DINOv3Error, match=r"missing tensor embeddings.patch_embeddings.bias"):
        d.DINOv3.load(path, d.Options())
    w = np.zeros((384, 3, 16, 16), np.float32)
    w[1, 0, 0, 0] = np.nan
    save_file({"embeddings.patch_embeddings.weight": w}, path)
    with pytest.raises(d.DINOv3Error, match=r"non-finite tensor embeddings.patch_embeddings.weight"):
        d.DINOv3.load(path, d.Options())
    save_file({"embeddings.patch_embeddings.weight": np.zeros((384, 3, 16, 16), np.int32)}, path)
    with pytest.raises(d.DINOv3Error, match=r"unsupported dtype I32 for embeddings.patch_embeddings.weight"):
        d.DINOv3.load(path, d.Options())


def test_malformed_safetensors_rejected(tmp_path):
    path = tmp_path / "bad.safetensors"
    for blob in [b"", b"\x05\x00\x00\x00\x00\x00\x00\x00{abc}", b"\xff" * 8 + b"{}",
                 (20).to_bytes(8, "little") + b'{"a":{"dtype":"F32"}}']:
        path.write_bytes(blob)
        with pytest.raises(d.DINOv3Error, match="safetensors|read"):
            d.DINOv3.load(str(path), d.Options())
    # declared size larger than the data
    hdr = b'{"embeddings.patch_embeddings.weight":{"dtype":"F32","shape":[384,3,16,16],"data_offsets":[0,1179648]}}'
    path.write_bytes(len(hdr).to_bytes(8, "little") + hdr + b"\0" * 100)
    with pytest.raises(d.DINOv3Error, match="offsets"):
        d.DINOv3.load(str(path), d.Options())


def test_pack_f16_kat():
    # weights.rs:152-169
    bits = d.pack_f16("weights", [0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65519.0, -65519.0])
    back = bits.view(np.float16).astype(np.float32)
    assert back.tolist() == [0.0, -0.0, 1.0, -1.0, 65504.0, -65504.0, 65504.0, -65504.0]
    assert np.signbit(back[1])
    with pytest.raises(d.DINOv3Error, match=r"tensor w\[2\] cannot be represented as finite float16: 65520"):
        d.pack_f16("w", [0.0, 1.0, 65520.0])


def test_pack_f16_matches_oracle():
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(1 << 18) * np.exp(rng.uniform(-20, 11, 1 << 18))).astype(np.float32)
    v = v[np.abs(v) < 65504]
    assert np.array_equal(d.pack_f16("x", v), oracle.f32_to_f16_bits(v))


def test_patchify_kat():
    # lib.rs:307-327
    img = np.arange(3 * 224 * 224, dtype=np.float32)
    out = d.patchify(img)
    for gy in (0, 5, 13):
        for gx in (0, 7, 13):
            for c in range(3):
                for dy in (0, 9, 15):
                    for dx in (0, 3, 15):
                        dst = (((gy * 14 + gx) * 3 + c) * 16 + dy) * 16 + dx
                        assert out.reshape(-1)[dst] == img[(c * 224 + gy * 16 + dy) * 224 + gx * 16 + dx]
    assert np.array_equal(out, oracle.patchify(img, 14))
    big = np.random.default_rng(0).standard_normal(2 * 3 * 512 * 512).astype(np.float32)
    assert np.array_equal(d.patchify(big, 512), oracle.patchify(big, 32))


def test_fragment_order_layout():
    # The kernels' activation layout (dinov3_engine.h): row m, columns
    # k8..k8+7 at ((m/32)*(K/16) + k8/16)*512 + ((k8/8)%2*32 + m%32)*8.
    from conftest import from_frag, to_frag

    rng = np.random.default_rng(2)
    for rows, k in [(1, 16), (33, 384), (201, 1536), (64, 32)]:
        a = rng.normal(size=(rows, k)).astype(np.float16)
        f = d.fragment_order(a)
        assert np.array_equal(f, to_frag(a).reshape(-1))
        assert np.array_equal(d.row_order(f, rows, k), a)
        assert np.array_equal(from_frag(f, rows, k), a)
        for m, k8 in [(0, 0), (rows - 1, k - 8), (rows // 2, (k // 2) & ~7)]:
            o = ((m // 32) * (k // 16) + k8 // 16) * 512 + ((k8 // 8) % 2 * 32 + m % 32) * 8
            assert np.array_equal(f[o:o + 8], a[m, k8:k8 + 8])
    assert not d.fragment_order(np.ones((3, 16), np.float16))[3 * 8:32 * 8].any()  # padding rows zero
    with pytest.raises(d.DINOv3Error, match="k % 16"):
        d.fragment_order(np.ones((2, 24), np.float16))


def test_random_weights_deterministic_and_shaped(weight_file):
    from safetensors.numpy import load_file

    t = load_file(weight_file(0))
    names = oracle.tensor_names()
    assert all(n in t for n in names)
    w = t["layer.3.mlp.up_proj.weight"]
    assert w.shape == (1536, 384)
    assert abs(w.std() - 0.02 * 0.8796) < 5e-4  # std of N(0,1) truncated at +-2 is 0.8796
    assert np.abs(w).max() <= 0.04 + 1e-9
    assert np.all(t["layer.0.layer_scale1.lambda1"] == np.float32(1e-5))
    assert np.all(t["layer.5.attention.v_proj.bias"] == 0) and np.all(t["norm.weight"] == 1)
    s = load_file(weight_file(1))
    assert np.all(s["layer.0.layer_scale2.lambda1"] == 1)
    assert 0.05 < s["layer.2.norm1.weight"].std() < 0.15 and s["layer.2.attention.q_proj.bias"].std() > 0.01
    # determinism: same seed -> identical bytes; different seed -> different values
    p2 = weight_file(0, seed=0)
    assert p2 == weight_file(0)
    other = load_file(weight_file(0, seed=5))
    assert not np.array_equal(other["layer.3.mlp.up_proj.weight"], w)


def test_random_pixels():
    a = d.random_pixels(1, 2)
    assert a.shape == (2, 3, 224, 224) and a.dtype == np.float32
    assert np.array_equal(a, d.random_pixels(1, 2))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1) < 0.01
    assert not np.array_equal(a, d.random_pixels(2, 2))


def test_hub_offline_miss_and_cache_hit(tmp_path, monkeypatch):
    # hub.rs:56-82: an offline miss names the file; a cache hit resolves the
    # pinned snapshot path without any server.
    monkeypatch.setenv("HF_HUB_CACHE", str(tmp_path))
    with pytest.raises(d.DINOv3Error) as e:
        d.hub_weights()
    assert "not cached" in str(e.value) and d.FILE in str(e.value)
    path = tmp_path / f"models--{d.REPO[0]}--{d.REPO[1]}" / "snapshots" / d.REVISION / d.FILE
    path.parent.mkdir(parents=True)
    path.write_bytes(b"cached model")
    assert d.hub_weights() == str(path)
    monkeypatch.delenv("HF_HUB_CACHE")
    monkeypatch.setenv("HF_HOME", str(tmp_path / "home"))
    (tmp_path / "home").mkdir()
    os.symlink(tmp_path, tmp_path / "home" / "hub")
    assert d.hub_weights().endswith(f"snapshots/{d.REVISION}/{d.FILE}")


def test_engine_open_without_gpu_reports_error():
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(d.DINOv3Error, match="no HIP device"):
        d.Engine(0)
