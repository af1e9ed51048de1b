"""The safetensors parser and the weight loader (csrc/safetensors.cpp,
csrc/weights.cpp) built host-only with AddressSanitizer and
UndefinedBehaviorSanitizer (clang++, no GPU code) and driven by
tests/host_sanitize.cpp over malformed files, the float16 packing KAT
(weights.rs:152-169), the seeded generator + loader, half-precision
checkpoints, and byte mutations of a valid header. The same malformed files
go through the library's own C ABI as well. Validation rules follow the
safetensors crate 0.6 (`read_metadata` / `Metadata::validate`): header at most
100,000,000 bytes, a UTF-8 JSON object starting with '{', string-valued
__metadata__, unique names, and data ranges that tile the data section."""
import json
import os
import subprocess

import numpy as np
import pytest

import dinov3_hrx as d

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"
ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:abort_on_error=0:exitcode=86",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1:exitcode=87")


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ not found")
    exe = str(tmp_path_factory.mktemp("asan") / "host_sanitize")
    csrc = os.path.join(ROOT, "dinov3-loom_amd", "csrc")
    subprocess.check_call([CLANG, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer",
                           "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                           "-I", os.path.join(ROOT, "include"), os.path.join(ROOT, "tests", "host_sanitize.cpp"),
                           os.path.join(csrc, "safetensors.cpp"), os.path.join(csrc, "weights.cpp"), "-o", exe])

    def run(*args, timeout=600):
        p = subprocess.run([exe, *map(str, args)], capture_output=True, text=True, env=ENV, timeout=timeout)
        assert p.returncode == 0, f"rc {p.returncode}\n{p.stdout[-2000:]}\n{p.stderr[-4000:]}"
        assert "ERROR: AddressSanitizer" not in p.stderr and "runtime error" not in p.stderr, p.stderr[-4000:]
        return p.stdout

    return run


def blob(header: str, data: bytes = b"") -> bytes:
    h = header.encode() if isinstance(header, str) else header
    return len(h).to_bytes(8, "little") + h + data


def t(name, dtype, shape, begin, end):
    return f'"{name}":{{"dtype":"{dtype}","shape":{json.dumps(shape)},"data_offsets":[{begin},{end}]}}'


# (name, file bytes, expected: "ok" or a substring of the error)
CASES = [
    ("empty", b"", "file too small"),
    ("short_json", blob("{abc}"), "invalid safetensors header"),
    ("huge_length", b"\xff" * 8 + b"{}", "header too large"),
    ("missing_fields", blob('{"a":{"dtype":"F32"}}'), "tensor a"),
    ("size_past_data", blob("{" + t("a", "F32", [384, 3, 16, 16], 0, 1179648) + "}", b"\0" * 100), "offsets of a"),
    ("one_tensor", blob("{" + t("a", "F32", [2], 0, 8) + "}", b"\0" * 8), "ok"),
    ("gap", blob("{" + t("a", "F32", [1], 0, 4) + "," + t("b", "F32", [1], 8, 12) + "}", b"\0" * 12), "offsets of b"),
    ("overlap", blob("{" + t("a", "F32", [2], 0, 8) + "," + t("b", "F32", [2], 4, 12) + "}", b"\0" * 12),
     "offsets of b"),
    ("unsorted_ok", blob("{" + t("b", "F32", [1], 4, 8) + "," + t("a", "F32", [1], 0, 4) + "}", b"\0" * 8), "ok"),
    ("trailing_bytes", blob("{" + t("a", "F32", [1], 0, 4) + "}", b"\0" * 8), "not exactly covered"),
    ("not_from_zero", blob("{" + t("a", "F32", [1], 4, 8) + "}", b"\0" * 8), "offsets of a"),
    ("duplicate", blob("{" + t("a", "F32", [1], 0, 4) + "," + t("a", "F32", [1], 4, 8) + "}", b"\0" * 8),
     "duplicate tensor a"),
    ("leading_space", blob(" {" + t("a", "F32", [1], 0, 4) + "}", b"\0" * 4), "does not start with {"),
    ("not_utf8", blob(b'{"\xff":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', b"\0" * 4), "not UTF-8"),
    ("metadata_ok", blob('{"__metadata__":{"format":"pt"},' + t("a", "F32", [1], 0, 4) + "}", b"\0" * 4), "ok"),
    ("metadata_number", blob('{"__metadata__":{"k":1},' + t("a", "F32", [1], 0, 4) + "}", b"\0" * 4),
     "__metadata__ value k"),
    ("leading_zero", blob('{"a":{"dtype":"F32","shape":[1],"data_offsets":[0,04]}}', b"\0" * 4),
     "invalid safetensors header"),
    ("float_shape", blob('{"a":{"dtype":"F32","shape":[1.0],"data_offsets":[0,4]}}', b"\0" * 4), "shape of a"),
    ("negative_shape", blob('{"a":{"dtype":"F32","shape":[-1],"data_offsets":[0,4]}}', b"\0" * 4), "shape of a"),
    ("f4_misaligned", blob("{" + t("a", "F4", [3], 0, 2) + "}", b"\0" * 2), "misaligned size of a"),
    ("f4_even", blob("{" + t("a", "F4", [4], 0, 2) + "}", b"\0" * 2), "ok"),
    ("zero_size", blob("{" + t("z", "F32", [0, 3], 0, 0) + "," + t("a", "F32", [1], 0, 4) + "}", b"\0" * 4), "ok"),
    ("unknown_dtype", blob("{" + t("a", "Q7", [1], 0, 4) + "}", b"\0" * 4), "unknown dtype Q7"),
    ("control_char", blob('{"a\x01":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', b"\0" * 4),
     "control character"),
    ("surrogate_pair", blob('{"\\ud83d\\ude00":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', b"\0" * 4), "ok"),
    ("lone_surrogate", blob('{"\\ud83d":{"dtype":"F32","shape":[1],"data_offsets":[0,4]}}', b"\0" * 4),
     "lone surrogate"),
    ("deep_nesting", blob('{"__metadata__":' + "[" * 100 + "]" * 100 + "}"), "nesting too deep"),
    ("overflow_shape", blob('{"a":{"dtype":"F32","shape":[4294967296,4294967296],"data_offsets":[0,4]}}',
                            b"\0" * 4), "shape of a"),
]


@pytest.fixture(scope="module")
def case_files(tmp_path_factory):
    d_ = tmp_path_factory.mktemp("malformed")
    paths = []
    for name, data, want in CASES:
        p = d_ / f"{name}.safetensors"
        p.write_bytes(data)
        paths.append((name, str(p), want))
    # A header length of 100,000,001 bytes (over the crate's cap, under
    # 100 MiB) in a file that really is that long (sparse).
    p = d_ / "header_over_cap.safetensors"
    with open(p, "wb") as f:
        f.write((100_000_001).to_bytes(8, "little") + b"{")
        f.truncate(8 + 100_000_001)
    paths.append(("header_over_cap", str(p), "header too large"))
    return paths


def test_sanitized_parser_on_malformed_files(driver, case_files):
    out = driver("parse", *[p for _, p, _ in case_files]).splitlines()
    assert len(out) == len(case_files)
    for (name, path, want), line in zip(case_files, out):
        assert line.startswith(path + ": "), line
        got = line[len(path) + 2:]
        if want == "ok":
            assert got.startswith("ok"), (name, got)
        else:
            assert got.startswith("error: ") and want in got, (name, got)


def test_library_rejects_malformed_files(case_files):
    # The same files through the C ABI: every malformed one fails while
    # parsing (before any tensor lookup or GPU work); the well-formed ones
    # parse and then miss the model's first tensor.
    for name, path, want in case_files:
        with pytest.raises(d.DINOv3Error) as e:
            d.DINOv3.load(path, d.Options(max_batch=1))
        if want == "ok":
            assert "missing tensor embeddings.patch_embeddings.weight" in str(e.value), name
        else:
            assert want in str(e.value), (name, str(e.value))


def test_sanitized_pack_kat_and_generator(driver, tmp_path):
    assert driver("pack-kat").strip() == "pack-kat ok"
    for preset in (0, 1):
        out = driver("generate", tmp_path / f"w{preset}.safetensors", preset)
        assert out.startswith("generate ok"), out


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_sanitized_half_checkpoint_packs_like_widened_f32(driver, tmp_path, weight_file, dtype):
    # weights.rs:30-45 widens F16/BF16 to f32 exactly, so a half-precision
    # checkpoint must pack to the same bytes as an F32 file holding the
    # widened values (every blob: f16 GEMM weights, fragment order, folded
    # LayerNorm constants, f32 vectors).
    import torch
    from safetensors.numpy import load_file, save_file
    from safetensors.torch import save_file as save_torch

    src = load_file(weight_file(1))
    tdt = torch.float16 if dtype == "F16" else torch.bfloat16
    half = {k: torch.from_numpy(v).to(tdt) for k, v in src.items()}
    save_torch(half, str(tmp_path / "half.safetensors"))
    save_file({k: v.to(torch.float32).numpy() for k, v in half.items()}, str(tmp_path / "wide.safetensors"))
    out = driver("same-pack", tmp_path / "half.safetensors", tmp_path / "wide.safetensors", 14)
    assert out.startswith("equal"), out
    # and a changed element is seen
    wide = {k: v.to(torch.float32).numpy() for k, v in half.items()}
    wide["layer.7.mlp.down_proj.weight"][3, 5] += 0.25
    save_file(wide, str(tmp_path / "wide2.safetensors"))
    out = driver("same-pack", tmp_path / "half.safetensors", tmp_path / "wide2.safetensors", 14)
    assert out.strip() == "differ l7_down_w", out


def test_sanitized_header_mutations(driver, tmp_path):
    hdr = "{" + ",".join([t("a", "F32", [3, 4], 0, 48), t("b", "F16", [5], 48, 58), t("c", "BF16", [2, 1], 58, 62)]) + "}"
    path = tmp_path / "small.safetensors"
    path.write_bytes(blob('{"__metadata__":{"format":"pt"},' + hdr[1:], bytes(range(62))))
    assert driver("parse", path).strip().endswith("ok 3 62")
    out = driver("mutate", path, 20000, 7)
    ok, rejected = [int(v.split("=")[1]) for v in out.split()[1:]]
    assert ok + rejected == 20000 and rejected > 10000, out
