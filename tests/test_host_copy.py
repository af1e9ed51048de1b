"""The forward pipeline's host copies (dinov3-loom_amd/csrc/host_copy.cpp:
parallel_copy and the copier thread) built host-only with ThreadSanitizer,
and again with AddressSanitizer + UndefinedBehaviorSanitizer (clang++, no
GPU code), driven by tests/host_copy_check.cpp: copy data and bounds at
sizes around the split unit, tickets, submission order (chained copies),
reads after wait() from the submitting thread, and the destructor running
queued copies. The GPU tests cover the same code inside forward()."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CLANG = "/opt/rocm/llvm/bin/clang++"
CSRC = os.path.join(ROOT, "dinov3-loom_amd", "csrc")


def build(tmp_path, sanitize, csrc=CSRC):
    if not os.path.exists(CLANG):
        pytest.skip("clang++ not found")
    exe = str(tmp_path / ("host_copy_" + sanitize.replace(",", "_")))
    subprocess.check_call([CLANG, "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", f"-fsanitize={sanitize}",
                           "-fno-sanitize-recover=all", "-I", csrc, os.path.join(ROOT, "tests", "host_copy_check.cpp"),
                           os.path.join(csrc, "host_copy.cpp"), "-o", exe, "-pthread"])
    return exe


def build_and_run(tmp_path, sanitize, env):
    exe = build(tmp_path, sanitize)
    p = subprocess.run([exe], capture_output=True, text=True, env=dict(os.environ, **env), timeout=600)
    assert p.returncode == 0, f"rc {p.returncode}\n{p.stdout[-2000:]}\n{p.stderr[-4000:]}"
    assert "WARNING: ThreadSanitizer" not in p.stderr and "ERROR: AddressSanitizer" not in p.stderr, p.stderr[-4000:]
    assert p.stdout.startswith("ok "), p.stdout
    return int(p.stdout.split()[1])


def test_host_copies_thread_sanitizer(tmp_path):
    checks = build_and_run(tmp_path, "thread", {"TSAN_OPTIONS": "halt_on_error=1:exitcode=88"})
    assert checks > 400


def test_host_copies_address_sanitizer(tmp_path):
    checks = build_and_run(tmp_path, "address,undefined",
                           {"ASAN_OPTIONS": "detect_leaks=1:exitcode=86", "UBSAN_OPTIONS": "halt_on_error=1:exitcode=87"})
    assert checks > 400


def test_the_thread_sanitizer_build_catches_a_planted_race(tmp_path):
    # The planted mistake, in a copy of the sources: the copier thread counts
    # a finished copy after releasing its lock, while wait() reads the count
    # under the lock on the submitting thread.
    copy = tmp_path / "csrc"
    copy.mkdir()
    for f in ("host_copy.hpp", "host_copy.cpp"):
        shutil.copy(os.path.join(CSRC, f), copy / f)
    src = (copy / "host_copy.cpp").read_text()
    good = "        lock.lock();\n        ++done_;\n"
    assert good in src
    (copy / "host_copy.cpp").write_text(src.replace(good, "        ++done_;\n        lock.lock();\n"))
    exe = build(tmp_path, "thread", str(copy))
    p = subprocess.run([exe], capture_output=True, text=True, timeout=600,
                       env=dict(os.environ, TSAN_OPTIONS="halt_on_error=1:exitcode=88"))
    assert p.returncode == 88 and "data race" in p.stderr, f"rc {p.returncode}\n{p.stderr[-2000:]}"
