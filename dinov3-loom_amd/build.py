"""Build recipe for libdinov3_hrx.so: every HIP kernel and host source of the
forward pass is compiled with hipcc for gfx950 (wave64) and linked into one
shared library that exports the C ABI of include/dinov3.h and
include/dinov3_engine.h; the command-line front end lib/dinov3-hrx
(csrc/cli.cpp) links against it. The machine-ceiling probes
(csrc/kernels/probe.hip, include/dinov3_probe.h) go into a library of their
own, lib/libdinov3_probe.so, which only bench.py and the tests load.

    python dinov3-loom_amd/build.py [-j N]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
LIB_DIR = os.path.join(HERE, "lib")
OBJ_DIR = os.path.join(LIB_DIR, "obj")
LIB_PATH = os.path.join(LIB_DIR, "libdinov3_hrx.so")
PROBE_LIB_PATH = os.path.join(LIB_DIR, "libdinov3_probe.so")
CLI_PATH = os.path.join(LIB_DIR, "dinov3-hrx")

PROBE_SOURCES = ["kernels/probe.hip"]
SOURCES = [
    "kernels/gemm.hip",
    "kernels/attention.hip",
    "kernels/norm.hip",
    "engine.cpp",
    "model.cpp",
    "host_copy.cpp",
    "weights.cpp",
    "safetensors.cpp",
]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
# Packed-FP32 instructions stay off in device code (hipcc forms them from
# plain float code otherwise); the host pass warns that it does not know the
# feature, which is harmless.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-I", os.path.join(ROOT, "include"),
          "-Wall", "-Wno-unused-function"]


def _compile_cmd(src: str) -> tuple[list[str], str]:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ_DIR, src.replace("/", "_") + ".o")
    lang = [] if src.endswith(".hip") else ["-x", "hip"]
    return [HIPCC, *COMMON, *DEVICE_FLAGS, *lang, "-c", path, "-o", obj], obj


def build(jobs: int = 8, verbose: bool = False) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    cmds = [_compile_cmd(s) for s in SOURCES + PROBE_SOURCES]
    running: list[tuple[subprocess.Popen, list[str]]] = []
    failed = []

    def reap(block: bool) -> None:
        for proc, cmd in list(running):
            if block or proc.poll() is not None:
                out, _ = proc.communicate()
                text = "\n".join(l for l in out.decode(errors="replace").splitlines() if "packed-fp32-ops" not in l)
                if proc.returncode != 0:
                    failed.append((cmd, text))
                elif verbose and text.strip():
                    print(text)
                running.remove((proc, cmd))

    for cmd, _ in cmds:
        while len(running) >= max(1, jobs):
            reap(block=False)
            if len(running) >= max(1, jobs):
                running[0][0].wait()
        if verbose:
            print(" ".join(cmd))
        running.append((subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT), cmd))
    while running:
        reap(block=True)
    if failed:
        msg = "\n\n".join(" ".join(c) + "\n" + t for c, t in failed)
        raise RuntimeError(f"hipcc failed:\n{msg}")
    probe_objs = [o for _, o in cmds[len(SOURCES):]]
    for path, objs in ((LIB_PATH, [o for _, o in cmds[:len(SOURCES)]]), (PROBE_LIB_PATH, probe_objs)):
        tmp = path + ".tmp"
        subprocess.check_call([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp])
        os.replace(tmp, path)
    build_cli()
    return LIB_PATH


def build_cli() -> str:
    """The command-line front end (csrc/cli.cpp, host code only) linked
    against the library next to it."""
    tmp = CLI_PATH + ".tmp"
    subprocess.check_call([os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-Wall", "-I", os.path.join(ROOT, "include"),
                           os.path.join(CSRC, "cli.cpp"), "-L", LIB_DIR, "-ldinov3_hrx", "-Wl,-rpath,$ORIGIN",
                           "-o", tmp])
    os.replace(tmp, CLI_PATH)
    return CLI_PATH


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("-j", type=int, default=8)
    ap.add_argument("-v", action="store_true")
    a = ap.parse_args()
    print(build(a.j, a.v))
    sys.exit(0)
