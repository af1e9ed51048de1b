"""Static check of the DMA waits in the kernels' K loops, on the gfx950
assembly this build produces (CPU only: hipcc cross-compiles).

The GEMM and attention kernels move weight stages (GEMMs) or K/V blocks
(attention) into LDS with DMA loads (`buffer_load_dwordx4 ... lds`) and end
each step with `s_waitcnt vmcnt(N)` + `s_barrier`, letting the N newest
vector-memory operations stay in flight. On this GPU DMA loads land in
issue order among themselves but are not ordered against register loads
(a two-buffer loop whose wait counted later register loads returned
different results from launch to launch), so such a wait proves that an
older stage has landed only if the N operations it lets stay in flight are
all DMA loads: every step issues its register loads before its DMA loads.
This test checks that rule on every barrier-ending wait with N > 0 of every
kernel, in the code the compiler actually emitted (a reordering by the
compiler or by a later edit of the K loop would break it silently, showing
only as rare run-to-run differences on the GPU). A negative control plants
the mistake in a copy of the GEMM core (the step's DMA issued before its
register loads) and checks that the test would catch it.

A second check on the same assembly: the attention kernels touch global
memory only through 16-byte Q fragment loads, buffer (DMA) loads and buffer
stores; everything else, such as the split-key kernel's hand-over between
its key halves, stays in LDS."""
import os
import re
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KERNELS = os.path.join(ROOT, "dinov3-loom_amd", "csrc", "kernels")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
# The flags of dinov3-loom_amd/build.py for device code.
FLAGS = ["-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang",
         "-packed-fp32-ops", "--cuda-device-only", "-S"]
VMEM = re.compile(r"^(global_|buffer_|flat_|scratch_)")


def assembly(src, out, include):
    subprocess.check_call([HIPCC, *FLAGS, "-I", os.path.join(ROOT, "include"), "-I", include, src, "-o", out],
                          stderr=subprocess.DEVNULL)
    kernels, cur = {}, None
    for line in open(out):
        m = re.match(r"^(_Z\S+):", line)
        if m and "kernel" in m.group(1):
            cur = m.group(1)
            kernels[cur] = []
            continue
        s = line.strip()
        if cur is None or not s or s.startswith((";", ".")):
            continue
        kernels[cur].append(s)
        if s.startswith("s_endpgm"):
            cur = None
    return kernels


def is_dma(ins):
    return ins.startswith("buffer_load") and " lds" in ins


def violations(instructions):
    """(checked waits, violations): for each `s_waitcnt vmcnt(N)` right
    before an `s_barrier` with N > 0, the N vector-memory instructions
    issued last before it must all be DMA loads."""
    checked, bad = 0, []
    for i, ins in enumerate(instructions):
        if not ins.startswith("s_barrier") or i == 0 or not instructions[i - 1].startswith("s_waitcnt"):
            continue
        m = re.search(r"vmcnt\((\d+)\)", instructions[i - 1])
        if not m or int(m.group(1)) == 0:
            continue
        n, tail = int(m.group(1)), []
        for prev in reversed(instructions[:i - 1]):
            if VMEM.match(prev):
                tail.append(prev)
                if len(tail) == n:
                    break
        checked += 1
        if len(tail) < n or not all(is_dma(t) for t in tail):
            bad.append((instructions[i - 1], tail))
    return checked, bad


@pytest.fixture(scope="module")
def hipcc():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not found")
    return HIPCC


def test_every_k_loop_wait_counts_dma_only(hipcc, tmp_path):
    found = {}
    for src in ("gemm.hip", "attention.hip"):
        for name, ins in assembly(os.path.join(KERNELS, src), str(tmp_path / (src + ".s")), KERNELS).items():
            checked, bad = violations(ins)
            assert not bad, f"{name}: {bad[:2]}"
            if any(is_dma(i) for i in ins):
                # every DMA-fed kernel has at least one wait that lets DMA stay in flight
                assert checked > 0, name
            short = re.sub(r"^_ZN3dhx(12_GLOBAL__N_1)?\d*(4gemm)?\d+", "", name)[:40]
            found[short] = checked
    print(found)
    for kernel in ("qkv_rope_kernel", "resid_kernel", "swiglu_kernel", "splitk_kernel", "attention_kernel",
                   "attention_split_kernel"):
        assert any(k.startswith(kernel) and v > 0 for k, v in found.items()), kernel


def test_the_check_catches_dma_issued_before_register_loads(hipcc, tmp_path):
    # The planted mistake: in a copy of the GEMM core, each K-loop step issues
    # its weight DMA before the next stage's activation loads.
    copy = tmp_path / "kernels"
    shutil.copytree(KERNELS, copy)
    core = copy / "gemm_core.hpp"
    text = core.read_text()
    right = ("        if (s + 1 < k_tiles) next.load(m0, n0, s + 1, tid);\n        compiler_fence();\n"
             "        if (more) wd.load(fill, n0, s + 2, tid);\n")
    wrong = ("        if (more) wd.load(fill, n0, s + 2, tid);\n        compiler_fence();\n"
             "        if (s + 1 < k_tiles) next.load(m0, n0, s + 1, tid);\n")
    assert text.count(right) == 1
    core.write_text(text.replace(right, wrong))
    kernels = assembly(str(copy / "gemm.hip"), str(tmp_path / "gemm_wrong.s"), str(copy))
    caught = [name for name, ins in kernels.items() if violations(ins)[1]]
    print(f"{len(caught)} of {len(kernels)} GEMM kernels flagged")
    for kernel in ("qkv_rope_kernel", "resid_kernel", "swiglu_kernel", "splitk_kernel"):
        assert any(kernel in name for name in caught), kernel


def test_attention_kernels_touch_global_memory_only_as_designed(hipcc, tmp_path):
    # A form of the split-key kernel's merge (its LDS buffers picked through
    # pointer tables declared inside a lambda's `if constexpr` branches) came
    # out of this compiler as 32-bit global stores and loads near address 0,
    # which fault on the GPU; every attention kernel is held to the designed
    # set of global-memory instructions (Q fragments as 16-byte loads, K and V
    # as DMA loads, the output as 16-byte buffer stores).
    kernels = assembly(os.path.join(KERNELS, "attention.hip"), str(tmp_path / "attention.s"), KERNELS)
    assert any("attention_split_kernel" in k for k in kernels)
    for name, ins in kernels.items():
        for i in ins:
            op = i.split()[0]
            if op.startswith(("global_", "flat_", "scratch_")):
                assert op == "global_load_dwordx4", f"{name}: {i}"
            elif op.startswith("buffer_store"):
                assert op == "buffer_store_dwordx4", f"{name}: {i}"
