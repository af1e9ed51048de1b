"""CPU regression test for the base address of the write-through store
descriptors (WtOut, dinov3-loom_amd/csrc/kernels/common.hpp): the two words
of the base come back from __builtin_amdgcn_readfirstlane as int, and each
must be widened through uint32_t. A low word with bit 31 set, widened as a
signed int, once produced bases of 0xffffffff'xxxxxxxx whose stores faulted.
tests/descriptor_base.cpp checks address_from_words, the helper WtOut uses,
on low words 0x7fffffff, 0x80000000, 0xffffffff and others with zero and
nonzero high words, and shows that the same cases reject the signed
widening."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


def test_address_from_words(tmp_path):
    if not (os.path.exists(HIPCC) or shutil.which("hipcc")):
        pytest.skip("hipcc not found")
    exe = str(tmp_path / "descriptor_base")
    subprocess.check_call([HIPCC, "-std=c++17", "-O2", "--offload-arch=gfx950", "--cuda-host-only",
                           "-I", os.path.join(ROOT, "dinov3-loom_amd", "csrc"),
                           os.path.join(ROOT, "tests", "descriptor_base.cpp"), "-o", exe])
    p = subprocess.run([exe], capture_output=True, text=True, timeout=60)
    print(p.stdout)
    assert p.returncode == 0, p.stdout + p.stderr
    assert "0 failures" in p.stdout
