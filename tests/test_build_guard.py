"""The gfx950 machine code this build produced, checked on the CPU.

Several kernels must round q * scale to f32 and then to f16 the same way, or a tree row no
longer equals its line and a fused step no longer equals its two calls. hipcc has contracted
that multiply-and-convert into one mixed-precision FMA (v_fma_mix*, a single rounding) despite
-ffp-contract=off, in some kernels and not others. The source keeps the two roundings with
an empty asm between them. This test reads the code objects the library's build left in
borrowed-compute_amd/_build and fails if any mixed-precision FMA reaches the attention object,
so a later compiler that finds another fold fails here before any GPU run.

It also checks that no object holds packed f32 arithmetic. The build turns it off with
-packed-fp32-ops, because some of its forms gave wrong results on these machines.
"""
import glob
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BUILD = os.path.join(ROOT, "borrowed-compute_amd", "_build")
LLVM = "/opt/rocm/llvm/bin"
TARGET = "hipv4-amdgcn-amd-amdhsa--gfx950"


def _disassemble(obj, tmp_path):
    """The gfx950 code object embedded in a host object (its .hip_fatbin bundle), as text."""
    fat = tmp_path / (os.path.basename(obj) + ".fatbin")
    host = tmp_path / (os.path.basename(obj) + ".host")
    code = tmp_path / (os.path.basename(obj) + ".co")
    subprocess.run([f"{LLVM}/llvm-objcopy", f"--dump-section=.hip_fatbin={fat}", obj, str(host)], check=True)
    subprocess.run([f"{LLVM}/clang-offload-bundler", "--type=o", f"--targets={TARGET}", f"--input={fat}",
                    f"--output={code}", "--unbundle"], check=True)
    return subprocess.run([f"{LLVM}/llvm-objdump", "-d", str(code)], capture_output=True, text=True,
                          check=True).stdout


def _objects():
    objs = sorted(glob.glob(os.path.join(BUILD, "*.o")))
    if not objs or not os.path.exists(f"{LLVM}/clang-offload-bundler"):
        pytest.skip("no library build in borrowed-compute_amd/_build (run __graft_entry__.build())")
    return objs


def _instructions(text, pattern):
    return [l.strip() for l in text.splitlines() if re.search(pattern, l)]


def test_attention_code_has_no_mixed_precision_fma(tmp_path):
    objs = [o for o in _objects() if os.path.basename(o) == "attention.o"]
    assert objs, "attention.o missing from the build"
    text = _disassemble(objs[0], tmp_path)
    assert len(_instructions(text, r"\bv_mfma_f32_16x16x32_f16\b")) > 100, "not the attention kernels"
    found = _instructions(text, r"\bv_fma_mix")
    assert not found, f"{len(found)} mixed-precision FMAs in attention.o, e.g. {found[:3]}"


def test_no_packed_f32_arithmetic(tmp_path):
    for obj in _objects():
        text = _disassemble(obj, tmp_path)
        found = _instructions(text, r"\bv_pk_(add|mul|fma)_f32\b")
        assert not found, f"{os.path.basename(obj)}: {found[:3]}"
