"""The built gfx950 code object of libvgx (CPU test: reads the library this
tree built, runs nothing on a GPU).

- No packed fp32 VALU forms: the Makefile builds the device code with
  -packed-fp32-ops, and this checks that the flag reached the device pass
  (hipcc -O3 forms them from float2 code otherwise).
- No private segment: every kernel's registers fit, nothing spills to
  per-lane scratch.
"""
import os
import re
import shutil
import subprocess

import pytest

from vgx import lib as vl

LLVM = "/opt/rocm/llvm/bin"


@pytest.fixture(scope="module")
def code_objects(tmp_path_factory):
    path = os.path.join(vl.PKG, "lib", "libvgx.so")
    if not os.path.exists(path):
        pytest.skip("libvgx is not built")
    if not os.path.exists(os.path.join(LLVM, "llvm-objdump")):
        pytest.skip("llvm-objdump missing")
    d = tmp_path_factory.mktemp("co")
    shutil.copy(path, d / "libvgx.so")
    subprocess.run([os.path.join(LLVM, "llvm-objdump"), "--offloading", "libvgx.so"], cwd=d, check=True,
                   stdout=subprocess.DEVNULL)
    cos = sorted(p for p in d.iterdir() if p.name.endswith("gfx950"))
    assert cos, "no gfx950 code object in libvgx.so"
    return cos


def test_no_packed_fp32(code_objects):
    packed = re.compile(r"\bv_pk_(add|mul|fma)_f32\b")
    n_kernels = 0
    for co in code_objects:
        asm = subprocess.run([os.path.join(LLVM, "llvm-objdump"), "-d", str(co)], check=True,
                             capture_output=True, text=True).stdout
        n_kernels += asm.count(">:\n")
        hits = packed.findall(asm)
        assert not hits, (co.name, len(hits))
    assert n_kernels > 100


def test_no_private_segment(code_objects):
    sizes = []
    for co in code_objects:
        notes = subprocess.run([os.path.join(LLVM, "llvm-readelf"), "--notes", str(co)], check=True,
                               capture_output=True, text=True).stdout
        sizes += [int(v) for v in re.findall(r"\.private_segment_fixed_size:\s*(\d+)", notes)]
    assert len(sizes) > 100
    assert max(sizes) == 0
