"""The C++ header is a source-level drop-in for reference callers.

`tests/compat/reference_style_caller.cpp` is written the way the reference's
own host code calls its API (include/branchcraft.hpp:8-74 of
Haaziq386/branchcraft-cuda; usage as in src/main.cu:130-133,194-199,286,504):
`half` buffers, `Inputs{q, k, v, pages, lengths, out}`, `kWarpsPerBlock` and
the five calls.  It must compile against include/branchcraft.hpp with g++
and with hipcc.  `branchcraft::auto_splits` must stay within the 16 splits
reference callers size Scratch for (src/paged_gqa.cu:126,134-142).
"""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
COMPAT = ROOT / "tests" / "compat"
ROCM = Path("/opt/rocm")
LIBDIR = ROOT / "branchcraft-cuda_amd" / "lib"
FLAGS = ["-std=c++17", "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}",
         f"-I{ROOT / 'include'}"]


def _compile(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    return proc


def test_reference_style_caller_compiles_with_gxx():
    _compile(["g++", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", *FLAGS,
              str(COMPAT / "reference_style_caller.cpp")])


@pytest.mark.skipif(shutil.which("hipcc") is None and not (ROCM / "bin" / "hipcc").exists(),
                    reason="hipcc not installed")
def test_reference_style_caller_compiles_with_hipcc():
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    _compile([hipcc, "-fsyntax-only", "-x", "c++", *FLAGS,
              str(COMPAT / "reference_style_caller.cpp")])


def test_auto_splits_ranges(tmp_path):
    exe = tmp_path / "auto_splits_range"
    _compile(["g++", "-O1", *FLAGS, str(COMPAT / "auto_splits_range.cpp"),
              f"-L{LIBDIR}", f"-L{ROCM / 'lib'}", f"-Wl,-rpath,{LIBDIR}",
              f"-Wl,-rpath,{ROCM / 'lib'}", "-lbranchcraft_hip", "-lamdhip64", "-o", str(exe)])
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout
    rows = [tuple(map(int, line.split())) for line in out.splitlines()]
    assert len(rows) == 10 * 10 * 4
    saw_above_16 = False
    for b, length, cus, capped, uncapped, c_abi in rows:
        assert 1 <= capped <= 16, (b, length, cus, capped)
        assert 1 <= c_abi <= 256, (b, length, cus, c_abi)
        assert uncapped == c_abi
        assert capped == min(c_abi, 16)
        saw_above_16 |= c_abi > 16
        if length < 512:
            # Short contexts stay whole (src/paged_gqa.cu:135) unless the
            # batch fills a wave of flat ranges (4 * CUs / 8 head blocks).
            ranges = 4 * cus // 8
            assert c_abi == (2 if ranges > 1 and b >= ranges else 1), (b, length, cus)
    # The MI355X policy does prefer more than 16 splits somewhere (C4-like
    # shapes), which is why the wrapper caps it.
    assert saw_above_16
