"""In-tree build of the Branchcraft MI355X libraries.

* ``lib/libbranchcraft_hip.so`` -- the HIP kernels for gfx950 and the C ABI
  declared in ``include/branchcraft.h`` (hipcc, one object per source).
* ``python/branchcraft_torch/_C.so`` -- the PyTorch dispatcher ops, a plain
  C++ translation unit compiled against PyTorch-ROCm and linked to the
  library above (no hipify step).

Run ``python branchcraft-cuda_amd/build.py`` or call :func:`build`.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIBDIR = PKG / "lib"
LIB = LIBDIR / "libbranchcraft_hip.so"
TORCH_EXT = PKG / "python" / "branchcraft_torch" / "_C.so"
HIP_SOURCES = ["decode.hip", "tree_verify.hip", "commit.hip", "slots.hip"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

# Packed-FP32 VALU forms (v_pk_{add,mul,fma}_f32) are switched off for every
# kernel; the compiler otherwise forms them from plain float code.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
]


def _run(cmd: list[str], cwd: Path | None = None) -> None:
    proc = subprocess.run(cmd, cwd=cwd, stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True)
    # hipcc's host pass does not know the packed-fp32 feature flag; drop
    # that known-harmless line from the log.
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "is not a recognized feature for this target" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def build_hip_library() -> Path:
    hipcc = shutil.which("hipcc") or str(ROCM / "bin" / "hipcc")
    BUILD.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = []
    procs = []
    for src in HIP_SOURCES:
        obj = BUILD / (Path(src).stem + ".o")
        objs.append(obj)
        cmd = [hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]
        procs.append((cmd, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT, text=True)))
    for cmd, proc in procs:
        out, _ = proc.communicate()
        out = "\n".join(line for line in out.splitlines()
                        if "is not a recognized feature for this target" not in line)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc failed: {' '.join(cmd)}\n{out}")
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *map(str, objs),
          "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_torch_extension() -> Path:
    import torch
    from torch.utils import cpp_extension

    inc = cpp_extension.include_paths()
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = ["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-DTORCH_EXTENSION_NAME=_C",
           f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}",
           *[f"-I{p}" for p in inc],
           str(CSRC / "torch_ops.cpp"),
           *[f"-L{p}" for p in libdirs], f"-L{LIBDIR}", f"-L{ROCM / 'lib'}",
           "-lbranchcraft_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           "-ltorch_hip", "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../lib",
           *[f"-Wl,-rpath,{p}" for p in libdirs],
           "-o", str(TORCH_EXT.with_suffix(".so.tmp"))]
    _run(cmd)
    os.replace(TORCH_EXT.with_suffix(".so.tmp"), TORCH_EXT)
    return TORCH_EXT


def build() -> None:
    build_hip_library()
    build_torch_extension()


if __name__ == "__main__":
    build()
    print(f"built {LIB} and {TORCH_EXT}", file=sys.stderr)
