"""Build libouro_hip.so (the C-ABI library) in-tree for gfx950.

Each ``csrc/*.hip`` file is compiled to an object in parallel, then linked
into ``ouroboros_amd/lib/libouro_hip.so``.  hipcc cross-compiles, so this runs
on a machine without a GPU.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "lib" / "libouro_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    # Keep the compiler from emitting packed-fp32 VALU instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]

# Flags for one source file only.  kquant.hip, tl1_mfma.hip: MFMA results
# in ordinary VGPRs (the accumulator-register form adds a copy per result
# read; measured faster in both).
FILE_FLAGS = {
    "kquant.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "tl1_mfma.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: Path, verbose: bool) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name; that warning
    # is expected and filtered out.
    noise = "'-packed-fp32-ops' is not a recognized feature"
    msgs = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{msgs}")
    if verbose and msgs.strip():
        print(msgs)
    return obj


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link libouro_hip.so; returns its path."""
    BUILD.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(lambda s: _compile(s, verbose), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs), "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


CPP_TEST_SRC = PKG.parent / "tests" / "cpp" / "reference_kats.cpp"
CPP_TEST_BIN = PKG.parent / "tests" / "cpp" / "reference_kats"


def build_cpp_tests(verbose: bool = False) -> Path:
    """Compile the C++ reference-KAT program against the C++ host mirror
    (include/ouro/infer.hpp) and libouro_hip.so; it runs where a GPU is present."""
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-std=c++17", "-Wall", f"-I{PKG.parent / 'include'}", str(CPP_TEST_SRC),
           "-o", str(CPP_TEST_BIN), f"-L{LIB.parent}", "-louro_hip",
           f"-Wl,-rpath,$ORIGIN/../../ouroboros_amd/lib", "-Wl,-rpath,/opt/rocm/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"C++ test build failed:\n{res.stdout}{res.stderr}")
    if verbose:
        print(f"built {CPP_TEST_BIN}")
    return CPP_TEST_BIN


if __name__ == "__main__":
    build_library(verbose=True)
    build_cpp_tests(verbose=True)
