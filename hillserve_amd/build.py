"""Build the gfx950 library in-tree: hillserve_amd/libhillserve_amd.so.

Every HIP source under hillserve_amd/csrc is compiled with hipcc for gfx950
(no other architecture), then linked into one shared library whose exported
symbols are the C ABI declared in include/hs_gpu.h.  The C++17 host adapters
(csrc/gqa_gpu.cpp) are linked into the same library, and their contract
test executable (tests/cpp/gqa_gpu_contracts) is linked against it.
Usage:  python -m hillserve_amd.build  (or __graft_entry__.build()).
"""
from __future__ import annotations

import concurrent.futures as futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "hillserve_amd"
CSRC = PKG / "csrc"
OBJ = ROOT / "_build" / "obj"
LIB = PKG / "libhillserve_amd.so"
# C++ contract tests of the host adapters (built next to their source)
CONTRACTS = ROOT / "tests" / "cpp" / "gqa_gpu_contracts"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
# host-only C++ that calls the HIP runtime API
HOST = [f"-I{ROCM / 'include'}", "-D__HIP_PLATFORM_AMD__", "-x", "c++"]

# Flags for device code.  -packed-fp32-ops keeps the compiler from forming
# v_pk_{add,mul,fma}_f32; -ffp-contract=off means every FMA in the kernels is
# one the source asks for (the bit-exact scorer depends on that).
COMMON = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
    "-ffp-contract=off",
    "-Wall",
    "-Wno-unused-command-line-argument",
]
DEVICE = [
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-munsafe-fp-atomics",
]

HIP_SOURCES = ["score.hip", "select.hip", "attention.hip", "pack.hip", "rehearsal.hip",
               "kv_store.hip", "runtime.hip"]
HOST_SOURCES = ["gqa_gpu.cpp", "host_common.cpp", "kv_image.cpp"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        sys.stderr.write(proc.stdout + proc.stderr)
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")
    noise = [
        line
        for line in (proc.stdout + proc.stderr).splitlines()
        if "packed-fp32-ops" not in line and line.strip()
    ]
    if noise:
        sys.stderr.write("\n".join(noise) + "\n")


def _compile(src: Path) -> Path:
    obj = OBJ / (src.name + ".o")
    if src.suffix == ".hip":
        cmd = [HIPCC, *COMMON, *DEVICE, "-c", str(src), "-o", str(obj)]
    else:  # host-only C++17 translation unit that calls the C ABI / HIP runtime
        cmd = [HIPCC, *COMMON, *HOST, "-c", str(src), "-o", str(obj)]
    _run(cmd)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile all sources and link the shared library; returns its path."""
    if not Path(HIPCC).exists() and shutil.which(HIPCC) is None:
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    OBJ.mkdir(parents=True, exist_ok=True)
    sources = [CSRC / s for s in HIP_SOURCES + HOST_SOURCES if (CSRC / s).exists()]
    jobs = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, sources))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB)
    test_src = CONTRACTS.with_suffix(".cpp")
    if test_src.exists():
        _run([HIPCC, *COMMON, *HOST, str(test_src), "-x", "none", "-o", str(CONTRACTS),
              f"-L{PKG}", "-lhillserve_amd", f"-L{ROCM / 'lib'}", "-lamdhip64",
              "-Wl,-rpath,$ORIGIN/../../hillserve_amd"])
    if verbose:
        print(f"built {LIB.relative_to(ROOT)} ({LIB.stat().st_size} bytes) for {ARCH}")
    return LIB


if __name__ == "__main__":
    build()
