"""AddressSanitizer + UndefinedBehaviorSanitizer builds of the host code, run
on the CPU (as the reference runs its CPU tests under ASan + UBSan,
CMakeLists.txt:10-14):

* the oracle (oracle/hs_oracle.c, with its malloc'd attention scratch),
  built with gcc and driven by every oracle test through HS_ORACLE_LIB;
* the C++ host adapters (hillserve_amd/csrc/gqa_gpu.cpp: the chunked-stream
  planner, pinned buffers, pread loops), the host error helpers and the
  SegmentedKVStore image writer (kv_image.cpp), built with g++ into the
  contract program, whose host-only cases (the reference planner's known
  answers, 200 random region lists, the image writer) run without a GPU.

Only g++ / gcc build these (no device code is sanitized); outputs go to a
temporary directory."""
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
SAN = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
       "-fno-omit-frame-pointer"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _gcc_file(name):
    return subprocess.run(["gcc", f"-print-file-name={name}"], capture_output=True, text=True,
                          check=True).stdout.strip()


def _no_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("CPU-only sanitizer run (a GPU is visible)")


def _clean(out):
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert "ERROR: LeakSanitizer" not in out, out[-4000:]


def test_oracle_under_asan_ubsan(tmp_path):
    lib = tmp_path / "liboracle_san.so"
    subprocess.run(["gcc", "-std=c11", "-fPIC", "-ffp-contract=off", "-Wall", *SAN, "-shared",
                    "-o", str(lib), str(ROOT / "oracle" / "hs_oracle.c"), "-lm", "-pthread"],
                   check=True)
    env = dict(os.environ)
    # the sanitizer runtime first; libstdc++ beside it, so that the compiled
    # reference (oracle/_ref, not instrumented) can throw through ASan's
    # __cxa_throw interceptor.  Python's own allocations are not leak-checked.
    env["LD_PRELOAD"] = f"{_gcc_file('libasan.so')} {_gcc_file('libstdc++.so.6')}"
    env["ASAN_OPTIONS"] = "detect_leaks=0:abort_on_error=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["HS_ORACLE_LIB"] = str(lib)
    tests = sorted(str(p) for p in (ROOT / "tests").glob("test_oracle_*.py"))
    tests.append(str(ROOT / "tests" / "test_golden.py"))
    proc = subprocess.run([sys.executable, "-m", "pytest", "-q", "-x", "-p", "no:cacheprovider",
                           "-m", "not gpu", *tests], capture_output=True, text=True, env=env,
                          cwd=str(ROOT), timeout=900)
    out = proc.stdout + proc.stderr
    _clean(out)
    assert proc.returncode == 0 and " passed" in out, out[-4000:]


def test_host_adapters_under_asan_ubsan(tmp_path):
    _no_gpu()
    exe = tmp_path / "contracts_san"
    csrc = ROOT / "hillserve_amd" / "csrc"
    lib_dir = ROOT / "hillserve_amd"
    assert (lib_dir / "libhillserve_amd.so").exists(), "run python -m hillserve_amd.build"
    # the instrumented host sources come first on the link line, so their
    # definitions serve the program; the library supplies the device entry
    # points, which the host-only cases never call
    subprocess.run(["g++", "-std=c++17", "-Wall", *SAN, f"-I{ROOT / 'include'}", f"-I{csrc}",
                    f"-I{ROCM / 'include'}", "-D__HIP_PLATFORM_AMD__",
                    str(ROOT / "tests" / "cpp" / "gqa_gpu_contracts.cpp"),
                    str(csrc / "gqa_gpu.cpp"), str(csrc / "host_common.cpp"),
                    str(csrc / "kv_image.cpp"), f"-L{lib_dir}", "-lhillserve_amd",
                    f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{lib_dir}:{ROCM / 'lib'}",
                    "-o", str(exe)], check=True)
    env = dict(os.environ)
    env["ASAN_OPTIONS"] = "abort_on_error=1:detect_leaks=1"
    env["UBSAN_OPTIONS"] = "halt_on_error=1:print_stacktrace=1"
    env["LSAN_OPTIONS"] = f"suppressions={ROOT / 'tests' / 'cpp' / 'lsan_hip_runtime.supp'}"
    proc = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=300)
    out = proc.stdout + proc.stderr
    _clean(out)
    # 77: every host-only case passed, then no GPU was found for the rest
    assert proc.returncode == 77 and "skipped" in proc.stdout, out[-4000:]
