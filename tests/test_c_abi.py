"""The C ABI from plain C (CPU only): include/hs_gpu.h compiles as strict C99
and C11 (-pedantic -Werror, no C++), and a C program linked against
libhillserve_amd.so calls entry points that answer without a GPU: the
version string, a workspace size, and argument rejections that return
HS_ERR_ARGUMENT with a message and touch no memory.  This is what a cgo, JNI
or ctypes binding of the library relies on."""
import os
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

PROGRAM = r'''
#include <stdio.h>
#include <string.h>
#include "hs_gpu.h"

int main(void) {
    int failures = 0;
    const char *v = hs_version();
    if (v == NULL || strstr(v, "gfx950") == NULL) { puts("version"); ++failures; }
    if (hs_gqa_select_workspace_bytes(32, 32768) == 0) { puts("workspace size"); ++failures; }
    /* an invalid token count is refused before any memory access
       (kernels/full_gqa_pipeline/kernel.cpp:251): null pointers are never read */
    if (hs_full_gqa_pipeline(NULL, NULL, NULL, 100, NULL) != HS_ERR_ARGUMENT) { puts("v3 count"); ++failures; }
    if (strlen(hs_last_error()) == 0) { puts("message"); ++failures; }
    if (hs_gqa_select(NULL, 0, 0, 0, 1.0f, 0.2f, 0, NULL, NULL, 0, NULL, NULL, NULL, NULL, NULL)
        != HS_ERR_ARGUMENT) { puts("select heads"); ++failures; }
    printf("{\"failures\":%d}\n", failures);
    return failures;
}
'''


def _no_gpu():
    import torch
    if torch.cuda.is_available():
        pytest.skip("CPU-only ABI check (a GPU is visible)")


@pytest.mark.parametrize("std", ["c99", "c11"])
def test_header_is_strict_c(tmp_path, std):
    src = tmp_path / "hdr.c"
    src.write_text('#include "hs_gpu.h"\nint main(void) { return 0; }\n')
    subprocess.run(["gcc", f"-std={std}", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    f"-I{ROOT / 'include'}", "-c", str(src), "-o", str(tmp_path / "hdr.o")],
                   check=True)


def test_c_program_links_and_calls(tmp_path):
    _no_gpu()
    lib_dir = ROOT / "hillserve_amd"
    assert (lib_dir / "libhillserve_amd.so").exists(), "run python -m hillserve_amd.build"
    src = tmp_path / "abi.c"
    src.write_text(PROGRAM)
    exe = tmp_path / "abi"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Wextra", "-pedantic", "-Werror",
                    f"-I{ROOT / 'include'}", str(src), f"-L{lib_dir}", "-lhillserve_amd",
                    f"-Wl,-rpath,{lib_dir}:{ROCM / 'lib'}", "-o", str(exe)], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert '"failures":0' in proc.stdout, proc.stdout
