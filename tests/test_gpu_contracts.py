"""The reference's own C++ contract cases, run through the C++17 host
adapters (include/hs_gqa.hpp) on the GPU, and the layer-pipelining C calls
against the single calls: tests/cpp/gqa_gpu_contracts."""
import json
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

CONTRACTS = Path(__file__).resolve().parent / "cpp" / "gqa_gpu_contracts"


def test_cpp_contracts(hs):
    assert CONTRACTS.exists(), "run python -m hillserve_amd.build"
    print(f"running {CONTRACTS.name}", flush=True)
    proc = subprocess.run([str(CONTRACTS)], capture_output=True, text=True, timeout=240)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    report = json.loads(proc.stdout.strip().splitlines()[-1])
    assert report["status"] == "passed" and report["cases"] > 100, report
