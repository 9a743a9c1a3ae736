"""Writes tests/golden/config1.npz from the reference's OWN hot-path code.

The vectors come from oracle/_ref/libhsref.so — FullGqaCpuScorer::score
(policy/full_gqa_cpu.cpp), the runtime scaling expression
(policy/full_gqa_runtime.cpp:571, evaluated with the reference's half
functions) and select_gqa_scores (policy/gqa_policy.cpp:47-70) — compiled from
/root/reference by oracle/Makefile.  Inputs are regenerated from the seed by
tests/hs_data.config1_inputs; their SHA-256 is stored to detect drift.

Q[32,128] ~ N(0,1), K[4096,8,128] ~ N(0,1) with 4
per-channel outliers x8, seed 0; alpha 0.1, cap ratio 0.2f.
Run:  python tests/golden/make_golden.py
"""
import hashlib
import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parent.parent))

import oracle  # noqa: E402
from hs_data import config1_inputs  # noqa: E402

N, ALPHA, RATIO = 4096, 0.1, 0.2


def digest(*arrays):
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def main():
    ref = oracle.ref()
    if ref is None:
        raise SystemExit("oracle/_ref is not built (needs /root/reference)")
    q, k, outliers = config1_inputs(0, N)
    raw = ref.score(q, k.reshape(-1), N, 1024, threads=4, impl=0)
    root = np.float32(math.sqrt(128.0))
    table = np.array([ref.L.hsref_half_bits(float(np.float32(ref.L.hsref_half_value(b)) / root))
                      for b in range(65536)], dtype=np.uint16)
    scaled = table[raw]
    rc, k_sel, ids, counts, tied = ref.select(scaled, 32, N, N, ALPHA, RATIO, width=N)
    assert rc == 0, k_sel
    np.savez_compressed(
        HERE / "config1.npz", inputs_sha256=np.array(digest(q, k)), outliers=outliers,
        raw=raw, scaled=scaled, k=np.array(k_sel), ids=ids, counts=counts,
        boundary_tied_heads=np.array(tied), alpha=np.array(ALPHA, dtype=np.float32),
        ratio=np.array(RATIO, dtype=np.float32), n=np.array(N))
    print(f"config1: k={k_sel} counts[0:4]={counts[:4]} tied={tied} "
          f"sha={digest(q, k)[:16]}")


if __name__ == "__main__":
    main()
