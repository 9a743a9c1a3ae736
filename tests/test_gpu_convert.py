"""Exhaustive checks of the device conversion units against the oracle."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def test_f32_to_f16_all_patterns(hs, port):
    # all 2^32 FP32 patterns through v_cvt_f16_f32, folded per high half
    dev = hs.ops.selftest_f16_checksums().cpu().numpy().view(np.uint64)
    host = port.f16_checksums(16)
    bad = np.nonzero(dev != host)[0]
    assert bad.size == 0, f"F16 conversion differs in {bad.size} chunks, first {bad[:8]}"


def test_scale_table_all_inputs(hs, port):
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dev = hs.ops.selftest_scale_table().cpu().numpy().view(np.uint16)
    host = port.scale(raw)
    # every input, inf and NaN included (NaN maps to the canonical sign|0x7e00)
    bad = np.nonzero(dev != host)[0]
    detail = [(hex(int(raw[i])), hex(int(dev[i])), hex(int(host[i]))) for i in bad[:12]]
    assert bad.size == 0, f"{bad.size} mismatches (input, device, oracle): {detail}"
