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


def test_pair_keys_all_finite_inputs(hs, port):
    # the selection's two-at-a-time order keys (scaled and raw) against the
    # oracle's order_key(scale(b)) / order_key(b) for every finite pattern
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    dev = hs.ops.selftest_key_table().cpu().numpy().view(np.uint16)
    finite = (raw & 0x7C00) != 0x7C00
    scaled = port.scale(raw)
    want_scaled = np.array([port.order_key(int(b)) for b in scaled], dtype=np.uint16)
    want_raw = np.array([port.order_key(int(b)) for b in raw], dtype=np.uint16)
    for row, want, label in ((0, want_scaled, "scaled"), (1, want_raw, "raw")):
        bad = np.nonzero((dev[row] != want) & finite)[0]
        detail = [(hex(int(raw[i])), hex(int(dev[row][i])), hex(int(want[i]))) for i in bad[:12]]
        assert bad.size == 0, f"{label}: {bad.size} mismatches (input, device, oracle): {detail}"
    # -0 and +0 share a key
    assert dev[0][0x8000] == dev[0][0] == 0x8000 and dev[1][0x8000] == dev[1][0] == 0x8000
