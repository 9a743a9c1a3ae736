"""GPU rehearsal-query producer (MFMA) against the FP64 oracle.

Parity is unpinned against the reference (ggml b6000 arithmetic is absent);
the bar here is the F16 output within 1e-3 of the largest |q| of the
sequence and, for every element of at least 1/64 of that largest |q|, within
2 F16 ulps of the F16-rounded FP64 value (the only roundings are FP32
accumulation and the final F16 conversion; on smaller values FP32
cancellation can exceed 2 ulps of their own size)."""
import ctypes

import numpy as np
import pytest
import torch

from hs_data import rng

pytestmark = pytest.mark.gpu

THETA, EPS = 500000.0, 1e-5


def bf16(x):
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def to_bf16_dev(bits):
    return torch.from_numpy(bits.view(np.int16)).cuda().view(torch.bfloat16)


def ulps(a, b):
    ia = a.astype(np.int32)
    ib = b.astype(np.int32)
    ka = np.where(ia & 0x8000, 0x8000 - (ia & 0x7FFF), 0x8000 + ia)
    kb = np.where(ib & 0x8000, 0x8000 - (ib & 0x7FFF), 0x8000 + ib)
    return np.abs(ka - kb)


@pytest.mark.parametrize("batch", [1, 3, 16])
def test_matches_fp64_oracle(hs, port, batch):
    g = rng(batch)
    hidden = bf16(g.standard_normal((batch, 4096)).astype(np.float32) * 3.0)
    wq = bf16(g.standard_normal((4096, 4096)).astype(np.float32) * 0.02)
    positions = [int(p) for p in g.integers(0, 32768, size=batch)]
    positions[0] = 0
    q, status = hs.ops.rehearsal_query(to_bf16_dev(hidden), to_bf16_dev(wq), positions,
                                       eps=EPS, theta=THETA)
    got = q.cpu().view(torch.int16).numpy().view(np.uint16).reshape(batch, 4096)
    assert np.all(status.cpu().numpy()[:, 0] == 0)
    for b in range(batch):
        ref = port.rehearsal(hidden[b], wq, positions[b], eps=EPS, theta=THETA).reshape(-1)
        val = got[b].view(np.float16).astype(np.float64)
        assert np.max(np.abs(val - ref)) <= 1e-3 * np.max(np.abs(ref)), b
        ref16 = ref.astype(np.float16).view(np.uint16)
        big = np.abs(ref) >= np.max(np.abs(ref)) / 64
        assert ulps(got[b][big], ref16[big]).max() <= 2, b


def test_status_flags(hs):
    hidden = np.full((3, 4096), bf16(1.0), dtype=np.uint16)
    hidden[1, 5] = 0x7F80  # +inf in sequence 1: nonfinite
    wq = np.zeros((4096, 4096), dtype=np.uint16)
    wq[:, :] = bf16(0.01)
    wq[7, :] = bf16(32.0)  # feature 7: 32 * 4096 = 131072 > 65504 for unit rows
    q, status = hs.ops.rehearsal_query(to_bf16_dev(hidden), to_bf16_dev(wq), [0, 0, 0],
                                       eps=EPS, theta=THETA)
    codes = status.cpu().numpy()[:, 0]
    assert codes[1] == hs.HS_ERR_NONFINITE
    assert codes[0] == hs.HS_ERR_OVERFLOW and codes[2] == hs.HS_ERR_OVERFLOW


def test_status_precedence_across_tiles_and_stale_status(hs):
    """One launch publishes every sequence's status itself (no clearing, no
    second launch): a NONFINITE found by one tile of a sequence outranks an
    OVERFLOW found by another tile, and a stale status word is replaced."""
    hidden = np.full((2, 4096), bf16(1.0), dtype=np.uint16)
    hidden[1, :2] = 0  # sequence 1 does not see Wq's huge columns 0 and 1
    wq = np.full((4096, 4096), bf16(0.01), dtype=np.uint16)
    wq[7, :] = bf16(32.0)          # feature 7 (tile 0): beyond F16 for both sequences
    wq[20, :2] = bf16(3.0e38)      # feature 20 (tile 1): 6e38 -> inf in FP32 for sequence 0
    hd, wd = to_bf16_dev(hidden), to_bf16_dev(wq)  # held until the launches are done
    for stale in (hs.HS_OK, hs.HS_ERR_NONFINITE):
        out = torch.empty((2, 32, 128), dtype=torch.float16, device="cuda")
        status = torch.full((2, 4), stale, dtype=torch.int32, device="cuda")
        status[:, 1] = -5  # a stamp-like k from an earlier call
        L = hs.lib()
        pos = (ctypes.c_uint32 * 2)(0, 0)
        hs.check(L.hs_rehearsal_query(hd.data_ptr(), wd.data_ptr(),
                                      ctypes.cast(pos, ctypes.c_void_p), 2, EPS, THETA,
                                      out.data_ptr(), status.data_ptr(), None, None))
        codes = status.cpu().numpy()[:, 0]
        assert codes[0] == hs.HS_ERR_NONFINITE and codes[1] == hs.HS_ERR_OVERFLOW, (stale, codes)
