"""Pins of the ordered-FP32 scorer and the scaling rule (oracle, CPU)."""
import math

import numpy as np
import pytest

from hs_data import H, KH, D, markers_v3, mixed_finite, rng, v3_sample


def brute_force(q, k, n, stride):
    """Per-score sequential FP32 loop in numpy (each op rounds to float32)."""
    qf = q.view(np.float16).astype(np.float32).reshape(H, D)
    rows = k.view(np.float16).astype(np.float32)
    out = np.empty((H, n), dtype=np.uint16)
    keys = np.stack([rows[t * stride: t * stride + KH * D].reshape(KH, D) for t in range(n)])
    for h in range(H):
        s = np.zeros(n, dtype=np.float32)
        kk = keys[:, h // 4, :]
        for c in range(D):
            s = (s + (qf[h, c] * kk[:, c]).astype(np.float32)).astype(np.float32)
        with np.errstate(over="ignore"):
            out[h] = s.astype(np.float16).view(np.uint16)
    return out


@pytest.mark.parametrize("n", [192, 256])
def test_reference_markers(port, n):
    # kernel_check.cpp:93-98 known answers
    q, k = markers_v3(n, rng(n))
    raw = port.score(q, k, n)
    t = np.arange(n)
    assert np.array_equal(raw[0], (t + 1).astype(np.uint16))
    assert np.array_equal(raw[28], (0x8000 | (t + 1)).astype(np.uint16))
    assert np.all(raw[31] == 0)


def test_cancellation_witness_closed_form(port):
    # 4096*4096 + 1 - 4096*4096: ordered FP32 gives 0 (16777217 rounds to even)
    q = np.zeros(4096, dtype=np.uint16)
    k = np.zeros(1024, dtype=np.uint16)
    q[0], q[1], q[2] = 0x6C00, 0x3C00, 0xEC00
    k[0], k[1], k[2] = 0x6C00, 0x3C00, 0x6C00
    raw = port.score(q, k, 1)
    assert raw[0, 0] == 0 and raw[1, 0] == 0  # head 1 shares KV head 0
    q2 = q.copy()
    q2[2] = 0
    assert port.score(q2, k, 1)[0, 0] == 0x7C00  # 16777217 overflows F16 to +inf


@pytest.mark.parametrize("stride", [1024, 2048])
@pytest.mark.parametrize("n", [1, 2, 7, 9, 17, 65])
def test_brute_force_small(port, n, stride):
    g = rng(1000 + n + stride)
    q = mixed_finite(g, H * D)
    k = mixed_finite(g, n * stride)
    assert np.array_equal(port.score(q, k, n, stride), brute_force(q, k, n, stride))


def test_head_channel_markers(port, ref):
    # kernel_check.cpp:126-132: wrong h/4 mapping or token addressing shows up
    n = 192
    q = np.zeros(4096, dtype=np.uint16)
    k = np.zeros(n * 1024, dtype=np.uint16)
    for h in range(32):
        q[h * 128 + (h * 7) % 128] = np.float16((h + 1) / 32).view(np.uint16)
    t, hh, c = np.meshgrid(np.arange(n), np.arange(8), np.arange(128), indexing="ij")
    k[:] = (((t * 1024 + hh * 128 + c) / 16384).astype(np.float16)).view(np.uint16).reshape(-1)
    assert np.array_equal(port.score(q, k, n), ref.score(q, k, n))
    assert np.array_equal(port.score(q, k, n), brute_force(q, k, n, 1024))


@pytest.mark.parametrize("impl,threads", [(1, 1), (2, 4), (0, 7)])
@pytest.mark.parametrize("stride", [1024, 2048])
@pytest.mark.parametrize("n", [1, 8, 17, 129, 1024])
def test_matches_compiled_reference(port, ref, impl, threads, stride, n):
    # policy/full_gqa_cpu.cpp scalar / AVX2 tiles, several thread splits
    g = rng(n * 7 + stride + impl)
    q = mixed_finite(g, H * D) if n % 2 else v3_sample(g, H * D)
    k = mixed_finite(g, n * stride) if n % 2 else v3_sample(g, n * stride)
    assert np.array_equal(port.score(q, k, n, stride),
                          ref.score(q, k, n, stride, threads=threads, impl=impl))


def test_scale_exhaustive(port, ref):
    # policy/full_gqa_runtime.cpp:571 over every F16 input, three ways.
    raw = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = port.scale(raw)
    finite = (raw & 0x7C00) != 0x7C00
    # (1) the reference's own expression through its own half functions
    root = np.float32(math.sqrt(128.0))
    assert root == np.sqrt(np.float32(128.0))
    ref_vals = np.array([ref.L.hsref_half_bits(float(np.float32(ref.L.hsref_half_value(int(b)))
                                                       / root)) for b in raw[finite]],
                        dtype=np.uint16)
    assert np.array_equal(got[finite], ref_vals)
    # (2) FP64 quotient rounded to FP32 (correct: 53 >= 2*24+2), then numpy F16 RNE
    x64 = raw[finite].view(np.float16).astype(np.float64)
    q32 = (x64 / np.float64(root)).astype(np.float32)
    assert np.array_equal(got[finite], q32.astype(np.float16).view(np.uint16))
