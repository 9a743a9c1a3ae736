"""Pins of the FP64 rehearsal-query restatement (oracle, CPU).

The arithmetic of the reference lives in ggml b6000 (absent), so
hso_rehearsal_f64 is pinned by closed forms that a transposed Wq, a wrong
RMS scale, a wrong RoPE pair or angle would each fail:
  * Wq a permutation matrix: y[o] = x_norm[perm[o]] (catches Wq^T);
  * one-hot hidden: x_norm = 64 e_j, so the rotated pair is 64 (cos, sin);
  * RoPE at position 0 is the identity; RoPE keeps each pair's norm;
  * the RMS norm is scale invariant (hidden * 2 gives the same output)."""
import math

import numpy as np

from hs_data import rng


def bf16(x):
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    return ((b + 0x7FFF + ((b >> 16) & 1)) >> 16).astype(np.uint16)


def bf16_value(b):
    return (np.asarray(b, dtype=np.uint32) << 16).view(np.float32).astype(np.float64)


THETA = 500000.0


def test_permutation_wq_and_identity_rope(port):
    g = rng(1)
    perm = g.permutation(4096)
    wq = np.zeros((4096, 4096), dtype=np.uint16)
    wq[np.arange(4096), perm] = bf16(1.0)
    hidden = bf16(g.standard_normal(4096))
    x = bf16_value(hidden)
    xn = x / math.sqrt(np.mean(x * x) + 1e-5)
    out = port.rehearsal(hidden, wq, 0, eps=1e-5, theta=THETA).reshape(-1)
    assert np.allclose(out, xn[perm], rtol=1e-12, atol=1e-12)


def test_one_hot_rotation(port):
    wq = np.zeros((4096, 4096), dtype=np.uint16)
    wq[np.arange(4096), np.arange(4096)] = bf16(1.0)
    for head, i, pos in [(0, 0, 1), (5, 7, 1000), (31, 63, 32767)]:
        j = head * 128 + 2 * i
        hidden = np.zeros(4096, dtype=np.uint16)
        hidden[j] = bf16(3.0)
        out = port.rehearsal(hidden, wq, pos, eps=0.0, theta=THETA)
        angle = pos * THETA ** (-2.0 * i / 128.0)
        assert math.isclose(out[head, 2 * i], 64 * math.cos(angle), rel_tol=1e-12, abs_tol=1e-12)
        assert math.isclose(out[head, 2 * i + 1], 64 * math.sin(angle), rel_tol=1e-12, abs_tol=1e-12)
        others = np.delete(out.reshape(-1), [j, j + 1])
        assert np.all(others == 0)


def test_rope_keeps_pair_norms_and_rms_scale_invariance(port):
    g = rng(2)
    wq = bf16(g.standard_normal((4096, 4096)).astype(np.float32) * 0.02)
    hidden = bf16(g.standard_normal(4096))
    base = port.rehearsal(hidden, wq, 0, eps=0.0, theta=THETA)
    rot = port.rehearsal(hidden, wq, 777, eps=0.0, theta=THETA)
    nb = np.hypot(base[:, 0::2], base[:, 1::2])
    nr = np.hypot(rot[:, 0::2], rot[:, 1::2])
    assert np.allclose(nb, nr, rtol=1e-12)
    doubled = bf16(bf16_value(hidden) * 2.0)  # exact in BF16
    again = port.rehearsal(doubled, wq, 777, eps=0.0, theta=THETA)
    assert np.allclose(again, rot, rtol=1e-12, atol=1e-15)
