"""Deterministic test inputs (numpy) shared by CPU and GPU tests."""
from __future__ import annotations

import numpy as np

H, KH, D = 32, 8, 128


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def f16_bits(x) -> np.ndarray:
    """float array -> F16 bit patterns (numpy rounds to nearest even)."""
    return np.asarray(x, dtype=np.float64).astype(np.float16).view(np.uint16)


def bits_f32(b) -> np.ndarray:
    return np.asarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


def v3_sample(g: np.random.Generator, size) -> np.ndarray:
    """Distribution of kernels/full_gqa_pipeline/kernel_check.cpp:33-38: finite
    mixed signs, exponent 0..16 (subnormals included), any mantissa."""
    sign = g.integers(0, 2, size=size, dtype=np.uint32) << 15
    exp = g.integers(0, 17, size=size, dtype=np.uint32) << 10
    man = g.integers(0, 1024, size=size, dtype=np.uint32)
    return (sign | exp | man).astype(np.uint16)


EDGE = np.array([0, 0x8000, 1, 0x8001, 0x03FF, 0x83FF, 0x0400, 0x8400, 0x3C00, 0xBC00,
                 0x7BFF, 0xFBFF, 0x3555, 0xB555], dtype=np.uint16)


def mixed_finite(g: np.random.Generator, size) -> np.ndarray:
    """Distribution of tests/full_gqa_cpu_tests.cpp:21-27: 1 in 5 from the edge
    list (subnormal, max finite, signed zero), else any finite F16."""
    word = g.integers(0, 2**32, size=size, dtype=np.uint64)
    edge = EDGE[(word >> 8) % len(EDGE)]
    other = (word & 0x83FF) | (((word >> 10) % 31) << 10)
    return np.where(word % 5 == 0, edge, other).astype(np.uint16)


def config1_inputs(seed: int = 0, n: int = 4096):
    """Q[32,128] ~ N(0,1); K[n,8,128] ~ N(0,1) with 4 fixed
    channels (per KV head) scaled x8; all F16."""
    g = rng(seed)
    q = f16_bits(g.standard_normal((H, D)))
    k = g.standard_normal((n, KH, D))
    outliers = np.sort(g.choice(D, size=4, replace=False))
    k[:, :, outliers] *= 8.0
    return q, f16_bits(k), outliers


def rope_keys(n: int, seed: int, theta: float = 500000.0, heads: int = KH) -> np.ndarray:
    """K[n, heads, 128] = RoPE(adjacent pairs, base theta, position t) of N(0,1), F16."""
    g = rng(seed)
    x = g.standard_normal((n, heads, D // 2, 2))
    i = np.arange(D // 2, dtype=np.float64)
    freq = theta ** (-2.0 * i / D)
    ang = np.arange(n, dtype=np.float64)[:, None] * freq[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    out = np.empty_like(x)
    out[..., 0] = x[..., 0] * c - x[..., 1] * s
    out[..., 1] = x[..., 0] * s + x[..., 1] * c
    return f16_bits(out.reshape(n, heads, D))


def pool_rows(k_bits: np.ndarray, v_bits: np.ndarray) -> np.ndarray:
    """Hot-pool rows of 4096 B: K[8][128] then V[8][128] per token (uint16 view)."""
    n = k_bits.shape[0]
    rows = np.empty((n, 2, KH, D), dtype=np.uint16)
    rows[:, 0] = k_bits.reshape(n, KH, D)
    rows[:, 1] = v_bits.reshape(n, KH, D)
    return rows.reshape(n, 2 * KH * D)


def to_dev(a: np.ndarray, dtype="f16"):
    """numpy -> CUDA torch tensor (F16 bits as float16, u32 as int32)."""
    import torch
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16)).view(torch.float16)
    elif a.dtype == np.uint32:
        t = torch.from_numpy(a.view(np.int32))
    else:
        t = torch.from_numpy(a)
    return t.cuda()


def from_dev(t) -> np.ndarray:
    """CUDA tensor -> numpy (float16 -> uint16 bits, int32 -> uint32)."""
    import torch
    c = t.detach().cpu()
    if c.dtype == torch.float16:
        return c.view(torch.int16).numpy().view(np.uint16)
    if c.dtype == torch.int32:
        return c.numpy().view(np.uint32)
    return c.numpy()


def markers_v3(n: int, g: np.random.Generator):
    """kernels/full_gqa_pipeline/kernel_check.cpp:79-92: v3 samples overwritten
    with the subnormal (head 0), negative subnormal (head 28) and ordered
    cancellation (head 31) markers."""
    q = v3_sample(g, 4096)
    k = v3_sample(g, n * 1024)
    q[:128] = 0
    q[0] = 0x3C00
    q[28 * 128: 29 * 128] = 0
    q[28 * 128 + 3] = 0x3C00
    q[31 * 128:] = 0
    q[31 * 128: 31 * 128 + 3] = [0x6C00, 0x3C00, 0xEC00]
    t = np.arange(n)
    k[t * 1024] = (t + 1).astype(np.uint16)
    last = (t * 8 + 7) * 128
    k[last] = 0x6C00
    k[last + 1] = 0x3C00
    k[last + 2] = 0x6C00
    k[last + 3] = (0x8000 | (t + 1)).astype(np.uint16)
    return q, k


def make_jobs(hs, ns, seed):
    """Device scoring jobs: a Gaussian query and RoPE-structured keys of n
    tokens each, with a head-0 tile-maximum buffer."""
    import torch
    jobs = []
    for i, n in enumerate(ns):
        q = torch.empty(4096, dtype=torch.float16, device="cuda")
        k = torch.empty(n * 1024, dtype=torch.float16, device="cuda")
        hs.ops.fill_gaussian(q, seed=seed + 2 * i)
        hs.ops.fill_rope_keys(k, n, 1024, 8, seed=seed + 2 * i + 1, theta=500000.0)
        jobs.append(dict(q16=q, keys=k, tokens=n,
                         head0_partial=torch.empty((n + 63) // 64, dtype=torch.int32,
                                                   device="cuda")))
    return jobs


def batch_ns(seed, count=16):
    """Sequence lengths of a batch: multiples of 64 in 8192..32768."""
    g = rng(seed)
    return [int(x) * 64 for x in g.integers(8192 // 64, 32768 // 64 + 1, size=count)]
