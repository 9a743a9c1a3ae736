"""Pins of the binary16 conversions and the order key (oracle, CPU)."""
import numpy as np

from hs_data import rng


def test_roundtrip_exhaustive_and_numpy_decode(port):
    # tests/policy_tests.cpp:8 — every non-NaN binary16 survives half->float->half.
    bits = np.arange(65536, dtype=np.uint32)
    values = np.array([port.half_value(b) for b in bits], dtype=np.float32)
    numpy_values = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(numpy_values)
    # independent decoder (numpy) agrees bit for bit on every non-NaN pattern
    assert np.array_equal(values[~nan].view(np.uint32), numpy_values[~nan].view(np.uint32))
    assert all(port.half_bits(float(v)) == int(b) for b, v in zip(bits[~nan], values[~nan]))


def test_rne_ties():
    import oracle
    p = oracle.port()
    # tests/policy_tests.cpp:9-10
    assert p.half_bits(1.00048828125) == p.half_bits(1.0)
    assert p.half_bits(1.00146484375) == p.half_bits(1.001953125)
    # overflow threshold: 65520 rounds to inf, just below stays max finite
    assert p.half_bits(65520.0) == 0x7C00
    assert p.half_bits(np.nextafter(np.float32(65520.0), np.float32(0))) == 0x7BFF
    # smallest subnormal boundary: 2^-25 ties to even (0), above rounds up
    assert p.half_bits(2.0 ** -25) == 0
    assert p.half_bits(float(np.nextafter(np.float32(2.0 ** -25), np.float32(1)))) == 1
    # NaN canonicalisation (host_policy.cpp:18)
    assert p.half_bits(float("nan")) & 0x7FFF == 0x7E00


def test_half_bits_all_fp32_patterns_against_f16c(port):
    # All 2^32 FP32 patterns (NaN excluded) against the x86 F16C converter.
    assert port.check_half_bits_f16c(8) == 0


def test_half_bits_matches_compiled_reference(port, ref):
    g = rng(11)
    words = g.integers(0, 2**32, size=20000, dtype=np.uint64).astype(np.uint32)
    floats = words.view(np.float32)
    for f in floats[:20000]:
        if np.isnan(f):
            continue
        assert port.half_bits(float(f)) == ref.L.hsref_half_bits(float(f))


def test_order_key_exhaustive(port):
    # tests/gqa_policy_tests.cpp:63-69: the key orders finite halves exactly like
    # their FP32 values, and -0/+0 share a key.
    finite = [b for b in range(65536) if (b & 0x7C00) != 0x7C00]
    values = np.array(finite, dtype=np.uint16).view(np.float16).astype(np.float64)
    keys = np.array([port.order_key(b) for b in finite])
    order = np.argsort(values, kind="stable")
    v, k = values[order], keys[order]
    assert np.all((k[1:] > k[:-1]) == (v[1:] > v[:-1]))
    assert np.all((k[1:] == k[:-1]) == (v[1:] == v[:-1]))
    assert port.order_key(0x0000) == port.order_key(0x8000) == 0x8000
