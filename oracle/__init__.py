"""CPU oracle of the HillServe sparse-KV hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and the cpu_baseline leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline).  The product package ``hillserve_amd`` never imports it.

``port``: ctypes binding of liboracle.so (our C restatement, hs_oracle.c).
``ref``:  ctypes binding of _ref/libhsref.so, the reference's own hot-path C++
          compiled from /root/reference by oracle/Makefile (absent when the
          reference tree was not available at build time).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
PORT_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libhsref.so"

_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


def build(reference: bool = True) -> None:
    """make -C oracle (the reference part only when /root/reference exists)."""
    target = "all" if reference else "oracle"
    subprocess.run(["make", "-s", "-C", str(HERE), target], check=True)


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_P)


class Port:
    """Our C restatement (hs_oracle.h)."""

    def __init__(self, path=PORT_PATH):
        if not Path(path).exists():
            build(reference=False)
        L = ctypes.CDLL(str(path))
        L.hso_half_value.restype = ctypes.c_float
        L.hso_half_value.argtypes = [ctypes.c_uint16]
        L.hso_half_bits.restype = ctypes.c_uint16
        L.hso_half_bits.argtypes = [ctypes.c_float]
        L.hso_order_key.restype = ctypes.c_uint16
        L.hso_order_key.argtypes = [ctypes.c_uint16]
        L.hso_score.argtypes = [_P, _P, _SZ, _SZ, _P, _SZ]
        L.hso_scale_one.restype = ctypes.c_uint16
        L.hso_scale_one.argtypes = [ctypes.c_uint16]
        L.hso_scale.argtypes = [_P, _P, _SZ]
        L.hso_select.argtypes = [_P, _SZ, _SZ, _SZ, ctypes.c_float, ctypes.c_float, ctypes.c_int,
                                 _P, _SZ, _P, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]
        L.hso_select_k.argtypes = [_P, _SZ, _SZ, _SZ, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_int, ctypes.POINTER(_SZ)]
        L.hso_history_cover.argtypes = [_P, _SZ, _SZ, _SZ, ctypes.c_float, ctypes.c_float,
                                        ctypes.c_int, _P, _SZ, ctypes.POINTER(_SZ), _P,
                                        ctypes.POINTER(_SZ)]
        L.hso_fnv1a64.restype = ctypes.c_uint64
        L.hso_fnv1a64.argtypes = [_P, _SZ]
        L.hso_kv_store_extent.restype = ctypes.c_uint64
        L.hso_kv_store_extent.argtypes = [_SZ, _SZ]
        L.hso_kv_store_header.argtypes = [_P, ctypes.c_uint64, _SZ, _SZ]
        L.hso_kv_record.argtypes = [_P, _P, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint32]
        L.hso_physical_union.argtypes = [_P, _P, _SZ, _SZ, _P, ctypes.POINTER(_SZ)]
        L.hso_pack.argtypes = [_P, _P, _SZ, _P, _SZ, _P, _SZ, _P, _SZ, _P, _P, _P]
        L.hso_gather_rows.argtypes = [_P, _P, _P, _SZ, _P, _P]
        L.hso_attention_f64.argtypes = [_P, _P, _SZ, _P, _P, _P, _SZ, _P]
        L.hso_rehearsal_f64.argtypes = [_P, _P, ctypes.c_double, ctypes.c_double,
                                        ctypes.c_uint64, _P]
        L.hso_f16_checksums.argtypes = [_P, ctypes.c_uint]
        L.hso_check_half_bits_f16c.restype = ctypes.c_longlong
        L.hso_check_half_bits_f16c.argtypes = [ctypes.c_uint]
        self.L = L

    def half_value(self, h):
        return self.L.hso_half_value(int(h))

    def half_bits(self, f):
        return self.L.hso_half_bits(float(f))

    def order_key(self, h):
        return self.L.hso_order_key(int(h))

    def score(self, q, k, n, stride_words=1024, out_stride=None):
        q = np.ascontiguousarray(q, dtype=np.uint16)
        k = np.ascontiguousarray(k, dtype=np.uint16)
        out_stride = n if out_stride is None else out_stride
        out = np.zeros((32, out_stride), dtype=np.uint16)
        rc = self.L.hso_score(_ptr(q), _ptr(k), stride_words, n, _ptr(out), out_stride)
        if rc:
            raise ValueError(f"hso_score rc={rc}")
        return out

    def scale(self, raw):
        raw = np.ascontiguousarray(raw, dtype=np.uint16)
        out = np.empty_like(raw)
        self.L.hso_scale(_ptr(raw), _ptr(out), raw.size)
        return out

    def select(self, scaled, heads, stride, n, alpha, ratio, fp32_counts=False):
        """-> (rc, k, ids[heads][k] u32, counts[heads] u32, tied)."""
        scaled = np.ascontiguousarray(scaled, dtype=np.uint16)
        k = _SZ(0)
        rc = self.L.hso_select_k(_ptr(scaled), heads, stride, n, ctypes.c_float(alpha),
                                 ctypes.c_float(ratio), int(fp32_counts), ctypes.byref(k))
        if rc:
            return rc, 0, None, None, 0
        width = max(1, k.value)
        ids = np.zeros((heads, width), dtype=np.uint32)
        counts = np.zeros(heads, dtype=np.uint32)
        k2, tied = _SZ(0), _SZ(0)
        rc = self.L.hso_select(_ptr(scaled), heads, stride, n, ctypes.c_float(alpha),
                               ctypes.c_float(ratio), int(fp32_counts), _ptr(ids), width,
                               _ptr(counts), ctypes.byref(k2), ctypes.byref(tied))
        return rc, k2.value, ids[:, : k2.value], counts, tied.value

    def history_cover(self, raw, heads, stride, position, alpha, ratio=0.2, fp32_counts=False):
        """prefetch_payload's cover (policy/full_gqa_runtime.cpp:299-344) of the
        RAW scores -> (rc, bound, ids[heads][bound] u32, physical u32)."""
        raw = np.ascontiguousarray(raw, dtype=np.uint16)
        width = max(1, position)
        ids = np.zeros((heads, width), dtype=np.uint32)
        physical = np.zeros(width, dtype=np.uint32)
        bound, np_out = _SZ(0), _SZ(0)
        rc = self.L.hso_history_cover(_ptr(raw), heads, stride, position, ctypes.c_float(alpha),
                                      ctypes.c_float(ratio), int(fp32_counts), _ptr(ids), width,
                                      ctypes.byref(bound), _ptr(physical), ctypes.byref(np_out))
        if rc:
            return rc, 0, None, None
        return rc, bound.value, ids[:, : bound.value], physical[: np_out.value]

    def fnv1a64(self, data):
        data = np.ascontiguousarray(data, dtype=np.uint8)
        return self.L.hso_fnv1a64(_ptr(data), data.size)

    def kv_store_image(self, request, layers, positions, layer, rows, first=0):
        """SegmentedKVStore image bytes with rows at positions first.. of layer."""
        rows = np.ascontiguousarray(rows, dtype=np.uint8).reshape(-1, 4096)
        image = np.zeros(self.L.hso_kv_store_extent(layers, positions), dtype=np.uint8)
        self.L.hso_kv_store_header(_ptr(image), request, layers, positions)
        rec = np.zeros(4128, dtype=np.uint8)
        for i, row in enumerate(rows):
            p = first + i
            self.L.hso_kv_record(_ptr(rec), _ptr(np.ascontiguousarray(row)), p, request, layer)
            off = 4096 + (layer * positions + p) * 4128
            image[off:off + 4128] = rec
        return image

    def physical_union(self, ids_rows, visible):
        stride = max(1, max(len(r) for r in ids_rows))
        ids = np.zeros((32, stride), dtype=np.uint32)
        lens = np.zeros(32, dtype=np.uintp)
        for h, r in enumerate(ids_rows):
            ids[h, : len(r)] = r
            lens[h] = len(r)
        out = np.zeros(visible, dtype=np.uint32)
        m = _SZ(0)
        rc = self.L.hso_physical_union(_ptr(ids), _ptr(lens), stride, visible, _ptr(out),
                                       ctypes.byref(m))
        return rc, out[: m.value]

    def pack(self, ids_rows, positions, physical, payload, count):
        stride = max(1, max(len(r) for r in ids_rows))
        ids = np.zeros((32, stride), dtype=np.uint32)
        lens = np.zeros(32, dtype=np.uintp)
        for h, r in enumerate(ids_rows):
            ids[h, : len(r)] = r
            lens[h] = len(r)
        pos = np.ascontiguousarray(positions, dtype=np.uint64)
        phys = np.ascontiguousarray(physical, dtype=np.uint32)
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        qpad = (len(pos) + 63) // 64 * 64
        k = np.zeros(count * 4096, dtype=np.uint16)
        v = np.zeros(count * 4096, dtype=np.uint16)
        mask = np.zeros(32 * qpad * count, dtype=np.float32)
        rc = self.L.hso_pack(_ptr(ids), _ptr(lens), stride, _ptr(pos), len(pos), _ptr(phys),
                             len(phys), _ptr(payload), count, _ptr(k), _ptr(v), _ptr(mask))
        return rc, k, v, mask

    def gather_rows(self, prefetched, misses, row_map, count):
        pre = np.ascontiguousarray(prefetched, dtype=np.uint16)
        mis = np.ascontiguousarray(misses, dtype=np.uint16)
        m = np.ascontiguousarray(row_map, dtype=np.int32)
        k = np.zeros(count * 4096, dtype=np.uint16)
        v = np.zeros(count * 4096, dtype=np.uint16)
        self.L.hso_gather_rows(_ptr(pre), _ptr(mis), _ptr(m), count, _ptr(k), _ptr(v))
        return k, v

    def attention(self, q32, pool, ids_rows, rows=None, row_bytes=4096):
        q = np.ascontiguousarray(q32, dtype=np.float32)
        pool = np.ascontiguousarray(pool, dtype=np.uint8)
        stride = max(1, max(len(r) for r in ids_rows))
        ids = np.zeros((32, stride), dtype=np.uint32)
        lens = np.zeros(32, dtype=np.uintp)
        for h, r in enumerate(ids_rows):
            ids[h, : len(r)] = r
            lens[h] = len(r)
        r = None if rows is None else np.ascontiguousarray(rows, dtype=np.int32)
        out = np.zeros((32, 128), dtype=np.float64)
        self.L.hso_attention_f64(_ptr(q), _ptr(pool), row_bytes, _ptr(r), _ptr(ids), _ptr(lens),
                                 stride, _ptr(out))
        return out

    def rehearsal(self, hidden_bf16, wq_bf16, pos, eps=1e-5, theta=500000.0):
        h = np.ascontiguousarray(hidden_bf16, dtype=np.uint16)
        w = np.ascontiguousarray(wq_bf16, dtype=np.uint16)
        out = np.zeros((32, 128), dtype=np.float64)
        self.L.hso_rehearsal_f64(_ptr(h), _ptr(w), eps, theta, pos, _ptr(out))
        return out

    def f16_checksums(self, threads=8):
        out = np.zeros(65536, dtype=np.uint64)
        self.L.hso_f16_checksums(_ptr(out), threads)
        return out

    def check_half_bits_f16c(self, threads=8):
        return self.L.hso_check_half_bits_f16c(threads)


class Ref:
    """The reference's own hot-path code (oracle/_ref/libhsref.so)."""

    def __init__(self, path=REF_PATH):
        if not Path(path).exists():
            raise FileNotFoundError(f"{path} not built (needs /root/reference at build time)")
        L = ctypes.CDLL(str(path))
        L.hsref_last_error.restype = ctypes.c_char_p
        L.hsref_half_value.restype = ctypes.c_float
        L.hsref_half_value.argtypes = [ctypes.c_uint16]
        L.hsref_half_bits.restype = ctypes.c_uint16
        L.hsref_half_bits.argtypes = [ctypes.c_float]
        L.hsref_scorer_new.restype = _P
        L.hsref_scorer_new.argtypes = [ctypes.c_uint, ctypes.c_int]
        L.hsref_scorer_free.argtypes = [_P]
        L.hsref_scorer_name.restype = ctypes.c_char_p
        L.hsref_scorer_name.argtypes = [_P]
        L.hsref_scorer_score.argtypes = [_P, _P, _P, _P, _SZ, _P]
        L.hsref_legacy_score.argtypes = [_P, _P, _SZ, _SZ, ctypes.c_uint, _P]
        L.hsref_select.argtypes = [_P, _SZ, _SZ, _SZ, ctypes.c_float, ctypes.c_float,
                                   ctypes.c_int, _P, _SZ, _P, ctypes.POINTER(_SZ),
                                   ctypes.POINTER(_SZ)]
        L.hsref_physical_union.argtypes = [_P, _P, _SZ, _SZ, _P, ctypes.POINTER(_SZ)]
        L.hsref_pack.argtypes = [_P, _P, _SZ, _P, _SZ, _P, _SZ, _P, _SZ, _P, _P, _P]
        L.hsref_checksum.restype = ctypes.c_uint64
        L.hsref_checksum.argtypes = [_P, _SZ]
        L.hsref_segmented_write.argtypes = [ctypes.c_char_p, ctypes.c_uint64, _SZ, ctypes.c_uint64,
                                            _SZ, _P, _SZ, ctypes.POINTER(ctypes.c_uint64)]
        self.L = L
        self._scorers = {}

    def error(self):
        return self.L.hsref_last_error().decode()

    def checksum(self, data):
        data = np.ascontiguousarray(data, dtype=np.uint8)
        return self.L.hsref_checksum(_ptr(data), data.size)

    def segmented_file(self, path, request, layers, positions, layer, rows):
        """Bytes of a SegmentedKVStore file holding rows [count][4096] at
        positions 0.. of `layer` (the reference's own writer)."""
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        extent = ctypes.c_uint64(0)
        rc = self.L.hsref_segmented_write(str(path).encode(), request, layers, positions, layer,
                                          _ptr(rows), rows.size // 4096, ctypes.byref(extent))
        if rc:
            raise RuntimeError(self.error())
        data = np.fromfile(str(path), dtype=np.uint8)
        assert data.size == extent.value
        return data

    def scorer(self, threads=1, impl=0):
        key = (threads, impl)
        if key not in self._scorers:
            h = self.L.hsref_scorer_new(threads, impl)
            if not h:
                raise RuntimeError(self.error())
            self._scorers[key] = h
        return self._scorers[key]

    def score(self, q, k, n, stride_words=1024, threads=1, impl=0, views=None):
        q = np.ascontiguousarray(q, dtype=np.uint16)
        k = np.ascontiguousarray(k, dtype=np.uint16)
        if views is None:
            views = [(0, n, stride_words)]
        total = sum(v[1] for v in views)
        vv = np.array(views, dtype=np.uint64).reshape(-1)
        out = np.zeros(32 * total, dtype=np.uint16)
        rc = self.L.hsref_scorer_score(self.scorer(threads, impl), _ptr(q), _ptr(k), _ptr(vv),
                                       len(views), _ptr(out))
        if rc:
            raise RuntimeError(self.error())
        return out.reshape(32, total)

    def select(self, scaled, heads, stride, n, alpha, ratio, fp32_counts=False, width=None):
        scaled = np.ascontiguousarray(scaled, dtype=np.uint16)
        width = max(1, n if width is None else width)
        ids = np.zeros((heads, width), dtype=np.uint32)
        counts = np.zeros(heads, dtype=np.uint32)
        k, tied = _SZ(0), _SZ(0)
        rc = self.L.hsref_select(_ptr(scaled), heads, stride, n, ctypes.c_float(alpha),
                                 ctypes.c_float(ratio), int(fp32_counts), _ptr(ids), width,
                                 _ptr(counts), ctypes.byref(k), ctypes.byref(tied))
        if rc:
            return rc, self.error(), None, None, 0
        return 0, k.value, ids[:, : k.value], counts, tied.value

    def physical_union(self, ids_rows, visible):
        stride = max(1, max(len(r) for r in ids_rows))
        ids = np.zeros((32, stride), dtype=np.uint32)
        lens = np.zeros(32, dtype=np.uintp)
        for h, r in enumerate(ids_rows):
            ids[h, : len(r)] = r
            lens[h] = len(r)
        out = np.zeros(visible, dtype=np.uint32)
        m = _SZ(0)
        rc = self.L.hsref_physical_union(_ptr(ids), _ptr(lens), stride, visible, _ptr(out),
                                         ctypes.byref(m))
        return rc, out[: m.value]

    def pack(self, ids_rows, positions, physical, payload, count):
        stride = max(1, max(len(r) for r in ids_rows))
        ids = np.zeros((32, stride), dtype=np.uint32)
        lens = np.zeros(32, dtype=np.uintp)
        for h, r in enumerate(ids_rows):
            ids[h, : len(r)] = r
            lens[h] = len(r)
        pos = np.ascontiguousarray(positions, dtype=np.uint64)
        phys = np.ascontiguousarray(physical, dtype=np.uint32)
        payload = np.ascontiguousarray(payload, dtype=np.uint8)
        qpad = (len(pos) + 63) // 64 * 64
        k = np.zeros(count * 4096, dtype=np.uint16)
        v = np.zeros(count * 4096, dtype=np.uint16)
        mask = np.zeros(32 * qpad * count, dtype=np.float32)
        rc = self.L.hsref_pack(_ptr(ids), _ptr(lens), stride, _ptr(pos), len(pos), _ptr(phys),
                               len(phys), _ptr(payload), count, _ptr(k), _ptr(v), _ptr(mask))
        return rc, k, v, mask


_port = None
_ref = None


def port() -> Port:
    """The restatement; HS_ORACLE_LIB names another build of hs_oracle.c (the
    sanitizer test runs the oracle tests against an ASan + UBSan build)."""
    global _port
    if _port is None:
        alt = os.environ.get("HS_ORACLE_LIB")
        _port = Port(alt) if alt else Port()
    return _port


def ref():
    """The compiled reference, or None when it was not built."""
    global _ref
    if _ref is None and REF_PATH.exists():
        _ref = Ref()
    return _ref
