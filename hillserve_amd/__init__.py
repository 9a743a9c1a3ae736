"""hillserve_amd — MI355X (gfx950) sparse-KV decode hot path.

Python access to the C ABI of ``include/hs_gpu.h`` (libhillserve_amd.so,
built in-tree by ``hillserve_amd.build``).  PyTorch is used only for device
memory and streams: every operation here is a HIP kernel of the native
library, and importing a wrapper without the library raises instead of
falling back to anything.

Layouts follow the reference contract (runtime/full_gqa_contract.hpp,
kernels/full_gqa_pipeline/ABI.json): 32 query heads, 8 KV heads, 128
channels, query head h reads KV head h/4.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libhillserve_amd.so")
HEADER = Path(__file__).resolve().parent.parent / "include" / "hs_gpu.h"

HS_OK = 0
HS_ERR_ARGUMENT = 1
HS_ERR_NONFINITE = 2
HS_ERR_THRESHOLD = 3
HS_ERR_COUNT = 4
HS_ERR_MEAN = 5
HS_ERR_ZERO_SELECTION = 6
HS_ERR_DUPLICATE = 7
HS_ERR_MISSING = 8
HS_ERR_HIP = 9
HS_ERR_UNSUPPORTED = 10
HS_ERR_OVERFLOW = 11
HS_ERR_CORRUPT = 12

HS_SELECT_SCALE_RAW = 1
HS_SELECT_FP32_COUNTS = 2
HS_SELECT_REQUIRE_K = 4
HS_SELECT_ID_ORDER = 8
HS_SELECT_COVER = 16
HS_SELECT_COUNTED = 32

ERROR_NAMES = {
    HS_ERR_ARGUMENT: "argument",
    HS_ERR_NONFINITE: "nonfinite score",
    HS_ERR_THRESHOLD: "F16 threshold overflow",
    HS_ERR_COUNT: "F16 count overflow",
    HS_ERR_MEAN: "F16 mean overflow",
    HS_ERR_ZERO_SELECTION: "zero selection",
    HS_ERR_DUPLICATE: "duplicate/future id",
    HS_ERR_MISSING: "missing KV row",
    HS_ERR_HIP: "HIP runtime",
    HS_ERR_UNSUPPORTED: "unsupported",
    HS_ERR_OVERFLOW: "F16 overflow",
    HS_ERR_CORRUPT: "corrupt cold record",
}


class HsError(RuntimeError):
    """A nonzero status from the native library."""

    def __init__(self, code: int, message: str = ""):
        self.code = code
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}".rstrip(": "))


class Status(ctypes.Structure):
    _fields_ = [
        ("code", ctypes.c_int32),
        ("k", ctypes.c_uint32),
        ("boundary_tied_heads", ctypes.c_uint32),
        ("head0_max_key", ctypes.c_uint32),
    ]


class ScoreJob(ctypes.Structure):
    """hs_score_job_t of include/hs_gpu.h."""
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("keys", ctypes.c_void_p),
        ("scores", ctypes.c_void_p),
        ("head0_partial", ctypes.c_void_p),
        ("key_stride_words", ctypes.c_uint32),
        ("tokens", ctypes.c_uint32),
        ("score_stride", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
    ]


class SelectJob(ctypes.Structure):
    """hs_select_job_t of include/hs_gpu.h."""
    _fields_ = [
        ("scores", ctypes.c_void_p),
        ("head0_partial", ctypes.c_void_p),
        ("ids", ctypes.c_void_p),
        ("counts", ctypes.c_void_p),
        ("member", ctypes.c_void_p),
        ("status", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("stride", ctypes.c_uint32),
        ("n", ctypes.c_uint32),
        ("ids_stride", ctypes.c_uint32),
        ("reserved", ctypes.c_uint32),
        ("current_q", ctypes.c_void_p),
        ("current_key", ctypes.c_void_p),
    ]


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32
_U64 = ctypes.c_uint64
_F = ctypes.c_float
_I = ctypes.c_int

SIGNATURES = {
    "hs_version": (ctypes.c_char_p, []),
    "hs_last_error": (ctypes.c_char_p, []),
    "hs_full_gqa_pipeline": (_I, [_P, _P, _P, _U32, _P]),
    "hs_gqa_score": (_I, [_P, _P, _SZ, _P, _U32, _U32, _P, _SZ, _P, _P]),
    "hs_gqa_score_batched": (_I, [_P, _U32, _P]),
    "hs_gqa_score_logits": (_I, [_P, _P, _P, _SZ, _P, _U32, _U32, _P, _SZ, _P, _P, _SZ, _P]),
    "hs_gqa_sparse_attention_logits": (_I, [_P, _SZ, _P, _SZ, _P, _U32, _P, _U32, _P, _P, _P]),
    "hs_gqa_select_workspace_bytes": (_SZ, [_U32, _U32]),
    "hs_gqa_select": (_I, [_P, _U32, _SZ, _U32, _F, _F, _U32, _P, _P, _SZ, _P, _P, _P, _P, _P]),
    "hs_gqa_select_batched": (_I, [_P, _U32, _U32, _F, _F, _U32, _P]),
    "hs_gqa_select_then_score": (_I, [_P, _U32, _U32, _F, _F, _U32, _P, _U32, _P]),
    "hs_gqa_attention_then_count": (_I, [_P, _P, _P, _SZ, _P, _U32, _P, _U32, _P, _P, _P, _U32,
                                         _U32, _F, _F, _U32, _P]),
    "hs_rehearsal_workspace_bytes": (_SZ, [_U32]),
    "hs_rehearsal_query": (_I, [_P, _P, _P, _U32, _F, _F, _P, _P, _P, _P]),
    "hs_kv_store_bytes": (_U64, [_U32, _U32]),
    "hs_kv_store_init": (_I, [_P, _U64, _U32, _U32]),
    "hs_kv_store_append": (_I, [_P, _U32, _U32, _P, _U32]),
    "hs_kv_cold_fetch_workspace_bytes": (_SZ, [_U32]),
    "hs_kv_cold_fetch": (_I, [_P, _U32, _P, _U32, _P, _P, _SZ, _P, _P, _P]),
    "hs_kv_cold_fetch_runs": (_I, [_P, _U32, _P, _P, _U32, _P, _P, _U32, _P, _P, _SZ, _P, _P, _P]),
    "hs_gqa_cold_plan": (_I, [_P, _U32, _U32, _P, _U32, _U32, _P, _P, _P, _P]),
    "hs_gqa_union_workspace_bytes": (_SZ, [_U32]),
    "hs_gqa_physical_union": (_I, [_P, _P, _SZ, _U32, _P, _P, _P, _P, _P]),
    "hs_gqa_pack": (_I, [_P, _P, _SZ, _U32, _P, _U32, _P, _P, _SZ, _P, _U32, _U32, _P, _P, _P, _P, _P]),
    "hs_gqa_gather_rows": (_I, [_P, _U32, _P, _U32, _P, _U32, _P, _P, _P, _P]),
    "hs_gqa_attention_workspace_bytes": (_SZ, [_U32]),
    "hs_gqa_sparse_attention": (_I, [_P, _P, _P, _SZ, _P, _U32, _P, _U32, _P, _P, _P]),
    "hs_decode_layer_workspace_bytes": (_SZ, [_U32]),
    "hs_decode_layer": (_I, [_P, _P, _P, _P, _SZ, _P, _U32, _U32, _F, _F, _U32, _P, _P, _SZ, _P, _P, _P, _P, _P]),
    "hs_decode_layer_noalloc": (_I, [_P, _P, _P, _P, _SZ, _P, _U32, _U32, _F, _F, _U32, _P, _P, _SZ, _P, _P, _P, _P]),
    "hs_selftest_f16_checksums": (_I, [_P, _P]),
    "hs_selftest_scale_table": (_I, [_P, _P]),
    "hs_selftest_key_table": (_I, [_P, _P]),
    "hs_fill_gaussian_f16": (_I, [_P, _SZ, _U64, _F, _P]),
    "hs_fill_rope_keys_f16": (_I, [_P, _U32, _SZ, _U32, _U64, _F, _P]),
}

_lib = None


def header_functions() -> list[str]:
    """Names of every function declared in include/hs_gpu.h."""
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hs_[a-z0-9_]+)\s*\(", text)))


def lib() -> ctypes.CDLL:
    """Load libhillserve_amd.so (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m hillserve_amd.build`; "
                "there is no fallback implementation")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def last_error() -> str:
    return lib().hs_last_error().decode()


def check(rc: int) -> None:
    if rc != HS_OK:
        raise HsError(rc, last_error())


from . import ops  # noqa: E402,F401  (torch-facing wrappers)
