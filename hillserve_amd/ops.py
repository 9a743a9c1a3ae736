"""Torch-tensor wrappers over the C ABI (device memory and streams only).

F16 data travel as ``torch.float16`` tensors (bit patterns are what the
kernels consume); uint32 ids/counts/bitmaps as ``torch.int32``.  Every
function enqueues on ``stream`` (default: torch's current stream) and
returns without synchronising, except ``read_status``.
"""
from __future__ import annotations

import ctypes
import math

import torch

from . import (HS_SELECT_COUNTED, HS_SELECT_COVER, HS_SELECT_FP32_COUNTS, HS_SELECT_ID_ORDER, HS_SELECT_REQUIRE_K, HS_SELECT_SCALE_RAW, HsError, check,
               lib)

H, KH, D = 32, 8, 128


def _p(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _s(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _need_cuda(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("hillserve_amd operates on device tensors only")


def workspace(nbytes: int, device="cuda") -> torch.Tensor:
    # scratch only: every kernel writes what it later reads (no clearing needed)
    return torch.empty(max(256, int(nbytes)), dtype=torch.uint8, device=device)


def _scratch(nbytes: int, device, stream) -> torch.Tensor:
    """A workspace the wrapper drops on return: recorded on the launch
    stream, so the caching allocator does not hand it out again while that
    stream's kernels still use it."""
    ws = workspace(nbytes, device)
    ws.record_stream(stream if stream is not None else torch.cuda.current_stream(ws.device))
    return ws


def new_status(device="cuda", stream=None) -> torch.Tensor:
    """A zeroed hs_status_t; zeroed on `stream` (default: the current
    stream), so the fill is ordered before the kernels that write it."""
    st = torch.empty(4, dtype=torch.int32, device=device)
    if stream is None:
        return st.zero_()
    with torch.cuda.stream(stream):
        return st.zero_()


def read_status(status: torch.Tensor) -> dict:
    """Synchronise on the status tensor and decode hs_status_t."""
    v = status.cpu().tolist()
    return {"code": int(v[0]), "k": int(v[1]) & 0xFFFFFFFF,
            "boundary_tied_heads": int(v[2]) & 0xFFFFFFFF,
            "head0_max_key": int(v[3]) & 0xFFFFFFFF}


# ---- scoring -----------------------------------------------------------------

def full_gqa_pipeline(q16, keys, tokens, out=None, stream=None):
    """V3 kernel ABI (hillserve_full_gqa_pipeline): scores F16[32, tokens]."""
    _need_cuda(q16, keys)
    if out is None:
        out = torch.empty((H, tokens), dtype=torch.float16, device=keys.device)
    check(lib().hs_full_gqa_pipeline(_p(q16), _p(keys), _p(out), tokens, _s(stream)))
    return out


def score(q16, keys, tokens, key_stride_words=1024, rows=None, out=None, score_stride=None,
          head0_partial=None, pool_rows=None, stream=None):
    """Ordered-FP32 raw GQA scores F16[32, score_stride] (columns < tokens)."""
    _need_cuda(q16, keys, rows, out, head0_partial)
    if score_stride is None:
        score_stride = tokens if out is None else out.shape[-1]
    if out is None:
        out = torch.empty((H, score_stride), dtype=torch.float16, device=keys.device)
    if pool_rows is None:
        pool_rows = keys.numel() // key_stride_words
    check(lib().hs_gqa_score(_p(q16), _p(keys), key_stride_words, _p(rows), pool_rows, tokens,
                             _p(out), score_stride, _p(head0_partial), _s(stream)))
    return out


def score_logits(q16, q32, keys, tokens, key_stride_words=1024, rows=None, out=None,
                 score_stride=None, head0_partial=None, logits=None, logit_stride=None,
                 pool_rows=None, stream=None):
    """hs_gqa_score_logits: the raw scores (as score) and, in the same pass,
    the attention dots logits F32 [32, logit_stride] of q32 F32 [32, 128].
    Returns (scores, logits)."""
    _need_cuda(q16, q32, keys, rows, out, head0_partial, logits)
    if score_stride is None:
        score_stride = tokens if out is None else out.shape[-1]
    if out is None:
        out = torch.empty((H, score_stride), dtype=torch.float16, device=keys.device)
    if logit_stride is None:
        logit_stride = tokens if logits is None else logits.shape[-1]
    if logits is None:
        logits = torch.empty((H, logit_stride), dtype=torch.float32, device=keys.device)
    if pool_rows is None:
        pool_rows = keys.numel() // key_stride_words
    check(lib().hs_gqa_score_logits(_p(q16), _p(q32), _p(keys), key_stride_words, _p(rows),
                                    pool_rows, tokens, _p(out), score_stride, _p(head0_partial),
                                    _p(logits), logit_stride, _s(stream)))
    return out, logits


# ---- selection ---------------------------------------------------------------

def score_batched(jobs, stream=None):
    """Score up to 16 (q16, keys, tokens) jobs in one launch.

    jobs: sequence of dicts with q16, keys, tokens and optional
    key_stride_words (1024), out, score_stride, head0_partial.  Returns the
    list of score tensors [32, score_stride]."""
    from . import ScoreJob
    table = (ScoreJob * max(1, len(jobs)))()
    outs = []
    for i, j in enumerate(jobs):
        _need_cuda(j["q16"], j["keys"])
        tokens = int(j["tokens"])
        stride = int(j.get("score_stride") or tokens)
        out = j.get("out")
        if out is None:
            out = torch.empty((32, stride), dtype=torch.float16, device=j["keys"].device)
        outs.append(out)
        table[i] = ScoreJob(_p(j["q16"]), _p(j["keys"]), _p(out), _p(j.get("head0_partial")),
                            int(j.get("key_stride_words", 1024)), tokens, stride, 0)
    check(lib().hs_gqa_score_batched(ctypes.cast(table, ctypes.c_void_p), len(jobs), _s(stream)))
    return outs


def _select_flags(scale_raw, fp32_counts, require_k, id_order, cover, counted=False):
    return ((HS_SELECT_SCALE_RAW if scale_raw else 0) | (HS_SELECT_FP32_COUNTS if fp32_counts else 0)
            | (HS_SELECT_REQUIRE_K if require_k else 0) | (HS_SELECT_ID_ORDER if id_order else 0)
            | (HS_SELECT_COVER if cover else 0) | (HS_SELECT_COUNTED if counted else 0))


def select_workspace_bytes(heads, n):
    return lib().hs_gqa_select_workspace_bytes(heads, n)


def select(scores, heads, stride, n, alpha, ratio, *, scale_raw=False, fp32_counts=False,
           require_k=False, id_order=False, cover=False, counted=False, head0_partial=None, ids=None,
           ids_stride=None, counts=None, member=None, status=None, ws=None, stream=None):
    """select_gqa_scores on device.  Returns (ids, counts, member, status).

    ids per head are in rank order (key desc, id asc), or ascending id order
    with id_order=True (same set, no rank sort).  cover=True selects the
    history cover of prefetch_payload (policy/full_gqa_runtime.cpp:299-344)
    over the n historical columns; status["k"] is then the cover bound.
    counted=True: the count launch already ran on this ws
    (attention_then_count)."""
    _need_cuda(scores)
    dev = scores.device
    cols = n + 1 if cover else n
    kmax = min(n, math.floor(float(cols) * float(ctypes.c_float(ratio).value)))
    if ids_stride is None:
        ids_stride = max(1, kmax)
    if ids is None:
        ids = torch.empty((heads, ids_stride), dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.empty(heads, dtype=torch.int32, device=dev)
    if status is None:
        status = new_status(dev, stream)
    if ws is None:
        ws = _scratch(select_workspace_bytes(heads, n), dev, stream)
    flags = _select_flags(scale_raw, fp32_counts, require_k, id_order, cover, counted)
    check(lib().hs_gqa_select(_p(scores), heads, stride, n, alpha, ratio, flags,
                              _p(head0_partial), _p(ids), ids_stride, _p(counts), _p(member),
                              _p(status), _p(ws), _s(stream)))
    return ids, counts, member, status


def _current(job):
    """(current_q, current_key) of a selection job dict: the current-token
    completion of column n - 1 (both or neither)."""
    q, key = job.get("current_q"), job.get("current_key")
    _need_cuda(q, key)
    return _p(q), _p(key)


def select_batched(jobs, heads, alpha, ratio, *, scale_raw=False, fp32_counts=False,
                   require_k=False, id_order=False, cover=False, stream=None):
    """Up to 16 selections sharing heads/alpha/ratio/flags in one batch.

    jobs: dicts with scores [heads, stride] and n, optional head0_partial,
    member (int32 [heads, ceil(n/32)]), current_q and current_key (the
    current-token completion of column n - 1: F16 [32, 128] query and the
    token's F16 [8, 128] K row; head0_partial then covers the n - 1 history
    columns).  Returns a list of
    (ids, counts, member, status) per job."""
    from . import SelectJob
    table = (SelectJob * max(1, len(jobs)))()
    results = []
    for i, j in enumerate(jobs):
        scores, n = j["scores"], int(j["n"])
        _need_cuda(scores)
        dev = scores.device
        stride = int(j.get("stride") or scores.shape[-1])
        cols = n + 1 if cover else n
        kmax = min(n, math.floor(float(cols) * float(ctypes.c_float(ratio).value)))
        ids_stride = max(1, kmax)
        ids = torch.empty((heads, ids_stride), dtype=torch.int32, device=dev)
        counts = torch.empty(heads, dtype=torch.int32, device=dev)
        status = new_status(dev, stream)
        ws = _scratch(select_workspace_bytes(heads, n), dev, stream)
        member = j.get("member")
        results.append((ids, counts, member, status, ws))
        table[i] = SelectJob(_p(scores), _p(j.get("head0_partial")), _p(ids), _p(counts),
                             _p(member), _p(status), _p(ws), stride, n, ids_stride, 0,
                             *_current(j))
    flags = _select_flags(scale_raw, fp32_counts, require_k, id_order, cover)
    check(lib().hs_gqa_select_batched(ctypes.cast(table, ctypes.c_void_p), len(jobs), heads,
                                      alpha, ratio, flags, _s(stream)))
    return [r[:4] for r in results]


def _select_table(jobs):
    """hs_select_job_t table over caller-owned buffers (scores, n, ids,
    status, ws; optional stride, head0_partial, counts, member, ids_stride,
    current_q, current_key)."""
    from . import SelectJob
    table = (SelectJob * max(1, len(jobs)))()
    for i, j in enumerate(jobs):
        _need_cuda(j["scores"], j["ids"], j["status"], j["ws"])
        stride = int(j.get("stride") or j["scores"].shape[-1])
        ids_stride = int(j.get("ids_stride") or j["ids"].shape[-1])
        table[i] = SelectJob(_p(j["scores"]), _p(j.get("head0_partial")), _p(j["ids"]),
                             _p(j.get("counts")), _p(j.get("member")), _p(j["status"]),
                             _p(j["ws"]), stride, int(j["n"]), ids_stride, 0, *_current(j))
    return table


def prepare_select_batched(jobs, heads, alpha, ratio, *, scale_raw=False, fp32_counts=False,
                           require_k=False, id_order=False, cover=False, counted=False,
                           stream=None):
    """Bind hs_gqa_select_batched to caller-owned buffers (as
    prepare_select_then_score): returns a callable that enqueues it."""
    table = _select_table(jobs)
    flags = _select_flags(scale_raw, fp32_counts, require_k, id_order, cover, counted)
    fn, tp, st, nj = lib().hs_gqa_select_batched, ctypes.cast(table, ctypes.c_void_p), _s(stream), len(jobs)
    keep = (jobs, table)

    def call():
        check(fn(tp, nj, heads, alpha, ratio, flags, st))
        return keep

    return call


def prepare_select_then_score(select_jobs, score_jobs, heads, alpha, ratio, *, scale_raw=False,
                              fp32_counts=False, require_k=False, id_order=False, cover=False,
                              counted=False, stream=None):
    """Bind hs_gqa_select_then_score to fixed buffers: returns a callable
    that enqueues the call (on `stream`, default the current stream at bind
    time) with job tables built once.  For a decode loop that reuses its
    buffers every step.

    select_jobs: dicts with scores, n and the caller's ids, status and ws
    (optional stride, head0_partial, counts, member, ids_stride);
    score_jobs: as score_batched, each with its own out (which must not
    overlap any selection buffer)."""
    from . import ScoreJob, SelectJob
    stable = (SelectJob * max(1, len(select_jobs)))()
    for i, j in enumerate(select_jobs):
        _need_cuda(j["scores"], j["ids"], j["status"], j["ws"])
        n = int(j["n"])
        stride = int(j.get("stride") or j["scores"].shape[-1])
        ids_stride = int(j.get("ids_stride") or j["ids"].shape[-1])
        stable[i] = SelectJob(_p(j["scores"]), _p(j.get("head0_partial")), _p(j["ids"]),
                              _p(j.get("counts")), _p(j.get("member")), _p(j["status"]),
                              _p(j["ws"]), stride, n, ids_stride, 0, *_current(j))
    ttable = (ScoreJob * max(1, len(score_jobs)))()
    for i, j in enumerate(score_jobs):
        _need_cuda(j["q16"], j["keys"], j["out"])
        tokens = int(j["tokens"])
        ttable[i] = ScoreJob(_p(j["q16"]), _p(j["keys"]), _p(j["out"]), _p(j.get("head0_partial")),
                             int(j.get("key_stride_words", 1024)), tokens,
                             int(j.get("score_stride") or tokens), 0)
    flags = _select_flags(scale_raw, fp32_counts, require_k, id_order, cover, counted)
    fn = lib().hs_gqa_select_then_score
    sp, tp, st = ctypes.cast(stable, ctypes.c_void_p), ctypes.cast(ttable, ctypes.c_void_p), _s(stream)
    ns, nt = len(select_jobs), len(score_jobs)
    keep = (select_jobs, score_jobs, stable, ttable)  # the tensors and tables outlive the callable

    def call():
        check(fn(sp, ns, heads, alpha, ratio, flags, tp, nt, st))
        return keep

    return call


def select_then_score(select_jobs, score_jobs, heads, alpha, ratio, stream=None, **flags):
    """One layer's selections and the next layer's scoring in one call
    (hs_gqa_select_then_score): the scoring runs on the CUs the per-head
    selection leaves idle.  Outputs equal select_batched then score_batched;
    arguments as prepare_select_then_score."""
    prepare_select_then_score(select_jobs, score_jobs, heads, alpha, ratio, stream=stream,
                              **flags)()


def prepare_attention_then_count(q32, pool, n, member, next_jobs, heads, alpha, ratio, *,
                                 out, ws, v_pool=None, row_bytes=4096, scale_raw=False,
                                 fp32_counts=False, require_k=False, id_order=False, cover=False,
                                 stream=None):
    """Bind hs_gqa_attention_then_count to fixed buffers (as
    prepare_select_then_score): this layer's sparse attention, and the count
    launch of the next layer's selections (next_jobs as in
    prepare_select_then_score; run them afterwards with counted=True)."""
    from . import SelectJob
    _need_cuda(q32, pool, member, out, ws, v_pool)
    kp, vp, row_bytes, pool_rows = _kv_pool(pool, v_pool, row_bytes)
    table = (SelectJob * max(1, len(next_jobs)))()
    for i, j in enumerate(next_jobs):
        _need_cuda(j["scores"], j["ids"], j["status"], j["ws"])
        stride = int(j.get("stride") or j["scores"].shape[-1])
        ids_stride = int(j.get("ids_stride") or j["ids"].shape[-1])
        table[i] = SelectJob(_p(j["scores"]), _p(j.get("head0_partial")), _p(j["ids"]),
                             _p(j.get("counts")), _p(j.get("member")), _p(j["status"]),
                             _p(j["ws"]), stride, int(j["n"]), ids_stride, 0, *_current(j))
    flags = _select_flags(scale_raw, fp32_counts, require_k, id_order, cover)
    fn = lib().hs_gqa_attention_then_count
    args = (_p(q32), kp, vp, row_bytes, None, pool_rows, _p(member), n, _p(out), _p(ws),
            ctypes.cast(table, ctypes.c_void_p), len(next_jobs), heads, alpha, ratio, flags,
            _s(stream))
    keep = (q32, pool, v_pool, member, out, ws, next_jobs, table)

    def call():
        check(fn(*args))
        return keep

    return call


def rehearsal_query(hidden, wq, positions, eps=1e-5, theta=500000.0, out=None, status=True,
                    stream=None):
    """Rehearsal query of a batch (<= 16 sequences) on MFMA.

    hidden: bfloat16 [batch, 4096]; wq: bfloat16 [4096, 4096] (out, in);
    positions: host ints.  Returns (q16 [batch, 32, 128], status or None)."""
    _need_cuda(hidden, wq)
    batch = hidden.shape[0]
    pos = (ctypes.c_uint32 * max(1, batch))(*[int(p) for p in positions])
    if out is None:
        out = torch.empty((batch, 32, 128), dtype=torch.float16, device=hidden.device)
    st = None
    if status:  # written by the launch itself: no clearing
        st = torch.empty((batch, 4), dtype=torch.int32, device=hidden.device)
    check(lib().hs_rehearsal_query(_p(hidden), _p(wq), ctypes.cast(pos, ctypes.c_void_p), batch,
                                   eps, theta, _p(out), _p(st), None, _s(stream)))
    return out, st


# ---- union / pack / gather -------------------------------------------------------

def physical_union(ids, lens, ids_stride, visible, stream=None):
    dev = ids.device
    out = torch.empty(visible, dtype=torch.int32, device=dev)
    out_n = torch.empty(1, dtype=torch.int32, device=dev)
    with torch.cuda.stream(stream if stream is not None else torch.cuda.current_stream()):
        out_n.zero_()
    status = new_status(dev, stream)
    ws = _scratch(lib().hs_gqa_union_workspace_bytes(visible), dev, stream)
    check(lib().hs_gqa_physical_union(_p(ids), _p(lens), ids_stride, visible, _p(out), _p(out_n),
                                      _p(status), _p(ws), _s(stream)))
    return out, out_n, status


def _kv_pool(pool, v_pool, row_bytes):
    """(K base, V base, row bytes, rows) of a hot pool: one tensor of the
    reference's 4096 B KV records (v_pool None), or K and V row arrays."""
    if v_pool is None:
        if row_bytes != 4096:
            raise ValueError("a single pool tensor holds 4096 B KV records")
        return (_p(pool), ctypes.c_void_p(pool.data_ptr() + 2048), 4096,
                pool.numel() * pool.element_size() // 4096)
    rows = min(pool.numel() * pool.element_size(), v_pool.numel() * v_pool.element_size())
    return _p(pool), _p(v_pool), row_bytes, rows // row_bytes


def pack(pool, ids, lens, ids_stride, positions, count, row_of_id=None, max_id=None,
         v_pool=None, row_bytes=4096, status=None, stream=None):
    """pack_gqa_workspace from the device hot pool -> (K, V, mask, status).
    pool: 4096 B KV records, or with v_pool the K and V row arrays.  status:
    any 8-byte aligned int32[4] (no clearing needed: the call stamps it)."""
    dev = pool.device
    nq = positions.numel()
    qpad = (nq + 63) // 64 * 64
    k = torch.empty(count * H * D, dtype=torch.float16, device=dev)
    v = torch.empty(count * H * D, dtype=torch.float16, device=dev)
    mask = torch.empty(H * qpad * count, dtype=torch.float32, device=dev)
    if status is None:
        status = torch.empty(4, dtype=torch.int32, device=dev)
    kp, vp, row_bytes, pool_rows = _kv_pool(pool, v_pool, row_bytes)
    if max_id is None:
        max_id = row_of_id.numel() if row_of_id is not None else pool_rows
    check(lib().hs_gqa_pack(kp, vp, row_bytes, pool_rows, _p(row_of_id), max_id, _p(ids), _p(lens),
                            ids_stride,
                            _p(positions), nq, count, _p(k), _p(v), _p(mask), _p(status),
                            _s(stream)))
    return k, v, mask, status


def gather_rows(prefetched, misses, row_map, count, status=None, stream=None):
    """GQAPrefetchCuda's gather_gqa on device rows -> (K, V, status); status
    as for pack (no clearing needed)."""
    dev = row_map.device
    k = torch.empty(count * H * D, dtype=torch.float16, device=dev)
    v = torch.empty(count * H * D, dtype=torch.float16, device=dev)
    if status is None:
        status = torch.empty(4, dtype=torch.int32, device=dev)
    rows_of = lambda t: 0 if t is None else t.numel() * t.element_size() // 4096
    check(lib().hs_gqa_gather_rows(_p(prefetched), rows_of(prefetched), _p(misses), rows_of(misses),
                                   _p(row_map), count, _p(k), _p(v), _p(status), _s(stream)))
    return k, v, status


# ---- attention / fused layer -------------------------------------------------------

def attention_workspace_bytes(n):
    return lib().hs_gqa_attention_workspace_bytes(n)


def sparse_attention(q32, pool, n, member, rows=None, out=None, ws=None, pool_rows=None,
                     v_pool=None, row_bytes=4096, stream=None):
    """pool: 4096 B KV records, or with v_pool the K and V row arrays."""
    _need_cuda(q32, pool, member, v_pool)
    dev = pool.device
    if out is None:
        out = torch.empty((H, D), dtype=torch.float32, device=dev)
    if ws is None:
        ws = _scratch(attention_workspace_bytes(n), dev, stream)
    kp, vp, row_bytes, rows_in_pool = _kv_pool(pool, v_pool, row_bytes)
    if pool_rows is None:
        pool_rows = rows_in_pool
    check(lib().hs_gqa_sparse_attention(_p(q32), kp, vp, row_bytes, _p(rows), pool_rows,
                                        _p(member), n, _p(out), _p(ws), _s(stream)))
    return out


def sparse_attention_logits(logits, v_pool, n, member, rows=None, out=None, ws=None,
                            pool_rows=None, row_bytes=2048, stream=None):
    """hs_gqa_sparse_attention_logits: attention from the scoring pass's dots
    (logits F32 [32, stride]) over the selected V rows of v_pool (rows of
    row_bytes)."""
    _need_cuda(logits, v_pool, member, rows)
    dev = v_pool.device
    if out is None:
        out = torch.empty((H, D), dtype=torch.float32, device=dev)
    if ws is None:
        ws = _scratch(attention_workspace_bytes(n), dev, stream)
    if pool_rows is None:
        pool_rows = v_pool.numel() * v_pool.element_size() // row_bytes
    check(lib().hs_gqa_sparse_attention_logits(_p(logits), logits.shape[-1], _p(v_pool), row_bytes,
                                               _p(rows), pool_rows, _p(member), n, _p(out), _p(ws),
                                               _s(stream)))
    return out


def decode_layer_workspace_bytes(n):
    return lib().hs_decode_layer_workspace_bytes(n)


def decode_layer(q16, q32, pool, n, alpha, ratio, *, rows=None, fp32_counts=False, scores=None,
                 ids=None, ids_stride=None, counts=None, out=None, status=None, ws=None,
                 pool_rows=None, v_pool=None, row_bytes=4096, stream=None):
    """score -> select -> sparse attention for one layer (all on device).
    pool: 4096 B KV records, or with v_pool the K and V arrays (row_bytes
    2048: the scorer streams K contiguously)."""
    dev = pool.device
    kmax = min(n, math.floor(float(n) * float(ctypes.c_float(ratio).value)))
    if ids_stride is None:
        ids_stride = max(1, kmax)
    if scores is None:
        scores = torch.empty((H, n), dtype=torch.float16, device=dev)
    if ids is None:
        ids = torch.empty((H, ids_stride), dtype=torch.int32, device=dev)
    if counts is None:
        counts = torch.empty(H, dtype=torch.int32, device=dev)
    if out is None:
        out = torch.empty((H, D), dtype=torch.float32, device=dev)
    if status is None:
        status = new_status(dev, stream)
    if ws is None:
        ws = _scratch(decode_layer_workspace_bytes(n), dev, stream)
    kp, vp, row_bytes, rows_in_pool = _kv_pool(pool, v_pool, row_bytes)
    if pool_rows is None:
        pool_rows = rows_in_pool
    check(lib().hs_decode_layer(_p(q16), _p(q32), kp, vp, row_bytes, _p(rows), pool_rows, n,
                                alpha, ratio,
                                HS_SELECT_FP32_COUNTS if fp32_counts else 0, _p(scores), _p(ids),
                                ids_stride, _p(counts), _p(out), _p(status), _p(ws), _s(stream)))
    return scores, ids, counts, out, status


def kv_cold_fetch(image, layer, positions, k_out, *, v_out=None, row_bytes=4096, status=None,
                  ws=None, stream=None):
    """Device read of cold records (hs_kv_cold_fetch) from a pinned
    SegmentedKVStore image: record i's K half to row i of k_out and its V
    half to row i of v_out (v_out None: k_out holds 4096 B records)."""
    _need_cuda(positions, k_out, v_out)
    if image.is_cuda or not image.is_pinned():
        raise ValueError("the store image must be pinned host memory")
    count = positions.numel()
    if v_out is None:
        if row_bytes != 4096:
            raise ValueError("a single output tensor holds 4096 B KV records")
        kp, vp = _p(k_out), ctypes.c_void_p(k_out.data_ptr() + 2048)
    else:
        kp, vp = _p(k_out), _p(v_out)
    if status is None:
        status = new_status(k_out.device, stream)
    if ws is None:
        ws = _scratch(lib().hs_kv_cold_fetch_workspace_bytes(count), k_out.device, stream)
    check(lib().hs_kv_cold_fetch(ctypes.c_void_p(image.data_ptr()), layer, _p(positions), count,
                                 kp, vp, row_bytes, _p(status), _p(ws), _s(stream)))
    return status


def cold_plan(member, heads, n, slot, staging_base, list_size, positions=None, rows=None,
              count=None, stream=None):
    """hs_gqa_cold_plan of one sequence -> (positions, rows, count): the
    selected tokens whose slot is negative, ascending (padded with
    0xffffffff to list_size), the row map (slot, staging_base + list index,
    or -1) and their count."""
    _need_cuda(member, slot)
    dev = member.device
    if positions is None:
        positions = torch.empty(list_size, dtype=torch.int32, device=dev)
    if rows is None:
        rows = torch.empty(n, dtype=torch.int32, device=dev)
    if count is None:
        count = torch.empty(1, dtype=torch.int32, device=dev)
    check(lib().hs_gqa_cold_plan(_p(member), heads, n, _p(slot), staging_base, list_size,
                                 _p(positions), _p(rows), _p(count), _s(stream)))
    return positions, rows, count


def cold_runs(positions):
    """(run_first, run_count) ctypes arrays of the consecutive runs of an
    ascending host list of positions."""
    firsts, counts = [], []
    for p in positions:
        p = int(p)
        if firsts and firsts[-1] + counts[-1] == p:
            counts[-1] += 1
        else:
            firsts.append(p)
            counts.append(1)
    n = max(1, len(firsts))
    return (ctypes.c_uint32 * n)(*firsts), (ctypes.c_uint32 * n)(*counts), len(firsts)


def kv_cold_fetch_runs(image, layer, runs, raw, positions, k_out, *, v_out=None, row_bytes=4096,
                       status=None, ws=None, stream=None):
    """hs_kv_cold_fetch_runs: the records of `runs` (from cold_runs) copied
    from the pinned image into `raw` (uint8, count x 4128) by the copy
    engines, then checked and split into k_out / v_out as kv_cold_fetch does;
    positions: the expected position of each staged record (device)."""
    _need_cuda(raw, positions, k_out, v_out)
    if image.is_cuda or not image.is_pinned():
        raise ValueError("the store image must be pinned host memory")
    first, count_arr, nruns = runs
    count = positions.numel()
    if v_out is None:
        if row_bytes != 4096:
            raise ValueError("a single output tensor holds 4096 B KV records")
        kp, vp = _p(k_out), ctypes.c_void_p(k_out.data_ptr() + 2048)
    else:
        kp, vp = _p(k_out), _p(v_out)
    if status is None:
        status = new_status(k_out.device, stream)
    if ws is None:
        ws = _scratch(lib().hs_kv_cold_fetch_workspace_bytes(count), k_out.device, stream)
    check(lib().hs_kv_cold_fetch_runs(ctypes.c_void_p(image.data_ptr()), layer,
                                      ctypes.cast(first, ctypes.c_void_p),
                                      ctypes.cast(count_arr, ctypes.c_void_p), nruns, _p(raw),
                                      _p(positions), count, kp, vp, row_bytes, _p(status), _p(ws),
                                      _s(stream)))
    return status


# ---- device checks and synthetic data -------------------------------------------------

def selftest_f16_checksums(stream=None):
    out = torch.empty(65536, dtype=torch.int64, device="cuda")
    check(lib().hs_selftest_f16_checksums(_p(out), _s(stream)))
    return out


def selftest_scale_table(stream=None):
    out = torch.empty(65536, dtype=torch.int16, device="cuda")
    check(lib().hs_selftest_scale_table(_p(out), _s(stream)))
    return out


def selftest_key_table(stream=None):
    """[2, 65536] order keys the selection computes two at a time: row 0 of
    the scaled values, row 1 of the raw ones (finite inputs only meaningful)."""
    out = torch.empty((2, 65536), dtype=torch.int16, device="cuda")
    check(lib().hs_selftest_key_table(_p(out), _s(stream)))
    return out


def fill_gaussian(t, seed, scale=1.0, stream=None):
    check(lib().hs_fill_gaussian_f16(_p(t), t.numel(), seed, scale, _s(stream)))
    return t


def fill_rope_keys(t, tokens, row_stride_words, heads_per_row, seed, theta=500000.0,
                   stream=None):
    check(lib().hs_fill_rope_keys_f16(_p(t), tokens, row_stride_words, heads_per_row, seed, theta,
                                      _s(stream)))
    return t


__all__ = [name for name in dir() if not name.startswith("_")] + ["HsError"]
