"""The C ABI library loads and exports every function include/hs_gpu.h
declares; host-side argument checks reject bad shapes before any GPU work
(no compute call is made here)."""
import ctypes
import subprocess
from pathlib import Path

import pytest


@pytest.fixture(scope="module")
def hs():
    import hillserve_amd
    hillserve_amd.lib()
    return hillserve_amd


def test_exports_every_declared_function(hs):
    declared = hs.header_functions()
    assert len(declared) >= 18
    missing = [name for name in declared if not hasattr(hs.lib(), name)]
    assert missing == []
    assert set(hs.SIGNATURES) == set(declared)


def test_version(hs):
    assert b"gfx950" in hs.lib().hs_version()


def test_v3_rejects_invalid_counts_without_access(hs):
    # kernels/full_gqa_pipeline/kernel_check.cpp:116-121: null Q/K/S with an
    # invalid N must be refused without touching memory.
    for n in [0, 1, 32, 63, 65, 32769, 0xFFFFFFFF]:
        assert hs.lib().hs_full_gqa_pipeline(None, None, None, n, None) == hs.HS_ERR_ARGUMENT
        assert "64<=N<=32768" in hs.last_error()


def test_select_rejects_bad_parameters(hs):
    fake = ctypes.c_void_p(0x1000)  # never dereferenced: shape checks come first
    L = hs.lib()
    args = dict(scores=fake, heads=32, stride=64, n=64, alpha=1.0, ratio=0.2, flags=0,
                partial=None, ids=fake, ids_stride=64, counts=None, member=None, status=fake,
                ws=fake, stream=None)

    def call(**kw):
        a = {**args, **kw}
        return L.hs_gqa_select(a["scores"], a["heads"], a["stride"], a["n"], a["alpha"],
                               a["ratio"], a["flags"], a["partial"], a["ids"], a["ids_stride"],
                               a["counts"], a["member"], a["status"], a["ws"], a["stream"])

    assert call(heads=0) == hs.HS_ERR_ARGUMENT
    assert call(heads=129) == hs.HS_ERR_ARGUMENT
    assert call(n=0) == hs.HS_ERR_ARGUMENT
    assert call(n=131073, stride=140000) == hs.HS_ERR_ARGUMENT
    assert call(stride=63) == hs.HS_ERR_ARGUMENT
    assert call(alpha=-1.0) == hs.HS_ERR_ARGUMENT
    assert call(alpha=float("inf")) == hs.HS_ERR_ARGUMENT
    assert call(ratio=0.0) == hs.HS_ERR_ARGUMENT
    assert call(ratio=1.5) == hs.HS_ERR_ARGUMENT
    assert call(ids_stride=11) == hs.HS_ERR_ARGUMENT  # floor(64*0.2f) = 12
    assert call(flags=64) == hs.HS_ERR_ARGUMENT
    assert call(scores=None) == hs.HS_ERR_ARGUMENT


def test_score_rejects_bad_shapes(hs):
    fake = ctypes.c_void_p(0x1000)
    L = hs.lib()
    assert L.hs_gqa_score(fake, fake, 1000, None, 0, 64, fake, 64, None, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_gqa_score(fake, fake, 1024, None, 0, 0, fake, 64, None, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_gqa_score(fake, fake, 1024, None, 0, 65537, fake, 70000, None, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_gqa_score(fake, fake, 1024, None, 0, 64, fake, 63, None, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_gqa_score(fake, ctypes.c_void_p(0x1008), 1024, None, 0, 64, fake, 64, None,
                          None) == hs.HS_ERR_ARGUMENT  # keys not 16-byte aligned


def test_pack_union_gather_reject_bad_shapes(hs):
    fake = ctypes.c_void_p(0x1000)
    L = hs.lib()
    assert L.hs_gqa_physical_union(fake, fake, 8, 0, fake, fake, fake, fake, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_gqa_physical_union(fake, fake, 8, 66049, fake, fake, fake, fake, None) == hs.HS_ERR_ARGUMENT
    pack = lambda nq, count, row_bytes=4096: L.hs_gqa_pack(
        fake, fake, row_bytes, 1, None, 1, fake, fake, 8, fake, nq, count, fake, fake, fake, fake,
        None)
    assert pack(0, 32) == hs.HS_ERR_ARGUMENT  # nq == 0
    assert pack(257, 32) == hs.HS_ERR_ARGUMENT  # nq > 256
    assert pack(1, 0) == hs.HS_ERR_ARGUMENT  # count == 0
    assert pack(1, 32, row_bytes=1024) == hs.HS_ERR_ARGUMENT  # a row holds 2048 B of K
    assert L.hs_gqa_gather_rows(fake, 1, fake, 1, fake, 0, fake, fake, fake, None) == hs.HS_ERR_ARGUMENT
    for row_bytes in (1000, 2056 - 1, 1 << 21):  # below 2048, not a multiple of 16, above 1 MiB
        assert L.hs_gqa_sparse_attention(fake, fake, fake, row_bytes, None, 0, fake, 64, fake,
                                         fake, None) == hs.HS_ERR_ARGUMENT
    misaligned = ctypes.c_void_p(0x1008)
    assert L.hs_gqa_sparse_attention(fake, fake, misaligned, 2048, None, 0, fake, 64, fake, fake,
                                     None) == hs.HS_ERR_ARGUMENT
    # the scorer streams K rows of 2048 or 4096 B only
    assert L.hs_decode_layer(fake, fake, fake, fake, 3072, None, 0, 64, 1.0, 0.2, 0, fake, fake,
                             16, fake, fake, fake, fake, None) == hs.HS_ERR_ARGUMENT
    assert L.hs_kv_cold_fetch(fake, 0, fake, 1, fake, fake, 1024, fake, fake,
                              None) == hs.HS_ERR_ARGUMENT


CONTRACTS = Path(__file__).resolve().parent / "cpp" / "gqa_gpu_contracts"


def test_cpp_adapters_exported(hs):
    # the C++17 host adapters (include/hs_gqa.hpp) live in the same library
    out = subprocess.run(["nm", "-D", "--defined-only", "-C", str(hs.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    for name in ("hillserve::gpu::FullGqaGpuScorer::score(", "hillserve::gpu::select_gqa_scores(",
                 "hillserve::gpu::gqa_physical_union(", "hillserve::gpu::pack_gqa_workspace(",
                 "hillserve::gpu::GpuScoreBackend::score_raw_gqa(", "hillserve::gpu::history_cover_gqa("):
        assert name in out, name


def test_cpp_contracts_binary_links():
    # built by hillserve_amd.build; without a GPU it reports "skipped" (77)
    import torch
    assert CONTRACTS.exists(), "run python -m hillserve_amd.build"
    if torch.cuda.is_available():
        pytest.skip("GPU visible: the contract run itself is a gpu test")
    proc = subprocess.run([str(CONTRACTS)], capture_output=True, text=True, timeout=60)
    assert proc.returncode == 77 and "skipped" in proc.stdout, proc.stdout + proc.stderr


def test_select_then_score_rejects_overlap(hs):
    # The scoring of the next layer runs beside the selection: its scores may
    # not land on the selection's scores, and nothing may alias a selection
    # output.  Every check is on the host, before any launch.
    L = hs.lib()
    MB = 1 << 20
    base = 0x10000000

    def sel(scores, ids, status, ws):
        return hs.SelectJob(scores, None, ids, None, None, status, ws, 4096, 4096, 819, 0)

    def sco(q, keys, out):
        return hs.ScoreJob(q, keys, out, None, 1024, 4096, 4096, 0)

    scores, ids, status, ws = base, base + MB, base + 2 * MB, base + 3 * MB
    q, keys, out = base + 8 * MB, base + 16 * MB, base + 32 * MB

    def call(s, t):
        st = (hs.SelectJob * 1)(s)
        tt = (hs.ScoreJob * 1)(t)
        return L.hs_gqa_select_then_score(ctypes.cast(st, ctypes.c_void_p), 1, 32, 5.0, 0.2, 0,
                                          ctypes.cast(tt, ctypes.c_void_p), 1, None)

    assert call(sel(scores, ids, status, ws), sco(q, keys, scores + 4096)) == hs.HS_ERR_ARGUMENT
    assert "selection input" in hs.last_error()
    assert call(sel(scores, ids, status, ws), sco(q, keys, ws)) == hs.HS_ERR_ARGUMENT
    assert "selection output" in hs.last_error()
    assert call(sel(scores, ids, status, ws), sco(ids, keys, out)) == hs.HS_ERR_ARGUMENT
    assert "scoring input" in hs.last_error()
    # the usual shape checks of both halves still apply
    assert call(sel(scores, ids, status, ws), sco(q, keys + 8, out)) == hs.HS_ERR_ARGUMENT
    bad = sel(scores, ids, status, ws)
    bad.ids_stride = 10
    assert call(bad, sco(q, keys, out)) == hs.HS_ERR_ARGUMENT


def test_attention_then_count_rejects_overlap(hs):
    L = hs.lib()
    MB = 1 << 20
    base = 0x20000000
    q, kp, vp, member, out, aws = (base + i * 4 * MB for i in range(6))
    scores, ws, status, ids = (base + 64 * MB + i * 8 * MB for i in range(4))

    def call(job, out_ptr=out, ws_ptr=aws, flags=hs.HS_SELECT_SCALE_RAW):
        t = (hs.SelectJob * 1)(job)
        return L.hs_gqa_attention_then_count(q, kp, vp, 2048, None, 0, member, 4096, out_ptr,
                                             ws_ptr, ctypes.cast(t, ctypes.c_void_p), 1, 32, 5.0,
                                             0.2, flags, None)

    def job(scores=scores, ws=ws, status=status):
        return hs.SelectJob(scores, None, ids, None, None, status, ws, 4096, 4096, 819, 0)

    assert call(job(ws=aws)) == hs.HS_ERR_ARGUMENT          # count workspace = attention records
    assert call(job(status=out)) == hs.HS_ERR_ARGUMENT      # status over the attention output
    assert call(job(scores=out)) == hs.HS_ERR_ARGUMENT      # next scores under the output
    assert call(job(scores=aws)) == hs.HS_ERR_ARGUMENT      # next scores under the records
    assert call(job(), flags=hs.HS_SELECT_SCALE_RAW | hs.HS_SELECT_COUNTED) == hs.HS_ERR_ARGUMENT
    assert call(job(), out_ptr=0) == hs.HS_ERR_ARGUMENT     # attention shape checks still apply


def test_layer_and_batch_checks_come_before_any_launch(hs):
    """Errors found on the host are returned before anything is enqueued, so
    no output is overwritten: on a machine without a GPU a launch would fail
    with a HIP error instead of HS_ERR_ARGUMENT."""
    L = hs.lib()
    fake = ctypes.c_void_p(0x1000)
    misaligned = ctypes.c_void_p(0x1008)

    def layer(v_pool=fake, q32=fake, ids_stride=16, row_bytes=2048):
        return L.hs_decode_layer(fake, q32, fake, v_pool, row_bytes, None, 0, 64, 1.0, 0.2, 0,
                                 fake, fake, ids_stride, fake, fake, fake, fake, None)

    assert layer(v_pool=misaligned) == hs.HS_ERR_ARGUMENT
    assert "pools" in hs.last_error()
    assert layer(q32=misaligned) == hs.HS_ERR_ARGUMENT  # the split query is read as float4
    assert layer(ids_stride=11) == hs.HS_ERR_ARGUMENT  # floor(64 * 0.2f) = 12 ids per head
    assert "ids_stride" in hs.last_error()
    # the dots' F32 query is read 16 bytes at a time
    assert L.hs_gqa_score_logits(fake, ctypes.c_void_p(0x1004), fake, 1024, None, 0, 64, fake, 64,
                                 None, fake, 64, None) == hs.HS_ERR_ARGUMENT
    # the copy-engine staging is read as 16-byte words
    assert L.hs_kv_cold_fetch_runs(fake, 0, fake, fake, 1, misaligned, fake, 1, fake, fake, 4096,
                                   fake, fake, None) == hs.HS_ERR_ARGUMENT
    assert "16-byte" in hs.last_error()


def test_batch_with_current_token_rejects_shared_scores(hs):
    """A job that completes its current token writes column n - 1 of its
    scores while the batch's other count groups read theirs."""
    L = hs.lib()
    MB = 1 << 20

    def job(base, scores_at, current):
        j = hs.SelectJob()
        j.scores = base + scores_at
        j.ids, j.status, j.workspace = base + 8 * MB, base + 9 * MB, base + 10 * MB
        j.stride, j.n, j.ids_stride = 4096, 4096, 4096
        if current:
            j.current_q, j.current_key = base + 20 * MB, base + 21 * MB
        return j

    # (only rejected calls here: a call that passed would launch kernels on
    # these fake addresses)
    for first_current in (True, False):
        jobs = (hs.SelectJob * 2)(job(0x10000000, 0, first_current),
                                  job(0x40000000, 0, not first_current))
        jobs[1].scores = jobs[0].scores + 64 * 1024  # inside job 0's rows
        assert L.hs_gqa_select_batched(jobs, 2, 32, 1.0, 0.2, 0, None) == hs.HS_ERR_ARGUMENT
        assert "share scores" in hs.last_error()
