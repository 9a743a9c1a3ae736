"""The scoring pass with the attention dots (hs_gqa_score_logits) and the
attention that reads V only (hs_gqa_sparse_attention_logits).

Bars: the raw scores and tile maxima equal the plain scorer's bit for bit;
the dots are within 1e-5 relative of an FP64 dot of the same F32 query and
F16 keys; the attention is within 2e-3 of the FP64 oracle on the same
selection, with and without a row map, and agrees
with the attention that reads K itself within 1e-3 (both round their
softmax weights to F16 once)."""
import numpy as np
import pytest
import torch

from hs_data import f16_bits, from_dev, pool_rows, rng, rope_keys, to_dev
from test_gpu_attention import member_words, rel_err

pytestmark = pytest.mark.gpu
TOL = 2e-3


@pytest.mark.parametrize("n,mapped", [(4096, False), (32768, False), (6000, True), (100, False)])
def test_scores_and_dots(hs, n, mapped):
    g = rng(610 + n)
    k = rope_keys(n, 611 + n)
    q16 = f16_bits(g.standard_normal((32, 128)))
    q32 = (g.standard_normal((32, 128)) * 2.0).astype(np.float32)
    keys, rows, perm = k, None, None
    if mapped:
        perm = g.permutation(n).astype(np.int32)
        keys = k[np.argsort(perm)]  # row perm[t] holds token t
        rows = to_dev(perm)
    kd = to_dev(keys.reshape(-1))
    part_a = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    part_b = torch.empty((n + 63) // 64, dtype=torch.int32, device="cuda")
    plain = hs.ops.score(to_dev(q16.reshape(-1)), kd, n, rows=rows, head0_partial=part_a)
    raw, dots = hs.ops.score_logits(to_dev(q16.reshape(-1)), torch.from_numpy(q32).cuda(), kd, n,
                                    rows=rows, head0_partial=part_b)
    assert np.array_equal(from_dev(raw), from_dev(plain))
    assert np.array_equal(from_dev(part_b), from_dev(part_a))
    kf = k.view(np.float16).astype(np.float64).reshape(n, 8, 128)
    qg = q32.astype(np.float64).reshape(8, 4, 128)  # query head 4g + j reads KV head g
    want = np.einsum("gjc,tgc->gjt", qg, kf).reshape(32, n)
    bound = np.einsum("gjc,tgc->gjt", np.abs(qg), np.abs(kf)).reshape(32, n)
    got = dots.cpu().numpy().astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-5 * bound + 1e-30)


@pytest.mark.parametrize("n,frac,mapped", [(4096, 0.2, False), (32768, 0.2, False),
                                           (5000, 0.14, True), (257, 0.5, False)])
def test_attention_from_dots(hs, port, n, frac, mapped):
    g = rng(620 + n)
    k = rope_keys(n, 621 + n)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    records = pool_rows(k, v)
    q32 = (g.standard_normal((32, 128)) * 1.5).astype(np.float32)
    ids = [np.sort(g.choice(n, size=max(1, int(n * frac)), replace=False)) for _ in range(32)]
    member = to_dev(member_words(ids, n).reshape(-1))
    rows, perm = None, None
    if mapped:
        perm = g.permutation(n).astype(np.int32)
        records = records[np.argsort(perm)]
        rows = to_dev(perm)
    k_rows = to_dev(np.ascontiguousarray(records[:, :1024]).reshape(-1))
    v_rows = to_dev(np.ascontiguousarray(records[:, 1024:]).reshape(-1))
    qd = torch.from_numpy(q32).cuda()
    q16 = to_dev(f16_bits(g.standard_normal((32, 128))).reshape(-1))
    _, dots = hs.ops.score_logits(q16, qd, k_rows, n, rows=rows)
    out = hs.ops.sparse_attention_logits(dots, v_rows, n, member, rows=rows)
    if mapped:
        # a pool declared at 4 GiB (2^21 rows of 2048 B) takes the kernel's
        # 64-bit row addressing instead of its buffer reads; the rows the map
        # names are the same, and so are the output's bits
        wide = hs.ops.sparse_attention_logits(dots, v_rows, n, member, rows=rows, pool_rows=1 << 21)
        assert torch.equal(wide, out)
    ref = port.attention(q32, records.view(np.uint8).reshape(-1), ids, rows=perm)
    got = out.cpu().numpy().astype(np.float64)
    assert rel_err(got, ref) <= TOL
    # against the attention that reads K itself (MFMA dots of a split query):
    # each form rounds its softmax weights to F16 once, and the two forms'
    # dots differ in their last bits, so a weight may round to the other
    # neighbour (2^-11 relative); over few rows that does not average out
    via_k = hs.ops.sparse_attention(qd, k_rows, n, member, rows=rows, v_pool=v_rows,
                                    row_bytes=2048).cpu().numpy().astype(np.float64)
    assert rel_err(got, via_k) <= 1e-3
