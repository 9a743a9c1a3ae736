"""End-to-end sparse decode layer on the GPU against the oracle.

BASELINE.json configs[0] against the golden fixture written by the compiled
reference; configs[2] (score N=32768 over the hot pool, select at the cap,
sparse attention) against the oracle: scores and ids bit-exact, attention
within 2e-3."""
from pathlib import Path

import numpy as np
import pytest
import torch

from hs_data import config1_inputs, f16_bits, from_dev, pool_rows, rng, rope_keys, to_dev
from test_gpu_attention import rel_err

pytestmark = pytest.mark.gpu
FIXTURE = Path(__file__).resolve().parent / "golden" / "config1.npz"


def test_config1_golden(hs):
    g = np.load(FIXTURE, allow_pickle=False)
    n = int(g["n"])
    q, k, _ = config1_inputs(0, n)
    partial = torch.zeros((n + 63) // 64, dtype=torch.int32, device="cuda")
    raw = hs.ops.score(to_dev(q), to_dev(k.reshape(-1)), n, head0_partial=partial)
    assert np.array_equal(from_dev(raw), g["raw"])
    ids, counts, _, status = hs.ops.select(raw, 32, n, n, float(g["alpha"]), float(g["ratio"]),
                                           scale_raw=True, head0_partial=partial)
    st = hs.ops.read_status(status)
    assert st["code"] == 0 and st["k"] == int(g["k"])
    assert st["boundary_tied_heads"] == int(g["boundary_tied_heads"])
    assert np.array_equal(from_dev(ids)[:, : st["k"]], g["ids"])
    assert np.array_equal(from_dev(counts), g["counts"])


@pytest.mark.parametrize("n,alpha", [(4096, 5.0), (32768, 5.0), (32768, 1.5)])
def test_config3_layer(hs, port, n, alpha):
    g = rng(3000 + n)
    k = rope_keys(n, 31 + n)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    q16 = f16_bits(g.standard_normal((32, 128)))
    q32 = g.standard_normal((32, 128)).astype(np.float32)
    scores, ids, counts, out, status = hs.ops.decode_layer(
        to_dev(q16), torch.from_numpy(q32).cuda(), to_dev(pool.reshape(-1)), n, alpha, 0.2)
    st = hs.ops.read_status(status)
    raw = port.score(q16, pool.reshape(-1), n, 2048)
    assert np.array_equal(from_dev(scores), raw)
    rc, kk, pids, pcounts, tied = port.select(port.scale(raw), 32, n, n, alpha, 0.2)
    assert st["code"] == 0 and st["k"] == kk and st["boundary_tied_heads"] == tied
    gids = from_dev(ids)[:, :kk]  # the layer lists each head's selection by ascending id
    assert np.array_equal(gids, np.sort(pids, axis=1)) and np.array_equal(from_dev(counts), pcounts)
    ref = port.attention(q32, pool.view(np.uint8).reshape(-1), [list(r) for r in pids])
    assert rel_err(out.cpu().numpy().astype(np.float64), ref) <= 2e-3
    if alpha == 5.0:
        assert kk == int(np.floor(n * np.float64(np.float32(0.2))))  # k reaches the cap


def test_layer_zero_selection_is_an_error(hs):
    n = 256
    g = rng(1)
    k = f16_bits(g.standard_normal((n, 8, 128)) * 0.01)
    k[7, 0, :] = f16_bits(np.full(128, 8.0))  # one token dominates head 0
    v = f16_bits(g.standard_normal((n, 8, 128)))
    pool = pool_rows(k, v)
    q16 = f16_bits(np.ones((32, 128)))
    q32 = np.ones((32, 128), dtype=np.float32)
    *_, status = hs.ops.decode_layer(to_dev(q16), torch.from_numpy(q32).cuda(),
                                     to_dev(pool.reshape(-1)), n, 0.5, 0.2)
    assert hs.ops.read_status(status)["code"] == hs.HS_ERR_ZERO_SELECTION


def test_layer_split_kv_arrays_equal_records(hs):
    # score over the K array's 2048 B rows and attention over the K and V
    # arrays: scores, ids, counts and output equal the 4096 B record layout's
    n = 32768
    g = rng(4242)
    k = rope_keys(n, 4243)
    v = f16_bits(g.standard_normal((n, 8, 128)))
    records = pool_rows(k, v)
    q16 = f16_bits(g.standard_normal((32, 128)))
    q32 = torch.from_numpy(g.standard_normal((32, 128)).astype(np.float32)).cuda()
    a = hs.ops.decode_layer(to_dev(q16), q32, to_dev(records.reshape(-1)), n, 5.0, 0.2)
    b = hs.ops.decode_layer(to_dev(q16), q32, to_dev(np.ascontiguousarray(records[:, :1024])), n,
                            5.0, 0.2, v_pool=to_dev(np.ascontiguousarray(records[:, 1024:])),
                            row_bytes=2048)
    sa, sb = hs.ops.read_status(a[4]), hs.ops.read_status(b[4])
    assert sa == sb and sa["code"] == 0
    kk = sa["k"]
    assert torch.equal(a[0], b[0])
    assert torch.equal(a[1][:, :kk], b[1][:, :kk])
    assert torch.equal(a[2], b[2]) and torch.equal(a[3], b[3])
