"""Pins the indexer oracle (restating cpu_lightning_indexer,
examples/deepseek_v4/lightning_indexer.py:199-335) with an independent triple-loop
brute force, the second formulation index_golden (example_lightning_indexer.py:137-144)
and invariants."""
import math

import pytest
import torch

from oracle.dsa_oracle import index_golden, indexer_scores, lightning_indexer


def brute_scores(q, k, w, aq, ak, mode):
    """Plain loops: score[t][s] = sum_h w[t][h] * max(0, sum_d q[t][h][d]*k[s][d])."""
    G, D = q.shape[1], q.shape[2]
    out = []
    for t in range(aq):
        if mode == 3:
            cl = ak - aq + t + 1
            vis = cl if cl > 0 else ak
        else:
            vis = ak
        row = []
        for s in range(ak):
            if s >= vis:
                row.append(-math.inf)
                continue
            tot = 0.0
            for h in range(G):
                dot = 0.0
                for d in range(D):
                    dot += float(q[t, h, d]) * float(k[s, d])
                tot += float(w[t, h]) * max(dot, 0.0)
            row.append(tot)
        out.append(row)
    return torch.tensor(out, dtype=torch.float64)


@pytest.mark.parametrize("aq,ak,mode", [(3, 37, 3), (5, 9, 0), (6, 4, 3)])
def test_scores_vs_bruteforce(aq, ak, mode):
    g = torch.Generator().manual_seed(aq * 100 + ak)
    q = torch.randn((aq, 4, 8), generator=g)
    k = torch.randn((ak, 8), generator=g)
    w = torch.randn((aq, 4), generator=g)
    got = indexer_scores(q, k, w, aq, ak, mode).double()
    ref = brute_scores(q, k, w, aq, ak, mode)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    assert torch.allclose(got[fin], ref[fin], rtol=1e-5, atol=1e-5)


def test_causal_rule_when_fewer_keys_than_queries():
    # lightning_indexer.py:309-310: a row whose causal length is <= 0 sees all ak keys
    q = torch.ones((6, 1, 2))
    k = torch.ones((4, 2))
    w = torch.ones((6, 1))
    sc = indexer_scores(q, k, w, 6, 4, 3)
    # cl = 4 - 6 + t + 1 = t - 1 -> rows 0 and 1 see all keys, row 2 sees 1 key
    assert torch.isfinite(sc[0]).all() and torch.isfinite(sc[1]).all()
    assert torch.isfinite(sc[2]).tolist() == [True, False, False, False]
    assert torch.isfinite(sc[5]).all()


def test_full_indexer_vs_bruteforce_topk():
    g = torch.Generator().manual_seed(7)
    B, S1, S2, N1, D, K = 2, 5, 40, 4, 128, 16
    q = torch.randn((B, S1, N1, D), generator=g)
    k = torch.randn((B, S2, 1, D), generator=g)
    w = torch.randn((B, S1, N1), generator=g)
    idx, scores, vals = lightning_indexer(q, k, w, sparse_count=K, sparse_mode=3)
    for b in range(B):
        ref = brute_scores(q[b], k[b, :, 0], w[b], S1, S2, 3)
        for t in range(S1):
            row = ref[t].tolist()
            order = sorted(range(S2), key=lambda i: (-row[i], i))[:K]
            exp = [i if row[i] > -1e30 else -1 for i in order]
            assert idx[b, t, 0].tolist() == exp


def test_second_formulation_index_golden_agrees():
    g = torch.Generator().manual_seed(3)
    B, S1, S2, G, D, K = 2, 6, 64, 8, 16, 10
    q5 = torch.randn((B, S1, 1, G, D), generator=g)
    k = torch.randn((B, S2, 1, D), generator=g)
    w5 = torch.randn((B, S1, 1, G, 1), generator=g)
    red, top = index_golden(q5, k, w5, K)
    idx, scores, _ = lightning_indexer(q5.view(B, S1, G, D), k, w5.view(B, S1, G), sparse_count=K, sparse_mode=0)
    assert torch.allclose(scores[:, 0], red[:, :, 0], rtol=1e-5, atol=1e-5)
    # random fp32 data has no ties: the index sets (and order) agree
    assert torch.equal(idx[:, :, 0], top[:, :, 0])


def test_invariants_scale_and_sign():
    g = torch.Generator().manual_seed(11)
    q = torch.randn((1, 4, 8, 128), generator=g)
    k = torch.randn((1, 50, 1, 128), generator=g)
    w = torch.randn((1, 4, 8), generator=g)
    _, s1, _ = lightning_indexer(q, k, w, sparse_count=8, sparse_mode=0)
    # positive per-key scale factors out of the ReLU
    c = torch.rand((1, 50), generator=g) + 0.1
    _, s2, _ = lightning_indexer(q, k, w, key_scale=c, sparse_count=8, sparse_mode=0)
    assert torch.allclose(s2[0, 0], s1[0, 0] * c[0].unsqueeze(0), rtol=1e-5, atol=1e-4)
    # all q.k <= 0 -> all logits are exactly 0
    _, s3, _ = lightning_indexer(q.abs(), -k.abs(), w, sparse_count=8, sparse_mode=0)
    assert torch.count_nonzero(s3) == 0


def test_fp8_dequant_identity():
    g = torch.Generator().manual_seed(13)
    k32 = torch.randn((1, 30, 1, 128), generator=g)
    scale = k32.abs().amax(-1) / 448
    k8 = (k32 / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    q = torch.randn((1, 3, 64, 128), generator=g).to(torch.float8_e4m3fn)
    w = torch.randn((1, 3, 64), generator=g) / 8
    _, s_fp8, _ = lightning_indexer(q, k8, w, key_scale=scale.view(1, 30), sparse_count=4, sparse_mode=0)
    kdq = k8.float() * scale.unsqueeze(-1)
    _, s_deq, _ = lightning_indexer(q.float(), kdq, w, sparse_count=4, sparse_mode=0)
    assert torch.allclose(s_fp8, s_deq, rtol=1e-5, atol=1e-4)
