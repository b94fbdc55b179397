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


def _varlen_case(seed, lens_q, lens_k, N1=4, D=128):
    """Ragged batches: per-batch queries / keys, as a list of tensors."""
    g = torch.Generator().manual_seed(seed)
    qs = [torch.randn((aq, N1, D), generator=g) for aq in lens_q]
    ks = [torch.randn((ak, 1, D), generator=g) for ak in lens_k]
    ws = [torch.randn((aq, N1), generator=g) for aq in lens_q]
    return qs, ks, ws


def _cumsum(lens):
    out, acc = [], 0
    for x in lens:
        acc += x
        out.append(acc)
    return torch.tensor(out, dtype=torch.int32)


@pytest.mark.parametrize("mode", [3, 0])
def test_tnd_layout_vs_bruteforce(mode):
    # TND query and key (lightning_indexer.py:48-84,111-150: prefix-sum lengths,
    # output [T, N2, K]); every row checked against the triple loop of its batch
    lens_q, lens_k, K = [3, 0, 5], [20, 7, 33], 12
    qs, ks, ws = _varlen_case(21 + mode, lens_q, lens_k)
    q, k, w = torch.cat(qs), torch.cat(ks), torch.cat(ws)
    idx, _, vals = lightning_indexer(q, k, w, actual_seq_lengths_query=_cumsum(lens_q),
                                     actual_seq_lengths_key=_cumsum(lens_k), layout_query="TND",
                                     layout_key="TND", sparse_count=K, sparse_mode=mode)
    assert idx.shape == (sum(lens_q), 1, K)
    row = 0
    for b, (aq, ak) in enumerate(zip(lens_q, lens_k)):
        if aq == 0:
            continue
        ref = brute_scores(qs[b], ks[b][:, 0], ws[b], aq, ak, mode)
        for t in range(aq):
            r = ref[t].tolist()
            order = sorted(range(ak), key=lambda i: (-r[i], i))[:K]
            exp = [i if r[i] > -1e30 else -1 for i in order] + [-1] * (K - min(K, ak))
            assert idx[row, 0].tolist() == exp, (b, t)
            row += 1


def test_tnd_equals_padded_bsnd():
    # the padded form of the same ragged batches (BSND with per-batch lengths)
    lens_q, lens_k, K = [4, 2], [30, 18], 8
    qs, ks, ws = _varlen_case(5, lens_q, lens_k)
    B, S1, S2 = 2, max(lens_q), max(lens_k)
    qp = torch.zeros((B, S1, 4, 128))
    kp = torch.zeros((B, S2, 1, 128))
    wp = torch.zeros((B, S1, 4))
    for b in range(B):
        qp[b, :lens_q[b]] = qs[b]
        kp[b, :lens_k[b]] = ks[b]
        wp[b, :lens_q[b]] = ws[b]
    ip, sp, _ = lightning_indexer(qp, kp, wp, actual_seq_lengths_query=torch.tensor(lens_q),
                                  actual_seq_lengths_key=torch.tensor(lens_k), sparse_count=K)
    it, st, _ = lightning_indexer(torch.cat(qs), torch.cat(ks), torch.cat(ws),
                                  actual_seq_lengths_query=_cumsum(lens_q),
                                  actual_seq_lengths_key=_cumsum(lens_k), layout_query="TND",
                                  layout_key="TND", sparse_count=K)
    row = 0
    for b in range(B):
        for t in range(lens_q[b]):
            assert torch.equal(it[row, 0], ip[b, t, 0])
            row += 1
    assert torch.equal(torch.nan_to_num(st, neginf=-1.0), torch.nan_to_num(sp, neginf=-1.0))


@pytest.mark.parametrize("block_size", [16, 64])
def test_paged_keys_equal_contiguous(block_size):
    # PA_BSND (lightning_indexer.py:271-292 golden gather bt[b, s // bs], s % bs):
    # the keys scattered over a shuffled page pool give the contiguous result
    g = torch.Generator().manual_seed(block_size)
    B, S1, S2, K = 2, 5, 100, 16
    q = torch.randn((B, S1, 4, 128), generator=g)
    k = torch.randn((B, S2, 1, 128), generator=g)
    w = torch.randn((B, S1, 4), generator=g)
    lens_k = [100, 77]
    nb = (S2 + block_size - 1) // block_size
    perm = torch.randperm(B * nb + 3, generator=g)
    pool = torch.randn((B * nb + 3, block_size, 1, 128), generator=g)
    bt = torch.full((B, nb + 2), -1, dtype=torch.int32)
    for b in range(B):
        for j in range(nb):
            page = int(perm[b * nb + j])
            bt[b, j] = page
            lo, hi = j * block_size, min(S2, (j + 1) * block_size)
            pool[page, :hi - lo] = k[b, lo:hi]
    ic, sc, _ = lightning_indexer(q, k, w, actual_seq_lengths_key=torch.tensor(lens_k), sparse_count=K)
    ipa, spa, _ = lightning_indexer(q, pool, w, actual_seq_lengths_key=torch.tensor(lens_k), block_table=bt,
                                    layout_key="PA_BSND", sparse_count=K)
    assert torch.equal(ipa, ic)
    assert torch.equal(torch.nan_to_num(spa, neginf=-1.0), torch.nan_to_num(sc, neginf=-1.0))


def test_block_sparse_logits_equal_indexer_scores_on_gathered_blocks():
    # HISA logits (examples/HISA/paged_block_sparse_mqa_attn_expert.py:425-468) against
    # the lightning-indexer score restatement run on the same keys gathered contiguously
    from oracle.dsa_oracle import block_sparse_indexer_logits
    g = torch.Generator().manual_seed(12)
    B, S, H, D, bs, topk, nb = 2, 3, 8, 16, 4, 5, 12
    q = torch.randn((B, S, H, D), generator=g)
    kv = torch.randn((nb, bs, 1, D), generator=g)
    w = torch.rand((B, S, H), generator=g)
    bt = torch.stack([torch.randperm(nb, generator=g)[:6] for _ in range(B)]).int()
    ctx = torch.tensor([21, 9], dtype=torch.int32)
    idx = torch.randint(0, 6, (B, S, topk), generator=g, dtype=torch.int32)
    got = block_sparse_indexer_logits(q, kv, idx, w, ctx, bt).view(B, S, topk, bs)
    for b in range(B):
        for s in range(S):
            for i in range(topk):
                lb = int(idx[b, s, i])
                keys = kv[int(bt[b, lb]), :, 0, :]
                ref = indexer_scores(q[b, s].unsqueeze(0), keys, w[b, s].unsqueeze(0), 1, bs, 0)[0]
                pos = lb * bs + torch.arange(bs)
                ref = torch.where(pos < int(ctx[b]), ref, torch.tensor(float("-inf")))
                torch.testing.assert_close(got[b, s, i], ref, rtol=1e-5, atol=1e-5)
