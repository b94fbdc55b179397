"""Pins the sparse-MLA oracle: per-(token, head) brute force, agreement of the gather
(examples/deepseek_v4/sparse_attention.py:171-198) and dense
(examples/sparse_flash_attention/example_sparse_flash_attn.py:255-292) restatements,
closed forms and invariants."""
import math

import pytest
import torch

from oracle.dsa_oracle import lse_combine, pa_to_contiguous, sparse_mla_fwd_dense, sparse_mla_fwd_gather


def brute_row(qrow, kv_rows, scale, d_v):
    """One (token, head): python loops over the valid rows."""
    scores = [scale * sum(float(a) * float(b) for a, b in zip(qrow, r)) for r in kv_rows]
    if not scores:
        return [0.0] * d_v, -math.inf
    m = max(scores)
    ex = [math.exp(s - m) for s in scores]
    den = sum(ex)
    out = [sum(e * float(r[d]) for e, r in zip(ex, kv_rows)) / den for d in range(d_v)]
    return out, m + math.log(den)


def _inputs(seed, B=1, S=4, Skv=40, H=3, D=24, topk=8):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, S, H, D), generator=g)
    kv = torch.randn((B, Skv, 1, D), generator=g)
    idx = torch.stack([torch.randperm(Skv, generator=g)[:topk] for _ in range(B * S)]).view(B, S, 1, topk).int()
    return q, kv, idx


def test_gather_vs_bruteforce_with_padding():
    q, kv, idx = _inputs(1)
    idx[0, 1, 0, 5:] = -1
    idx[0, 2, 0, 2] = 40  # out-of-range sentinel (example_sparse_flash_attn.py:303)
    out, lse = sparse_mla_fwd_gather(q, kv, idx, 0.3, d_v=16, is_causal=False)
    for s in range(4):
        rows = [kv[0, i, 0].tolist() for i in idx[0, s, 0].tolist() if 0 <= i < 40]
        for h in range(3):
            o, l = brute_row(q[0, s, h].tolist(), rows, 0.3, 16)
            assert torch.allclose(out[0, s, h], torch.tensor(o), rtol=1e-5, atol=1e-5)
            assert abs(float(lse[0, s, h]) - l) < 1e-4


def test_gather_equals_dense_form():
    q, kv, idx = _inputs(2, B=2, S=6, Skv=64, H=4, D=576, topk=16)
    # causal: indices within [0, q_start + s]; q_start = Skv - S
    S, Skv = 6, 64
    for b in range(2):
        for s in range(S):
            lim = Skv - S + s
            idx[b, s, 0] = torch.randperm(lim + 1)[:16].int()
    o1, l1 = sparse_mla_fwd_gather(q, kv, idx, None, is_causal=True)
    o2, l2 = sparse_mla_fwd_dense(q, kv, idx)
    assert torch.allclose(o1, o2, rtol=1e-4, atol=1e-5)
    assert torch.allclose(l1, l2, rtol=1e-5, atol=1e-5)


def test_single_valid_index_closed_form():
    q, kv, idx = _inputs(3)
    idx[:] = -1
    idx[0, 0, 0, 3] = 17
    out, lse = sparse_mla_fwd_gather(q, kv, idx, 0.5, d_v=16, is_causal=False)
    assert torch.allclose(out[0, 0], kv[0, 17, 0, :16].expand(3, 16))
    exp_lse = 0.5 * (q[0, 0] @ kv[0, 17, 0])
    assert torch.allclose(lse[0, 0], exp_lse, rtol=1e-5)
    # rows with no valid index: out 0, lse -inf
    assert torch.count_nonzero(out[0, 1:]) == 0
    assert torch.isinf(lse[0, 1:]).all() and (lse[0, 1:] < 0).all()


def test_permutation_invariance_and_logsumexp():
    q, kv, idx = _inputs(4, D=576, topk=32, Skv=100)
    perm = torch.randperm(32)
    o1, l1 = sparse_mla_fwd_gather(q, kv, idx, None, is_causal=False)
    o2, l2 = sparse_mla_fwd_gather(q, kv, idx[..., perm].contiguous(), None, is_causal=False)
    assert torch.allclose(o1, o2, rtol=1e-5, atol=1e-6) and torch.allclose(l1, l2)
    sc = torch.einsum("shd,skd->shk", q[0], kv[0, idx[0, :, 0].long(), 0]) * 576 ** -0.5
    assert torch.allclose(l1[0], torch.logsumexp(sc, dim=-1), rtol=1e-5, atol=1e-5)


def test_causal_mask_drops_future_indices():
    q, kv, idx = _inputs(5, S=2, Skv=10, topk=4)
    idx[0, 0, 0] = torch.tensor([0, 8, 9, 1])  # q_start = 8: row 0 may see <= 8
    o1, _ = sparse_mla_fwd_gather(q, kv, idx, 0.2, d_v=8, is_causal=True)
    idx2 = idx.clone()
    idx2[0, 0, 0, 2] = -1
    o2, _ = sparse_mla_fwd_gather(q, kv, idx2, 0.2, d_v=8, is_causal=False)
    assert torch.allclose(o1[0, 0], o2[0, 0])


def test_paged_equals_contiguous():
    g = torch.Generator().manual_seed(6)
    B, ctx, bs, D = 2, 96, 16, 32
    nb = ctx // bs
    pool = torch.randn((B * nb + 3, bs, 1, D), generator=g)
    bt = torch.randperm(B * nb + 3, generator=g)[: B * nb].view(B, nb).int()
    q = torch.randn((B, 1, 4, D), generator=g)
    idx = torch.stack([torch.randperm(ctx, generator=g)[:20] for _ in range(B)]).view(B, 1, 1, 20).int()
    o1, l1 = sparse_mla_fwd_gather(q, pool, idx, 0.1, d_v=16, block_table=bt, is_causal=False)
    kvc = torch.stack([pa_to_contiguous(pool, bt[b], ctx) for b in range(B)])
    o2, l2 = sparse_mla_fwd_gather(q, kvc, idx, 0.1, d_v=16, is_causal=False)
    assert torch.allclose(o1, o2) and torch.allclose(l1, l2)


def test_sink_reduces_to_plain_at_minus_inf_and_matches_formula():
    q, kv, idx = _inputs(7)
    o0, l0 = sparse_mla_fwd_gather(q, kv, idx, 0.3, d_v=16, is_causal=False)
    o1, l1 = sparse_mla_fwd_gather(q, kv, idx, 0.3, d_v=16, is_causal=False,
                                   attn_sink=torch.full((3,), -float("inf")))
    assert torch.allclose(o0, o1) and torch.allclose(l0, l1)
    sink = torch.tensor([0.5, -1.0, 2.0])
    o2, l2 = sparse_mla_fwd_gather(q, kv, idx, 0.3, d_v=16, is_causal=False, attn_sink=sink)
    # sparse_attention.py:180-187: denominator gains exp(sink); lse = logaddexp(lse, sink)
    assert torch.allclose(l2, torch.logaddexp(l0, sink.view(1, 1, 3)), rtol=1e-5, atol=1e-5)
    assert torch.allclose(o2, o0 * torch.exp(l0 - l2).unsqueeze(-1), rtol=1e-5, atol=1e-6)


def test_lse_combine_of_split_index_sets():
    q, kv, idx = _inputs(8, D=64, topk=16, Skv=64)
    o, l = sparse_mla_fwd_gather(q, kv, idx, 0.2, d_v=16, is_causal=False)
    oa, la = sparse_mla_fwd_gather(q, kv, idx[..., :7].contiguous(), 0.2, d_v=16, is_causal=False)
    ob, lb = sparse_mla_fwd_gather(q, kv, idx[..., 7:].contiguous(), 0.2, d_v=16, is_causal=False)
    oc, lc = lse_combine([oa, ob], [la, lb])
    assert torch.allclose(oc, o, rtol=1e-5, atol=1e-6) and torch.allclose(lc, l, rtol=1e-6)


def test_bf16_probability_rounding_stays_close():
    q, kv, idx = _inputs(9, D=576, topk=64, Skv=128)
    o1, _ = sparse_mla_fwd_gather(q, kv, idx, None, is_causal=False)
    o2, _ = sparse_mla_fwd_gather(q, kv, idx, None, is_causal=False, p_dtype=torch.bfloat16)
    assert torch.allclose(o1, o2, rtol=2e-2, atol=2e-2)


# ---------------------------------------------------------------- DeepSeek-V4 sparse flash MLA
from oracle.dsa_oracle import sparse_flash_mla_v4, unpack_pages, v4_compressed_positions  # noqa: E402


def test_v4_compressed_positions_hand_worked():
    idx = torch.tensor([[[5, 0, 9, 2, -1, 1]]], dtype=torch.int32).view(1, 1, 1, 6)
    # act_kv 40, act_q 1, s 0: t = (40 - 1 + 0 + 1) // 4 = 10; the first min(6, 10) entries up to the -1
    assert v4_compressed_positions(idx.view(1, 1, 6), 0, 0, 40, 1, 4) == [5, 0, 9, 2]
    # t = (12 - 1 + 0 + 1) // 4 = 3: only the first min(K, t) = 3 entries are read
    # (5, 0, 9), and of those only 0 lies below t
    assert v4_compressed_positions(idx.view(1, 1, 6), 0, 0, 12, 1, 4) == [0]
    # t = 5 reads 5, 0, 9, 2, -1: 0 and 2 (5 is not < 5)
    assert v4_compressed_positions(idx.view(1, 1, 6), 0, 0, 20, 1, 4) == [0, 2]
    # the -1 ends the list even when later entries would be in range
    assert v4_compressed_positions(idx.view(1, 1, 6), 0, 0, 400, 1, 4) == [5, 0, 9, 2]
    # dense (no list): all positions below t
    assert v4_compressed_positions(None, 0, 0, 12, 1, 4) == [0, 1, 2]
    assert v4_compressed_positions(None, 0, 0, 2, 4, 4) == []


def _v4_small(seed, scenario):
    g = torch.Generator().manual_seed(seed)
    B, N1, D, win = 2, 4, 32, 6
    act_q, act_kv = [5, 3], [17, 9]
    S = max(act_q)
    q = torch.randn((B, N1, S, D), generator=g).to(torch.bfloat16)
    ori = torch.randn((B, 1, max(act_kv), D), generator=g).to(torch.bfloat16)
    cmp = torch.randn((B, 1, max(act_kv) // 2, D), generator=g).to(torch.bfloat16) if scenario >= 2 else None
    lists = None
    if scenario == 3:
        lists = torch.randint(0, 8, (B, S, 1, 5), generator=g, dtype=torch.int32)
        lists[0, 1, 0, 3] = -1
    sinks = torch.randn(N1, generator=g)
    return dict(q=q, ori=ori, cmp=cmp, lists=lists, sinks=sinks, act_q=act_q, act_kv=act_kv, win=win, ratio=2,
                scale=D ** -0.5)


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_v4_agrees_with_gather_formulation(scenario):
    c = _v4_small(30 + scenario, scenario)
    out, lse = sparse_flash_mla_v4(c["q"], c["ori"], c["sinks"], act_q_lens=c["act_q"], act_kv_lens=c["act_kv"],
                                   softmax_scale=c["scale"], cmp_k_bnsd=c["cmp"], cmp_sparse_indices=c["lists"],
                                   cmp_ratio=c["ratio"], ori_win_left=c["win"] - 1)
    B, N1, S, D = c["q"].shape
    n_ori = c["ori"].shape[2]
    for b in range(B):
        keys = c["ori"][b, 0] if c["cmp"] is None else torch.cat([c["ori"][b, 0], c["cmp"][b, 0]])
        for s in range(c["act_q"][b]):
            sg = c["act_kv"][b] - c["act_q"][b] + s
            sel = list(range(max(sg - c["win"] + 1, 0), sg + 1))
            if c["cmp"] is not None:
                sel += [n_ori + p for p in v4_compressed_positions(c["lists"], b, s, c["act_kv"][b], c["act_q"][b],
                                                                   c["ratio"])]
            idx = torch.full((1, 1, 1, 32), -1, dtype=torch.int32)
            idx[0, 0, 0, :len(sel)] = torch.tensor(sel, dtype=torch.int32)
            ro, rl = sparse_mla_fwd_gather(c["q"][b, :, s].unsqueeze(0).unsqueeze(0), keys.view(1, -1, 1, D), idx,
                                           c["scale"], d_v=D, attn_sink=c["sinks"], p_dtype=torch.bfloat16)
            torch.testing.assert_close(out[b, :, s].float(), ro[0, 0], rtol=2e-2, atol=2e-2)
            torch.testing.assert_close(lse[b, :, s], rl[0, 0], rtol=1e-5, atol=1e-5)


def test_v4_closed_forms():
    # a row before any key (act_kv < act_q): out 0 and lse = sink; a row seeing one
    # key k with score x: out = k e^x / (e^x + e^sink), lse = ln(e^x + e^sink)
    g = torch.Generator().manual_seed(3)
    N1, D = 2, 16
    q = torch.randn((1, N1, 3, D), generator=g).to(torch.bfloat16)
    ori = torch.randn((1, 1, 1, D), generator=g).to(torch.bfloat16)
    sinks = torch.tensor([0.3, -2.0])
    out, lse = sparse_flash_mla_v4(q, ori, sinks, act_q_lens=[3], act_kv_lens=[1], softmax_scale=0.5,
                                   ori_win_left=0)
    # rows 0, 1 sit before the cache (positions -2, -1); row 2 sees key 0 only
    assert torch.equal(out[0, :, :2].float(), torch.zeros(N1, 2, D))
    torch.testing.assert_close(lse[0, :, 0], sinks)
    x = (q[0, :, 2].float() @ ori[0, 0, 0].float()) * 0.5
    w = torch.exp(x) / (torch.exp(x) + torch.exp(sinks))
    torch.testing.assert_close(out[0, :, 2].float(), (w.unsqueeze(1) * ori[0, 0, 0].float()), rtol=1e-2, atol=1e-2)
    torch.testing.assert_close(lse[0, :, 2], torch.logaddexp(x, sinks), rtol=1e-5, atol=1e-5)


def test_unpack_pages_roundtrip():
    g = torch.Generator().manual_seed(4)
    pool = torch.randn((5, 4, 1, 3), generator=g)
    bt = torch.tensor([[3, 0, -1], [1, 4, 2]], dtype=torch.int32)
    u = unpack_pages(pool, bt, 10)
    assert torch.equal(u[0, 0, 0:4], pool[3, :, 0]) and torch.equal(u[0, 0, 4:8], pool[0, :, 0])
    assert torch.equal(u[0, 0, 8:10], torch.zeros(2, 3))
    assert torch.equal(u[1, 0, 8:10], pool[2, :2, 0])
