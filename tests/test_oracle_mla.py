"""Pins the sparse-MLA oracle: per-(token, head) brute force, agreement of the gather
(examples/deepseek_v4/sparse_attention.py:171-198) and dense
(examples/sparse_flash_attention/example_sparse_flash_attn.py:255-292) restatements,
closed forms and invariants."""
import math

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
