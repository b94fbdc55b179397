"""The whole-output GPU checkers (tests/fullsize.py), exercised on the CPU: they
accept the oracle's own answers and reject answers with a planted mistake."""
import pytest
import torch

from fullsize import check_mla_tokens, check_topk_rows
from oracle.dsa_oracle import sparse_mla_fwd_gather, stable_topk


def test_topk_checker_accepts_oracle_and_rejects_swaps():
    g = torch.Generator().manual_seed(7)
    x = torch.randn((6, 300), generator=g)
    x[1, 10:20] = 0.5          # ties broken by lower index
    x[2, 5] = -0.0             # -0.0 ties +0.0
    x[2, 6] = 0.0
    x[3, 200:] = float("-inf")  # fewer valid entries than K -> -1 padding
    lens = torch.tensor([300, 300, 300, 300, 37, 300])
    ref, _ = stable_topk(x, 64, row_len=lens)
    check_topk_rows(ref, x, lens, 64, chunk=4)
    bad = ref.clone()
    bad[1, [3, 4]] = bad[1, [4, 3]]  # two tied entries out of index order
    with pytest.raises(AssertionError):
        check_topk_rows(bad, x, lens, 64, chunk=4)
    bad = ref.clone()
    bad[4, 40] = 5                   # a -1 pad replaced
    with pytest.raises(AssertionError):
        check_topk_rows(bad, x, lens, 64, chunk=4)


def test_mla_checker_accepts_oracle_and_rejects_a_moved_token():
    g = torch.Generator().manual_seed(8)
    T, H, Skv, topk, D = 9, 8, 256, 64, 576
    q = (torch.randn((1, T, H, D), generator=g) * 0.5).to(torch.bfloat16)
    kv = (torch.randn((1, Skv, 1, D), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(Skv, generator=g)[:topk] for _ in range(T)]).int()
    idx[3, 10:] = -1
    q_start = Skv - T
    out, lse = sparse_mla_fwd_gather(q, kv, idx.view(1, T, 1, topk), D ** -0.5, q_start_index_s=q_start,
                                     is_causal=True, p_dtype=torch.bfloat16)
    kv0 = kv[0, :, 0]
    limit = q_start + torch.arange(T)
    check_mla_tokens(out[0].to(torch.bfloat16), lse[0], q[0], lambda t0, t1, ii: kv0[ii], idx, limit, Skv,
                     D ** -0.5, heads=range(H), chunk=4)
    moved = out[0].clone()
    moved[[2, 5]] = moved[[5, 2]]   # two tokens' outputs swapped
    with pytest.raises(AssertionError):
        check_mla_tokens(moved.to(torch.bfloat16), lse[0], q[0], lambda t0, t1, ii: kv0[ii], idx, limit, Skv,
                         D ** -0.5, heads=range(H), chunk=4)
