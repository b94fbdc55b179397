"""Whole-output checks at the benchmark configurations' full sizes, in plain torch on
the GPU (test infrastructure, not the product path).

The sampled oracle checks in the GPU tests pin the arithmetic; these pin the
mapping of rows and tokens to workgroups, over every row and every token:

* top-k: every row's indices against ``torch.sort(descending=True, stable=True)``
  of the kernel's own logits (the golden's ``argsort(-score, stable=True)``,
  examples/deepseek_v4/lightning_indexer.py:316-325), entries <= -1e30 -> -1;
* sparse MLA: every token's ``lse`` and ``out`` on a fixed set of heads that
  covers the first and last head of every 32-head wave, recomputed in fp32 from
  the gathered rows (P rounded to the input dtype before P.V, as the golden does,
  sparse_flash_mla_golden.py:143), ``out`` at atol = rtol = 2e-2 and ``lse`` at 1e-3.
"""
from __future__ import annotations

from typing import Callable, Optional, Sequence

import torch

HEADS_PROBE = (0, 31, 32, 63, 64, 95, 96, 127)
OUT_TOL = dict(rtol=2e-2, atol=2e-2)
LSE_TOL = dict(rtol=1e-3, atol=1e-3)


def check_topk_rows(idx: torch.Tensor, logits: torch.Tensor, row_len: Optional[torch.Tensor], K: int,
                    chunk: int = 128, what: str = "top-k") -> None:
    """``idx [R, K]`` int32 against the stable descending sort of ``logits [R, N]``
    restricted to each row's first ``row_len[r]`` columns (all N when None)."""
    R, N = logits.shape
    assert idx.shape == (R, K), f"{what}: indices {tuple(idx.shape)} for {R} rows of {K}"
    cols = torch.arange(N, device=logits.device)
    for r0 in range(0, R, chunk):
        r1 = min(R, r0 + chunk)
        x = logits[r0:r1] + 0.0  # -0.0 -> +0.0: the two tie, as in the golden's comparison
        if row_len is not None:
            x = torch.where(cols.unsqueeze(0) < row_len[r0:r1].view(-1, 1), x, float("-inf"))
        v, i = torch.sort(x, dim=1, descending=True, stable=True)
        kk = min(K, N)
        ref = torch.full((r1 - r0, K), -1, dtype=torch.int32, device=idx.device)
        ref[:, :kk] = torch.where(v[:, :kk] > -1e30, i[:, :kk], -1).to(torch.int32)
        if not torch.equal(idx[r0:r1], ref):
            bad = (idx[r0:r1] != ref).any(dim=1).nonzero().flatten()
            raise AssertionError(f"{what}: {bad.numel()} of rows {r0}..{r1 - 1} differ (first: row {r0 + int(bad[0])})")


def check_mla_tokens(out: torch.Tensor, lse: torch.Tensor, q: torch.Tensor, gather: Callable,
                     indices: torch.Tensor, limit: Optional[torch.Tensor], skv: int, sm_scale: float,
                     heads: Sequence[int] = HEADS_PROBE, chunk: int = 64, what: str = "sparse MLA") -> None:
    """Every token of ``out [T, H, 512]`` / ``lse [T, H]`` on ``heads``.

    ``q [T, H, Dqk]``; ``indices [T, topk]``; ``gather(tok0, tok1, safe_idx)``
    returns the KV rows ``[t, topk, Dqk]`` of tokens tok0..tok1-1 for the clamped
    indices; an index is valid when ``0 <= idx < skv`` and (``limit [T]`` given)
    ``idx <= limit[t]``."""
    T = q.shape[0]
    hs = torch.tensor(list(heads), device=q.device)
    for t0 in range(0, T, chunk):
        t1 = min(T, t0 + chunk)
        ii = indices[t0:t1].long()
        valid = (ii >= 0) & (ii < skv)
        if limit is not None:
            valid &= ii <= limit[t0:t1].view(-1, 1)
        safe = torch.where(valid, ii, torch.zeros_like(ii))
        rows = gather(t0, t1, safe).float() * valid.unsqueeze(-1)           # [t, topk, Dqk]
        qq = q[t0:t1].index_select(1, hs).float()                         # [t, h, Dqk]
        s = torch.bmm(qq, rows.transpose(1, 2).contiguous()) * sm_scale    # [t, h, topk]
        s = s.masked_fill(~valid.unsqueeze(1), float("-inf"))
        m = s.amax(dim=-1, keepdim=True)
        m = torch.where(torch.isfinite(m), m, torch.zeros_like(m))
        p = torch.exp(s - m)
        den = p.sum(dim=-1)
        ref_lse = torch.where(den > 0, m.squeeze(-1) + torch.log(den.clamp_min(1e-38)),
                              torch.full_like(den, float("-inf")))
        pv = p.to(q.dtype).float()
        ref_out = torch.bmm(pv, rows[..., :512].contiguous()) / den.clamp_min(1e-38).unsqueeze(-1)
        ref_out = torch.where((den > 0).unsqueeze(-1), ref_out, torch.zeros_like(ref_out))
        got_o = out[t0:t1].index_select(1, hs).float()
        got_l = lse[t0:t1].index_select(1, hs)
        try:
            torch.testing.assert_close(got_l, ref_lse, **LSE_TOL)
            torch.testing.assert_close(got_o, ref_out, **OUT_TOL)
        except AssertionError as e:
            raise AssertionError(f"{what}: tokens {t0}..{t1 - 1}: {e}") from None
