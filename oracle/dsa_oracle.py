"""CPU oracle for the DeepSeek Sparse Attention path (indexer -> top-k -> sparse MLA).

TEST INFRASTRUCTURE ONLY.  This module restates, in plain PyTorch on the CPU, the
torch/numpy goldens that tilelang-ascend ships with its examples.  Only the test
suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or as the timed CPU baseline).  The product
path (``dsa.api``) never imports or calls anything here, and fails loudly when
its HIP library is missing.

Every function cites the reference file:line it follows (paths relative to the
tilelang-ascend checkout).  How each function is pinned (independent brute-force
loops on tiny shapes, the reference's known-answer tests, closed forms and
invariants) is listed in the ``PINNED_BY`` table at the bottom; the tests in
``tests/test_oracle_*.py`` execute those checks.  No function here is unpinned.

Conventions shared with the HIP kernels:

* fp32 scores; natural-log LSE ``lse = m + log(sum(exp(s - m)))``
  (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_golden.py:147-149).
* top-k order is ``argsort(-score, stable=True)``: descending value, ties to the
  lower index; selected entries with value <= -1e30 become index -1
  (examples/deepseek_v4/lightning_indexer.py:316-325).
* sparse-MLA indices: -1 and any index outside [0, Skv) select nothing
  (examples/deepseek_v4/sparse_attention.py:171-177,195 handles -1;
  examples/sparse_flash_attention/example_sparse_flash_attn.py:303 pads with the
  out-of-range sentinel Skv).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import torch

NEG_INF = float("-inf")
INVALID_SCORE = -1e30  # lightning_indexer.py:321  (topv <= -1e30 -> index -1)


# ---------------------------------------------------------------------------
# top-k
# ---------------------------------------------------------------------------
def stable_topk(scores: torch.Tensor, k: int, *, pad_invalid: bool = True,
                row_len: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """Row-wise top-k of fp32 ``scores [R, N]`` in stable descending order.

    Follows examples/deepseek_v4/lightning_indexer.py:316-325:
    ``sorted_order = argsort(-score, stable=True)``; take ``kk = min(K, N)``;
    entries whose value is <= -1e30 become index -1; columns past ``kk`` stay -1
    (the golden pre-fills indices with -1, :259-263).

    ``row_len`` (optional, int [R]) restricts row r to its first ``row_len[r]``
    columns, as the golden restricts each batch row to ``[:ak]`` (:297-314).
    ``pad_invalid=False`` keeps the raw indices (torch.topk-style, the
    topk_selector example's ``ref_program``, example_topk_selector.py:57-58).
    Returns ``(indices int32 [R, k], values fp32 [R, k])``; unfilled values are -inf.
    """
    scores = scores.to(torch.float32)
    R, N = scores.shape
    idx_out = torch.full((R, k), -1, dtype=torch.int32)
    val_out = torch.full((R, k), NEG_INF, dtype=torch.float32)
    if row_len is None:
        lens = [N] * R
    else:
        lens = [int(x) for x in row_len.tolist()]
    # group rows with the same length so torch does the sorting in bulk
    by_len = {}
    for r, L in enumerate(lens):
        by_len.setdefault(min(L, N), []).append(r)
    for L, rows in by_len.items():
        if L <= 0:
            continue
        rows_t = torch.tensor(rows, dtype=torch.long)
        s = scores[rows_t, :L]
        order = torch.argsort(-s, dim=1, stable=True)
        kk = min(k, L)
        topi = order[:, :kk]
        topv = s.gather(1, topi)
        topi = topi.to(torch.int32)
        if pad_invalid:
            topi = torch.where(topv <= INVALID_SCORE, torch.full_like(topi, -1), topi)
        idx_out[rows_t, :kk] = topi
        val_out[rows_t, :kk] = topv
    return idx_out, val_out


# ---------------------------------------------------------------------------
# lightning indexer
# ---------------------------------------------------------------------------
def dequant_fp8(x: torch.Tensor, scale: Optional[torch.Tensor]) -> torch.Tensor:
    """fp8-e4m3 (or any float) -> fp32, times an optional per-token scale over the
    last dim.  Because every scale is > 0, ``scale*ReLU(x) == ReLU(scale*x)``, so
    the fp8 indexer with per-key scale equals the reference golden run on the
    dequantised key (lightning_indexer.py:304-305)."""
    xf = x.to(torch.float32)
    if scale is not None:
        sc = scale.to(torch.float32)
        if sc.numel() != xf[..., 0].numel():
            raise ValueError(f"scale has {sc.numel()} entries, key has {xf[..., 0].numel()} tokens")
        xf = xf * sc.reshape(xf.shape[:-1]).unsqueeze(-1)
    return xf


def _prefix(lens: Sequence[int]) -> list:
    out = [0]
    for x in lens:
        out.append(out[-1] + int(x))
    return out


def indexer_scores(q: torch.Tensor, k: torch.Tensor, w: torch.Tensor, aq: int, ak: int,
                   sparse_mode: int, row_chunk: int = 64) -> torch.Tensor:
    """Masked logits for one (batch, kv-head) group.

    q ``[aq, G, D]`` fp32, k ``[ak, D]`` fp32, w ``[aq, G]`` fp32 -> ``[aq, ak]`` fp32.
    ``score = sum_g relu(q @ k^T) * w`` (lightning_indexer.py:303-305); causal mask
    for sparse_mode 3 with the golden's rule that a row whose causal length is <= 0
    sees every key (:307-314).  Computed ``row_chunk`` query rows at a time: the
    golden's ``[aq, G, ak]`` intermediate would not fit in memory at 32K-128K keys.
    """
    out = torch.empty((aq, ak), dtype=torch.float32)
    kt = k.t().contiguous()
    for r0 in range(0, aq, row_chunk):
        r1 = min(aq, r0 + row_chunk)
        qk = torch.relu(torch.matmul(q[r0:r1], kt))           # [r, G, ak]
        out[r0:r1] = torch.matmul(w[r0:r1].unsqueeze(1), qk).squeeze(1)
    if sparse_mode == 3:
        s1 = torch.arange(aq)
        cl = ak - aq + s1 + 1
        s2_valid = torch.where(cl > 0, cl, torch.full_like(cl, ak))
    else:
        s2_valid = torch.full((aq,), ak)
    mask = torch.arange(ak)[None, :] < s2_valid[:, None]
    out.masked_fill_(~mask, NEG_INF)
    return out


def lightning_indexer(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor, *,
                      key_scale: Optional[torch.Tensor] = None,
                      actual_seq_lengths_query: Optional[torch.Tensor] = None,
                      actual_seq_lengths_key: Optional[torch.Tensor] = None,
                      block_table: Optional[torch.Tensor] = None,
                      layout_query: str = "BSND", layout_key: str = "BSND",
                      sparse_count: int = 2048, sparse_mode: int = 3,
                      block_size: Optional[int] = None, return_scores: bool = True,
                      row_chunk: int = 64):
    """Restatement of ``cpu_lightning_indexer`` (examples/deepseek_v4/lightning_indexer.py:199-335).

    Layouts: query BSND ``[B,S1,N1,D]`` or TND ``[T,N1,D]`` (prefix-sum lengths);
    key BSND ``[B,S2,N2,D]``, TND ``[T,N2,D]`` (prefix-sum lengths) or PA_BSND
    ``[blocks, block_size, N2, D]`` with ``block_table [B, max_blocks]`` (:217-292).
    ``key_scale`` (extension for fp8 keys) has the key's shape without D.
    Returns ``(indices int32, full_scores fp32 [B,N2,S1,max_ak] or None, values fp32)``.
    Unlike the golden, ``values`` stay fp32 (fp8 has no useful value dtype).
    """
    is_tnd = layout_query == "TND"
    is_pa = layout_key == "PA_BSND"
    is_tnd_key = layout_key == "TND"
    q = query.detach().cpu()
    k = dequant_fp8(key.detach().cpu(), None if key_scale is None else key_scale.detach().cpu())
    w = weights.detach().cpu().to(torch.float32)
    if is_tnd:
        q_tot, N1, D = q.shape
        asq_raw = [int(x) for x in actual_seq_lengths_query.tolist()]
        B = len(asq_raw)
    else:
        B, S1, N1, D = q.shape
        q_tot = B * S1
        asq_raw = ([S1] * B if actual_seq_lengths_query is None
                   else [int(x) for x in actual_seq_lengths_query.tolist()])
    if is_pa:
        N2 = k.shape[2]
        bs = int(block_size) if block_size else k.shape[1]
        ask_raw = [int(x) for x in actual_seq_lengths_key.tolist()]
    elif is_tnd_key:
        N2 = k.shape[1]
        ask_raw = [int(x) for x in actual_seq_lengths_key.tolist()]
    else:
        N2 = k.shape[2]
        ask_raw = ([k.shape[1]] * B if actual_seq_lengths_key is None
                   else [int(x) for x in actual_seq_lengths_key.tolist()])
    G = N1 // N2
    K = sparse_count
    # TND lengths are prefix sums, BSND/PA lengths are per batch (:271-283)
    q_off = [0] + asq_raw if is_tnd else _prefix(asq_raw)
    k_off = [0] + ask_raw if is_tnd_key else _prefix(ask_raw)
    aqs = [q_off[b + 1] - q_off[b] for b in range(B)]
    aks = [k_off[b + 1] - k_off[b] for b in range(B)]
    S1 = max(aqs) if is_tnd else q.shape[1]
    if is_tnd:
        indices = torch.full((q_tot, N2, K), -1, dtype=torch.int32)
        values = torch.full((q_tot, N2, K), NEG_INF, dtype=torch.float32)
    else:
        indices = torch.full((B, S1, N2, K), -1, dtype=torch.int32)
        values = torch.full((B, S1, N2, K), NEG_INF, dtype=torch.float32)
    max_ak = max(aks) if aks else 0
    full_scores = (torch.full((B, N2, S1, max_ak), NEG_INF, dtype=torch.float32)
                   if return_scores else None)
    qf = q.to(torch.float32)
    for b in range(B):
        aq, ak = aqs[b], aks[b]
        if aq == 0 or ak == 0:
            continue
        qo, ko = q_off[b], k_off[b]
        for n2 in range(N2):
            if is_tnd:
                qb = qf[qo:qo + aq, n2 * G:(n2 + 1) * G, :]
                wb = w[qo:qo + aq, n2 * G:(n2 + 1) * G]
            else:
                qb = qf[b, :aq, n2 * G:(n2 + 1) * G, :]
                wb = w[b, :aq, n2 * G:(n2 + 1) * G]
            if is_pa:
                s2 = torch.arange(ak)
                bids = block_table.detach().cpu()[b, s2 // bs].long()
                kb = k[bids, s2 % bs, n2, :]
            elif is_tnd_key:
                kb = k[ko:ko + ak, n2, :]
            else:
                kb = k[b, :ak, n2, :]
            score = indexer_scores(qb, kb, wb, aq, ak, sparse_mode, row_chunk)
            if full_scores is not None:
                full_scores[b, n2, :aq, :ak] = score
            topi, topv = stable_topk(score, K)
            if is_tnd:
                indices[qo:qo + aq, n2] = topi
                values[qo:qo + aq, n2] = topv
            else:
                indices[b, :aq, n2] = topi
                values[b, :aq, n2] = topv
    return indices, full_scores, values


def index_golden(q: torch.Tensor, k: torch.Tensor, weights: torch.Tensor, top_k: int):
    """Second indexer formulation, restating ``index_golden``
    (examples/lightning_indexer/example_lightning_indexer.py:137-144):
    q ``[B,S1,N2,G,D]``, k ``[B,S2,N2,D]``, weights ``[B,S1,N2,G,1]``; no mask;
    ``torch.topk`` (sorted) over the head-reduced score.  Returns
    ``(reduced scores [B,S1,N2,S2], indices int32 [B,S1,N2,top_k])``."""
    score_1 = torch.einsum("bsmgd,btmd->bmsgt", q.float(), k.float()).relu()
    score = score_1.permute(0, 2, 1, 3, 4)
    reduce_res = torch.sum(score * weights.float(), dim=3)            # [B,S1,N2,S2]
    top = torch.topk(reduce_res, top_k, dim=3, largest=True, sorted=True)
    return reduce_res, top.indices.to(torch.int32)


# ---------------------------------------------------------------------------
# sparse MLA forward
# ---------------------------------------------------------------------------
def _valid_index_mask(idx: torch.Tensor, skv: int, limit: Optional[torch.Tensor]) -> torch.Tensor:
    valid = (idx >= 0) & (idx < skv)
    if limit is not None:
        valid &= idx <= limit
    return valid


def sparse_mla_fwd_gather(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor,
                          sm_scale: Optional[float] = None, *, d_v: int = 512,
                          block_table: Optional[torch.Tensor] = None,
                          q_start_index_s: Optional[int] = None, is_causal: bool = False,
                          attn_sink: Optional[torch.Tensor] = None,
                          p_dtype: Optional[torch.dtype] = None, token_chunk: int = 16):
    """Sparse MLA forward, gather formulation, returning ``(out, lse)``.

    Follows ``gather_sparse_kv`` / ``sparse_softmax_with_sink`` / ``sparse_attn``
    (examples/deepseek_v4/sparse_attention.py:171-198): gather the indexed rows of
    the single latent KV head, ``-1`` rows contribute nothing (score -inf), scores
    ``q.k * scale`` in fp32, softmax, ``P @ V`` with ``V = kv[..., :d_v]``.
    LSE follows sparse_flash_mla_golden.py:147-149 (``lse = m + log(sum)``; with a
    sink the sum starts at 1 with ``m = sink``, :115-117).
    ``p_dtype=torch.bfloat16`` rounds the un-normalised probabilities before the
    PV product as sparse_flash_mla_golden.py:143 does.

    Shapes: q ``[B,S,H,Dqk]``; kv ``[B,Skv,1,Dqk]`` or, with ``block_table``, a page
    pool ``[blocks, block_size, 1, Dqk]`` addressed as
    ``pool[block_table[b, i // bs], i % bs]`` (bench_sfa/sparse_flash_attn_pa_no_cv_pipeline.py:196-200);
    indices ``[B,S,1,topk]`` int32.  Out-of-range indices (>= Skv, e.g. the
    sentinel of example_sparse_flash_attn.py:303) are treated like -1.
    ``is_causal`` additionally drops indices above ``q_start_index_s + s``
    (default ``Skv - S``), the mask of example_sparse_flash_attn.py:261-275 and
    the validity rule of sparse_flash_attn_pa_no_cv_pipeline.py:185.
    A row with no valid index returns out = 0 and lse = -inf (without a sink).
    """
    B, S, H, Dqk = q.shape
    topk = indices.shape[-1]
    idx = indices.reshape(B, S, topk).to(torch.int64)
    if block_table is not None:
        bs = kv.shape[1]
        skv = block_table.shape[1] * bs
    else:
        skv = kv.shape[1]
    if sm_scale is None:
        sm_scale = Dqk ** -0.5
    if q_start_index_s is None:
        q_start_index_s = skv - S
    out = torch.zeros((B, S, H, d_v), dtype=torch.float32)
    lse = torch.full((B, S, H), NEG_INF, dtype=torch.float32)
    for b in range(B):
        for s0 in range(0, S, token_chunk):
            s1 = min(S, s0 + token_chunk)
            ii = idx[b, s0:s1]                                         # [t, topk]
            limit = (torch.arange(s0, s1) + q_start_index_s).unsqueeze(1) if is_causal else None
            valid = _valid_index_mask(ii, skv, limit)
            safe = torch.where(valid, ii, torch.zeros_like(ii))
            if block_table is not None:
                bt = block_table[b].to(torch.int64)
                rows = kv[bt[safe // bs], safe % bs, 0, :]
            else:
                rows = kv[b, safe, 0, :]                               # [t, topk, Dqk]
            rows = rows.to(torch.float32) * valid.unsqueeze(-1)
            qq = q[b, s0:s1].to(torch.float32)                         # [t, H, Dqk]
            sc = torch.matmul(qq, rows.transpose(1, 2)) * sm_scale     # [t, H, topk]
            sc = sc.masked_fill(~valid.unsqueeze(1), NEG_INF)
            m = sc.amax(dim=-1)                                        # [t, H]
            if attn_sink is not None:
                m = torch.maximum(m, attn_sink.to(torch.float32).view(1, H))
            m_safe = torch.where(torch.isinf(m) & (m < 0), torch.zeros_like(m), m)
            p = torch.exp(sc - m_safe.unsqueeze(-1))
            denom = p.sum(dim=-1)
            if attn_sink is not None:
                denom = denom + torch.exp(attn_sink.to(torch.float32).view(1, H) - m_safe)
            if p_dtype is not None:
                p = p.to(p_dtype).to(torch.float32)
            o = torch.matmul(p, rows[..., :d_v])                       # [t, H, d_v]
            has = denom > 0
            out[b, s0:s1] = torch.where(has.unsqueeze(-1), o / denom.clamp_min(1e-38).unsqueeze(-1),
                                        torch.zeros_like(o))
            lse[b, s0:s1] = torch.where(has, m_safe + torch.log(denom.clamp_min(1e-38)),
                                        torch.full_like(denom, NEG_INF))
    return out, lse


def sparse_mla_fwd_dense(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor,
                         q_start_index_s: Optional[int] = None, kv_stride: int = 1,
                         sm_scale: Optional[float] = None, d_v: int = 512):
    """Dense masked formulation, restating ``ref_sparse_attention_fwd_interface``
    (examples/sparse_flash_attention/example_sparse_flash_attn.py:255-292), plus LSE.

    The index set is scattered into a ``[S, Skv+1]`` mask (the last column absorbs
    the out-of-range sentinel and is dropped), ANDed with the causal mask
    ``q_start + i >= j``, then a full softmax over all keys.  ``-1`` entries are
    mapped to the sentinel first (``scatter`` cannot take -1).  Duplicate indices
    collapse to one key here, unlike the gather form; the inputs used for
    cross-checking hold no duplicates.  Returns fp32 ``(out [B,S,H,d_v], lse [B,S,H])``.
    """
    qf = q.float()
    kvf = kv.float()
    b, sq, h, dim_q = qf.shape
    _, sk, g, _ = kvf.shape
    if q_start_index_s is None:
        q_start_index_s = sk * kv_stride - sq
    idx = indices.to(torch.int64).transpose(1, 2)                 # [b, g, sq, topk]
    idx = torch.where((idx < 0) | (idx >= sk), torch.full_like(idx, sk), idx)
    causal = (torch.arange(q_start_index_s, sq + q_start_index_s).view(-1, 1)
              >= torch.arange(kv_stride - 1, sk * kv_stride, kv_stride).view(1, -1))
    mask = torch.zeros(b, g, sq, sk + 1, dtype=torch.bool).scatter(3, idx, True)[..., :-1]
    mask = mask & causal.view(1, 1, sq, sk)
    mask[:, :, :kv_stride - 1, 0] = True
    mask = mask.view(b, g, 1, sq, sk)
    qv = qf.view(b, sq, g, -1, dim_q)
    score = torch.einsum("bmghd,bngd->bghmn", qv, kvf)
    sm_scale = dim_q ** -0.5 if sm_scale is None else sm_scale
    score = score.masked_fill(~mask, NEG_INF).mul(sm_scale)
    lse = torch.logsumexp(score, dim=-1)                            # [b, g, h/g, sq]
    p = score.softmax(dim=-1)
    o = torch.einsum("bghmn,bngd->bmghd", p, kvf[..., :d_v])
    lse = lse.reshape(b, h, sq).transpose(1, 2).contiguous()
    return o.reshape(b, sq, h, d_v), lse


def pa_to_contiguous(pool: torch.Tensor, block_table: torch.Tensor, seq_len: int) -> torch.Tensor:
    """Page pool ``[blocks, bs, 1, D]`` + one block-table row -> ``[seq_len, 1, D]``
    (sfa_golden.py:5-12, ``pa_to_bsnd`` for one batch row)."""
    bs = pool.shape[1]
    nblk = (seq_len + bs - 1) // bs
    rows = pool[block_table[:nblk].long()].reshape(nblk * bs, *pool.shape[2:])
    return rows[:seq_len]


# ---------------------------------------------------------------------------
# LSE combine across key splits (what a context-parallel shard merge does)
# ---------------------------------------------------------------------------
def lse_combine(outs: Sequence[torch.Tensor], lses: Sequence[torch.Tensor]):
    """Merge partial attention results over disjoint key subsets:
    ``lse = logsumexp_p(lse_p)``, ``out = sum_p exp(lse_p - lse) * out_p``."""
    L = torch.stack([x.float() for x in lses])
    lse = torch.logsumexp(L, dim=0)
    wts = torch.exp(L - lse.unsqueeze(0))
    wts = torch.nan_to_num(wts, nan=0.0)
    out = sum(wts[i].unsqueeze(-1) * outs[i].float() for i in range(len(outs)))
    return out, lse


# ---------------------------------------------------------------------------
# block-sparse indexer logits (HISA second stage)
# ---------------------------------------------------------------------------
def block_sparse_indexer_logits(q: torch.Tensor, kv_cache: torch.Tensor, topk_block_indices: torch.Tensor,
                                weights: torch.Tensor, context_lens: torch.Tensor,
                                block_tables: torch.Tensor) -> torch.Tensor:
    """``ref_paged_block_sparse_mqa_attn`` (examples/HISA/paged_block_sparse_mqa_attn_expert.py:425-468)
    restated over tokens: q ``[B, S, H, D]``, kv_cache ``[blocks, bs, 1, D]``,
    indices ``[B, S, topk]`` logical blocks -> fp32 ``[B, S, topk * bs]``; score
    ``sum_h w_h ReLU(q_h . k)`` of each key of the block, -inf at positions
    ``>= context_lens[b]``."""
    B, S, H, D = q.shape
    topk = topk_block_indices.shape[-1]
    bs = kv_cache.shape[1]
    out = torch.empty((B, S, topk, bs), dtype=torch.float32)
    pos = torch.arange(bs)
    for b in range(B):
        ctx = int(context_lens[b])
        for s in range(S):
            lb = topk_block_indices[b, s].long()                       # [topk]
            pages = block_tables[b, lb].long()
            keys = kv_cache[pages, :, 0, :].float()                    # [topk, bs, D]
            sc = torch.relu(torch.einsum("hd,tjd->thj", q[b, s].float(), keys))
            logit = (sc * weights[b, s].float().view(1, H, 1)).sum(dim=1)   # [topk, bs]
            logit[(lb.view(-1, 1) * bs + pos.view(1, -1)) >= ctx] = NEG_INF
            out[b, s] = logit
    return out.view(B, S, topk * bs)


# ---------------------------------------------------------------------------
# DeepSeek-V4 sparse flash MLA (window over the original KV + compressed KV)
# ---------------------------------------------------------------------------
def v4_compressed_positions(cmp_sparse_indices: Optional[torch.Tensor], b: int, s: int, act_kv: int, act_q: int,
                            cmp_ratio: int, K: Optional[int] = None) -> list:
    """Compressed positions query row ``s`` of batch ``b`` attends to
    (sparse_flash_mla_golden.py:16-53 with sparse_block_size 1, and the dense
    branch :120-122): threshold ``t = floor((act_kv - act_q + s + 1) / cmp_ratio)``;
    without a list all of ``0 .. t - 1``; with one, its first ``min(K, t)`` entries
    up to the first -1, each kept when ``< t`` and ``< floor(act_kv / cmp_ratio)``."""
    thr = (act_kv - act_q + s + 1) // cmp_ratio
    if cmp_sparse_indices is None:
        return list(range(max(thr, 0)))
    lst = cmp_sparse_indices[b, s].reshape(-1).tolist()
    K = len(lst) if K is None else K
    cmp_act = act_kv // cmp_ratio
    pos = []
    for i in range(min(K, max(thr, 0))):
        e = lst[i]
        if e == -1:
            break
        if 0 <= e < thr and e < cmp_act:
            pos.append(e)
    return pos


def sparse_flash_mla_v4(q_bnsd: torch.Tensor, ori_k_bnsd: torch.Tensor, sinks: torch.Tensor, *,
                        act_q_lens: Sequence[int], act_kv_lens: Sequence[int], softmax_scale: float,
                        cmp_k_bnsd: Optional[torch.Tensor] = None,
                        cmp_sparse_indices: Optional[torch.Tensor] = None, cmp_ratio: Optional[int] = None,
                        ori_win_left: int = 127, s2_tile: int = 512):
    """DeepSeek-V4 sparse flash MLA, the golden's loop restated
    (sparse_flash_mla_golden.py:56-153): per query row, the window
    ``[max(sg - ori_win_left, 0), sg]`` of the original keys (``sg = act_kv - act_q +
    s``) then the compressed keys of :func:`v4_compressed_positions`, in tiles of
    ``s2_tile`` with a running maximum that starts at the sink (sum starts at 1),
    probabilities rounded to q's dtype before the P.V product; K = V.
    q ``[B, N1, S, D]``, keys ``[B, 1, S_kv, D]``, sparse indices ``[B, S, 1, K]``.
    Returns ``(out [B, N1, S, D] in q's dtype, lse [B, N1, S] fp32)``; rows past
    ``act_q`` stay zero."""
    B, N1, S, D = q_bnsd.shape
    dtype = q_bnsd.dtype
    out = torch.zeros_like(q_bnsd)
    lse = torch.zeros((B, N1, S), dtype=torch.float32)
    sink = sinks.to(torch.float32)
    for b in range(B):
        aq, akv = int(act_q_lens[b]), int(act_kv_lens[b])
        for s in range(aq):
            sg = akv - aq + s
            q = q_bnsd[b, :, s, :].to(torch.float32)
            keys = [ori_k_bnsd[b, 0, max(sg - ori_win_left, 0):sg + 1, :].to(torch.float32)]
            if cmp_k_bnsd is not None:
                pos = v4_compressed_positions(cmp_sparse_indices, b, s, akv, aq, cmp_ratio)
                keys.append(cmp_k_bnsd[b, 0, pos, :].to(torch.float32))
            m = sink.clone()
            l = torch.ones(N1, dtype=torch.float32)
            acc = torch.zeros((N1, D), dtype=torch.float32)
            for kk in keys:
                for t0 in range(0, kk.shape[0], s2_tile):
                    kt = kk[t0:t0 + s2_tile]
                    sc = (q @ kt.t()) * softmax_scale
                    m_new = torch.maximum(m, sc.amax(dim=1))
                    alpha = torch.exp(m - m_new)
                    p = torch.exp(sc - m_new.unsqueeze(1))
                    l = alpha * l + p.sum(dim=1)
                    acc = acc * alpha.unsqueeze(1) + p.to(dtype).to(torch.float32) @ kt
                    m = m_new
            out[b, :, s, :] = (acc / l.unsqueeze(1)).to(dtype)
            lse[b, :, s] = m + torch.log(l)
    return out, lse


def unpack_pages(pool: torch.Tensor, block_table: torch.Tensor, length: int) -> torch.Tensor:
    """Page pool ``[blocks, bs, N2, D]`` + table ``[B, max_blocks]`` -> ``[B, N2, length, D]``
    (sparse_flash_mla_golden.py:175-198; missing pages stay zero)."""
    nb, bs, N2, D = pool.shape
    B = block_table.shape[0]
    out = pool.new_zeros((B, N2, length, D))
    for b in range(B):
        for i in range(block_table.shape[1]):
            page = int(block_table[b, i])
            lo = i * bs
            if page < 0 or lo >= length:
                continue
            hi = min(lo + bs, length)
            out[b, :, lo:hi, :] = pool[page, :hi - lo].permute(1, 0, 2)
    return out


# ---------------------------------------------------------------------------
# row quantisation (the producer of the indexer's fp8 operands; int8 act quant)
# ---------------------------------------------------------------------------
FP8_MAX = 448.0


def pow2_ceil(v: torch.Tensor) -> torch.Tensor:
    """``2 ** ceil(log2(v))`` for positive normal fp32 ``v``, exactly: the bit rule
    of fast_log2_ceil / fast_pow2 (examples/deepseek_v4/act_quant.py:93-107),
    exponent plus one when any mantissa bit is set.  The golden writes it as
    ``2 ** torch.ceil(torch.log2(...))`` (:131-132); the two differ only where
    fp32 log2 rounds a value just above a power of two down onto it."""
    m, e = torch.frexp(v.to(torch.float32))           # v = m * 2^e, m in [0.5, 1)
    k = torch.where(m == 0.5, e - 1, e)
    return torch.ldexp(torch.ones_like(v, dtype=torch.float32), k)


def act_quant_int8(x: torch.Tensor, round_scale: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantisation, ``act_quant_torch`` (act_quant.py:110-149):
    ``s = max(absmax, 1e-4) / 127`` (power of two with ``round_scale``),
    ``y = round(clamp(x / s, -127, 127))`` (round half to even).  2-D ``[M, N]`` ->
    ``(y [M, N] int8, s [M, 1])``; 3-D ``[b, s, N]`` -> scales ``[b, s, 1]``."""
    shape = x.shape
    x2 = x.reshape(-1, shape[-1]).to(torch.float32)
    amax = torch.clamp(x2.abs().amax(dim=1, keepdim=True), min=1e-4)
    scales = amax / 127.0
    if round_scale:
        scales = pow2_ceil(scales)
    y = torch.round(torch.clamp(x2 / scales, -127, 127)).to(torch.float16).to(torch.int8)
    return y.view(shape), scales.view(*shape[:-1], 1)


def quant_fp8_rows(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row fp8 e4m3fn quantisation over the last dim:
    ``s = max(absmax / 448, FLT_MIN)``, ``y = e4m3fn(x / s)`` (round to nearest even,
    torch's float8 conversion).  Returns ``(y, s)`` with ``s`` of shape ``x.shape[:-1]``.
    This is the key quantisation whose scale is the indexer's ``key_scale``."""
    x32 = x.to(torch.float32)
    s = torch.clamp(x32.abs().amax(dim=-1) / FP8_MAX, min=torch.finfo(torch.float32).tiny)
    return (x32 / s.unsqueeze(-1)).to(torch.float8_e4m3fn), s


def indexer_q_quant_fp8(q: torch.Tensor, weights: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Indexer query producer: one fp8 scale per (token, head) folded into the head
    weights, ``w' = w * s``, so that ``w' * ReLU(q8 . k) = w * ReLU((s q8) . k)``
    (the score of lightning_indexer.py:199-335 with the dequantised query)."""
    q8, s = quant_fp8_rows(q)
    return q8, weights.to(torch.float32) * s


def fp8_e4m3fn_nearest(v: torch.Tensor) -> torch.Tensor:
    """Brute-force round-to-nearest-even onto the finite e4m3fn grid (enumerates
    the 254 finite codes); used to pin torch's float8 conversion on in-range values."""
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(torch.float8_e4m3fn)
    grid = codes.to(torch.float32)
    fin = torch.isfinite(grid)
    grid, codes = grid[fin], codes[fin]
    d = (v.to(torch.float32).reshape(-1, 1) - grid.reshape(1, -1)).abs()
    best = d.min(dim=1, keepdim=True).values
    cand = d == best
    # a tie sits between two neighbours: prefer the even mantissa code, and keep
    # the sign of v for zero
    even = (codes.view(torch.uint8) & 1) == 0
    pick = torch.where(cand & even, 1, 0) * 2 + cand.int()
    out = codes[pick.argmax(dim=1)].view(torch.uint8).clone()
    zero = (out & 0x7F) == 0  # rounded to zero: the sign follows v
    out[zero] = torch.where(torch.signbit(v.reshape(-1)[zero]), 0x80, 0x00).to(torch.uint8)
    return out.view(torch.float8_e4m3fn).view(v.shape)


PINNED_BY = {
    "stable_topk": "brute force sorted(key=(-v, i)); known answers restated from "
                   "test_topk/test_sort (arange N=51 K=10, N=131); ties, +-0.0, -inf rows, "
                   "short rows -> -1 (tests/test_oracle_topk.py, tests/golden/topk_*.npz)",
    "indexer_scores/lightning_indexer": "triple-loop brute force on tiny shapes; second "
                   "formulation index_golden; invariants: positive key scaling, all-negative "
                   "q.k -> 0, masked -> -inf, fp8 dequant identity (tests/test_oracle_indexer.py)",
    "sparse_mla_fwd_gather": "per-(token, head) brute force; agreement with the dense "
                   "formulation; single valid index -> out = v, lse = score; permutation "
                   "invariance; LSE == logsumexp (tests/test_oracle_mla.py)",
    "sparse_mla_fwd_dense": "agreement with the gather form and brute force",
    "lse_combine": "split a row's index set in two, combine == unsplit result",
    "block_sparse_indexer_logits": "the a1 restatement (indexer_scores) on the gathered blocks' keys "
                   "(independent code), masked positions (tests/test_oracle_indexer.py)",
    "sparse_flash_mla_v4": "the gather formulation on the same key sets (independent code), "
                   "closed forms (no key: out 0 and lse = sink; one key: out = v e^s / (e^s + e^sink)), "
                   "compressed-position rules against hand-worked lists (tests/test_oracle_mla.py)",
    "act_quant_int8/pow2_ceil": "the golden's torch formula (2**ceil(log2)) on random rows, "
                   "the reference test's tolerance (act_quant.py:162-163), max |y| = 127 at the "
                   "row maximum, |x - y s| <= s / 2, half-to-even ties on constructed rows, "
                   "power-of-two bounds s/2 < v <= s (tests/test_oracle_quant.py)",
    "quant_fp8_rows": "torch's float8 conversion against a brute-force nearest-even search "
                   "over the e4m3fn grid for every bf16 value in range, max |y| = 448 at the "
                   "row maximum, power-of-two equivariance, the indexer's key recipe",
    "indexer_q_quant_fp8": "indexer scores with (q8, w s) equal those with the dequantised "
                   "query s q8 and w, to fp32 rounding",
}
