"""Seeded synthetic inputs for the DSA path, in the shapes of the benchmark configs.

Every generator draws from one ``torch.Generator`` seeded with ``seed``, in the
order documented on the function, on ``device``.  Tests run the CPU checker on
copies of the very same tensors, so both sides see identical bytes.

Configs (B = batch, S = query tokens, Skv = keys, H = query heads):
  1  sparse MLA small     B=1 S=128 Skv=4096 H=16 topk=512, causal index ranges
  2  indexer + top-k      B=1 S1=4096 S2=32768, 64 index heads x 128, fp8, top 2048
  3  sparse MLA decode    B=64 S=1 H=128, 64K paged context (64-token pages), topk 2048
  4  sparse MLA prefill   B=1 S=Skv=16384 H=128 topk 2048, row i draws from [0, i]
  5  full layer at 128K   indexer over S2=131072 with a 4096-token tail chunk, top-k,
                          sparse MLA on that chunk; plus a B=32 decode step
"""

from __future__ import annotations

from typing import Optional

import torch

FP8 = torch.float8_e4m3fn
D_QK, D_V = 576, 512


def _gen(seed: int, device) -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def causal_indices(S: int, Skv: int, topk: int, q_start: int, gen: torch.Generator,
                   device="cpu", row_chunk: int = 512) -> torch.Tensor:
    """int32 ``[S, topk]``: row i holds ``min(q_start+i+1, Skv, topk)`` distinct
    indices drawn uniformly from ``[0, q_start + i]`` (clipped to Skv), padded with -1.
    Sampling = the first entries of a uniform random order of the allowed keys."""
    out = torch.full((S, topk), -1, dtype=torch.int32, device=device)
    cols = torch.arange(Skv, device=device)
    for r0 in range(0, S, row_chunk):
        r1 = min(S, r0 + row_chunk)
        keys = torch.rand((r1 - r0, Skv), generator=gen, device=device)
        limit = (torch.arange(r0, r1, device=device) + q_start).unsqueeze(1)
        keys = torch.where(cols.unsqueeze(0) <= limit, keys, torch.full_like(keys, 2.0))
        order = torch.argsort(keys, dim=1)[:, :topk]
        n_ok = torch.clamp(limit + 1, max=min(Skv, topk))            # valid count per row
        pos = torch.arange(order.shape[1], device=device).unsqueeze(0)
        out[r0:r1, :order.shape[1]] = torch.where(pos < n_ok, order, torch.full_like(order, -1)).to(torch.int32)
    return out


def mla_prefill(B=1, S=128, Skv=4096, H=16, topk=512, seed=1, d_qk=D_QK, q_start: Optional[int] = None,
                device="cpu"):
    """Config 1 (defaults) and config 4 (S=Skv=16384, H=128, topk=2048, q_start=0).
    Draw order: q, kv, then the index rows.  q, kv ~ N(0,1)*0.5 in bf16."""
    g = _gen(seed, device)
    q = (torch.randn((B, S, H, d_qk), generator=g, device=device) * 0.5).to(torch.bfloat16)
    kv = (torch.randn((B, Skv, 1, d_qk), generator=g, device=device) * 0.5).to(torch.bfloat16)
    if q_start is None:
        q_start = Skv - S
    idx = torch.stack([causal_indices(S, Skv, topk, q_start, g, device) for _ in range(B)])
    return dict(q=q, kv=kv, indices=idx.unsqueeze(2).contiguous(), sm_scale=d_qk ** -0.5, q_start=q_start)


def mla_decode(B=64, ctx=65536, H=128, topk=2048, block_size=64, seed=3, d_qk=D_QK, device="cpu",
               pool_blocks: Optional[int] = None):
    """Config 3: paged decode.  Draw order: q, the page pool, one permutation of
    the pool's pages (batch b takes pages [b*nb, (b+1)*nb) of it), then per batch
    a random order of [0, ctx) whose first topk entries are the indices."""
    g = _gen(seed, device)
    nb = (ctx + block_size - 1) // block_size
    nblocks = pool_blocks if pool_blocks is not None else B * nb
    q = (torch.randn((B, 1, H, d_qk), generator=g, device=device) * 0.5).to(torch.bfloat16)
    pool = (torch.randn((nblocks, block_size, 1, d_qk), generator=g, device=device) * 0.5).to(torch.bfloat16)
    perm = torch.randperm(nblocks, generator=g, device=device).to(torch.int32)
    if nblocks >= B * nb:
        bt = perm[: B * nb].view(B, nb).contiguous()
    else:
        bt = perm.repeat((B * nb + nblocks - 1) // nblocks)[: B * nb].view(B, nb).contiguous()
    idx = torch.stack([torch.randperm(ctx, generator=g, device=device)[:topk] for _ in range(B)])
    idx = idx.to(torch.int32).view(B, 1, 1, topk).contiguous()
    seq_len = torch.full((B,), ctx, dtype=torch.int32, device=device)
    return dict(q=q, kv=pool, indices=idx, block_table=bt, seq_len_kv=seq_len,
                sm_scale=d_qk ** -0.5, q_start=ctx - 1)


def indexer_fp8(B=1, S1=4096, S2=32768, H=64, D=128, seed=2, device="cpu"):
    """Config 2 (defaults) / config 5 (S2=131072).  Draw order: q (N(0,1) -> e4m3),
    k32 (N(0,1)), w (N(0,1)/8).  Keys are quantised per token:
    scale = absmax/448, k = e4m3(k32 / scale)."""
    g = _gen(seed, device)
    q = torch.randn((B, S1, H, D), generator=g, device=device).to(FP8)
    k32 = torch.randn((B, S2, 1, D), generator=g, device=device)
    w = torch.randn((B, S1, H), generator=g, device=device) / 8
    scale = k32.abs().amax(dim=-1) / 448.0                      # [B, S2, 1]
    scale = torch.clamp(scale, min=torch.finfo(torch.float32).tiny)
    k = (k32 / scale.unsqueeze(-1)).to(FP8)
    return dict(q=q.contiguous(), k=k.contiguous(), w=w.contiguous(), key_scale=scale.view(B, S2).contiguous())


def flash_mla_v4(scenario=3, B=1, S1=1024, N1=64, D=512, K=512, cmp_ratio=4, block_size=128,
                 seqused_kv=None, cu_seqlens_q=None, seed=42, win_left=127):
    """A DeepSeek-V4 sparse flash MLA case shaped like the reference's fast scenarios
    (sparse_flash_mla_golden.py:384-461: "swa" scenario 1, "hca" 2 with cmp_ratio
    128, "csa" 3 with K = 512): TND queries (cu_seqlens_q), q ~ U(-10, 10), original
    keys ~ U(-10, 10) and compressed keys ~ U(-5, 10) in shuffled pages of
    ``block_size``, sinks ~ U(-1, 1), per-row top-K compressed lists (a random
    permutation of the visible compressed positions, -1 padded).  Draw order:
    q, original keys, page permutation, compressed keys, its permutation, lists, sinks."""
    g = _gen(seed, "cpu")
    if cu_seqlens_q is None:
        cu_seqlens_q = [S1 * i for i in range(B + 1)]
    lens = [cu_seqlens_q[i + 1] - cu_seqlens_q[i] for i in range(B)]
    if seqused_kv is None:
        seqused_kv = list(lens)
    T = cu_seqlens_q[-1]
    bf = torch.bfloat16
    q = (torch.rand((T, N1, D), generator=g) * 20 - 10).to(bf)

    def paged(n_tok, lo, hi):
        mx = max(max(n_tok), 1)
        logical = (torch.rand((B, mx, D), generator=g) * (hi - lo) + lo).to(bf)
        nbs = [(n + block_size - 1) // block_size for n in n_tok]
        nblocks = max(sum(nbs), 1) + 2
        perm = torch.randperm(nblocks, generator=g)
        table = torch.full((B, max(max(nbs), 1)), -1, dtype=torch.int32)
        pool = torch.zeros((nblocks, block_size, 1, D), dtype=bf)
        c = 0
        for b in range(B):
            for i in range(nbs[b]):
                page = int(perm[c]); c += 1
                table[b, i] = page
                lo_, hi_ = i * block_size, min((i + 1) * block_size, n_tok[b])
                pool[page, :hi_ - lo_, 0] = logical[b, lo_:hi_]
        return pool, table

    ori_pa, ori_bt = paged(seqused_kv, -10, 10)
    case = dict(q=q, ori_kv=ori_pa, ori_block_table=ori_bt, cu_seqlens_q=torch.tensor(cu_seqlens_q, dtype=torch.int32),
                seqused_kv=torch.tensor(seqused_kv, dtype=torch.int32), cmp_kv=None, cmp_block_table=None,
                cmp_sparse_indices=None, cmp_ratio=cmp_ratio if scenario >= 2 else None,
                softmax_scale=0.04419417, ori_win_left=win_left, topk_cmp=None)
    if scenario >= 2:
        cmp_seqs = [n // cmp_ratio for n in seqused_kv]
        case["cmp_kv"], case["cmp_block_table"] = paged(cmp_seqs, -5, 10)
    if scenario == 3:
        idx = torch.full((T, 1, K), -1, dtype=torch.int32)
        for b in range(B):
            for s in range(lens[b]):
                cur = max(0, (seqused_kv[b] - lens[b] + s + 1) // cmp_ratio)
                perm = torch.randperm(cur, generator=g).to(torch.int32) if cur > 0 else torch.empty(0, dtype=torch.int32)
                take = min(cur, K)
                idx[cu_seqlens_q[b] + s, 0, :take] = perm[:take]
        case["cmp_sparse_indices"] = idx
        case["topk_cmp"] = K
    case["sinks"] = torch.rand(N1, generator=g) * 2 - 1
    return case
