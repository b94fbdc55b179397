"""GPU parity of the lightning indexer on the reference wrapper's own input dtypes
(fp16 / bf16 q and k, weights in q's dtype or fp32, 1..64 index heads) and of the
fp8 path with fewer than 64 heads.

The four cases are the reference's own examples (examples/deepseek_v4/
lightning_indexer.py:1568-1640: BSND+BSND, BSND+PA_BSND, TND+TND, TND+PA_BSND, with
its uniform(-1, 1) inputs and |uniform| weights) and the acceptance rule is its
own _check_result (:1394-1503), restated below: index sets may differ only where
the scores lie within 1e-4 relative of the K-th score, and (non-paged keys) the
sorted top-K values agree within rtol 0.005 / atol 2.5e-5 after an fp16
conversion on at least 95 % of the entries.  The logits themselves are checked
against the oracle at 1e-4 of the row's largest magnitude (both accumulate the
exact 16-bit products in fp32; only the order of the additions differs)."""
import math

import numpy as np
import pytest
import torch

import dsa
from oracle.dsa_oracle import lightning_indexer as ref_indexer

pytestmark = pytest.mark.gpu


def _rand(rng, shape, dtype):
    return torch.tensor(rng.uniform(-1, 1, shape), dtype=dtype)


def _build_pa(k_bsnd, act_k, block_size, block_num, seed=42):
    # the reference's own scatter (lightning_indexer.py:1505-1532): shuffled pages,
    # a [B, block_num] table padded with -1
    B, S2_max, N2, D = k_bsnd.shape
    perm = np.random.RandomState(seed).permutation(block_num).astype(np.int32)
    bt = np.full((B, block_num), -1, dtype=np.int32)
    k_pa = torch.zeros((block_num, block_size, N2, D), dtype=k_bsnd.dtype)
    c = 0
    for b in range(B):
        for i in range(math.ceil(act_k[b] / block_size)):
            bt[b, i] = perm[c]
            c += 1
            s0, s1 = i * block_size, min((i + 1) * block_size, act_k[b])
            k_pa[int(bt[b, i]), : s1 - s0] = k_bsnd[b, s0:s1]
    return k_pa, torch.from_numpy(bt)


def _check_result(g_idx, g_scores, g_val, t_idx, t_val, asq, layout_query, is_pa):
    K = g_idx.shape[-1]
    g_flat, t_flat = g_idx.reshape(-1, K), t_idx.reshape(-1, K)
    if layout_query == "TND":
        q_off = [0] + [int(x) for x in asq.tolist()]
        rows = []
        for b in range(len(q_off) - 1):
            rows += [(b, s) for s in range(q_off[b + 1] - q_off[b])]
    else:
        B, S1 = g_idx.shape[0], g_idx.shape[1]
        rows = [(b, s) for b in range(B) for s in range(S1)]
    fail = 0
    for r, (b, s) in enumerate(rows):
        gs = set(x for x in g_flat[r].tolist() if x >= 0)
        ts = set(x for x in t_flat[r].tolist() if x >= 0)
        if gs == ts:
            continue
        row = g_scores[b, 0, s]
        bound = min(float(row[i]) for i in gs) if gs else float("-inf")
        for i in gs ^ ts:
            sc = float(row[i])
            re = (0.0 if sc == 0 else float("inf")) if bound == 0 else abs(sc - bound) / abs(bound)
            fail += re > 1e-4
    assert fail == 0, f"{fail} differing indices outside 1e-4 of the K-th score"
    if not is_pa:
        g = torch.sort(g_val.reshape(-1, K).float(), dim=-1, descending=True)[0].to(torch.float16).float()
        t = torch.sort(t_val.reshape(-1, K).float(), dim=-1, descending=True)[0].to(torch.float16).float()
        bad = (~torch.isclose(g, t, rtol=0.005, atol=0.000025, equal_nan=True)).float().mean().item()
        assert bad < 0.05, f"{bad * 100:.2f} % of the top-K values off"


def _run(gpu, q, k, w, asq, ask, bt, lq, lk, K, mode):
    is_pa = lk == "PA_BSND"
    d = lambda t: None if t is None else t.to(gpu)  # noqa: E731
    idx, val, logits = dsa.lightning_indexer(d(q), d(k), d(w), actual_seq_lengths_query=d(asq),
                                             actual_seq_lengths_key=d(ask), block_table=d(bt), layout_query=lq,
                                             layout_key=lk, sparse_count=K, sparse_mode=mode,
                                             return_value=not is_pa, return_logits=True)
    torch.cuda.synchronize()
    if not is_pa:
        assert val.dtype == q.dtype  # the golden's values are in q's dtype
    g_idx, g_scores, g_val = ref_indexer(q, k, w, actual_seq_lengths_query=asq, actual_seq_lengths_key=ask,
                                         block_table=bt, layout_query=lq, layout_key=lk, sparse_count=K,
                                         sparse_mode=mode)
    _check_result(g_idx, g_scores, g_val, idx.cpu(), None if is_pa else val.cpu(), asq, lq, is_pa)
    # logits against the oracle's, row by row, over the row's visible keys
    lg = logits.cpu().reshape(-1, logits.shape[-1])
    r = 0
    q_off = [0] + [int(x) for x in asq.tolist()] if lq == "TND" else None
    nb = len(q_off) - 1 if q_off else q.shape[0]
    for b in range(nb):
        ns = (q_off[b + 1] - q_off[b]) if q_off else q.shape[1]
        for s in range(ns):
            ref = g_scores[b, 0, s]
            n = int(torch.isfinite(ref).sum())
            if n:
                scale = float(ref[:n].abs().max()) + 1e-30
                err = float((lg[r, :n] - ref[:n]).abs().max())
                assert err <= 1e-4 * scale, f"row {r}: logit error {err} vs row scale {scale}"
            r += 1
    return idx


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_example_bsnd_bsnd(gpu, dtype):
    # Example 1 (:1571-1583): B=2, S1=3, S2=32768, N1=64, TOP_K=2048, mode 3
    rng = np.random.RandomState(1)
    B, S1, S2, N1, D, K = 2, 3, 32768, 64, 128, 2048
    print(f"indexer {dtype} example 1 bsnd+bsnd", flush=True)
    q, k = _rand(rng, (B, S1, N1, D), dtype), _rand(rng, (B, S2, 1, D), dtype)
    w = _rand(rng, (B, S1, N1), dtype).abs()
    asq, ask = torch.full((B,), S1, dtype=torch.int32), torch.full((B,), S2, dtype=torch.int32)
    _run(gpu, q, k, w, asq, ask, None, "BSND", "BSND", K, 3)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_example_bsnd_pa(gpu, dtype):
    # Example 2 (:1586-1610): B=2, S1=1, N1=8, block_size 128, 32 blocks, act_k [1024, 2048], mode 0
    rng = np.random.RandomState(2)
    B, S1, N1, D, K, bs, nblk = 2, 1, 8, 128, 2048, 128, 32
    act_k = [1024, 2048]
    print(f"indexer {dtype} example 2 bsnd+pa", flush=True)
    q, w = _rand(rng, (B, S1, N1, D), dtype), _rand(rng, (B, S1, N1), dtype).abs()
    k_pa, bt = _build_pa(_rand(rng, (B, max(act_k), 1, D), dtype), act_k, bs, nblk)
    _run(gpu, q, k_pa, w, torch.full((B,), S1, dtype=torch.int32), torch.tensor(act_k, dtype=torch.int32), bt,
         "BSND", "PA_BSND", K, 0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_example_tnd_tnd(gpu, dtype):
    # Example 3 (:1613-1622): B=8, S1=64, S2=3072, N1=24, TOP_K=2048, mode 0, prefix sums
    rng = np.random.RandomState(3)
    B, S1, S2, N1, D, K = 8, 64, 3072, 24, 128, 2048
    print(f"indexer {dtype} example 3 tnd+tnd", flush=True)
    q, k = _rand(rng, (B * S1, N1, D), dtype), _rand(rng, (B * S2, 1, D), dtype)
    w = _rand(rng, (B * S1, N1), dtype).abs()
    asq = torch.cumsum(torch.full((B,), S1, dtype=torch.int32), dim=0).int()
    ask = torch.cumsum(torch.full((B,), S2, dtype=torch.int32), dim=0).int()
    _run(gpu, q, k, w, asq, ask, None, "TND", "TND", K, 0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_example_tnd_pa(gpu, dtype):
    # Example 4 (:1625-1650): B=2, N1=8, act_q [1024, 2048], act_k [4096, 8192],
    # block_size 128, 128 blocks, mode 0
    rng = np.random.RandomState(4)
    B, N1, D, K, bs, nblk = 2, 8, 128, 2048, 128, 128
    act_q, act_k = [1024, 2048], [4096, 8192]
    print(f"indexer {dtype} example 4 tnd+pa", flush=True)
    q, w = _rand(rng, (sum(act_q), N1, D), dtype), _rand(rng, (sum(act_q), N1), dtype).abs()
    k_pa, bt = _build_pa(_rand(rng, (B, max(act_k), 1, D), dtype), act_k, bs, nblk)
    asq = torch.cumsum(torch.tensor(act_q, dtype=torch.int32), dim=0).int()
    _run(gpu, q, k_pa, w, asq, torch.tensor(act_k, dtype=torch.int32), bt, "TND", "PA_BSND", K, 0)


def test_causal_signed_weights_fp32(gpu):
    # causal rows (mode 3) with signed fp32 weights and N(0, 1) bf16 inputs, a
    # partial last key tile, two batch rows of different key lengths
    g = torch.Generator().manual_seed(5)
    B, S1, S2, N1, D, K = 2, 37, 5000, 64, 128, 512
    print("indexer bf16 causal signed weights", flush=True)
    q = torch.randn((B, S1, N1, D), generator=g).to(torch.bfloat16)
    k = torch.randn((B, S2, 1, D), generator=g).to(torch.bfloat16)
    w = torch.randn((B, S1, N1), generator=g) / 8
    ask = torch.tensor([S2, 4321], dtype=torch.int32)
    _run(gpu, q, k, w, torch.full((B,), S1, dtype=torch.int32), ask, None, "BSND", "BSND", K, 3)


def test_fp8_fewer_heads(gpu):
    # the fp8 path with N1 = 24 (zero-padded to the kernel's 64 heads)
    from dsa import inputs
    inp = inputs.indexer_fp8(B=1, S1=16, S2=3000, seed=6)
    q, w = inp["q"][:, :, :24].contiguous(), inp["w"][:, :, :24].contiguous()
    print("indexer fp8 N1=24", flush=True)
    idx, _, logits = dsa.lightning_indexer(q.to(gpu), inp["k"].to(gpu), w.to(gpu), key_scale=inp["key_scale"].to(gpu),
                                           sparse_count=256, return_logits=True)
    torch.cuda.synchronize()
    ri, rs, _ = ref_indexer(q, inp["k"], w, key_scale=inp["key_scale"], sparse_count=256)
    lg = logits.cpu()[0]
    for t in range(16):
        ref = rs[0, 0, t]
        n = int(torch.isfinite(ref).sum())
        scale = float(ref[:n].abs().max())
        assert float((lg[t, :n] - ref[:n]).abs().max()) <= 1e-2 * scale, f"row {t}"


def test_full_length_key_chunks(gpu):
    # 2048 causal bf16 rows x 140000 keys: 256 workgroups of 8 tokens keep the
    # longest key chunk (131072 keys; two chunks per block, the second of 8928
    # keys), so every row crosses a chunk boundary.  Logits of three rows against
    # the oracle's formula at 1e-4 of the row's largest magnitude; every row's
    # indices against the stable sort of the kernel's own logits.
    from fullsize import check_topk_rows
    g = torch.Generator(device=gpu).manual_seed(11)
    S1, S2, N1, D, K = 2048, 140000, 64, 128, 2048
    q_start = S2 - S1
    print(f"indexer bf16 full-length chunks S1={S1} S2={S2}", flush=True)
    q = torch.randn((1, S1, N1, D), generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn((1, S2, 1, D), generator=g, device=gpu).to(torch.bfloat16)
    w = torch.randn((1, S1, N1), generator=g, device=gpu) / 8
    idx, _, logits = dsa.lightning_indexer(q, k, w, sparse_count=K, sparse_mode=3, return_logits=True)
    torch.cuda.synchronize()
    kc = k[0, :, 0].float().cpu()
    for t in (0, 1100, S1 - 1):
        n = q_start + t + 1
        ref = (w[0, t].cpu().unsqueeze(1) * torch.relu(q[0, t].float().cpu() @ kc[:n].T)).sum(0)
        got = logits[0, t, :n].cpu()
        assert float((got - ref).abs().max()) <= 1e-4 * float(ref.abs().max()), f"row {t}"
    check_topk_rows(idx.view(S1, K), logits.view(S1, S2), q_start + 1 + torch.arange(S1, device=gpu), K,
                    chunk=64, what="bf16 full-length chunks top-k")


def test_paged_long_rows_group_maxima(gpu):
    # bf16 keys in shuffled 128-key pages, two sequences of 70000 / 66000 keys,
    # causal rows: at least 2 K groups of 16 keys per row, so the logits kernel
    # writes the group maxima and the top-k reads only the groups that can hold a
    # top-K key.  Paged and contiguous keys give bit-identical logits and indices;
    # every row's indices equal the stable sort of the kernel's own logits; two
    # rows' logits against the formula.
    from fullsize import check_topk_rows
    rng = np.random.RandomState(9)
    B, S1, N1, D, K, bs = 2, 24, 64, 128, 2048, 128
    act_k = [70000, 66000]
    nblk = sum((a + bs - 1) // bs for a in act_k)
    print(f"indexer bf16 paged long rows act_k={act_k}", flush=True)
    g = torch.Generator().manual_seed(9)
    q = torch.randn((B, S1, N1, D), generator=g).to(torch.bfloat16)
    w = torch.randn((B, S1, N1), generator=g) / 8
    k = torch.randn((B, max(act_k), 1, D), generator=g).to(torch.bfloat16)
    k_pa, bt = _build_pa(k, act_k, bs, nblk, seed=9)
    asq = torch.full((B,), S1, dtype=torch.int32)
    ask = torch.tensor(act_k, dtype=torch.int32)
    d = lambda t: t.to(gpu)  # noqa: E731
    idx_p, _, lg_p = dsa.lightning_indexer(d(q), d(k_pa), d(w), actual_seq_lengths_query=d(asq),
                                           actual_seq_lengths_key=d(ask), block_table=d(bt), layout_key="PA_BSND",
                                           sparse_count=K, sparse_mode=3, return_logits=True)
    idx_c, _, lg_c = dsa.lightning_indexer(d(q), d(k), d(w), actual_seq_lengths_query=d(asq),
                                           actual_seq_lengths_key=d(ask), sparse_count=K, sparse_mode=3,
                                           return_logits=True)
    torch.cuda.synchronize()
    L = torch.tensor([act_k[b] - S1 + s + 1 for b in range(B) for s in range(S1)], dtype=torch.int32, device=gpu)
    lp, lc = lg_p.reshape(B * S1, -1), lg_c.reshape(B * S1, -1)
    n = min(lp.shape[1], lc.shape[1])
    keep = torch.arange(n, device=gpu).unsqueeze(0) < L.view(-1, 1)
    assert torch.equal(torch.where(keep, lp[:, :n], 0.), torch.where(keep, lc[:, :n], 0.)), "paged logits differ"
    assert torch.equal(idx_p, idx_c), "paged indices differ"
    check_topk_rows(idx_p.reshape(B * S1, K), lc[:, :n].contiguous(), L, K, chunk=48, what="bf16 paged top-k")
    for b, s in ((0, 0), (1, S1 - 1)):
        nl = act_k[b] - S1 + s + 1
        ref = (w[b, s].unsqueeze(1) * torch.relu(q[b, s].float() @ k[b, :nl, 0].float().T)).sum(0)
        got = lc[b * S1 + s, :nl].cpu()
        assert float((got - ref).abs().max()) <= 1e-4 * float(ref.abs().max()), f"row ({b}, {s})"


@pytest.mark.parametrize("n1,S2", [(8, 70000), (24, 70000), (64, 70007)])
def test_few_heads_long_rows(gpu, n1, S2):
    # N1 <= 32 (the reference examples' head counts) on rows long enough for the
    # group-maxima top-k: the one-tile kernel with group maxima (and 64 heads on a
    # key count that ends inside a 16-key group).  Every row's
    # indices against the stable sort of the kernel's logits; two rows' logits
    # against the formula.
    from fullsize import check_topk_rows
    g = torch.Generator(device=gpu).manual_seed(n1)
    S1, K = 24, 2048  # S2 = 70007: the rows' last 16-key group is partial
    print(f"indexer bf16 N1={n1} long rows S2={S2}", flush=True)
    q = torch.randn((1, S1, n1, 128), generator=g, device=gpu).to(torch.bfloat16)
    k = torch.randn((1, S2, 1, 128), generator=g, device=gpu).to(torch.bfloat16)
    w = torch.randn((1, S1, n1), generator=g, device=gpu) / 8
    idx, _, logits = dsa.lightning_indexer(q, k, w, sparse_count=K, sparse_mode=3, return_logits=True)
    torch.cuda.synchronize()
    L = S2 - S1 + 1 + torch.arange(S1, device=gpu)
    check_topk_rows(idx.view(S1, K), logits.view(S1, S2), L, K, chunk=24, what=f"N1={n1} top-k")
    kc = k[0, :, 0].float().cpu()
    for t in (0, S1 - 1):
        n = S2 - S1 + t + 1
        ref = (w[0, t].cpu().unsqueeze(1) * torch.relu(q[0, t].float().cpu() @ kc[:n].T)).sum(0)
        got = logits[0, t, :n].cpu()
        assert float((got - ref).abs().max()) <= 1e-4 * float(ref.abs().max()), f"row {t}"


@pytest.mark.parametrize("n1", [1, 32, 33])
def test_head_tile_boundary(gpu, n1):
    # head counts at the one-tile / two-tile boundary (N1 <= 32 computes one
    # 32-head tile): logits against the oracle, indices under the reference rule
    rng = np.random.RandomState(100 + n1)
    B, S1, S2, K = 2, 20, 3000, 512
    print(f"indexer bf16 N1={n1} head-tile boundary", flush=True)
    q = _rand(rng, (B, S1, n1, 128), torch.bfloat16)
    k = _rand(rng, (B, S2, 1, 128), torch.bfloat16)
    w = _rand(rng, (B, S1, n1), torch.bfloat16).abs()
    _run(gpu, q, k, w, torch.full((B,), S1, dtype=torch.int32), torch.tensor([S2, 2500], dtype=torch.int32), None,
         "BSND", "BSND", K, 3)
