"""GPU parity of the fp8 lightning indexer.

Logits: within 1e-2 relative of the oracle for every logit whose
magnitude is at least 2 % of its row's RMS; smaller logits (cancellations of the
signed head weights) within 2e-4 of the row RMS.  Indices: the top-k of the GPU's
own logits is bit-exact with the oracle's stable top-k of the same logits; against
the oracle's logits the reference's own acceptance rule applies
(examples/deepseek_v4/lightning_indexer.py:1394-1503: differing indices must lie
within 1e-4 relative of the K-th score)."""
import pytest
import torch

import dsa
from dsa import inputs
from oracle.dsa_oracle import lightning_indexer as ref_indexer
from oracle.dsa_oracle import stable_topk
from fullsize import check_topk_rows

pytestmark = pytest.mark.gpu


def _logit_close(got, ref):
    """1e-2 relative for every logit at or above a floor of 2 % of its row's RMS;
    below the floor (near-cancellations of the signed head weights, where a
    relative bound says nothing) the error must stay under 1e-2 of the floor."""
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got)), "masked positions differ"
    rms = torch.sqrt(torch.mean(torch.where(fin, ref, 0) ** 2, dim=-1, keepdim=True))
    floor = 2e-2 * rms
    err = (got - ref).abs()
    big = (ref.abs() >= floor) & fin
    rel = (err / ref.abs().clamp_min(1e-30))[big]
    max_rel = float(rel.max()) if rel.numel() else 0.0
    print(f"indexer logits: max relative error {max_rel:.3e} over {rel.numel()} entries above the floor", flush=True)
    assert max_rel <= 1e-2, f"max relative error {max_rel}"
    bad = (err > 1e-2 * floor) & fin & ~big
    assert not bad.any(), f"{int(bad.sum())} logits below the floor off by more than 1e-2 of it"


def _case(gpu, B, S1, S2, seed, K=2048, mode=3, act_q=None, act_k=None):
    print(f"indexer case B={B} S1={S1} S2={S2} K={K} mode={mode}", flush=True)
    inp = inputs.indexer_fp8(B=B, S1=S1, S2=S2, seed=seed)
    dev = {k: v.to(gpu) for k, v in inp.items()}
    idx, vals, logits = dsa.lightning_indexer(dev["q"], dev["k"], dev["w"], key_scale=dev["key_scale"],
                                              actual_seq_lengths_query=act_q, actual_seq_lengths_key=act_k,
                                              sparse_count=K, sparse_mode=mode, return_value=True,
                                              return_logits=True)
    torch.cuda.synchronize()
    ri, rscores, rv = ref_indexer(inp["q"], inp["k"], inp["w"], key_scale=inp["key_scale"],
                                  actual_seq_lengths_query=act_q, actual_seq_lengths_key=act_k,
                                  sparse_count=K, sparse_mode=mode)
    return idx.cpu(), vals.cpu(), logits.cpu(), ri, rscores, rv


@pytest.mark.parametrize("B,S1,S2,mode", [(1, 64, 4096, 3), (2, 40, 1000, 3), (1, 33, 2500, 0), (1, 16, 9000, 3)])
def test_logits_and_indices(gpu, B, S1, S2, mode):
    idx, vals, logits, ri, rscores, rv = _case(gpu, B, S1, S2, seed=S1 + S2, mode=mode)
    for b in range(B):
        L = torch.isfinite(rscores[b, 0]).sum(dim=-1)  # visible keys per row
        for t in range(S1):
            n = int(L[t])
            _logit_close(logits[b, t, :n], rscores[b, 0, t, :n])
    # bit-exact top-k given identical logits
    flat = logits.view(B * S1, S2)
    row_len = torch.isfinite(rscores[:, 0]).sum(dim=-1).view(-1).int()
    ti, tv = stable_topk(flat, idx.shape[-1], row_len=row_len)
    assert torch.equal(idx.view(B * S1, -1), ti)
    assert torch.equal(torch.nan_to_num(vals.view(B * S1, -1), neginf=-3e38), torch.nan_to_num(tv, neginf=-3e38))
    # reference acceptance rule against the oracle's own logits
    K = idx.shape[-1]
    for r in range(B * S1):
        b, t = divmod(r, S1)
        gs = set(x for x in ri[b, t, 0].tolist() if x >= 0)
        ts = set(x for x in idx[b, t, 0].tolist() if x >= 0)
        if gs == ts:
            continue
        row = rscores[b, 0, t]
        bound = min(float(row[i]) for i in gs)
        for i in gs ^ ts:
            assert abs(float(row[i]) - bound) <= 1e-4 * abs(bound) + 1e-6, f"row {r} index {i}"


def test_actual_lengths(gpu):
    act_q = torch.tensor([20, 7], dtype=torch.int32)
    act_k = torch.tensor([3000, 100], dtype=torch.int32)
    idx, vals, logits, ri, rscores, rv = _case(gpu, 2, 24, 3000, seed=5, K=512, act_q=act_q, act_k=act_k)
    # rows past act_q are all -1; batch 1 sees at most 100 keys
    assert (idx[0, 20:] == -1).all() and (idx[1, 7:] == -1).all()
    assert (idx[1, :7, 0, 100:] == -1).all()
    for b in range(2):
        for t in range(int(act_q[b])):
            gs = set(x for x in ri[b, t, 0].tolist() if x >= 0)
            ts = set(x for x in idx[b, t, 0].tolist() if x >= 0)
            assert gs == ts or len(gs ^ ts) <= 2


def test_config2_rows_sample(gpu):
    # config 2 shapes; the oracle runs on a sample of query rows of the same inputs
    inp = inputs.indexer_fp8(B=1, S1=4096, S2=32768, seed=2)
    dev = {k: v.to(gpu) for k, v in inp.items()}
    print("indexer config2 full run", flush=True)
    idx, vals, logits = dsa.lightning_indexer(dev["q"], dev["k"], dev["w"], key_scale=dev["key_scale"],
                                              sparse_count=2048, return_value=True, return_logits=True)
    torch.cuda.synchronize()
    rows = [0, 1, 777, 2048, 4095]
    q = inp["q"][:, rows]
    w = inp["w"][:, rows]
    kdq = inp["k"].float() * inp["key_scale"].view(1, -1, 1, 1)
    for j, t in enumerate(rows):
        L = 32768 - 4096 + t + 1
        qk = torch.relu(torch.einsum("hd,sd->hs", q[0, j].float(), kdq[0, :L, 0]))
        ref = (w[0, j].unsqueeze(1) * qk).sum(0)
        _logit_close(logits[0, t, :L].cpu(), ref)
        ti, _ = stable_topk(logits[0, t, :L].cpu().unsqueeze(0), 2048)
        assert torch.equal(idx[0, t, 0].cpu(), ti[0])
    # every row's top-k against the stable sort of the same logits, on the GPU
    lens = 32768 - 4096 + 1 + torch.arange(4096, device=gpu)
    check_topk_rows(idx.view(4096, 2048), logits.view(4096, 32768), lens, 2048, what="config 2 top-k")


@pytest.mark.parametrize("K,mode", [(4096, 3), (8192, 3), (8192, 0)])
def test_sparse_count_above_2048_long_rows(gpu, K, mode):
    # sparse_count multiples of 1024 up to 8192 (lightning_indexer.py:1240-1241) at
    # 131072 keys: more than 2K / 16 groups reach the threshold, so the rows take
    # the streamed top-k instead of the group-maxima path; every row's indices
    # against the stable sort of the same logits, and sampled logits against the oracle
    S1, S2 = 64, 131072
    print(f"indexer sparse_count={K} mode={mode} S1={S1} S2={S2}", flush=True)
    inp = inputs.indexer_fp8(B=1, S1=S1, S2=S2, seed=K + mode, device=gpu)
    idx, _, logits = dsa.lightning_indexer(inp["q"], inp["k"], inp["w"], key_scale=inp["key_scale"],
                                           sparse_count=K, sparse_mode=mode, return_logits=True)
    torch.cuda.synchronize()
    assert tuple(idx.shape) == (1, S1, 1, K)
    lens = (S2 - S1 + 1 + torch.arange(S1, device=gpu)) if mode == 3 else None
    check_topk_rows(idx.view(S1, K), logits.view(S1, S2), lens, K, what=f"sparse_count {K}")
    kdq = inp["k"][0, :, 0].float().cpu() * inp["key_scale"][0].cpu().unsqueeze(1)
    for t in (0, S1 - 1):
        L = S2 - S1 + t + 1 if mode == 3 else S2
        qk = torch.relu(inp["q"][0, t].float().cpu() @ kdq[:L].T)
        ref = (inp["w"][0, t].cpu().unsqueeze(1) * qk).sum(0)
        _logit_close(logits[0, t, :L].cpu(), ref)


def _ragged_fp8(seed, lens_q, lens_k, D=128, H=64):
    """Ragged fp8 batches with per-key scales (the config-2 recipe per batch)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((sum(lens_q), H, D), generator=g).to(inputs.FP8)
    k32 = torch.randn((sum(lens_k), 1, D), generator=g)
    w = torch.randn((sum(lens_q), H), generator=g) / 8
    scale = torch.clamp(k32.abs().amax(dim=-1) / 448.0, min=torch.finfo(torch.float32).tiny)  # [T2, 1]
    k = (k32 / scale.unsqueeze(-1)).to(inputs.FP8)
    return q, k, w, scale.view(-1)


def _cum(lens):
    return torch.tensor([sum(lens[:i + 1]) for i in range(len(lens))], dtype=torch.int32)


@pytest.mark.parametrize("mode", [3, 0])
def test_tnd_layout(gpu, mode):
    # TND query and key (varlen rows read in place); reference layout contract
    # lightning_indexer.py:48-84,111-150,1256-1262,1365-1368
    lens_q, lens_k, K = [40, 0, 17, 64], [2500, 300, 1024, 4000], 256
    q, k, w, ks = _ragged_fp8(31 + mode, lens_q, lens_k)
    print(f"indexer TND lens_q={lens_q} lens_k={lens_k} mode={mode}", flush=True)
    cq, ck = _cum(lens_q), _cum(lens_k)
    idx, vals, logits = dsa.lightning_indexer(q.to(gpu), k.to(gpu), w.to(gpu), key_scale=ks.to(gpu),
                                              actual_seq_lengths_query=cq.to(gpu), actual_seq_lengths_key=ck.to(gpu),
                                              layout_query="TND", layout_key="TND", sparse_count=K,
                                              sparse_mode=mode, return_value=True, return_logits=True)
    torch.cuda.synchronize()
    assert idx.shape == (sum(lens_q), 1, K) and logits.shape == (sum(lens_q), max(lens_k))
    ri, rscores, rv = ref_indexer(q, k, w, key_scale=ks, actual_seq_lengths_query=cq, actual_seq_lengths_key=ck,
                                  layout_query="TND", layout_key="TND", sparse_count=K, sparse_mode=mode)
    logits, idx = logits.cpu(), idx.cpu()
    row = 0
    for b, (aq, ak) in enumerate(zip(lens_q, lens_k)):
        for t in range(aq):
            ref = rscores[b, 0, t, :ak]
            n = int(torch.isfinite(ref).sum())
            _logit_close(logits[row, :n].unsqueeze(0), ref[:n].unsqueeze(0))
            ti, _ = stable_topk(logits[row, :n].unsqueeze(0), K)
            assert torch.equal(idx[row, 0], ti[0]), (b, t)
            row += 1


@pytest.mark.parametrize("block_size", [16, 64, 128])
def test_paged_keys_match_contiguous(gpu, block_size):
    # PA_BSND keys through a shuffled block table (lightning_indexer.py:271-292):
    # identical inputs laid out contiguously give bit-identical logits and indices
    B, S1, S2, K = 3, 20, 3000, 512
    inp = inputs.indexer_fp8(B=B, S1=S1, S2=S2, seed=40 + block_size)
    lens_k = torch.tensor([3000, 1234, 2049], dtype=torch.int32)
    g = torch.Generator().manual_seed(block_size)
    nb = (S2 + block_size - 1) // block_size
    nblocks = B * nb + 5
    perm = torch.randperm(nblocks, generator=g)
    pool = torch.zeros((nblocks, block_size, 1, 128), dtype=torch.uint8).view(inputs.FP8)
    pscale = torch.ones((nblocks, block_size))
    bt = torch.full((B, nb + 1), -1, dtype=torch.int32)
    kf = inp["k"].view(torch.uint8)
    for b in range(B):
        for j in range(nb):
            page = int(perm[b * nb + j])
            bt[b, j] = page
            lo, hi = j * block_size, min(S2, (j + 1) * block_size)
            pool.view(torch.uint8)[page, :hi - lo] = kf[b, lo:hi]
            pscale[page, :hi - lo] = inp["key_scale"][b, lo:hi]
    print(f"indexer PA block_size={block_size}", flush=True)
    d = {k: v.to(gpu) for k, v in inp.items()}
    ic, vc, lc = dsa.lightning_indexer(d["q"], d["k"], d["w"], key_scale=d["key_scale"],
                                       actual_seq_lengths_key=lens_k.to(gpu), sparse_count=K,
                                       return_value=True, return_logits=True)
    ip, _, lp = dsa.lightning_indexer(d["q"], pool.to(gpu), d["w"], key_scale=pscale.to(gpu),
                                      actual_seq_lengths_key=lens_k.to(gpu), block_table=bt.to(gpu),
                                      layout_key="PA_BSND", sparse_count=K, return_logits=True)
    torch.cuda.synchronize()
    assert torch.equal(ip.cpu(), ic.cpu())
    # and against the oracle run on the paged layout itself
    ri, rs, _ = ref_indexer(inp["q"], pool, inp["w"], key_scale=pscale, actual_seq_lengths_key=lens_k,
                            block_table=bt, layout_key="PA_BSND", sparse_count=K)
    lp, lc = lp.cpu(), lc.cpu()
    for b in range(B):
        for t in range(S1):
            n = int(torch.isfinite(rs[b, 0, t]).sum())  # keys row t sees (unseen ones are not written)
            assert torch.equal(lp[b, t, :n], lc[b, t, :n]), (b, t)
            _logit_close(lp[b, t, :n], rs[b, 0, t, :n])
            gs = set(x for x in ri[b, t, 0].tolist() if x >= 0)
            ts = set(x for x in ic.cpu()[b, t, 0].tolist() if x >= 0)
            assert len(gs ^ ts) <= 2, (b, t)


def test_tnd_query_with_paged_keys(gpu):
    # decode-like: one or a few query rows per sequence (TND) over paged fp8 caches
    lens_q, lens_k, K, bs = [1, 1, 3, 1], [5000, 70, 2048, 9000], 2048, 64
    q, k, w, ks = _ragged_fp8(77, lens_q, lens_k)
    nbs = [(x + bs - 1) // bs for x in lens_k]
    nblocks = sum(nbs) + 2
    g = torch.Generator().manual_seed(3)
    perm = torch.randperm(nblocks, generator=g)
    pool = torch.zeros((nblocks, bs, 1, 128), dtype=torch.uint8)
    pscale = torch.ones((nblocks, bs))
    bt = torch.full((4, max(nbs)), -1, dtype=torch.int32)
    kf, off, pi = k.view(torch.uint8), 0, 0
    for b, ak in enumerate(lens_k):
        for j in range(nbs[b]):
            page = int(perm[pi]); pi += 1
            bt[b, j] = page
            lo, hi = j * bs, min(ak, (j + 1) * bs)
            pool[page, :hi - lo] = kf[off + lo:off + hi]
            pscale[page, :hi - lo] = ks[off + lo:off + hi]
        off += ak
    pool = pool.view(inputs.FP8)
    cq = _cum(lens_q)
    print("indexer TND query + PA keys", flush=True)
    idx, _, logits = dsa.lightning_indexer(q.to(gpu), pool.to(gpu), w.to(gpu), key_scale=pscale.to(gpu),
                                           actual_seq_lengths_query=cq.to(gpu),
                                           actual_seq_lengths_key=torch.tensor(lens_k).to(gpu),
                                           block_table=bt.to(gpu), layout_query="TND", layout_key="PA_BSND",
                                           sparse_count=K, return_logits=True)
    torch.cuda.synchronize()
    ri, rscores, _ = ref_indexer(q, pool, w, key_scale=pscale, actual_seq_lengths_query=cq,
                                 actual_seq_lengths_key=torch.tensor(lens_k), block_table=bt,
                                 layout_query="TND", layout_key="PA_BSND", sparse_count=K)
    logits, idx = logits.cpu(), idx.cpu()
    row = 0
    for b, (aq, ak) in enumerate(zip(lens_q, lens_k)):
        for t in range(aq):
            ref = rscores[b, 0, t, :ak]
            n = int(torch.isfinite(ref).sum())
            _logit_close(logits[row, :n].unsqueeze(0), ref[:n].unsqueeze(0))
            ti, _ = stable_topk(logits[row, :n].unsqueeze(0), K)
            assert torch.equal(idx[row, 0], ti[0]), (b, t)
            row += 1


@pytest.mark.parametrize("S2,mode", [(131072, 3), (70000, 0)])
def test_long_rows_group_max_selection(gpu, S2, mode):
    # rows of >= 2 K groups of 16 keys: the indexer emits the group maxima and the
    # top-k reads only the groups that can hold a top-K key; the indices equal the
    # stable top-k of the same GPU logits (and the logits-only + plain top-k run)
    inp = inputs.indexer_fp8(B=1, S1=24, S2=S2, seed=S2 + mode)
    d = {k: v.to(gpu) for k, v in inp.items()}
    print(f"indexer long rows S2={S2} mode={mode}", flush=True)
    idx, vals, logits = dsa.lightning_indexer(d["q"], d["k"], d["w"], key_scale=d["key_scale"], sparse_count=2048,
                                              sparse_mode=mode, return_value=True, return_logits=True)
    torch.cuda.synchronize()
    lg = logits.cpu().view(24, S2)
    L = torch.tensor([S2 - 24 + t + 1 if mode == 3 else S2 for t in range(24)], dtype=torch.int32)
    ti, tv = stable_topk(lg, 2048, row_len=L)
    assert torch.equal(idx.cpu().view(24, -1), ti)
    assert torch.equal(vals.cpu().view(24, -1), tv)
    # a few rows' logits against the oracle
    kdq = inp["k"].float() * inp["key_scale"].view(1, -1, 1, 1)
    for t in (0, 23):
        n = int(L[t])
        qk = torch.relu(torch.einsum("hd,sd->hs", inp["q"][0, t].float(), kdq[0, :n, 0]))
        ref = (inp["w"][0, t].unsqueeze(1) * qk).sum(0)
        _logit_close(lg[t, :n], ref)


def test_full_length_key_chunks(gpu):
    # 2048 query rows x 140000 keys: 128 token blocks keep the longest key chunk
    # (131072 keys; two chunks per block, the second of 8928 keys), so a workgroup
    # runs 2048 tiles and every row crosses a chunk boundary.  Logits of the first,
    # a middle and the last row against the oracle; every row's indices (the
    # group-maxima top-k) against the stable sort of the kernel's own logits.
    S1, S2, K = 2048, 140000, 2048
    q_start = S2 - S1
    inp = inputs.indexer_fp8(B=1, S1=S1, S2=S2, seed=140, device=gpu)
    print(f"indexer full-length chunks S1={S1} S2={S2}", flush=True)
    idx, _, logits = dsa.lightning_indexer(inp["q"], inp["k"], inp["w"], key_scale=inp["key_scale"],
                                           sparse_count=K, sparse_mode=3, return_logits=True)
    torch.cuda.synchronize()
    kdq = inp["k"][0, :, 0].float().cpu() * inp["key_scale"][0].cpu().unsqueeze(1)
    for t in (0, 1100, S1 - 1):
        n = q_start + t + 1
        qk = torch.relu(inp["q"][0, t].float().cpu() @ kdq[:n].T)
        ref = (inp["w"][0, t].cpu().unsqueeze(1) * qk).sum(0)
        _logit_close(logits[0, t, :n].cpu().unsqueeze(0), ref.unsqueeze(0))
    check_topk_rows(idx.view(S1, K), logits.view(S1, S2), q_start + 1 + torch.arange(S1, device=gpu), K,
                    chunk=64, what="full-length chunks top-k")


def test_group_maxima_are_exact(gpu):
    # the indexer's 16-key group maxima equal the maxima of the logits it wrote
    # (every group that holds a visible key; -inf past a row's causal length)
    from dsa import _lib
    S1, S2 = 24, 4100
    inp = inputs.indexer_fp8(B=1, S1=S1, S2=S2, seed=77)
    d = {k: v.to(gpu) for k, v in inp.items()}
    ng = (S2 + 15) // 16
    logits = torch.empty((S1, S2), device=gpu)
    rl = torch.empty((S1,), dtype=torch.int32, device=gpu)
    gm = torch.full((S1, ng), float("nan"), device=gpu)
    print("indexer group maxima", flush=True)
    _lib.check(_lib.lib().dsa_indexer_logits_fp8_group_max(
        d["q"].data_ptr(), d["k"].data_ptr(), d["key_scale"].data_ptr(), d["w"].data_ptr(), None, None, 1, S1, S2,
        64, 128, 3, logits.data_ptr(), S2, rl.data_ptr(), gm.data_ptr(), ng,
        torch.cuda.current_stream().cuda_stream), "group max")
    torch.cuda.synchronize()
    lg, gm, rl = logits.cpu(), gm.cpu(), rl.cpu()
    for t in range(S1):
        L = int(rl[t])
        row = torch.full((ng * 16,), float("-inf"))
        row[:L] = lg[t, :L]
        want = row.view(ng, 16).amax(dim=1)
        n = (L + 15) // 16
        assert torch.equal(gm[t, :n], want[:n]), t


def test_varlen_long_rows_use_group_maxima(gpu):
    # TND rows over prefix-summed keys long enough (>= 2 K groups of 16) for the
    # fused selection; indices equal the stable top-k of the GPU's own logits
    lens_q, lens_k, K = [3, 2], [70000, 66000], 2048
    q, k, w, ks = _ragged_fp8(91, lens_q, lens_k)
    cq, ck = _cum(lens_q), _cum(lens_k)
    print("indexer varlen long rows", flush=True)
    idx, vals, logits = dsa.lightning_indexer(q.to(gpu), k.to(gpu), w.to(gpu), key_scale=ks.to(gpu),
                                              actual_seq_lengths_query=cq.to(gpu), actual_seq_lengths_key=ck.to(gpu),
                                              layout_query="TND", layout_key="TND", sparse_count=K, sparse_mode=3,
                                              return_value=True, return_logits=True)
    torch.cuda.synchronize()
    logits, idx, vals = logits.cpu(), idx.cpu(), vals.cpu()
    row = 0
    for b, (aq, ak) in enumerate(zip(lens_q, lens_k)):
        for t in range(aq):
            n = ak - aq + t + 1
            ti, tv = stable_topk(logits[row, :n].unsqueeze(0), K)
            assert torch.equal(idx[row, 0], ti[0]) and torch.equal(vals[row, 0], tv[0]), (b, t)
            row += 1


# ---- the decode form (batch rows of at most 4 query tokens: one wave per token
# and key chunk, keys loaded straight into registers)
@pytest.mark.parametrize("B,S1,S2,mode,scaled", [(8, 1, 9000, 0, True), (8, 1, 9000, 3, False),
                                                  (2, 4, 5000, 3, True), (3, 2, 700, 0, True)])
def test_decode_form(gpu, B, S1, S2, mode, scaled):
    from dsa import _lib
    inp = inputs.indexer_fp8(B=B, S1=S1, S2=S2, seed=B * 100 + S1 + mode)
    act_k = torch.tensor([S2 - 37 * b for b in range(B)], dtype=torch.int32)
    act_q = torch.tensor([S1 - (b % S1) for b in range(B)], dtype=torch.int32)
    ks = inp["key_scale"] if scaled else None
    print(f"indexer decode form B={B} S1={S1} S2={S2} mode={mode} scaled={scaled}", flush=True)
    d = {k: v.to(gpu) for k, v in inp.items()}
    aq_d, ak_d = act_q.to(gpu), act_k.to(gpu)  # held: the launch reads them asynchronously
    ng = (S2 + 15) // 16
    logits = torch.empty((B * S1, S2), device=gpu)
    rl = torch.full((B * S1,), -7, dtype=torch.int32, device=gpu)
    gm = torch.empty((B * S1, ng), device=gpu)
    _lib.check(_lib.lib().dsa_indexer_logits_fp8_group_max(
        d["q"].data_ptr(), d["k"].data_ptr(), d["key_scale"].data_ptr() if scaled else None, d["w"].data_ptr(),
        aq_d.data_ptr(), ak_d.data_ptr(), B, S1, S2, 64, 128, mode, logits.data_ptr(), S2,
        rl.data_ptr(), gm.data_ptr(), ng, torch.cuda.current_stream().cuda_stream), "decode form")
    torch.cuda.synchronize()
    logits, rl, gm = logits.cpu(), rl.cpu(), gm.cpu()
    _, rscores, _ = ref_indexer(inp["q"], inp["k"], inp["w"], key_scale=ks, actual_seq_lengths_query=act_q,
                                actual_seq_lengths_key=act_k, sparse_count=64, sparse_mode=mode)
    for b in range(B):
        for t in range(S1):
            r = b * S1 + t
            ref = rscores[b, 0, t]
            n = int(torch.isfinite(ref).sum())
            assert int(rl[r]) == n, (b, t)  # rows past act_q: 0
            if n == 0:
                continue
            _logit_close(logits[r, :n], ref[:n])
            row = torch.full((ng * 16,), float("-inf"))
            row[:n] = logits[r, :n]
            m = (n + 15) // 16
            assert torch.equal(gm[r, :m], row.view(ng, 16).amax(dim=1)[:m]), (b, t)


def test_decode_form_shared_pool(gpu):
    # 32 single-token rows, each through its own block table onto one shared page
    # pool (the layer's decode step): bit-identical to the contiguous layout, and
    # the fused top-k equals the stable top-k of the logits
    B, S2, bs, K = 32, 20000, 64, 2048
    inp = inputs.indexer_fp8(B=1, S1=B, S2=S2, seed=123)
    q = inp["q"].view(B, 1, 64, 128)
    w = inp["w"].view(B, 1, 64)
    nb = (S2 + bs - 1) // bs
    pool = torch.zeros((nb, bs, 1, 128), dtype=torch.uint8)
    pool.view(-1, 128)[:S2] = inp["k"].view(torch.uint8).view(S2, 128)
    pscale = torch.zeros((nb, bs))
    pscale.view(-1)[:S2] = inp["key_scale"].view(-1)
    bt = torch.arange(nb, dtype=torch.int32).repeat(B, 1)
    kc = inp["k"].expand(B, S2, 1, 128).contiguous()
    kscale = inp["key_scale"].expand(B, S2).contiguous()
    print("indexer decode form, 32 rows over one shared pool", flush=True)
    # (PA_BSND takes no return_value, lightning_indexer.py:1235-1236)
    ip, _, lp = dsa.lightning_indexer(q.to(gpu), pool.view(inputs.FP8).to(gpu), w.to(gpu), key_scale=pscale.to(gpu),
                                      actual_seq_lengths_key=torch.full((B,), S2, dtype=torch.int32).to(gpu),
                                      block_table=bt.to(gpu), layout_key="PA_BSND", sparse_count=K, sparse_mode=0,
                                      return_logits=True)
    ic, vc, lc = dsa.lightning_indexer(q.to(gpu), kc.to(gpu), w.to(gpu), key_scale=kscale.to(gpu), sparse_count=K,
                                       sparse_mode=0, return_value=True, return_logits=True)
    torch.cuda.synchronize()
    lp, lc, ip, ic, vc = lp.cpu(), lc.cpu(), ip.cpu(), ic.cpu(), vc.cpu()
    assert torch.equal(lp, lc) and torch.equal(ip, ic)
    ti, tv = stable_topk(lc.view(B, S2), K)
    assert torch.equal(ic.view(B, K), ti) and torch.equal(vc.view(B, K), tv)
    # one row against the oracle
    _, rs, _ = ref_indexer(q[:1], kc[:1], w[:1], key_scale=kscale[:1], sparse_count=K, sparse_mode=0)
    _logit_close(lp[0, 0], rs[0, 0, 0])


def test_paged_long_chunks_match_contiguous(gpu):
    # enough query rows for 16384-key chunks (the paged form keeps a chunk's pool
    # rows in LDS): paged and contiguous layouts give bit-identical logits, and
    # sampled rows match the oracle
    from dsa import _lib
    B, S1, S2, bs = 4, 512, 20000, 64
    inp = inputs.indexer_fp8(B=B, S1=S1, S2=S2, seed=404)
    nb = (S2 + bs - 1) // bs
    g = torch.Generator().manual_seed(404)
    perm = torch.randperm(B * nb, generator=g)
    pool = torch.zeros((B * nb, bs, 128), dtype=torch.uint8)
    pscale = torch.zeros((B * nb, bs))
    bt = perm.view(B, nb).int().contiguous()
    kf = inp["k"].view(torch.uint8).view(B, S2, 128)
    for b in range(B):
        for j in range(nb):
            lo, hi = j * bs, min(S2, (j + 1) * bs)
            pool[bt[b, j], :hi - lo] = kf[b, lo:hi]
            pscale[bt[b, j], :hi - lo] = inp["key_scale"][b, lo:hi]
    d = {k: v.to(gpu) for k, v in inp.items()}
    pool_d, ps_d, bt_d = pool.to(gpu), pscale.to(gpu), bt.to(gpu)
    lc = torch.empty((B * S1, S2), device=gpu)
    lp = torch.empty((B * S1, S2), device=gpu)
    rl = torch.empty((B * S1,), dtype=torch.int32, device=gpu)
    rl2 = torch.empty((B * S1,), dtype=torch.int32, device=gpu)
    st = torch.cuda.current_stream().cuda_stream
    print("indexer paged long chunks", flush=True)
    L = _lib.lib()
    _lib.check(L.dsa_indexer_logits_fp8(d["q"].data_ptr(), d["k"].data_ptr(), d["key_scale"].data_ptr(), d["w"].data_ptr(),
                                        None, None, B, S1, S2, 64, 128, 3, lc.data_ptr(), S2, rl.data_ptr(), st), "contiguous")
    _lib.check(L.dsa_indexer_logits_fp8_varlen(d["q"].data_ptr(), pool_d.data_ptr(), ps_d.data_ptr(), d["w"].data_ptr(),
                                               None, 0, None, 0, bt_d.data_ptr(), bs, nb, B * nb * bs, B, S1, S2, 64, 128,
                                               3, lp.data_ptr(), S2, rl2.data_ptr(), st), "paged")
    torch.cuda.synchronize()
    lc, lp, rl = lc.cpu(), lp.cpu(), rl.cpu()
    assert torch.equal(rl, rl2.cpu())
    vis = torch.arange(S2)[None, :] < rl[:, None].long()
    assert torch.equal(lc[vis], lp[vis])
    for b, t in ((0, 0), (1, 300), (3, S1 - 1)):
        _, rs, _ = ref_indexer(inp["q"][b:b + 1, t:t + 1], inp["k"][b:b + 1, :S2 - S1 + t + 1], inp["w"][b:b + 1, t:t + 1],
                               key_scale=inp["key_scale"][b:b + 1, :S2 - S1 + t + 1], sparse_count=64, sparse_mode=0)
        n = S2 - S1 + t + 1
        assert int(rl[b * S1 + t]) == n
        _logit_close(lc[b * S1 + t, :n], rs[0, 0, 0, :n])
