"""GPU parity of the sparse-MLA kernel against the oracle.

Tolerances: out within bf16 atol = rtol = 2e-2, LSE
within 1e-3 (absolute and relative).  The oracle rounds the probabilities to bf16
before the PV product as sparse_flash_mla_golden.py:143 does."""
import pytest
import torch

import dsa
from dsa import inputs
from oracle.dsa_oracle import sparse_mla_fwd_dense, sparse_mla_fwd_gather

pytestmark = pytest.mark.gpu

OUT_TOL = dict(rtol=2e-2, atol=2e-2)
LSE_TOL = dict(rtol=1e-3, atol=1e-3)


def _check(inp, gpu, **kw):
    q, kv, idx = inp["q"], inp["kv"], inp["indices"]
    print(f"mla case q={tuple(q.shape)} kv={tuple(kv.shape)} topk={idx.shape[-1]} kw={kw}", flush=True)
    out, lse = dsa.sparse_mla_fwd(q.to(gpu), kv.to(gpu), idx.to(gpu), inp.get("sm_scale"),
                                  **{k: (v.to(gpu) if torch.is_tensor(v) else v) for k, v in kw.items()})
    torch.cuda.synchronize()
    ref_kw = {k: v for k, v in kw.items() if k in ("block_table", "q_start_index_s", "is_causal", "attn_sink")}
    if "seq_len_kv" in kw:
        pass  # every index in these cases is below seq_len_kv
    ro, rl = sparse_mla_fwd_gather(q, kv, idx, inp.get("sm_scale"), p_dtype=torch.bfloat16, **ref_kw)
    torch.testing.assert_close(out.float().cpu(), ro, **OUT_TOL)
    torch.testing.assert_close(lse.cpu(), rl, **LSE_TOL)
    return out.cpu(), lse.cpu()


def test_config1_small(gpu):
    inp = inputs.mla_prefill()  # config 1: B=1 S=128 Skv=4096 H=16 topk=512
    _check(inp, gpu, is_causal=True)


@pytest.mark.parametrize("splits", [1, 2, 3, 8])
def test_splits_agree(gpu, splits):
    inp = inputs.mla_prefill(B=2, S=8, Skv=2048, H=128, topk=1024, seed=11)
    _check(inp, gpu, num_splits=splits)


def test_minus_one_padding_and_sentinel(gpu):
    inp = inputs.mla_prefill(B=1, S=64, Skv=64, H=32, topk=128, seed=12, q_start=0)
    idx = inp["indices"]
    assert (idx == -1).any()
    idx[0, 5, 0, 0] = 64          # out-of-range sentinel Skv
    idx[0, 6, 0, :] = -1          # a row with nothing to attend to
    out, lse = _check(inp, gpu, is_causal=True)
    assert torch.count_nonzero(out[0, 6]) == 0 and torch.isinf(lse[0, 6]).all()


@pytest.mark.parametrize("S,topk,q_start", [(320, 256, 0), (3, 64, 0), (40, 64, 30), (24, 64, 100)])
def test_128_heads_short_causal_rows(gpu, S, topk, q_start):
    # one causal sequence through the 128-head form: the rows whose list ends in
    # -1 padding stop after their last valid key, and the short rows are dealt to
    # the XCDs apart from the long ones; holes, front padding, a row with nothing
    # valid and indices past the causal bound must all keep their meaning
    inp = inputs.mla_prefill(B=1, S=S, Skv=q_start + S, H=128, topk=topk, seed=17, q_start=q_start)
    idx = inp["indices"]
    g = torch.Generator().manual_seed(5)
    holes = torch.rand(idx.shape, generator=g) < 0.1
    idx[holes] = -1
    r = min(S - 1, 2)
    idx[0, r, 0, :] = -1                      # nothing to attend to
    if S > 10:
        row = idx[0, 9, 0].clone()
        idx[0, 9, 0, :] = -1
        idx[0, 9, 0, -4:] = row[:4]           # valid keys only at the end of the list
        idx[0, 10, 0, -1] = q_start + 11      # past the causal bound: masked
    out, lse = _check(inp, gpu, is_causal=True, q_start_index_s=q_start)
    assert torch.count_nonzero(out[0, r]) == 0 and torch.isinf(lse[0, r]).all()


def test_prefill_list_order_cases(gpu):
    # multi-token lists are gathered in index order (64 buckets of each list's
    # index range, -1 entries dropped): duplicates, a one-value list, narrow and
    # very wide ranges, holes and a lone valid entry keep their meaning, and two
    # launches give bit-identical results (the order is a function of the list)
    S, Skv, topk = 8, 200000, 512
    inp = inputs.mla_prefill(B=1, S=S, Skv=Skv, H=128, topk=topk, seed=21, q_start=Skv - S)
    g = torch.Generator().manual_seed(21)
    idx = torch.randint(0, Skv, (1, S, 1, topk), generator=g, dtype=torch.int32)
    idx[0, 1, 0] = torch.randint(0, Skv, (topk // 2,), generator=g, dtype=torch.int32).repeat(2)  # duplicates
    idx[0, 2, 0] = 777                                                        # one value, 512 times
    idx[0, 3, 0] = torch.randint(1000, 1040, (topk,), generator=g, dtype=torch.int32)  # span < 64
    idx[0, 4, 0, : topk // 2] = torch.arange(topk // 2, dtype=torch.int32)    # both ends of the range
    idx[0, 4, 0, topk // 2:] = torch.arange(Skv - topk // 2, Skv, dtype=torch.int32)
    idx[0, 5, 0, ::2] = -1                                                    # holes
    idx[0, 6, 0] = -1
    idx[0, 6, 0, topk // 2] = 4242                                            # one valid entry
    idx[0, 7] = idx[0, 7, :, torch.randperm(topk, generator=g)]               # a shuffled list
    inp["indices"] = idx
    out, lse = _check(inp, gpu, is_causal=False)
    out2, lse2 = dsa.sparse_mla_fwd(inp["q"].to(gpu), inp["kv"].to(gpu), idx.to(gpu), inp["sm_scale"],
                                    is_causal=False)
    torch.cuda.synchronize()
    assert torch.equal(out, out2.cpu()) and torch.equal(lse, lse2.cpu())
    # the one-value row: the softmax over 512 copies of one key is that key's value row
    torch.testing.assert_close(out[0, 2].float(), inp["kv"][0, 777, 0, :512].float().expand(128, 512),
                               rtol=1e-2, atol=1e-2)


def test_causal_mask_applies(gpu):
    inp = inputs.mla_prefill(B=1, S=16, Skv=512, H=16, topk=64, seed=13)
    g = torch.Generator().manual_seed(0)
    inp["indices"] = torch.randint(0, 512, (1, 16, 1, 64), generator=g, dtype=torch.int32)
    _check(inp, gpu, is_causal=True, q_start_index_s=100)
    _check(inp, gpu, is_causal=False)


def test_paged_decode_small(gpu):
    inp = inputs.mla_decode(B=4, ctx=4096, H=128, topk=512, block_size=64, seed=14)
    _check(inp, gpu, block_table=inp["block_table"], seq_len_kv=inp["seq_len_kv"], is_causal=False)


@pytest.mark.parametrize("B,topk", [(1, 2048), (1, 640), (1, 192), (1, 128), (3, 2048), (15, 1024), (8, 96)])
def test_latency_bound_decode_splits(gpu, B, topk):
    # a handful of decode rows takes the automatic split count of a latency-bound
    # launch (down to 64-key splits; a list of <= 128 keys unsplit): every row
    # against the oracle, including lists that end in -1 padding
    inp = inputs.mla_decode(B=B, ctx=8192, H=128, topk=topk, block_size=64, seed=40 + B + topk)
    inp["indices"][0, 0, 0, topk - topk // 5:] = -1
    _check(inp, gpu, block_table=inp["block_table"], seq_len_kv=inp["seq_len_kv"], is_causal=False)


def test_d512_with_sink(gpu):
    inp = inputs.mla_prefill(B=1, S=16, Skv=256, H=64, topk=128, seed=15, d_qk=512)
    g = torch.Generator().manual_seed(1)
    sink = torch.randn(64, generator=g)
    _check(inp, gpu, attn_sink=sink, is_causal=False)


@pytest.mark.parametrize("sink_value,splits,rising", [(-30.0, 1, True), (-30.0, 2, True), (2.0, 1, True),
                                                      (None, 1, True), (-30.0, 1, False), (-30.0, 2, False)])
def test_128_heads_rising_scores_with_sink(gpu, sink_value, splits, rising):
    # 128 heads (the 4-wave form) with scores that grow (or shrink) along the index
    # list, so that the reference maximum is raised in the first step (a sink far
    # below the scores) and, rising, again in later steps, with O rescaled behind
    # the P.V in flight; shrinking, the first step carries most of the weight and
    # no later step raises the reference
    inp = inputs.mla_prefill(B=1, S=4, Skv=4096, H=128, topk=2048, seed=21)
    g = torch.Generator().manual_seed(2)
    # the ramp scales the 64 rope dims only (scores move, values keep their size)
    pos = torch.arange(4096, dtype=torch.float32) / 4096
    ramp = 1.0 + 40.0 * (pos if rising else 1.0 - pos)
    kv = inp["kv"].float()
    kv[..., 512:] *= ramp.view(1, -1, 1, 1)
    inp["kv"] = kv.to(torch.bfloat16)
    inp["indices"] = torch.sort(inp["indices"], dim=-1)[0]
    kw = dict(is_causal=True, num_splits=splits)
    if sink_value is not None:
        kw["attn_sink"] = torch.full((128,), sink_value) + 0.1 * torch.randn(128, generator=g)
    _check(inp, gpu, **kw)


def test_head_count_not_multiple_of_16(gpu):
    inp = inputs.mla_prefill(B=1, S=4, Skv=300, H=20, topk=96, seed=16)
    _check(inp, gpu)


@pytest.mark.parametrize("H,topk,splits", [(64, 2048, 1), (64, 1024, 2), (96, 256, 1), (48, 512, 4)])
def test_workgroup_forms(gpu, H, topk, splits):
    # <= 64 heads: 4-wave workgroups (two per CU) unless their LDS does not fit
    # (d_qk 576 with 2048-key lists: the 128-head form with idle waves); 65-127
    # heads: the 128-head form with some waves idle; with and without splits
    inp = inputs.mla_prefill(B=1, S=6, Skv=4096, H=H, topk=topk, seed=18 + H + topk)
    _check(inp, gpu, is_causal=False, num_splits=splits)


def test_reference_factory_fp16_sentinel_convention(gpu):
    # sparse_attention_fwd pads indices with the sentinel Skv (example_sparse_flash_attn.py:303)
    inp = inputs.mla_prefill(B=1, S=32, Skv=1024, H=128, topk=256, seed=17, q_start=900)
    idx = inp["indices"].clone()
    idx[idx < 0] = 1024
    kern = dsa.sparse_attention_fwd(heads=128, dim=512, tail_dim=64, topk=256, kv_stride=1)
    out = kern(inp["q"].to(gpu), inp["kv"].to(gpu), idx.to(gpu)).float().cpu()
    ro, _ = sparse_mla_fwd_gather(inp["q"], inp["kv"], inp["indices"], None, q_start_index_s=900,
                                  is_causal=True, p_dtype=torch.bfloat16)
    torch.testing.assert_close(out, ro, **OUT_TOL)


@pytest.mark.parametrize("S,sk,kv_stride,topk", [(64, 512, 4, 128), (16, 4, 4, 64), (40, 96, 2, 64)])
def test_reference_factory_kv_stride(gpu, S, sk, kv_stride, topk):
    # compressed KV rows (kv_stride > 1): the golden's causal rule over compressed
    # positions, q_start = sk * kv_stride - S, and key 0 kept for the first
    # kv_stride - 1 rows, listed or not (example_sparse_flash_attn.py:255-292);
    # lists hold future keys, padded with the sentinel sk; row 0's list omits key 0
    # (and is full when sk > topk), the other rows list it
    g = torch.Generator().manual_seed(100 + S + kv_stride)
    q = torch.randn((1, S, 128, 576), generator=g).to(torch.bfloat16)
    kv = torch.randn((1, sk, 1, 576), generator=g).to(torch.bfloat16)
    idx = torch.full((1, S, 1, topk), sk, dtype=torch.int32)
    n = min(topk, sk)
    for t in range(S):
        if t == 0:
            perm = (torch.randperm(sk - 1, generator=g) + 1)[:n]
        else:
            perm = torch.randperm(sk, generator=g)[:n]
            if not (perm == 0).any():
                perm[0] = 0
        idx[0, t, 0, :perm.numel()] = perm.to(torch.int32)
    print(f"factory kv_stride={kv_stride} S={S} sk={sk}", flush=True)
    kern = dsa.sparse_attention_fwd(heads=128, dim=512, tail_dim=64, topk=topk, kv_stride=kv_stride)
    out = kern(q.to(gpu), kv.to(gpu), idx.to(gpu)).float().cpu()
    ro, _ = sparse_mla_fwd_dense(q, kv, idx, kv_stride=kv_stride, sm_scale=576 ** -0.5)
    torch.testing.assert_close(out, ro, **OUT_TOL)


@pytest.mark.parametrize("block_size", [64, 128])
def test_paged_prefill_per_batch_lengths(gpu, block_size):
    # paged KV for prefill with per-batch KV lengths, the reference's masked PA
    # kernel (example_sparse_flash_attn_mask_pa.py:216-236,398-426): index i of batch
    # b is valid when i != -1 and i <= kv_len[b] - S + s; the row is
    # pool[block_table[b, i // block_size], i % block_size]
    B, S, H, topk = 2, 48, 128, 512
    kv_len = [3000, 1100]
    g = torch.Generator().manual_seed(block_size)
    nb = [(n + block_size - 1) // block_size for n in kv_len]
    nblocks = sum(nb) + 3
    pool = torch.randn((nblocks, block_size, 1, 576), generator=g).to(torch.bfloat16)
    perm = torch.randperm(nblocks, generator=g)
    bt = torch.full((B, max(nb) + 1), -1, dtype=torch.int32)
    q = torch.randn((B, S, H, 576), generator=g).to(torch.bfloat16)
    idx = torch.full((B, S, 1, topk), -1, dtype=torch.int32)
    contig = torch.zeros((B, max(kv_len), 1, 576), dtype=torch.bfloat16)
    pi = 0
    for b in range(B):
        for j in range(nb[b]):
            bt[b, j] = int(perm[pi]); pi += 1
            lo, hi = j * block_size, min(kv_len[b], (j + 1) * block_size)
            contig[b, lo:hi] = pool[bt[b, j], :hi - lo]
        for t in range(S):
            vis = kv_len[b] - S + t + 1
            sel = torch.randperm(vis, generator=g)[:topk]
            idx[b, t, 0, :len(sel)] = sel.int()
    idx[0, 3, 0, 7] = kv_len[0] - S + 3 + 5   # a future index: masked by the causal rule
    print(f"mla paged prefill block_size={block_size} kv_len={kv_len}", flush=True)
    kvl = torch.tensor(kv_len, dtype=torch.int32)
    out, lse = dsa.sparse_mla_fwd(q.to(gpu), pool.to(gpu), idx.to(gpu), block_table=bt.to(gpu),
                                  seq_len_kv=kvl.to(gpu), is_causal=True)
    oc, lc = dsa.sparse_mla_fwd(q.to(gpu), contig.to(gpu), idx.to(gpu), seq_len_kv=kvl.to(gpu), is_causal=True)
    torch.cuda.synchronize()
    # the same rows in the same order: bit-identical to the contiguous layout
    assert torch.equal(out.cpu(), oc.cpu()) and torch.equal(lse.cpu(), lc.cpu())
    for b in range(B):
        ro, rl = sparse_mla_fwd_gather(q[b:b + 1], pool, idx[b:b + 1], None, block_table=bt[b:b + 1],
                                       q_start_index_s=kv_len[b] - S, is_causal=True, p_dtype=torch.bfloat16)
        torch.testing.assert_close(out[b:b + 1].float().cpu(), ro, **OUT_TOL)
        torch.testing.assert_close(lse[b:b + 1].cpu(), rl, **LSE_TOL)


@pytest.mark.parametrize("rope,T,act_q", [(True, 3, 3), (True, 4, 3), (False, 2, 2)])
def test_sparse_attn_tilelang_signature(gpu, rope, T, act_q):
    # bench_sfa.py:9-56 recipe: TND query, PA_BSND key (value = key), N(0, 0.5)
    # inputs, indices = topk of uniform noise over the first act_kv_s keys, an identity
    # block table, scale 0.5; rows past actual_seq_lengths_query are zero here
    g = torch.Generator().manual_seed(40 + T)
    N, D, Dr, bs, KV_S, act_kv, topk = 128, 512, 64, 128, 6400, 2560, 2048
    query = (torch.randn((T, N, D), generator=g) * 0.5).bfloat16()
    key = (torch.randn((KV_S // bs, bs, 1, D), generator=g) * 0.5).bfloat16()
    qr = (torch.randn((T, N, Dr), generator=g) * 0.5).bfloat16() if rope else None
    kr = (torch.randn((KV_S // bs, bs, 1, Dr), generator=g) * 0.5).bfloat16() if rope else None
    idx = torch.topk(torch.rand((T, 1, act_kv), generator=g), topk, dim=-1).indices.int()
    # padded rows past act_q hold NaN / Inf (as an uninitialised buffer may): their
    # output rows must still come back as zeros
    query[act_q:, :, 0] = float("nan")
    query[act_q:, :, 1] = float("inf")
    bt = torch.arange(KV_S // bs, dtype=torch.int32).view(1, -1)
    aq, ak = torch.tensor([act_q], dtype=torch.int32), torch.tensor([act_kv], dtype=torch.int32)
    print(f"sparse_attn_tilelang rope={rope} T={T} act_q={act_q}", flush=True)
    dv = lambda t: None if t is None else t.to(gpu)
    out = dsa.sparse_attn_tilelang(query=dv(query), key=dv(key), value=dv(key), sparse_indices=dv(idx),
                                   scale_value=0.5, sparse_block_size=1, actual_seq_lengths_query=dv(aq),
                                   actual_seq_lengths_kv=dv(ak), query_rope=dv(qr), key_rope=dv(kr),
                                   layout_query="TND", layout_kv="PA_BSND", sparse_mode=0, block_table=dv(bt),
                                   attention_mode=2)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (T, N, D) and out.dtype == torch.bfloat16
    q = torch.cat((query, qr), -1) if rope else query
    kv = torch.cat((key, kr), -1) if rope else key
    ro, _ = sparse_mla_fwd_gather(q[:act_q].unsqueeze(0), kv, idx[:act_q].unsqueeze(0), 0.5, block_table=bt,
                                  q_start_index_s=act_kv - act_q, is_causal=True, p_dtype=torch.bfloat16)
    torch.testing.assert_close(out[:act_q].float().cpu(), ro[0], **OUT_TOL)
    assert torch.equal(out[act_q:].float().cpu(), torch.zeros_like(out[act_q:].float().cpu()))


@pytest.mark.parametrize("H,splits", [(128, 1), (128, 4), (64, 2), (16, 1)])
def test_fp16_forms(gpu, H, splits):
    # fp16 q / kv through both workgroup forms (H > 64: 32-head waves; H <= 64:
    # paired 64-head workgroups), with and without split partials; the oracle
    # rounds P to fp16 as the reference golden does (p.type(v.dtype))
    inp = inputs.mla_prefill(B=2, S=8, Skv=2048, H=H, topk=1024, seed=21)
    q, kv = inp["q"].to(torch.float16), inp["kv"].to(torch.float16)
    print(f"mla fp16 H={H} splits={splits}", flush=True)
    out, lse = dsa.sparse_mla_fwd(q.to(gpu), kv.to(gpu), inp["indices"].to(gpu), inp["sm_scale"], num_splits=splits)
    torch.cuda.synchronize()
    assert out.dtype == torch.float16
    ro, rl = sparse_mla_fwd_gather(q, kv, inp["indices"], inp["sm_scale"], p_dtype=torch.float16)
    torch.testing.assert_close(out.float().cpu(), ro, **OUT_TOL)
    torch.testing.assert_close(lse.cpu(), rl, **LSE_TOL)


def test_fp16_paged_decode(gpu):
    inp = inputs.mla_decode(B=4, ctx=4096, H=128, topk=512, block_size=64, seed=22)
    q, kv = inp["q"].to(torch.float16), inp["kv"].to(torch.float16)
    print("mla fp16 paged decode", flush=True)
    out, lse = dsa.sparse_mla_fwd(q.to(gpu), kv.to(gpu), inp["indices"].to(gpu), inp["sm_scale"],
                                  block_table=inp["block_table"].to(gpu), seq_len_kv=inp["seq_len_kv"].to(gpu),
                                  is_causal=False)
    torch.cuda.synchronize()
    ro, rl = sparse_mla_fwd_gather(q, kv, inp["indices"], inp["sm_scale"], block_table=inp["block_table"],
                                   p_dtype=torch.float16)
    torch.testing.assert_close(out.float().cpu(), ro, **OUT_TOL)
    torch.testing.assert_close(lse.cpu(), rl, **LSE_TOL)


def test_mixed_dtypes_rejected(gpu):
    inp = inputs.mla_prefill(B=1, S=4, Skv=256, H=16, topk=64, seed=23)
    with pytest.raises(ValueError, match="both"):
        dsa.sparse_mla_fwd(inp["q"].to(gpu), inp["kv"].to(gpu).to(torch.float16), inp["indices"].to(gpu))

