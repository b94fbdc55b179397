"""GPU parity of the block-sparse indexer logits (HISA second stage) against the
oracle restatement of ref_paged_block_sparse_mqa_attn
(examples/HISA/paged_block_sparse_mqa_attn_expert.py:425-468), at the reference
test's tolerance (rtol = atol = 1e-2, :561) and the indexer's logit bound
(|gpu - ref| <= 1e-2 |ref| + 1e-2 rms of the row); masked positions exactly -inf."""
import pytest
import torch

import dsa
from oracle.dsa_oracle import block_sparse_indexer_logits as ref_logits

pytestmark = pytest.mark.gpu


def _case(seed, batch, seq_len, heads, bs, topk, nblocks, max_blocks, dtype):
    # the reference test's recipe (:502-513): U(0, 1) inputs, a context length of
    # at least one block, an identity block table, random logical blocks in range
    g = torch.Generator().manual_seed(seed)
    q = torch.rand((batch, seq_len, heads, 128), generator=g).to(dtype)
    kv = torch.rand((nblocks, bs, 1, 128), generator=g).to(dtype)
    w = torch.rand((batch, seq_len, heads), generator=g).to(dtype)
    ctx = torch.randint(bs, nblocks * bs + 1, (batch,), generator=g, dtype=torch.int32)
    bt = torch.arange(max_blocks, dtype=torch.int32).unsqueeze(0).expand(batch, -1).contiguous()
    mlb = min((int(ctx.max()) + bs - 1) // bs, max_blocks)
    idx = torch.randint(0, mlb, (batch, seq_len, topk), generator=g, dtype=torch.int32)
    return q, kv, w, ctx, bt, idx


@pytest.mark.parametrize("batch,seq_len,heads,bs,topk,dtype", [
    (1, 1, 32, 128, 64, torch.float16),      # the reference's defaults (:572-580)
    (4, 2, 32, 128, 16, torch.float16),
    (2, 3, 64, 64, 8, torch.bfloat16),
    (3, 1, 16, 32, 12, torch.float16),
    # grids of >= 256 workgroups group a token's blocks four (or two) to a
    # workgroup: ragged last groups, and 256-key blocks (two tile rounds per wave)
    (64, 1, 32, 128, 13, torch.float16),
    (40, 1, 16, 64, 13, torch.bfloat16),
    (16, 4, 16, 256, 16, torch.float16),
])
def test_matches_reference(gpu, batch, seq_len, heads, bs, topk, dtype):
    nblocks, max_blocks = 64, 64
    q, kv, w, ctx, bt, idx = _case(batch * 100 + heads, batch, seq_len, heads, bs, topk, nblocks, max_blocks, dtype)
    print(f"block-sparse logits B={batch} S={seq_len} H={heads} bs={bs} topk={topk} {dtype}", flush=True)
    # the reference factory takes top-k counts divisible by 4 (:70); the direct
    # entry any count
    kern = (dsa.paged_block_sparse_mqa_attn_return_logits(batch, seq_len, nblocks, bs, topk, heads, 128, max_blocks)
            if topk % 4 == 0 else dsa.block_sparse_indexer_logits)
    T = batch * seq_len
    got = kern(q.view(T, heads, 128).to(gpu), kv.to(gpu), idx.view(T, topk).to(gpu), w.view(T, heads).to(gpu),
               ctx.to(gpu), bt.to(gpu))
    torch.cuda.synchronize()
    got = got.cpu().view(batch, seq_len, topk * bs)
    ref = ref_logits(q, kv, idx, w, ctx, bt)
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    torch.testing.assert_close(got[fin], ref[fin], rtol=1e-2, atol=1e-2)
    rms = torch.sqrt((torch.where(fin, ref, 0) ** 2).mean())
    assert ((got - ref).abs()[fin] <= 1e-2 * ref.abs()[fin] + 1e-2 * rms).all()


def test_paged_and_out_of_table_blocks(gpu):
    # a shuffled block table, a short context and block ids outside the table:
    # those blocks are entirely -inf
    g = torch.Generator().manual_seed(5)
    batch, heads, bs, topk, nblocks, max_blocks = 2, 32, 128, 8, 40, 16
    q = torch.rand((batch, 1, heads, 128), generator=g).half()
    kv = torch.rand((nblocks, bs, 1, 128), generator=g).half()
    w = torch.rand((batch, 1, heads), generator=g).half()
    ctx = torch.tensor([1000, 130], dtype=torch.int32)
    bt = torch.stack([torch.randperm(nblocks, generator=g)[:max_blocks] for _ in range(batch)]).int()
    idx = torch.randint(0, 8, (batch, 1, topk), generator=g, dtype=torch.int32)
    idx[0, 0, 3] = max_blocks + 2
    print("block-sparse logits paged / out-of-table", flush=True)
    got = dsa.block_sparse_indexer_logits(q.view(batch, heads, 128).to(gpu), kv.to(gpu), idx.view(batch, topk).to(gpu),
                                          w.view(batch, heads).to(gpu), ctx.to(gpu), bt.to(gpu))
    torch.cuda.synchronize()
    got = got.cpu()
    assert torch.isinf(got[0, 3]).all()
    keep = torch.ones(topk, dtype=torch.bool)
    keep[3] = False
    ref = ref_logits(q, kv, idx.clamp(max=max_blocks - 1), w, ctx, bt).view(batch, topk, bs)
    fin = torch.isfinite(ref)
    g0 = got[0, keep]
    assert torch.equal(torch.isfinite(g0), fin[0, keep])
    torch.testing.assert_close(g0[fin[0, keep]], ref[0, keep][fin[0, keep]], rtol=1e-2, atol=1e-2)
    assert torch.equal(torch.isfinite(got[1]), fin[1])
    torch.testing.assert_close(got[1][fin[1]], ref[1][fin[1]], rtol=1e-2, atol=1e-2)
