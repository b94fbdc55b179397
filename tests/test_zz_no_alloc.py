"""The allocation-free sparse MLA entry point (dsa_sparse_mla_fwd_noalloc) against
dsa_sparse_mla_fwd with a caller workspace: two calls in a row on one GPU, the
second smaller, both through the C ABI; the results must be bit-identical (same
kernels, same split choice), so the fixed scratch array is shared and reused
correctly between calls."""
import pytest
import torch

import dsa
from dsa import inputs
from dsa._lib import lib

pytestmark = pytest.mark.gpu


def _noalloc(d, H=128, topk=2048):
    L = lib()
    q, pool, idx, bt, kvl = d["q"], d["kv"], d["indices"], d["block_table"], d["seq_len_kv"]
    B = q.shape[0]
    out = torch.empty((B, 1, H, 512), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, 1, H), dtype=torch.float32, device=q.device)
    st = torch.cuda.current_stream(q.device).cuda_stream
    rc = L.dsa_sparse_mla_fwd_noalloc(q.data_ptr(), pool.data_ptr(), idx.data_ptr(), bt.data_ptr(), kvl.data_ptr(),
                                      None, None, B, 1, H, 576, 512, pool.shape[0] * pool.shape[1], pool.shape[1],
                                      bt.shape[1], topk, d["sm_scale"], 0, 0, out.data_ptr(), lse.data_ptr(), st)
    assert rc == 0, L.dsa_last_error().decode()
    return out, lse


def test_noalloc_matches_workspace_entry_twice(gpu):
    L = lib()
    results = []
    for B, ctx, seed in ((16, 8192, 31), (3, 4096, 32)):  # the second call is smaller
        print(f"noalloc decode B={B} ctx={ctx}", flush=True)
        d = {k: (v.to(gpu) if torch.is_tensor(v) else v)
             for k, v in inputs.mla_decode(B=B, ctx=ctx, seed=seed).items()}
        need = L.dsa_sparse_mla_workspace_bytes(B, 1, 128, 2048, 0)
        assert 0 < need <= (64 << 20)  # these calls do use the scratch array
        o1, l1 = _noalloc(d)
        o2, l2 = dsa.sparse_mla_fwd(d["q"], d["kv"], d["indices"], d["sm_scale"], block_table=d["block_table"],
                                    seq_len_kv=d["seq_len_kv"], is_causal=False)
        torch.cuda.synchronize()
        assert torch.equal(o1.cpu(), o2.cpu()), f"out differs at B={B}"
        assert torch.equal(l1.cpu(), l2.cpu()), f"lse differs at B={B}"
        results.append(o1)
    assert results[1].shape[0] == 3


def test_noalloc_rejects_oversized_request(gpu):
    L = lib()
    # 1000 tokens x 8 splits x 128 heads of partials = 1.06 GB > the 64 MiB scratch
    rc = L.dsa_sparse_mla_fwd_noalloc(None, None, None, None, None, None, None, 1000, 1, 128, 576, 512, 4096, 0, 0,
                                      2048, 0.04, 0, 8, None, None, None)
    assert rc == 2 and b"scratch" in L.dsa_last_error()
