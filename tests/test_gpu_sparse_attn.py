"""GPU parity of the DeepSeek-V4 ``sparse_attn_kernel`` API (sparse attention with a
per-head sink over a contiguous [b, n, d] KV, examples/deepseek_v4/sparse_attention.py)
against the oracle's gather formulation, which restates that file's golden
(gather_sparse_kv / sparse_softmax_with_sink / sparse_attn, :171-198) with fp32
probabilities.  Tolerance: the reference test's rtol = atol = 1e-2
(examples/deepseek_v4/test_sparse_attention.py:49)."""
import pytest
import torch

import dsa
from oracle.dsa_oracle import sparse_mla_fwd_gather

pytestmark = pytest.mark.gpu


def _golden(q, kv, sink, idx, scale):
    out, _ = sparse_mla_fwd_gather(q, kv.unsqueeze(2), idx.unsqueeze(2), scale, is_causal=False, attn_sink=sink)
    return out


def _inputs(seed, b, m, n, h, d, topk):
    # the reference test's recipe (sparse_attention.py:200-206): randn q / kv in bf16,
    # randn fp32 sinks, randint(0, n) indices (repeats allowed)
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((b, m, h, d), generator=g).bfloat16()
    kv = torch.randn((b, n, d), generator=g).bfloat16()
    sink = torch.randn((h,), generator=g)
    idx = torch.randint(0, n, (b, m, topk), generator=g, dtype=torch.int32)
    return q, kv, sink, idx


def test_reference_shape(gpu):
    # test_sparse_attention.py:27-33: b=1, m=n=256, h=64, d=512, topk=128, scale d^-0.5
    b, m, n, h, d, topk = 1, 256, 256, 64, 512, 128
    q, kv, sink, idx = _inputs(42, b, m, n, h, d, topk)
    print("sparse_attn_kernel reference shape", flush=True)
    kern = dsa.sparse_attn_kernel(h=h, d=d, scale=d ** -0.5)
    got = kern(q.to(gpu), kv.to(gpu), sink.to(gpu), idx.to(gpu))
    torch.cuda.synchronize()
    assert got.dtype == torch.float32 and tuple(got.shape) == (b, m, h, d)
    torch.testing.assert_close(got.cpu(), _golden(q, kv, sink, idx, d ** -0.5), rtol=1e-2, atol=1e-2)


def test_unused_slots_and_default_scale(gpu):
    # -1 slots select nothing (gather_sparse_kv zeroes them and the score mask is
    # -inf, :171-177 and :195); a ragged top-k, two batches, 16 heads, the
    # factory's default scale d^-0.5 (:34)
    b, m, n, h, d, topk = 2, 5, 300, 16, 512, 70
    q, kv, sink, idx = _inputs(7, b, m, n, h, d, topk)
    g = torch.Generator().manual_seed(8)
    idx[torch.rand(idx.shape, generator=g) < 0.3] = -1
    idx[1, 2, 1:] = -1  # a row with a single key: out = that key's value row
    print("sparse_attn_kernel -1 slots", flush=True)
    got = dsa.sparse_attn_kernel(h=h, d=d)(q.to(gpu), kv.to(gpu), sink.to(gpu), idx.to(gpu)).cpu()
    ref = _golden(q, kv, sink, idx, d ** -0.5)
    torch.testing.assert_close(got, ref, rtol=1e-2, atol=1e-2)
    # with a sink, the single key's weight is 1 / (1 + exp(sink - score))
    j = int(idx[1, 2, 0])
    s = (q[1, 2].float() @ kv[1, j].float()) * d ** -0.5
    wgt = 1.0 / (1.0 + torch.exp(sink - s))
    torch.testing.assert_close(got[1, 2], wgt[:, None] * kv[1, j].float()[None, :], rtol=1e-2, atol=1e-2)


def test_functional_form_matches_factory(gpu):
    b, m, n, h, d, topk = 1, 3, 64, 32, 512, 16
    q, kv, sink, idx = _inputs(3, b, m, n, h, d, topk)
    args = [t.to(gpu) for t in (q, kv, sink, idx)]
    a = dsa.sparse_attn(*args, 0.05)
    c = dsa.sparse_attn_kernel(h=h, d=d, scale=0.05)(*args)
    torch.cuda.synchronize()
    assert torch.equal(a, c)
