"""GPU parity of the row quantisers against the oracle: bit-exact codes and
scales (integer / byte work), through the C ABI via the Python layer."""
import pytest
import torch

import dsa
from dsa import inputs
from oracle.dsa_oracle import act_quant_int8, indexer_q_quant_fp8, quant_fp8_rows

pytestmark = pytest.mark.gpu


def _bytes(t):
    return t.view(torch.uint8) if t.dtype != torch.int8 else t


@pytest.mark.parametrize("rows,cols", [(1000, 128), (37, 1024), (5, 7168), (64, 8), (3, 4104), (0, 128)])
def test_fp8_rows_bit_exact(gpu, rows, cols):
    # cols 7168 and 4104 take more steps per lane than stay in registers (re-read pass)
    print(f"quant fp8 rows={rows} cols={cols}", flush=True)
    g = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn((rows, cols), generator=g) * torch.exp(torch.randn((rows, 1), generator=g) * 6))
    x = x.to(torch.bfloat16)
    if rows > 4:
        x[1] = 0
        x[2, :] = 1e-38
        x[3, ::3] = -0.0
    y, s = dsa.quant_fp8(x.to(gpu))
    torch.cuda.synchronize()
    ry, rs = quant_fp8_rows(x)
    assert torch.equal(_bytes(y.cpu()), _bytes(ry))
    assert torch.equal(s.cpu(), rs)


def test_fp8_conversion_every_bf16_in_range(gpu):
    # rows whose maximum is 448 have scale 1, so x / s = x: every finite bf16 value
    # of magnitude <= 448 goes through the hardware conversion once
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = bits[torch.isfinite(bits.float()) & (bits.float().abs() <= 448)]
    n = v.numel()
    cols = 128
    rows = (n + cols - 2) // (cols - 1)
    x = torch.zeros((rows, cols), dtype=torch.bfloat16)
    x[:, 0] = 448.0
    flat = torch.zeros(rows * (cols - 1), dtype=torch.bfloat16)
    flat[:n] = v
    x[:, 1:] = flat.view(rows, cols - 1)
    print(f"quant fp8 conversion sweep values={n}", flush=True)
    y, s = dsa.quant_fp8(x.to(gpu))
    torch.cuda.synchronize()
    assert (s.cpu() == 1.0).all()
    assert torch.equal(_bytes(y.cpu()), _bytes(x.float().to(torch.float8_e4m3fn)))


@pytest.mark.parametrize("round_scale", [False, True])
def test_act_quant_int8_reference_case(gpu, round_scale):
    # the reference's own test (examples/deepseek_v4/act_quant.py:150-163): M, N = 128, 1024
    g = torch.Generator().manual_seed(42)
    x = torch.randn((128, 1024), generator=g).to(torch.bfloat16)
    print(f"act_quant int8 round_scale={round_scale}", flush=True)
    kern = dsa.act_quant_kernel_int8_optimized(1024, block_M=16, block_N=1024, round_scale=round_scale)
    Y, S = kern(x.to(gpu))
    torch.cuda.synchronize()
    ry, rs = act_quant_int8(x, round_scale=round_scale)
    assert torch.equal(Y.cpu(), ry) and torch.equal(S.cpu(), rs.view(-1))
    torch.testing.assert_close(Y.cpu(), ry, rtol=1e-2, atol=1)


def test_act_quant_int8_3d_and_ties(gpu):
    g = torch.Generator().manual_seed(7)
    x = (torch.randn((3, 50, 256), generator=g) * 3).to(torch.bfloat16)
    x[0, 0] = 0
    x[1, 2, :8] = torch.tensor([127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 3.5])
    x[1, 2, 8:] = 0
    y, s = dsa.act_quant(x.to(gpu))
    torch.cuda.synchronize()
    ry, rs = act_quant_int8(x)
    assert y.shape == x.shape and s.shape == (3, 50, 1)
    assert torch.equal(y.cpu(), ry) and torch.equal(s.cpu(), rs)
    assert y[1, 2, :8].cpu().tolist() == [127, 0, 2, 2, 0, -2, 126, 4]


def test_q_quant_fold(gpu):
    g = torch.Generator().manual_seed(8)
    T, H, D = 33, 64, 128
    q = (torch.randn((T, H, D), generator=g) * 3).to(torch.bfloat16)
    w = torch.randn((T, H), generator=g) / 8
    print("indexer q quant", flush=True)
    q8, wf = dsa.indexer_q_quant_fp8(q.to(gpu), w.to(gpu))
    torch.cuda.synchronize()
    rq, rw = indexer_q_quant_fp8(q, w)
    assert torch.equal(_bytes(q8.cpu()), _bytes(rq)) and torch.equal(wf.cpu(), rw)


def test_append_into_paged_cache_then_index(gpu):
    # bf16 keys -> quantise-on-append into a shuffled page pool -> the indexer on
    # PA_BSND keys gives exactly what it gives on the same keys quantised in place
    B, S1, bs, K = 2, 16, 64, 256
    lens = [1500, 700]
    g = torch.Generator().manual_seed(9)
    k = [torch.randn((n, 128), generator=g).to(torch.bfloat16) for n in lens]
    nb = [(n + bs - 1) // bs for n in lens]
    nblocks = sum(nb) + 4
    perm = torch.randperm(nblocks, generator=g)
    bt = torch.full((B, max(nb)), -1, dtype=torch.int32)
    pi = 0
    for b in range(B):
        for j in range(nb[b]):
            bt[b, j] = int(perm[pi]); pi += 1
    pool = torch.full((nblocks, bs, 1, 128), 0x7F, dtype=torch.uint8).view(torch.float8_e4m3fn).to(gpu)
    pscale = torch.full((nblocks, bs), -1.0).to(gpu)
    btg = bt.to(gpu)
    print("append keys into paged pool", flush=True)
    # append in two steps per batch (prefill, then a few decode tokens), as a cache fills
    for b in range(B):
        for lo, hi in ((0, lens[b] - 3), (lens[b] - 3, lens[b])):
            pos = torch.arange(lo, hi)
            slots = dsa.paged_slots(btg, torch.full_like(pos, b), pos, bs)
            dsa.indexer_k_append_fp8(k[b][lo:hi].to(gpu), pool, pscale, slots)
    # slots that must be dropped: -1 and past the pool
    dsa.indexer_k_append_fp8(torch.ones((2, 128), dtype=torch.bfloat16, device=gpu), pool, pscale,
                             torch.tensor([-1, nblocks * bs], device=gpu))
    torch.cuda.synchronize()
    poolc, psc = pool.cpu(), pscale.cpu()
    for b in range(B):
        ry, rs = quant_fp8_rows(k[b])
        pos = torch.arange(lens[b])
        rows = bt[b, pos // bs].long() * bs + pos % bs
        assert torch.equal(_bytes(poolc.view(-1, 128)[rows]), _bytes(ry))
        assert torch.equal(psc.view(-1)[rows], rs)
    used = torch.zeros(nblocks * bs, dtype=torch.bool)
    for b in range(B):
        pos = torch.arange(lens[b])
        used[bt[b, pos // bs].long() * bs + pos % bs] = True
    assert (_bytes(poolc.view(-1, 128)[~used]) == 0x7F).all() and (psc.view(-1)[~used] == -1.0).all()
    # the indexer reads the appended cache exactly like the contiguous quantised keys
    inp = inputs.indexer_fp8(B=B, S1=S1, S2=max(lens), seed=10)
    q, w = inp["q"].to(gpu), inp["w"].to(gpu)
    kc = torch.zeros((B, max(lens), 1, 128), dtype=torch.float8_e4m3fn)
    sc = torch.ones((B, max(lens)))
    for b in range(B):
        ry, rs = quant_fp8_rows(k[b])
        kc[b, :lens[b], 0] = ry
        sc[b, :lens[b]] = rs
    lk = torch.tensor(lens, dtype=torch.int32, device=gpu)
    ip, _ = dsa.lightning_indexer(q, pool, w, key_scale=pscale, actual_seq_lengths_key=lk, block_table=btg,
                                  layout_key="PA_BSND", sparse_count=K)
    ic, _ = dsa.lightning_indexer(q, kc.to(gpu), w, key_scale=sc.to(gpu), actual_seq_lengths_key=lk,
                                  sparse_count=K)
    torch.cuda.synchronize()
    assert torch.equal(ip.cpu(), ic.cpu())


def test_rejections(gpu):
    with pytest.raises(ValueError, match="multiple of 8"):
        dsa.quant_fp8(torch.zeros((4, 12), dtype=torch.bfloat16, device=gpu))
    with pytest.raises(ValueError, match="bfloat16"):
        dsa.act_quant(torch.zeros((4, 16), device=gpu))
    with pytest.raises(ValueError, match="slots"):
        pool = torch.zeros((2, 16, 1, 128), dtype=torch.uint8, device=gpu).view(torch.float8_e4m3fn)
        dsa.indexer_k_append_fp8(torch.zeros((3, 128), dtype=torch.bfloat16, device=gpu), pool,
                                 torch.zeros((2, 16), device=gpu), torch.zeros(2, dtype=torch.int64, device=gpu))
