"""GPU parity of the top-k kernel against the oracle: bit-exact indices (and values)."""
import pytest
import torch

import dsa
from oracle.dsa_oracle import stable_topk

pytestmark = pytest.mark.gpu


def _run(x_cpu, k, gpu, row_len=None, pad_invalid=True):
    print(f"topk case rows={x_cpu.shape[0]} cols={x_cpu.shape[1]} k={k}", flush=True)
    x = x_cpu.to(gpu)
    rl = None if row_len is None else row_len.to(gpu)
    idx, val = dsa.topk_selector(x, k, row_len=rl, pad_invalid=pad_invalid, return_values=True)
    torch.cuda.synchronize()
    ri, rv = stable_topk(x_cpu, k, pad_invalid=pad_invalid, row_len=row_len)
    return idx.cpu(), val.cpu(), ri, rv


def _assert_exact(gi, gv, ri, rv):
    bad = (gi != ri).any(dim=1).nonzero().flatten().tolist()
    assert not bad, f"{len(bad)} rows differ, first {bad[:5]}"
    assert torch.equal(torch.nan_to_num(gv, neginf=-3e38), torch.nan_to_num(rv, neginf=-3e38))


@pytest.mark.parametrize("rows,cols,k", [(64, 4096, 2048), (1024, 1024, 128), (7, 333, 50),
                                         (3, 20000, 2048), (4, 32768, 2048)])
def test_random_rows(gpu, rows, cols, k):
    # shapes of example_topk_selector.py:124-141 plus the register-resident limit
    g = torch.Generator().manual_seed(rows * 7 + cols)
    x = torch.randn((rows, cols), generator=g)
    _assert_exact(*_run(x, k, gpu))


def test_streamed_long_rows(gpu):
    g = torch.Generator().manual_seed(1)
    x = torch.randn((3, 131072), generator=g)
    _assert_exact(*_run(x, 2048, gpu))


def test_streamed_ties_and_specials(gpu):
    # long rows through the sampled-threshold path where the candidate group holds
    # tie groups larger than a bucket (ordered by the bitonic fallback), NaN, +inf
    # groups and values straddling zero (value-linear buckets)
    g = torch.Generator().manual_seed(5)
    x = torch.round(torch.randn((5, 131072), generator=g) * 4) / 4
    x[1, ::7] = float("nan")
    x[2, :1000] = float("inf")
    x[3] = torch.randn(131072, generator=g) * 1e-30
    x[4] = torch.randn(131072, generator=g) - 2.1  # the K-th value sits near zero
    _assert_exact(*_run(x, 2048, gpu))
    y = torch.round(torch.randn((4, 32768), generator=g) * 8) / 8
    y[1] = torch.randn(32768, generator=g) + 0.01 * torch.arange(32768) % 3
    _assert_exact(*_run(y, 2048, gpu))


def test_known_answer_arange(gpu):
    # test_topk / test_sort (test_tilelang_ascend_language_elementwise.py:4218-4248, 4059-4086)
    x = torch.arange(0, 51, dtype=torch.float32).reshape(1, 51)
    gi, gv, _, _ = _run(x, 10, gpu)
    assert gi[0].tolist() == list(range(50, 40, -1))
    x = torch.arange(0, 131, dtype=torch.float32).reshape(1, 131)
    gi, _, _, _ = _run(x, 131, gpu)
    assert gi[0].tolist() == list(range(130, -1, -1))


def test_heavy_ties(gpu):
    g = torch.Generator().manual_seed(2)
    x = torch.randint(-2, 3, (8, 40000), generator=g).float()  # five values: every group is huge
    x[1] = 0.0
    x[2, ::2] = -0.0
    _assert_exact(*_run(x, 2048, gpu))
    x2 = torch.randint(-1, 2, (4, 9000), generator=g).float()
    _assert_exact(*_run(x2, 2048, gpu))


def test_masked_and_short_rows(gpu):
    g = torch.Generator().manual_seed(3)
    x = torch.randn((6, 5000), generator=g)
    x[0, 100:] = float("-inf")
    x[1, :] = float("-inf")
    x[2, 4000:] = -1e31
    row_len = torch.tensor([5000, 5000, 5000, 1000, 0, 2048], dtype=torch.int32)
    _assert_exact(*_run(x, 2048, gpu, row_len=row_len))
    gi, _, ri, _ = _run(x, 2048, gpu, pad_invalid=False)
    assert torch.equal(gi, ri)


def test_large_k_and_k_above_n(gpu):
    g = torch.Generator().manual_seed(4)
    x = torch.randn((3, 30000), generator=g)
    _assert_exact(*_run(x, 8192, gpu))
    x = torch.randn((2, 700), generator=g)
    _assert_exact(*_run(x, 1024, gpu))


def test_simple_topk_selector_factory(gpu):
    g = torch.Generator().manual_seed(0)
    x = torch.randn((64, 4096), generator=g)
    kern = dsa.simple_topk_selector(64, 4096, 2048, 512)
    idx = kern(x.to(gpu)).cpu()
    ref = torch.topk(x, 2048, dim=-1)[1]
    # the reference example's check (example_topk_selector.py:61-86): per-row set equality
    for r in range(64):
        assert set(idx[r].tolist()) == set(ref[r].tolist())


def _group_max(x, row_len=None):
    # exact maxima of 16-element groups within each row's length (NaN ignored,
    # -inf for groups past it), the bound the indexer emits
    R, N = x.shape
    ng = (N + 15) // 16
    pad = torch.full((R, ng * 16), float("-inf"))
    pad[:, :N] = x
    if row_len is not None:
        pad[torch.arange(ng * 16)[None, :] >= row_len[:, None].long()] = float("-inf")
    pad = torch.where(torch.isnan(pad), torch.tensor(float("-inf")), pad)
    return pad.view(R, ng, 16).amax(dim=-1).contiguous()


@pytest.mark.parametrize("cols,k", [(131072, 2048), (70001, 2048), (65536, 512), (40000, 1024)])
def test_group_max_path(gpu, cols, k):
    # the threshold from group maxima, then only the groups reaching it are read;
    # rows of fewer than 2 k groups take the streamed path: identical results
    g = torch.Generator().manual_seed(cols + k)
    x = torch.randn((6, cols), generator=g)
    x[1] = torch.round(x[1] * 4) / 4                  # tie groups
    x[2, ::5] = float("nan")
    x[3, : cols // 2] = float("-inf")                 # half the row masked
    x[4] = -x[4].abs()                                # all negative; zeros below
    x[4, 100:140] = -0.0
    x[5, 7::16] = 50.0 + torch.arange(len(range(7, cols, 16))) * 1e-3  # one large value per group
    row_len = torch.tensor([cols, cols - 5, cols, cols, cols - 17, cols], dtype=torch.int32)
    gm = _group_max(x, row_len)
    print(f"topk group-max case cols={cols} k={k}", flush=True)
    gi, gv = dsa.topk_selector(x.to(gpu), k, row_len=row_len.to(gpu), group_max=gm.to(gpu), return_values=True)
    torch.cuda.synchronize()
    ri, rv = stable_topk(x, k, row_len=row_len)
    _assert_exact(gi.cpu(), gv.cpu(), ri, rv)


def test_group_max_overflow_and_loose_bounds(gpu):
    # every group reaching the bound (a constant row): the group list overflows
    # and the exact passes decide; bounds above the true maxima stay correct
    g = torch.Generator().manual_seed(11)
    x = torch.randn((3, 131072), generator=g)
    x[0] = 1.0
    gm = _group_max(x)
    gm[1] += 0.5                                      # loose upper bounds
    gm[2, ::3] = float("inf")
    print("topk group-max overflow / loose bounds", flush=True)
    gi, gv = dsa.topk_selector(x.to(gpu), 2048, group_max=gm.to(gpu), return_values=True)
    torch.cuda.synchronize()
    ri, rv = stable_topk(x, 2048)
    _assert_exact(gi.cpu(), gv.cpu(), ri, rv)


def test_decode_shape_rows(gpu):
    # the decode step's top-k: 32 rows x 131072 logits with group maxima; random
    # rows, ties (values on a 1/8 and a 1/2 grid), short and masked rows, a row of
    # mostly equal values (its group list overflows) and a block of equal maxima,
    # all bit-exact against the stable sort
    R, N, K = 32, 131072, 2048
    g = torch.Generator().manual_seed(32)
    x = torch.randn((R, N), generator=g)
    x[1] = torch.round(x[1] * 8) / 8
    x[2, 70000:] = float("-inf")
    x[3, :] = 0.25
    x[3, ::997] = 1.0
    x[4, 5000:6000] = 3.0
    x[5] = torch.round(x[5] * 2) / 2
    row_len = torch.full((R,), N, dtype=torch.int32)
    row_len[6] = 40000
    row_len[7] = 2 * 16 * K + 3
    gm = _group_max(x, row_len)
    print("topk decode shape 32 x 131072", flush=True)
    gi, gv = dsa.topk_selector(x.to(gpu), K, row_len=row_len.to(gpu), group_max=gm.to(gpu), return_values=True)
    torch.cuda.synchronize()
    ri, rv = stable_topk(x, K, row_len=row_len)
    _assert_exact(gi.cpu(), gv.cpu(), ri, rv)
