"""Pins oracle.stable_topk (restating lightning_indexer.py:316-325) without retyping it:
brute force with Python's sorted(), the reference's known-answer tests, edge cases."""
import math

import pytest
import torch

from oracle.dsa_oracle import stable_topk


def brute_topk(row, k, pad_invalid=True):
    """Python sorted() on (-value, index); -0.0 == 0.0 compare equal in Python too."""
    order = sorted(range(len(row)), key=lambda i: (-row[i] if not math.isnan(row[i]) else math.inf, i))
    idx = [-1] * k
    val = [-math.inf] * k
    for p, i in enumerate(order[:k]):
        v = row[i]
        idx[p] = -1 if (pad_invalid and v <= -1e30) else i
        val[p] = v
    return idx, val


def _check(x, k, pad_invalid=True):
    gi, gv = stable_topk(x, k, pad_invalid=pad_invalid)
    for r in range(x.shape[0]):
        row = [float(v) for v in x[r].tolist()]
        bi, bv = brute_topk(row, k, pad_invalid)
        assert gi[r].tolist() == bi, f"row {r}"
        got = gv[r].tolist()
        for a, b in zip(got, bv):
            assert (a == b) or (math.isnan(a) and math.isnan(b)) or (math.isinf(a) and math.isinf(b))


def test_known_answer_topk_arange():
    # test_topk (testing/python/language/test_tilelang_ascend_language_elementwise.py:4218-4248):
    # arange(51), K=10 -> values 50..41, indices 50..41
    x = torch.arange(0, 51, dtype=torch.float32).reshape(1, 51)
    idx, val = stable_topk(x, 10)
    assert idx[0].tolist() == list(range(50, 40, -1))
    assert val[0].tolist() == [float(v) for v in range(50, 40, -1)]


def test_known_answer_sort_arange():
    # test_sort (:4059-4086): arange(131) sorted descending, indices follow
    x = torch.arange(0, 131, dtype=torch.float32).reshape(1, 131)
    idx, val = stable_topk(x, 131)
    assert idx[0].tolist() == list(range(130, -1, -1))
    assert val[0].tolist() == [float(v) for v in range(130, -1, -1)]


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_vs_bruteforce(seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((6, 300), generator=g)
    _check(x, 37)


def test_ties_go_to_lower_index():
    g = torch.Generator().manual_seed(5)
    x = torch.randint(-3, 4, (5, 200), generator=g).float()
    _check(x, 50)
    idx, _ = stable_topk(torch.zeros(1, 20), 5)
    assert idx[0].tolist() == [0, 1, 2, 3, 4]


def test_signed_zero_ties():
    x = torch.tensor([[-0.0, 0.0, -0.0, 1.0, 0.0]])
    idx, _ = stable_topk(x, 5)
    assert idx[0].tolist() == [3, 0, 1, 2, 4]


def test_masked_entries_become_minus_one():
    x = torch.full((2, 10), float("-inf"))
    x[0, 3] = 1.0
    x[0, 7] = 2.0
    x[1, :] = -1e31  # <= -1e30 is invalid too
    idx, val = stable_topk(x, 4)
    assert idx[0].tolist() == [7, 3, -1, -1]
    assert idx[1].tolist() == [-1, -1, -1, -1]
    idx2, _ = stable_topk(x, 4, pad_invalid=False)
    assert idx2[0].tolist() == [7, 3, 0, 1]


def test_short_rows_and_row_len():
    x = torch.arange(10, dtype=torch.float32).repeat(3, 1)
    idx, _ = stable_topk(x, 6, row_len=torch.tensor([10, 4, 0]))
    assert idx[0].tolist() == [9, 8, 7, 6, 5, 4]
    assert idx[1].tolist() == [3, 2, 1, 0, -1, -1]
    assert idx[2].tolist() == [-1] * 6
    idx, _ = stable_topk(torch.ones(1, 3), 5)
    assert idx[0].tolist() == [0, 1, 2, -1, -1]


def test_nan_sorts_last():
    x = torch.tensor([[1.0, float("nan"), 3.0, float("-inf"), 2.0]])
    idx, _ = stable_topk(x, 5, pad_invalid=False)
    assert idx[0].tolist() == [2, 4, 0, 3, 1]
