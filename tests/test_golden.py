"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_fixtures.py with brute-force loops) against the CPU oracle and,
on a GPU, against the HIP kernels called through the C ABI."""

import os

import numpy as np
import pytest
import torch

from oracle import dsa_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _bf16(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16)


def _fp8(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.copy()).view(torch.float8_e4m3fn)


# ----------------------------------------------------------------------------- CPU
def test_topk_fixture_known_answers():
    z = _load("topk_small.npz")
    # the reference's own answers (test_topk / test_sort on arange inputs)
    assert z["indices"][0, :10].tolist() == list(range(50, 40, -1))
    assert z["indices"][1, :131].tolist() == list(range(130, -1, -1))


def test_oracle_topk_vs_fixture():
    z = _load("topk_small.npz")
    idx, val = O.stable_topk(torch.from_numpy(z["x"]), int(z["k"]),
                             row_len=torch.from_numpy(z["row_len"]))
    assert torch.equal(idx, torch.from_numpy(z["indices"]))
    assert torch.equal(val, torch.from_numpy(z["values"]))


def test_oracle_indexer_vs_fixture():
    z = _load("indexer_small.npz")
    q, k = _fp8(z["q"]), _fp8(z["k"])
    B, S2, D = k.shape
    idx, scores, _ = O.lightning_indexer(q, k.view(B, S2, 1, D), torch.from_numpy(z["weights"]),
                                         key_scale=torch.from_numpy(z["key_scale"]).view(B, S2, 1),
                                         sparse_count=int(z["sparse_count"]), sparse_mode=3)
    ref = torch.from_numpy(z["logits"])
    got = scores[:, 0]
    fin = torch.isfinite(ref)
    assert torch.equal(fin, torch.isfinite(got))
    torch.testing.assert_close(got[fin], ref[fin], rtol=1e-5, atol=1e-5)
    assert torch.equal(idx[:, :, 0], torch.from_numpy(z["indices"]))


def test_oracle_mla_vs_fixture():
    z = _load("mla_small.npz")
    q, kv = _bf16(z["q"]), _bf16(z["kv"])
    idx = torch.from_numpy(z["indices"])
    for fn in ("gather", "dense"):
        if fn == "gather":
            out, lse = O.sparse_mla_fwd_gather(q, kv, idx, float(z["sm_scale"]),
                                               q_start_index_s=int(z["q_start"]), is_causal=True,
                                               p_dtype=torch.bfloat16)
            torch.testing.assert_close(lse, torch.from_numpy(z["lse"]), rtol=1e-5, atol=1e-5)
        else:
            out, lse = O.sparse_mla_fwd_dense(q, kv, idx, q_start_index_s=int(z["q_start"]),
                                              sm_scale=float(z["sm_scale"]))
            torch.testing.assert_close(lse, torch.from_numpy(z["lse"]), rtol=1e-5, atol=1e-5)
        torch.testing.assert_close(out.float(), torch.from_numpy(z["out_f32"]), rtol=2e-2, atol=2e-2)


# ----------------------------------------------------------------------------- GPU
@pytest.mark.gpu
def test_gpu_topk_vs_fixture(gpu):
    import dsa
    z = _load("topk_small.npz")
    dev = torch.device("cuda:0")
    x = torch.from_numpy(z["x"]).to(dev)
    idx, val = dsa.topk_selector(x, int(z["k"]), row_len=torch.from_numpy(z["row_len"]).to(dev),
                                 return_values=True)
    assert torch.equal(idx.cpu(), torch.from_numpy(z["indices"]))
    assert torch.equal(val.cpu(), torch.from_numpy(z["values"]))


@pytest.mark.gpu
def test_gpu_indexer_vs_fixture(gpu):
    import dsa
    z = _load("indexer_small.npz")
    dev = torch.device("cuda:0")
    q, k = _fp8(z["q"]).to(dev), _fp8(z["k"]).to(dev)
    B, S2, D = k.shape
    w = torch.from_numpy(z["weights"]).to(dev)
    ks = torch.from_numpy(z["key_scale"]).to(dev)
    logits, row_len = dsa.indexer_logits(q, k.view(B, S2, 1, D), w, key_scale=ks)
    logits, row_len = logits.cpu(), row_len.cpu()
    ref = torch.from_numpy(z["logits"])
    fin = torch.isfinite(ref)
    # logits are defined on each row's visible prefix, which is exactly where the fixture is finite
    assert torch.equal(fin.sum(-1).to(torch.int32), row_len)
    lg = logits[fin]
    r = ref[fin]
    assert torch.isfinite(lg).all()
    assert ((lg - r).abs() <= 1e-2 * r.abs() + 1e-2 * r.pow(2).mean().sqrt()).all()
    # top-k on the fixture's own logits is bit-exact
    idx = dsa.topk_selector(torch.from_numpy(z["logits"][0]).to(dev), int(z["sparse_count"]))
    assert torch.equal(idx.cpu(), torch.from_numpy(z["indices"][0]))


@pytest.mark.gpu
def test_gpu_mla_vs_fixture(gpu):
    import dsa
    z = _load("mla_small.npz")
    dev = torch.device("cuda:0")
    q, kv = _bf16(z["q"]).to(dev), _bf16(z["kv"]).to(dev)
    idx = torch.from_numpy(z["indices"]).to(dev)
    out, lse = dsa.sparse_mla_fwd(q, kv, idx, float(z["sm_scale"]),
                                  q_start_index_s=int(z["q_start"]))
    torch.testing.assert_close(out.float().cpu(), torch.from_numpy(z["out_f32"]), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(lse.cpu(), torch.from_numpy(z["lse"]), rtol=1e-3, atol=1e-3)
