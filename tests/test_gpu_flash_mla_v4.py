"""GPU parity of the DeepSeek-V4 sparse flash MLA (window + compressed KV, sinks)
against the oracle restatement of sparse_flash_mla_golden.py:56-153, under the
reference's own acceptance contract (check_result / check_lse,
sparse_flash_mla_golden.py:606-663: bf16 rtol 2^-7 / atol 1e-4 for out and
rtol 0.015 / atol 0.005 for lse, on at least 99.5 % of the elements, max
normalised error < 10), plus a bound on every element: out within 1 % of the
output range, lse within 2e-2."""
import numpy as np
import pytest
import torch

import dsa
from dsa import inputs
from oracle.dsa_oracle import sparse_flash_mla_v4, unpack_pages

pytestmark = pytest.mark.gpu


def _contract(real, expt, rtol, atol):
    real = real.detach().cpu().float().numpy().ravel()
    expt = expt.detach().cpu().float().numpy().ravel()
    ok = np.isclose(real, expt, rtol=rtol, atol=atol, equal_nan=True)
    frac = ok.mean() * 100.0
    floor = (1.0 / (1 << 14)) / 0.005
    den = np.maximum(np.maximum(np.abs(real), np.abs(expt)), floor) + 1e-9
    max_rel = float((np.abs(real - expt) / den)[~ok].max()) if (~ok).any() else 0.0
    assert frac >= 99.5, f"{frac:.3f}% within tolerance"
    assert max_rel < 10.0, f"max normalised error {max_rel}"


def _reference(case):
    cu = case["cu_seqlens_q"].tolist()
    B = len(cu) - 1
    lens = [cu[i + 1] - cu[i] for i in range(B)]
    S = max(lens)
    kvl = case["seqused_kv"].tolist()
    T, N1, D = case["q"].shape
    q_bnsd = torch.zeros((B, N1, S, D), dtype=case["q"].dtype)
    for b in range(B):
        q_bnsd[b, :, :lens[b]] = case["q"][cu[b]:cu[b + 1]].permute(1, 0, 2)
    ori = unpack_pages(case["ori_kv"], case["ori_block_table"], max(kvl))
    cmp = idx = None
    if case["cmp_kv"] is not None:
        cmp = unpack_pages(case["cmp_kv"], case["cmp_block_table"], max(max(kvl) // case["cmp_ratio"], 1))
    if case["cmp_sparse_indices"] is not None:
        K = case["cmp_sparse_indices"].shape[-1]
        idx = torch.full((B, S, 1, K), -1, dtype=torch.int32)
        for b in range(B):
            idx[b, :lens[b]] = case["cmp_sparse_indices"][cu[b]:cu[b + 1]]
    out, lse = sparse_flash_mla_v4(q_bnsd, ori, case["sinks"], act_q_lens=lens, act_kv_lens=kvl,
                                   softmax_scale=case["softmax_scale"], cmp_k_bnsd=cmp, cmp_sparse_indices=idx,
                                   cmp_ratio=case["cmp_ratio"], ori_win_left=case["ori_win_left"])
    ro = torch.cat([out[b, :, :lens[b]].permute(1, 0, 2) for b in range(B)])
    rl = torch.cat([lse[b, :, :lens[b]].permute(1, 0) for b in range(B)])
    return ro, rl


def _run(case, gpu, layout_q="TND"):
    d = lambda t: None if t is None else t.to(gpu)  # noqa: E731
    q = case["q"]
    kw = dict(ori_kv=d(case["ori_kv"]), cmp_kv=d(case["cmp_kv"]), cmp_sparse_indices=d(case["cmp_sparse_indices"]),
              ori_block_table=d(case["ori_block_table"]), cmp_block_table=d(case["cmp_block_table"]),
              seqused_kv=d(case["seqused_kv"]), sinks=d(case["sinks"]), softmax_scale=case["softmax_scale"],
              cmp_ratio=case["cmp_ratio"], ori_win_left=case["ori_win_left"], return_softmax_lse=True,
              topk_cmp=case["topk_cmp"])
    if layout_q == "TND":
        out, lse = dsa.sparse_flash_mla(q.to(gpu), cu_seqlens_q=d(case["cu_seqlens_q"]), layout_q="TND", **kw)
    else:
        B = case["cu_seqlens_q"].numel() - 1
        S = q.shape[0] // B
        ci = kw["cmp_sparse_indices"]
        if ci is not None:
            kw["cmp_sparse_indices"] = ci.view(B, S, 1, -1)
        out, lse = dsa.sparse_flash_mla(q.view(B, S, *q.shape[1:]).to(gpu), layout_q="BSND", **kw)
        out, lse = out.reshape(B * S, *out.shape[2:]), lse.reshape(B * S, -1)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


def _check(case, gpu, layout_q="TND"):
    out, lse = _run(case, gpu, layout_q)
    assert out.dtype == case["q"].dtype
    ro, rl = _reference(case)
    if case["q"].dtype == torch.bfloat16:  # check_result / check_lse, sparse_flash_mla_golden.py:606-663
        _contract(out, ro, 0.0078125, 0.0001)
        _contract(lse, rl, 0.015, 0.005)
    else:
        _contract(out, ro, 0.005, 0.000025)
        _contract(lse, rl, 0.01, 0.001)
    # and no element outside the contract's share is far off: within 1 % of the
    # output range (values here are up to 10; bf16 steps there are 2^-4)
    scale = float(ro.float().abs().max())
    assert float((out.float() - ro.float()).abs().max()) <= 1e-2 * scale
    torch.testing.assert_close(lse, rl, rtol=2e-2, atol=2e-2)


@pytest.mark.parametrize("name,scenario,cmp_ratio", [("swa", 1, 4), ("hca", 2, 128), ("csa", 3, 4)])
def test_reference_fast_scenarios(gpu, name, scenario, cmp_ratio):
    # FAST_SCENARIOS of sparse_flash_mla_golden.py:384-461: B=1, S=1024, N1=64, D=512, K=512
    case = inputs.flash_mla_v4(scenario=scenario, cmp_ratio=cmp_ratio, seed=42)
    print(f"flash mla v4 {name}", flush=True)
    _check(case, gpu)


@pytest.mark.parametrize("name,scenario,cmp_ratio", [("swa", 1, 4), ("hca", 2, 128), ("csa", 3, 4)])
def test_reference_fast_scenarios_fp16(gpu, name, scenario, cmp_ratio):
    # the same cases in fp16, the other dtype the API maps (sparse_flash_mla_api.py:16-21),
    # under check_result / check_lse's fp16 tolerances; the bf16 inputs convert exactly
    case = inputs.flash_mla_v4(scenario=scenario, cmp_ratio=cmp_ratio, seed=42)
    for k in ("q", "ori_kv", "cmp_kv"):
        if case[k] is not None:
            case[k] = case[k].to(torch.float16)
    print(f"flash mla v4 fp16 {name}", flush=True)
    _check(case, gpu)


@pytest.mark.parametrize("scenario", [1, 2, 3])
def test_varlen_batches_with_long_caches(gpu, scenario):
    # ragged TND rows over caches longer than the query chunk (prefill tails and
    # decode-like single rows), compressed ratio 4, K = 256
    case = inputs.flash_mla_v4(scenario=scenario, B=3, cu_seqlens_q=[0, 100, 101, 133],
                               seqused_kv=[700, 3001, 160], K=256, cmp_ratio=4, block_size=64, seed=7)
    print(f"flash mla v4 varlen scenario {scenario}", flush=True)
    _check(case, gpu)


def test_bsnd_layout_and_decode(gpu):
    case = inputs.flash_mla_v4(scenario=3, B=4, cu_seqlens_q=[0, 2, 4, 6, 8], seqused_kv=[8193, 4000, 130, 2],
                               K=512, cmp_ratio=4, seed=9)
    print("flash mla v4 bsnd decode", flush=True)
    _check(case, gpu, layout_q="BSND")
    _check(case, gpu, layout_q="TND")


def test_argument_checks(gpu):
    case = inputs.flash_mla_v4(scenario=1, S1=16, seed=1)
    with pytest.raises(AssertionError, match="ori_win_right"):
        dsa.sparse_flash_mla(case["q"].to(gpu), ori_kv=case["ori_kv"].to(gpu), ori_block_table=case["ori_block_table"],
                             cu_seqlens_q=case["cu_seqlens_q"], seqused_kv=case["seqused_kv"], sinks=case["sinks"],
                             softmax_scale=0.04, ori_win_right=1)
    with pytest.raises(AssertionError, match="cu_seqlens_q"):
        dsa.sparse_flash_mla(case["q"].to(gpu), ori_kv=case["ori_kv"].to(gpu), ori_block_table=case["ori_block_table"],
                             seqused_kv=case["seqused_kv"], sinks=case["sinks"], softmax_scale=0.04)
    with pytest.raises(ValueError, match="N1=64"):
        q = case["q"][:, :32].contiguous()
        dsa.sparse_flash_mla(q.to(gpu), ori_kv=case["ori_kv"].to(gpu), ori_block_table=case["ori_block_table"],
                             cu_seqlens_q=case["cu_seqlens_q"], seqused_kv=case["seqused_kv"], sinks=case["sinks"][:32],
                             softmax_scale=0.04)
