"""The quantisation oracle, pinned without a GPU: the reference golden's own
formula and tolerance (examples/deepseek_v4/act_quant.py:110-163), closed-form
properties, and torch's float8 conversion checked against a brute-force
nearest-even search over the e4m3fn grid."""
import math

import torch

from oracle.dsa_oracle import (act_quant_int8, fp8_e4m3fn_nearest, indexer_q_quant_fp8, indexer_scores,
                               pow2_ceil, quant_fp8_rows)


def _golden_int8(x, round_scale):
    # the golden's expression as act_quant.py:125-140 writes it (torch log2 for round_scale)
    x2 = x.float()
    amax = torch.clamp(x2.abs().amax(dim=1, keepdim=True), min=1e-4)
    s = 2 ** torch.ceil(torch.log2(amax / 127.0)) if round_scale else amax / 127.0
    return torch.round(torch.clamp(x2 / s, -127, 127)).to(torch.float16).to(torch.int8), s


def test_int8_matches_golden_formula_and_reference_tolerance():
    g = torch.Generator().manual_seed(0)
    x = torch.randn((128, 1024), generator=g).to(torch.bfloat16)  # the reference test's shape (:153-163)
    for rs in (False, True):
        y, s = act_quant_int8(x, round_scale=rs)
        gy, gs = _golden_int8(x, rs)
        assert torch.equal(y, gy) and torch.equal(s, gs)
        torch.testing.assert_close(y, gy, rtol=1e-2, atol=1)


def test_int8_properties():
    g = torch.Generator().manual_seed(1)
    x = (torch.randn((64, 256), generator=g) * torch.rand((64, 1), generator=g) * 10).to(torch.bfloat16)
    x[3] = 0
    y, s = act_quant_int8(x)
    xf = x.float()
    # the row maximum maps to +-127, every element within half a step
    am = xf.abs().argmax(dim=1)
    live = xf.abs().amax(dim=1) > 1e-4
    assert (y.abs().gather(1, am.view(-1, 1)).view(-1)[live] == 127).all()
    assert ((xf - y.float() * s).abs() <= s / 2 + xf.abs() * 1e-6).all()
    assert (y[3] == 0).all() and math.isclose(float(s[3]), 1e-4 / 127, rel_tol=1e-6)
    # ties round half to even: a row scaled so that x / s lands on k + 0.5
    r = torch.tensor([[127.0, 0.5, 1.5, 2.5, -0.5, -1.5, 126.5, 3.5]])
    yr, sr = act_quant_int8(r)
    assert float(sr) == 1.0
    assert yr[0].tolist() == [127, 0, 2, 2, 0, -2, 126, 4]


def test_pow2_ceil_bounds_and_golden():
    g = torch.Generator().manual_seed(2)
    v = torch.exp(torch.randn(10000, generator=g) * 10)
    p = pow2_ceil(v)
    assert ((p >= v) & (p / 2 < v)).all()
    assert torch.equal(torch.log2(p), torch.round(torch.log2(p)))  # powers of two
    # exact powers of two map to themselves
    e = torch.ldexp(torch.ones(40), torch.arange(-20, 20))
    assert torch.equal(pow2_ceil(e), e)
    # agrees with the golden's 2 ** ceil(log2 v) away from the fp32-log2 rounding band
    far = (v / (2 ** torch.floor(torch.log2(v))) - 1).abs() > 1e-5
    assert torch.equal(p[far], (2 ** torch.ceil(torch.log2(v)))[far])


def test_fp8_conversion_is_nearest_even_for_every_bf16_in_range():
    bits = torch.arange(0, 1 << 16, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    v = bits.float()
    v = v[torch.isfinite(v) & (v.abs() <= 448)]
    got = v.to(torch.float8_e4m3fn).view(torch.uint8)
    ref = fp8_e4m3fn_nearest(v).view(torch.uint8)
    assert torch.equal(got, ref)


def test_fp8_rows_properties():
    g = torch.Generator().manual_seed(3)
    x = (torch.randn((50, 128), generator=g) * torch.exp(torch.randn((50, 1), generator=g) * 5)).to(torch.bfloat16)
    x[7] = 0
    y, s = quant_fp8_rows(x)
    xf = x.float()
    live = xf.abs().amax(dim=1) > 0
    am = xf.abs().argmax(dim=1)
    assert (y.float().abs().gather(1, am.view(-1, 1)).view(-1)[live] == 448).all()
    assert float(s[7]) == torch.finfo(torch.float32).tiny and (y[7].float() == 0).all()
    # dequantised error within half an fp8 step (3 mantissa bits: 2^-4 relative), plus subnormal floor
    err = (xf - y.float() * s.unsqueeze(1)).abs()
    assert (err <= xf.abs() * 2 ** -4 + s.unsqueeze(1) * 2 ** -10).all()
    # scaling a row by a power of two leaves y alone and scales s
    y2, s2 = quant_fp8_rows((xf * 8).to(torch.bfloat16))
    assert torch.equal(y2.view(torch.uint8), y.view(torch.uint8)) and torch.equal(s2[live], s[live] * 8)


def test_q_fold_preserves_indexer_scores():
    g = torch.Generator().manual_seed(4)
    T, H, D, S2 = 6, 64, 128, 40
    q = torch.randn((T, H, D), generator=g).to(torch.bfloat16)
    w = torch.randn((T, H), generator=g) / 8
    k = torch.randn((S2, D), generator=g)
    q8, wf = indexer_q_quant_fp8(q, w)
    _, s = quant_fp8_rows(q)
    deq = q8.float() * s.unsqueeze(-1)
    a = indexer_scores(q8.float(), k, wf, T, S2, 0)
    b = indexer_scores(deq, k, w, T, S2, 0)
    torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
