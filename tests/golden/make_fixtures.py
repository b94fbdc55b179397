"""Writes the golden fixtures of this directory (run from the repo root:
``python tests/golden/make_fixtures.py``).

The reference holds no vector files: every reference test regenerates its
expectations from seeded inputs.  These fixtures freeze small seeded cases with
expectations computed here by brute force -- explicit loops in float64, written
independently of ``oracle/`` -- from the reference's definitions:

* top-k:   ``argsort(-score, stable=True)[:K]``, values <= -1e30 -> -1, -1 padding
           (examples/deepseek_v4/lightning_indexer.py:316-325), including the
           reference's own known answers (arange N=51, K=10 -> 50..41 and the
           arange N=131 full sort; testing/python/language/
           test_tilelang_ascend_language_elementwise.py:4059-4086,4218-4248);
* indexer: ``Σ_h w·ReLU(q_h·k_s)·scale_s`` with the right-down causal mask
           (lightning_indexer.py:303-314);
* sparse MLA: softmax over the selected rows with P rounded to bf16 before PV
           and ``lse = m + ln Σ`` (examples/sparse_flash_attention/
           example_sparse_flash_attn.py:255-292; examples/deepseek_v4/
           sparse_flash_mla/sparse_flash_mla_golden.py:143-149).

Arrays are stored with numpy (no pickles): bf16 as uint16 bit patterns, fp8 e4m3
as uint8 bit patterns.
"""

from __future__ import annotations

import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def _bf16_bits(t: torch.Tensor) -> np.ndarray:
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def _bf16_round(x: float) -> float:
    return float(torch.tensor(x, dtype=torch.float32).to(torch.bfloat16).to(torch.float32))


def _brute_topk(row, k, L=None, pad_invalid=True):
    n = len(row) if L is None else min(L, len(row))
    order = sorted(range(n), key=lambda i: (-row[i], i))
    idx = [-1] * k
    val = [-math.inf] * k
    for p, i in enumerate(order[:k]):
        val[p] = row[i]
        idx[p] = -1 if (pad_invalid and row[i] <= -1e30) else i
    return idx, val


def topk_fixture(path):
    rows, lens, K = [], [], 131  # K = 131: the arange N=131 row is fully sorted
    N = 300
    g = torch.Generator().manual_seed(11)
    # 0: the reference's known answer, arange N=51 (first 51 columns), K=10 -> 50..41
    r = [-math.inf] * N
    r[:51] = [float(i) for i in range(51)]
    rows.append(r); lens.append(51)
    # 1: arange N=131 (full descending sort is the reference's test_sort answer)
    r = [-math.inf] * N
    r[:131] = [float(i) for i in range(131)]
    rows.append(r); lens.append(131)
    # 2: heavy ties: values from a set of 5
    rows.append([float(v) for v in torch.randint(0, 5, (N,), generator=g).tolist()]); lens.append(N)
    # 3: +0.0 / -0.0 ties mixed with negatives
    r = [0.0 if i % 3 == 0 else (-0.0 if i % 3 == 1 else -1.0 - i) for i in range(N)]
    rows.append(r); lens.append(N)
    # 4: fewer than K valid entries (rest -inf / <= -1e30)
    r = [-math.inf] * N
    for i in range(0, N, 11):
        r[i] = float(torch.randn(1, generator=g))
    r[5] = -2e30
    rows.append(r); lens.append(N)
    # 5: a short row (row_len 40 < K) of random values
    rows.append(torch.randn(N, generator=g).tolist()); lens.append(40)
    # 6, 7: random rows, full length
    for _ in range(2):
        rows.append(torch.randn(N, generator=g).tolist()); lens.append(N)
    x = np.asarray(rows, dtype=np.float32)
    idx = np.zeros((len(rows), K), np.int32)
    val = np.zeros((len(rows), K), np.float32)
    for r in range(len(rows)):
        a, b = _brute_topk([float(v) for v in x[r]], K, lens[r])
        idx[r], val[r] = a, b
    np.savez(path, x=x, row_len=np.asarray(lens, np.int32), k=np.int32(K), indices=idx, values=val)


def indexer_fixture(path):
    B, S1, S2, N1, D, K = 1, 8, 300, 64, 128, 64
    g = torch.Generator().manual_seed(12)
    q = torch.randn((B, S1, N1, D), generator=g).to(torch.float8_e4m3fn)
    k32 = torch.randn((B, S2, D), generator=g)
    scale = k32.abs().amax(-1) / 448.0
    k8 = (k32 / scale.unsqueeze(-1)).to(torch.float8_e4m3fn)
    w = torch.randn((B, S1, N1), generator=g) / 8
    qf = q.to(torch.float64).numpy()
    kf = k8.to(torch.float64).numpy()
    sc = scale.to(torch.float64).numpy()
    wf = w.to(torch.float64).numpy()
    logits = np.full((B, S1, S2), -np.inf, np.float64)
    for t in range(S1):
        vis = S2 - S1 + t + 1  # right-down causal, aq = S1, ak = S2
        for s in range(vis):
            acc = 0.0
            for h in range(N1):
                d = float(np.dot(qf[0, t, h], kf[0, s]))
                acc += wf[0, t, h] * max(d, 0.0)
            logits[0, t, s] = acc * sc[0, s]
    lg32 = logits.astype(np.float32)
    idx = np.zeros((B, S1, K), np.int32)
    for t in range(S1):
        a, _ = _brute_topk([float(v) for v in lg32[0, t]], K)
        idx[0, t] = a
    np.savez(path, q=q.view(torch.uint8).numpy(), k=k8.view(torch.uint8).numpy(),
             key_scale=scale.numpy().astype(np.float32), weights=w.numpy().astype(np.float32),
             logits=lg32, indices=idx, sparse_count=np.int32(K))


def mla_fixture(path):
    B, S, H, DQK, DV, SKV, TOPK = 1, 4, 16, 576, 512, 96, 40
    g = torch.Generator().manual_seed(13)
    q = (torch.randn((B, S, H, DQK), generator=g) * 0.5).to(torch.bfloat16)
    kv = (torch.randn((B, SKV, 1, DQK), generator=g) * 0.5).to(torch.bfloat16)
    q_start = SKV - S
    idx = torch.full((B, S, 1, TOPK), -1, dtype=torch.int32)
    for s in range(S):
        cand = torch.randperm(q_start + s + 1, generator=g)[: TOPK - 6 + s].to(torch.int32)
        idx[0, s, 0, : cand.numel()] = cand
    idx[0, 1, 0, TOPK - 1] = SKV       # the reference's out-of-range sentinel: selects nothing
    idx[0, 2, 0, 3] = -1               # a -1 inside the list
    sm_scale = DQK ** -0.5
    qf = q.to(torch.float64).numpy()
    kvf = kv.to(torch.float64).numpy()
    out = np.zeros((B, S, H, DV), np.float64)
    lse = np.zeros((B, S, H), np.float64)
    for s in range(S):
        sel = [int(j) for j in idx[0, s, 0].tolist() if 0 <= j < SKV and j <= q_start + s]
        for h in range(H):
            sc = [sm_scale * float(np.dot(qf[0, s, h], kvf[0, j, 0])) for j in sel]
            m = max(sc)
            den = sum(math.exp(v - m) for v in sc)
            lse[0, s, h] = m + math.log(den)
            acc = np.zeros(DV, np.float64)
            for v, j in zip(sc, sel):
                p = _bf16_round(math.exp(v - m) / den)
                acc += p * kvf[0, j, 0, :DV]
            out[0, s, h] = acc
    out_bf16 = _bf16_bits(torch.from_numpy(out).to(torch.float32))
    np.savez(path, q=_bf16_bits(q), kv=_bf16_bits(kv), indices=idx.numpy(), q_start=np.int32(q_start),
             sm_scale=np.float32(sm_scale), out=out_bf16, out_f32=out.astype(np.float32),
             lse=lse.astype(np.float32))


def main():
    topk_fixture(os.path.join(HERE, "topk_small.npz"))
    indexer_fixture(os.path.join(HERE, "indexer_small.npz"))
    mla_fixture(os.path.join(HERE, "mla_small.npz"))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
