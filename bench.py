"""Benchmark of the MI355X DSA path (one GPU).

Default workload = the full DSA layer at 128K context:
  prefill chunk: lightning indexer (fp8, 64 heads x 128) of 4096 tail queries over
                 131072 keys -> top-2048 -> sparse MLA (H=128, d_qk=576, d_v=512) on
                 the chunk with those indices;
  decode step:   32 single-token queries at position 131072 over the same cache
                 (32 block tables on one 64-token page pool) through all three kernels.
One step = both.  Inputs are synthetic (seeded), resident in HBM before timing.
Prints one JSON line.  ``value`` = sparse-MLA TFLOP/s of the prefill chunk
(2*H*topk*(576+512) FLOP per token / MLA kernel time); the indexer / top-k times
per call are reported beside it.  ``roofline`` is for the kernel with the largest
share of the step.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "tilelang-ascend_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0
PEAK_FP8_TFLOPS = 5000.0
PEAK_HBM_GBS = 8000.0
METRIC = "sparse-MLA TFLOPS (% MFMA peak) + indexer/top-k µs @H=128, topk=2048"

H, DQK, DV, TOPK, IDX_HEADS, IDX_DIM = 128, 576, 512, 2048, 64, 128


def mla_flops(tokens: int) -> float:
    return 2.0 * H * TOPK * (DQK + DV) * tokens


def indexer_flops_causal(S1: int, S2: int) -> float:
    # valid (query, key) pairs under the right-down causal mask, 2*64*128 FLOP each
    pairs = sum(S2 - S1 + t + 1 for t in range(S1))
    return 2.0 * IDX_HEADS * IDX_DIM * pairs


class Layer:
    """Preallocated buffers and C-ABI launches for one DSA layer step."""

    def __init__(self, S1: int, S2: int, dec_b: int, seed: int = 5):
        import torch
        from dsa import inputs, lib

        self.torch = torch
        self.L = lib()
        dev = torch.device("cuda:0")
        self.dev = dev
        self.S1, self.S2, self.dec_b = S1, S2, dec_b
        ix = inputs.indexer_fp8(B=1, S1=S1, S2=S2, seed=seed, device=dev)
        self.iq, self.ik, self.iw, self.iks = ix["q"], ix["k"], ix["w"], ix["key_scale"]
        g = torch.Generator(device=dev)
        g.manual_seed(seed + 100)
        self.q = (torch.randn((1, S1, H, DQK), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        self.kv = (torch.randn((1, S2, 1, DQK), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        self.logits = torch.empty((S1, S2), dtype=torch.float32, device=dev)
        self.row_len = torch.empty((S1,), dtype=torch.int32, device=dev)
        # maxima of 16-key groups, emitted by the indexer and read by the top-k
        self.ld_g = (S2 + 15) // 16
        self.gmax = torch.empty((S1, self.ld_g), dtype=torch.float32, device=dev)
        self.idx = torch.empty((1, S1, 1, TOPK), dtype=torch.int32, device=dev)
        self.out = torch.empty((1, S1, H, DV), dtype=torch.bfloat16, device=dev)
        self.lse = torch.empty((1, S1, H), dtype=torch.float32, device=dev)
        self.q_start = torch.full((1,), S2 - S1, dtype=torch.int32, device=dev)
        # decode: dec_b queries at position S2 over the same cache, paged (64-token pages)
        self.bs = 64
        self.pool = self.kv.view(S2 // self.bs, self.bs, 1, DQK)
        self.bt = torch.arange(S2 // self.bs, dtype=torch.int32, device=dev).repeat(dec_b, 1).contiguous()
        self.dq_idx = torch.randn((1, dec_b, IDX_HEADS, IDX_DIM), generator=g, device=dev).to(inputs.FP8)
        self.dw = torch.randn((1, dec_b, IDX_HEADS), generator=g, device=dev) / 8
        self.dlogits = torch.empty((dec_b, S2), dtype=torch.float32, device=dev)
        self.drow = torch.empty((dec_b,), dtype=torch.int32, device=dev)
        self.dgmax = torch.empty((dec_b, self.ld_g), dtype=torch.float32, device=dev)
        self.didx = torch.empty((dec_b, 1, 1, TOPK), dtype=torch.int32, device=dev)
        self.dq = (torch.randn((dec_b, 1, H, DQK), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        self.dout = torch.empty((dec_b, 1, H, DV), dtype=torch.bfloat16, device=dev)
        self.dlse = torch.empty((dec_b, 1, H), dtype=torch.float32, device=dev)
        self.dlen = torch.full((dec_b,), S2, dtype=torch.int32, device=dev)
        self.mla_ws_bytes = self.L.dsa_sparse_mla_workspace_bytes(1, S1, H, TOPK, 0)
        self.dec_ws_bytes = self.L.dsa_sparse_mla_workspace_bytes(dec_b, 1, H, TOPK, 0)
        self.ws = torch.empty((max(self.mla_ws_bytes, self.dec_ws_bytes, 1),), dtype=torch.uint8, device=dev)
        self.names = ["indexer", "topk", "mla", "dec_indexer", "dec_topk", "dec_mla"]
        self.stream = torch.cuda.current_stream(dev).cuda_stream

    def _chk(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {self.L.dsa_last_error().decode()}")

    def launch(self, i: int):
        L, st = self.L, self.stream
        if i == 0:
            self._chk(L.dsa_indexer_logits_fp8_group_max(
                self.iq.data_ptr(), self.ik.data_ptr(), self.iks.data_ptr(), self.iw.data_ptr(), None, None, 1,
                self.S1, self.S2, IDX_HEADS, IDX_DIM, 3, self.logits.data_ptr(), self.S2, self.row_len.data_ptr(),
                self.gmax.data_ptr(), self.ld_g, st), "indexer")
        elif i == 1:
            self._chk(L.dsa_topk_f32_group_max(self.logits.data_ptr(), self.S1, self.S2, self.S2,
                                               self.row_len.data_ptr(), self.gmax.data_ptr(), self.ld_g, TOPK, 1,
                                               self.idx.data_ptr(), None, st), "topk")
        elif i == 2:
            self._chk(L.dsa_sparse_mla_fwd(self.q.data_ptr(), self.kv.data_ptr(), self.idx.data_ptr(), None, None,
                                           self.q_start.data_ptr(), None, 1, self.S1, H, DQK, DV, self.S2, 0, 0,
                                           TOPK, DQK ** -0.5, 1, 0, self.out.data_ptr(), self.lse.data_ptr(),
                                           self.ws.data_ptr(), self.ws.numel(), st), "mla")
        elif i == 3:
            self._chk(L.dsa_indexer_logits_fp8_group_max(
                self.dq_idx.data_ptr(), self.ik.data_ptr(), self.iks.data_ptr(), self.dw.data_ptr(), None, None, 1,
                self.dec_b, self.S2, IDX_HEADS, IDX_DIM, 0, self.dlogits.data_ptr(), self.S2, self.drow.data_ptr(),
                self.dgmax.data_ptr(), self.ld_g, st), "dec_indexer")
        elif i == 4:
            self._chk(L.dsa_topk_f32_group_max(self.dlogits.data_ptr(), self.dec_b, self.S2, self.S2,
                                               self.drow.data_ptr(), self.dgmax.data_ptr(), self.ld_g, TOPK, 1,
                                               self.didx.data_ptr(), None, st), "dec_topk")
        elif i == 5:
            self._chk(L.dsa_sparse_mla_fwd(self.dq.data_ptr(), self.pool.data_ptr(), self.didx.data_ptr(),
                                           self.bt.data_ptr(), self.dlen.data_ptr(), None, None, self.dec_b, 1, H,
                                           DQK, DV, self.S2, self.bs, self.bt.shape[1], TOPK, DQK ** -0.5, 1, 0,
                                           self.dout.data_ptr(), self.dlse.data_ptr(), self.ws.data_ptr(),
                                           self.ws.numel(), st), "dec_mla")

    def step(self, events=None):
        for i in range(len(self.names)):
            if events is not None:
                events[i][0].record()
            self.launch(i)
            if events is not None:
                events[i][1].record()


def _time_launches(fn, steps: int, warmup: int = 2) -> float:
    """Mean microseconds per call of fn() on the current stream (HIP events on that stream)."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return 1e3 * sum(a.elapsed_time(b) for a, b in evs) / steps


def target_configs(L, steps: int) -> dict:
    """The single-kernel north-star shapes beside the layer step: sparse-MLA decode
    (B=64, 64K paged context) and prefill (Sq=Skv=16384), and indexer + top-k at
    32K (B=1, 4096 x 32768).  Seeded inputs generated on the GPU, resident in HBM."""
    import torch

    from dsa import inputs

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    res = {}

    def chk(rc, what):
        if rc != 0:
            raise RuntimeError(f"{what}: {L.dsa_last_error().decode()}")

    # config 3: decode, B=64, 64K context in 64-token pages, top-2048
    d = inputs.mla_decode(device=dev)
    B = d["q"].shape[0]
    out = torch.empty((B, 1, H, DV), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, 1, H), dtype=torch.float32, device=dev)
    wsb = L.dsa_sparse_mla_workspace_bytes(B, 1, H, TOPK, 0)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    bt = d["block_table"]

    def dec():
        chk(L.dsa_sparse_mla_fwd(d["q"].data_ptr(), d["kv"].data_ptr(), d["indices"].data_ptr(), bt.data_ptr(),
                                 d["seq_len_kv"].data_ptr(), None, None, B, 1, H, DQK, DV, d["kv"].shape[0] * 64,
                                 64, bt.shape[1], TOPK, DQK ** -0.5, 0, 0, out.data_ptr(), lse.data_ptr(),
                                 ws.data_ptr(), ws.numel(), st), "decode")

    us = _time_launches(dec, steps)
    dec_bytes = B * TOPK * (DQK * 2) + B * H * DQK * 2 + B * TOPK * 4 + bt.numel() * 4 + B * H * (DV * 2 + 4)
    res["decode_b64_64k"] = {"us": round(us, 2), "gbs": round(dec_bytes / us / 1e3, 1),
                             "frac_of_hbm": round(dec_bytes / us / 1e3 / PEAK_HBM_GBS, 4),
                             "algorithmic_bytes": dec_bytes}
    del d, out, lse, ws, bt
    torch.cuda.empty_cache()

    # config 4: prefill, Sq = Skv = 16384, causal index ranges, top-2048
    p = inputs.mla_prefill(B=1, S=16384, Skv=16384, H=H, topk=TOPK, seed=4, q_start=0, device=dev)
    S = p["q"].shape[1]
    out = torch.empty((1, S, H, DV), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((1, S, H), dtype=torch.float32, device=dev)
    qs = torch.zeros((1,), dtype=torch.int32, device=dev)

    def pre():
        chk(L.dsa_sparse_mla_fwd(p["q"].data_ptr(), p["kv"].data_ptr(), p["indices"].data_ptr(), None, None,
                                 qs.data_ptr(), None, 1, S, H, DQK, DV, S, 0, 0, TOPK, DQK ** -0.5, 1, 1,
                                 out.data_ptr(), lse.data_ptr(), None, 0, st), "prefill")

    us = _time_launches(pre, max(2, steps // 2))
    fl = mla_flops(S)
    res["prefill_16k"] = {"us": round(us, 1), "tflops": round(fl / us / 1e6, 1),
                          "frac_of_bf16_peak": round(fl / us / 1e6 / PEAK_BF16_TFLOPS, 4)}
    del p, out, lse
    torch.cuda.empty_cache()

    # config 2: indexer + top-k, 4096 x 32768
    S1, S2 = 4096, 32768
    ix = inputs.indexer_fp8(B=1, S1=S1, S2=S2, seed=2, device=dev)
    logits = torch.empty((S1, S2), dtype=torch.float32, device=dev)
    rl = torch.empty((S1,), dtype=torch.int32, device=dev)
    idx = torch.empty((S1, TOPK), dtype=torch.int32, device=dev)

    def ind():
        chk(L.dsa_indexer_logits_fp8(ix["q"].data_ptr(), ix["k"].data_ptr(), ix["key_scale"].data_ptr(),
                                     ix["w"].data_ptr(), None, None, 1, S1, S2, IDX_HEADS, IDX_DIM, 3,
                                     logits.data_ptr(), S2, rl.data_ptr(), st), "indexer32k")

    def tk():
        chk(L.dsa_topk_f32(logits.data_ptr(), S1, S2, S2, rl.data_ptr(), TOPK, 1, idx.data_ptr(), None, st),
            "topk32k")

    ui = _time_launches(ind, steps)
    ut = _time_launches(tk, steps)
    fi = indexer_flops_causal(S1, S2)
    tb = 4.0 * sum(S2 - S1 + t + 1 for t in range(S1)) + 4.0 * S1 * TOPK
    res["indexer_topk_32k"] = {"indexer_us": round(ui, 1), "topk_us": round(ut, 1),
                               "indexer_frac_of_fp8_peak": round(fi / ui / 1e6 / PEAK_FP8_TFLOPS, 4),
                               "topk_frac_of_hbm": round(tb / ut / 1e3 / PEAK_HBM_GBS, 4)}
    del ix, logits, rl, idx
    torch.cuda.empty_cache()

    # the fp8 producers of the indexer's operands: a 128K-token key cache and the
    # 4096-token query chunk (64 heads, scales folded into the weights); HBM bound
    g = torch.Generator(device=dev).manual_seed(6)
    kb = torch.randn((131072, IDX_DIM), generator=g, device=dev).to(torch.bfloat16)
    k8 = torch.empty(kb.shape, dtype=torch.uint8, device=dev)
    ks = torch.empty((131072,), dtype=torch.float32, device=dev)
    qb = torch.randn((4096, IDX_HEADS, IDX_DIM), generator=g, device=dev).to(torch.bfloat16)
    wq = torch.randn((4096, IDX_HEADS), generator=g, device=dev)
    q8 = torch.empty(qb.shape, dtype=torch.uint8, device=dev)
    wo = torch.empty_like(wq)

    def kq():
        chk(L.dsa_quant_fp8_rows(kb.data_ptr(), kb.shape[0], IDX_DIM, k8.data_ptr(), ks.data_ptr(), st), "kquant")

    def qq():
        chk(L.dsa_indexer_q_quant_fp8(qb.data_ptr(), wq.data_ptr(), 4096, IDX_HEADS, IDX_DIM, q8.data_ptr(),
                                      wo.data_ptr(), st), "qquant")

    uk = _time_launches(kq, steps)
    uq = _time_launches(qq, steps)
    kbytes = kb.numel() * 3 + ks.numel() * 4
    qbytes = qb.numel() * 3 + wq.numel() * 8
    del kb, k8, ks, qb, wq, q8, wo
    torch.cuda.empty_cache()
    res["indexer_decode"] = indexer_decode_configs(L, steps)
    res["flash_mla_v4"] = flash_mla_v4_configs(L, steps)
    res["block_sparse_indexer"] = block_sparse_indexer_configs(L, steps)
    res["fp8_producers"] = {"key_cache_128k_us": round(uk, 2),
                            "key_cache_frac_of_hbm": round(kbytes / uk / 1e3 / PEAK_HBM_GBS, 4),
                            "query_4096_us": round(uq, 2),
                            "query_frac_of_hbm": round(qbytes / uq / 1e3 / PEAK_HBM_GBS, 4),
                            "algorithmic_bytes": {"key_cache": kbytes, "query": qbytes}}
    return res


def indexer_decode_configs(L, steps: int) -> dict:
    """Indexer logits for a decode batch: 32 sequences x one query row x 128K keys
    each (distinct key caches, 553 MB of fp8 keys + scales), the indexer's decode
    form; HBM bound (132 B per key read once, 4 B per logit written)."""
    import torch

    from dsa import inputs

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    B, S2 = 32, 131072
    ix = inputs.indexer_fp8(B=B, S1=1, S2=S2, seed=9, device=dev)
    lg = torch.empty((B, S2), device=dev)
    rl = torch.empty((B,), dtype=torch.int32, device=dev)
    gm = torch.empty((B, S2 // 16), device=dev)

    def run():
        rc = L.dsa_indexer_logits_fp8_group_max(ix["q"].data_ptr(), ix["k"].data_ptr(), ix["key_scale"].data_ptr(),
                                                ix["w"].data_ptr(), None, None, B, 1, S2, IDX_HEADS, IDX_DIM, 0,
                                                lg.data_ptr(), S2, rl.data_ptr(), gm.data_ptr(), S2 // 16, st)
        if rc != 0:
            raise RuntimeError(L.dsa_last_error().decode())

    us = _time_launches(run, steps)
    byts = B * S2 * (IDX_DIM + 4 + 4) + B * S2 // 16 * 4
    del ix, lg, rl, gm
    torch.cuda.empty_cache()
    return {"b32_128k_distinct_us": round(us, 1), "gbs": round(byts / us / 1e3, 1),
            "frac_of_hbm": round(byts / us / 1e3 / PEAK_HBM_GBS, 4), "algorithmic_bytes": byts}


def block_sparse_indexer_configs(L, steps: int) -> dict:
    """Block-sparse indexer logits (examples/HISA/paged_block_sparse_mqa_attn_expert.py):
    the reference test's defaults (batch 1, one token, 32 heads x 128, 128-key blocks,
    top-64 blocks of a 1024-block cache), and batches of 64 and 512 tokens with the
    same shapes; HBM bound: 256 B per key read + 4 B per logit written (algorithmic
    bytes: tokens that pick the same block read it again, from L2 or HBM)."""
    import torch

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    g = torch.Generator(device=dev).manual_seed(8)
    for name, batch in (("reference_default", 1), ("decode_b64", 64), ("tokens_512", 512)):
        H, bs, topk, nb = 32, 128, 64, 1024
        q = torch.rand((batch, H, 128), generator=g, device=dev).half()
        kv = torch.rand((nb, bs, 1, 128), generator=g, device=dev).half()
        w = torch.rand((batch, H), generator=g, device=dev).half()
        ctx = torch.full((batch,), nb * bs, dtype=torch.int32, device=dev)
        bt = torch.stack([torch.randperm(nb, generator=g, device=dev) for _ in range(batch)]).int()
        idx = torch.randint(0, nb, (batch, topk), generator=g, device=dev, dtype=torch.int32)
        out = torch.empty((batch, topk, bs), dtype=torch.float32, device=dev)

        def run():
            rc = L.dsa_block_sparse_indexer_logits(q.data_ptr(), kv.data_ptr(), idx.data_ptr(), w.data_ptr(),
                                                   ctx.data_ptr(), bt.data_ptr(), batch, 1, H, 128, topk, nb, bs, nb,
                                                   0, out.data_ptr(), st)
            if rc != 0:
                raise RuntimeError(L.dsa_last_error().decode())

        us = _time_launches(run, steps)
        byts = batch * topk * bs * (256 + 4) + batch * H * 258
        res[name] = {"us": round(us, 2), "gbs": round(byts / us / 1e3, 1),
                     "frac_of_hbm": round(byts / us / 1e3 / PEAK_HBM_GBS, 4)}
    return res


def flash_mla_v4_configs(L, steps: int) -> dict:
    """DeepSeek-V4 sparse flash MLA at the reference's benchmark shapes
    (examples/deepseek_v4/sparse_flash_mla/bench_mark.md: B=1, N1=64, D=512, block 128,
    window 127, K=512, cmp_ratio 4 (swa / csa) or 128 (hca); prefill S = 8192, decode
    one row against 8193 keys).  FLOP = 4 * N1 * D per attended (row, key)."""
    import torch

    from dsa import inputs

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    for name, scen, ratio in (("swa", 1, 4), ("hca", 2, 128), ("csa", 3, 4)):
        for mode, S, kv in (("prefill", 8192, 8192), ("decode", 1, 8193)):
            c = inputs.flash_mla_v4(scenario=scen, S1=S, seqused_kv=[kv], cmp_ratio=ratio, K=512, seed=11)
            T = S
            q = c["q"].to(dev)
            ori, obt = c["ori_kv"].to(dev), c["ori_block_table"].to(dev)
            cmp = c["cmp_kv"].to(dev) if c["cmp_kv"] is not None else None
            cbt = c["cmp_block_table"].to(dev) if cmp is not None else None
            ci = c["cmp_sparse_indices"].view(T, -1).to(dev) if c["cmp_sparse_indices"] is not None else None
            n_cmp = 512 if scen == 3 else (kv // ratio if scen == 2 else 0)
            qp = torch.zeros((1,), dtype=torch.int32, device=dev)
            aq = torch.full((1,), S, dtype=torch.int32, device=dev)
            kvl = torch.full((1,), kv, dtype=torch.int32, device=dev)
            sk = c["sinks"].to(dev)
            out = torch.empty((T, 64, 512), dtype=torch.bfloat16, device=dev)
            lse = torch.empty((T, 64), dtype=torch.float32, device=dev)
            wsb = L.dsa_sparse_flash_mla_workspace_bytes(T, 64, 127, n_cmp)
            ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)

            def run():
                rc = L.dsa_sparse_flash_mla(
                    q.data_ptr(), T, 64, 512, qp.data_ptr(), aq.data_ptr(), kvl.data_ptr(), 1, ori.data_ptr(),
                    ori.shape[0], ori.shape[1], obt.data_ptr(), obt.shape[1], cmp.data_ptr() if cmp is not None else None,
                    cmp.shape[0] if cmp is not None else 0, cmp.shape[1] if cmp is not None else 0,
                    cbt.data_ptr() if cbt is not None else None, cbt.shape[1] if cbt is not None else 0,
                    ci.data_ptr() if ci is not None else None, 512 if scen == 3 else 0, n_cmp, ratio,
                    sk.data_ptr(), 0.04419417, 127, out.data_ptr(), lse.data_ptr(), ws.data_ptr(), wsb, st)
                if rc != 0:
                    raise RuntimeError(f"flash_mla_v4 {name}: {L.dsa_last_error().decode()}")

            us = _time_launches(run, max(2, steps // 2))
            keys = 0
            for s_ in range(S):
                sg = kv - S + s_
                keys += min(sg + 1, 128)
                thr = (sg + 1) // ratio
                keys += 0 if scen == 1 else (thr if scen == 2 else min(512, thr))
            fl = 4.0 * 64 * 512 * keys
            res[f"{name}_{mode}"] = {"us": round(us, 2), "tflops": round(fl / us / 1e6, 2)}
            del c, q, ori, obt, cmp, cbt, ci, out, lse, ws
    torch.cuda.empty_cache()
    return res


def cpu_baseline(S1: int, S2: int, budget_rows: int = 2048, mla_tokens: int = 4096) -> dict:
    """Time the CPU oracle on a bounded sample of the same workload and scale it."""
    import torch

    from dsa import inputs
    from oracle.dsa_oracle import indexer_scores, sparse_mla_fwd_gather, stable_topk

    threads = torch.get_num_threads()
    ix = inputs.indexer_fp8(B=1, S1=budget_rows, S2=S2, seed=5)
    k = ix["k"][0, :, 0].float() * ix["key_scale"][0].unsqueeze(1)
    t0 = time.perf_counter()
    # the sample rows are the last ones of the chunk: they see (almost) all keys
    sc = indexer_scores(ix["q"][0].float(), k, ix["w"][0], budget_rows, S2, 3)
    t1 = time.perf_counter()
    stable_topk(sc, TOPK)
    t2 = time.perf_counter()
    g = torch.Generator().manual_seed(5)
    q = (torch.randn((1, mla_tokens, H, DQK), generator=g) * 0.5).to(torch.bfloat16)
    kv = (torch.randn((1, S2, 1, DQK), generator=g) * 0.5).to(torch.bfloat16)
    idx = torch.stack([torch.randperm(S2 - S1, generator=g)[:TOPK] for _ in range(mla_tokens)]).int()
    t3 = time.perf_counter()
    sparse_mla_fwd_gather(q, kv, idx.view(1, mla_tokens, 1, TOPK), None, is_causal=False,
                          p_dtype=torch.bfloat16)
    t4 = time.perf_counter()
    scale_rows = S1 / budget_rows
    return {
        "value": mla_flops(mla_tokens) / (t4 - t3) / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (torch CPU): indexer+top-k on {budget_rows} of {S1} query rows x {S2} keys, "
                   f"sparse MLA on {mla_tokens} of {S1} tokens; value = MLA TFLOP/s on the sample"),
        "indexer_topk_us_scaled": (t2 - t0) * scale_rows * 1e6,
        "mla_us_scaled": (t4 - t3) * (S1 / mla_tokens) * 1e6,
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
    }


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--s1", type=int, default=4096)
    ap.add_argument("--s2", type=int, default=131072)
    ap.add_argument("--dec-batch", type=int, default=32)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-targets", action="store_true",
                    help="skip the single-kernel decode / prefill / 32K indexer timings")
    ap.add_argument("--traffic", default=os.path.join(ROOT, "profiles", "traffic_indexer_layer128k.txt"),
                    help="rocprofv3 --pmc summary holding the dominant kernel's HBM bytes per launch")
    ap.add_argument("--traffic-run", action="store_true",
                    help="for rocprofv3 --pmc: one 1 GiB device copy (counter calibration), then one "
                         "layer step; prints no benchmark line")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported on this path "
              "(each GPU box has one GPU)", file=sys.stderr)
        return 2
    import torch

    layer = Layer(args.s1, args.s2, args.dec_batch)
    torch.cuda.synchronize()
    if args.traffic_run:
        src = torch.ones((1 << 28,), dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        layer.step()
        torch.cuda.synchronize()
        print("traffic run: copy of 1073741824 bytes, then one layer step", flush=True)
        return 0
    for _ in range(args.warmup):
        layer.step()
    torch.cuda.synchronize()
    n = len(layer.names)
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
           for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        layer.step(evs[s])
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = {name: 1e3 * sum(evs[s][i][0].elapsed_time(evs[s][i][1]) for s in range(args.steps)) / args.steps
           for i, name in enumerate(layer.names)}  # microseconds per call
    ms_per_step = wall * 1e3 / args.steps

    S1, S2 = args.s1, args.s2
    f_mla = mla_flops(S1)
    f_idx = indexer_flops_causal(S1, S2)
    mla_tflops = f_mla / (per["mla"] * 1e-6) / 1e12
    idx_tflops = f_idx / (per["indexer"] * 1e-6) / 1e12
    topk_bytes = 4.0 * sum(S2 - S1 + t + 1 for t in range(S1)) + 4.0 * S1 * TOPK
    topk_gbs = topk_bytes / (per["topk"] * 1e-6) / 1e9

    kern = {"indexer": ("mfma", idx_tflops, PEAK_FP8_TFLOPS, "TFLOP/s"),
            "mla": ("mfma", mla_tflops, PEAK_BF16_TFLOPS, "TFLOP/s"),
            "topk": ("hbm", topk_gbs, PEAK_HBM_GBS, "GB/s")}
    dom = max(kern, key=lambda k: per[k])
    bound, ach, peak, unit = kern[dom]
    traffic = None
    if os.path.exists(args.traffic):
        try:
            with open(args.traffic) as f:
                for line in f:
                    if line.startswith("hbm_bytes_per_launch"):
                        traffic = float(line.split("=", 1)[1])
        except (OSError, ValueError):
            traffic = None
    res = {
        "metric": METRIC,
        "value": round(mla_tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16 (MLA) / fp8-e4m3 (indexer) / fp32 (top-k keys)",
        "data": "synthetic (seeded N(0,1) inputs, random-init; no checkpoints)",
        "config": {"workload": "dsa_layer_128k (BASELINE config 5)", "prefill_chunk_tokens": S1,
                   "context_tokens": S2, "heads": H, "d_qk": DQK, "d_v": DV, "topk": TOPK,
                   "index_heads": IDX_HEADS, "index_dim": IDX_DIM, "decode_batch": args.dec_batch,
                   "page_size": 64},
        "mla_frac_of_bf16_peak": round(mla_tflops / PEAK_BF16_TFLOPS, 4),
        "indexer_us": round(per["indexer"], 2),
        "topk_us": round(per["topk"], 2),
        "indexer_topk_us": round(per["indexer"] + per["topk"], 2),
        "indexer_tflops": round(idx_tflops, 2),
        "indexer_frac_of_fp8_peak": round(idx_tflops / PEAK_FP8_TFLOPS, 4),
        "topk_gbs": round(topk_gbs, 1),
        "mla_us": round(per["mla"], 2),
        "decode_us": {"indexer": round(per["dec_indexer"], 2), "topk": round(per["dec_topk"], 2),
                      "mla": round(per["dec_mla"], 2)},
        "roofline": {"kernel": dom, "bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
                     "frac": round(ach / peak, 4), "traffic": traffic},
    }
    if not args.no_targets:
        lib_handle = layer.L
        del layer
        torch.cuda.empty_cache()
        res["target_configs"] = target_configs(lib_handle, args.steps)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(S1, S2)
    print(json.dumps(res))
    return 0


if __name__ == "__main__":
    sys.exit(main())
