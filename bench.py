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


DEC_BYTES = 64 * TOPK * (DQK * 2) + 64 * H * DQK * 2 + 64 * TOPK * 4 + 64 * 1024 * 4 + 64 * H * (DV * 2 + 4)


def decode_config3(L, runs: int) -> dict:
    """Config 3, sparse-MLA decode: B=64 single-token queries over 64K-token contexts
    in 64-token pages of one 4.8 GB pool, top-2048 uniform indices; mean microseconds
    per call (HIP events on the launch stream) over ``runs`` calls after 2 warm-ups."""
    import torch

    from dsa import inputs

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    d = inputs.mla_decode(device=dev)
    B = d["q"].shape[0]
    out = torch.empty((B, 1, H, DV), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((B, 1, H), dtype=torch.float32, device=dev)
    wsb = L.dsa_sparse_mla_workspace_bytes(B, 1, H, TOPK, 0)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    bt = d["block_table"]

    def dec():
        rc = L.dsa_sparse_mla_fwd(d["q"].data_ptr(), d["kv"].data_ptr(), d["indices"].data_ptr(), bt.data_ptr(),
                                  d["seq_len_kv"].data_ptr(), None, None, B, 1, H, DQK, DV, d["kv"].shape[0] * 64,
                                  64, bt.shape[1], TOPK, DQK ** -0.5, 0, 0, out.data_ptr(), lse.data_ptr(),
                                  ws.data_ptr(), ws.numel(), st)
        if rc != 0:
            raise RuntimeError(f"decode: {L.dsa_last_error().decode()}")

    us = _time_launches(dec, runs)
    dec_bytes = B * TOPK * (DQK * 2) + B * H * DQK * 2 + B * TOPK * 4 + bt.numel() * 4 + B * H * (DV * 2 + 4)
    assert dec_bytes == DEC_BYTES
    return {"us": round(us, 2), "gbs": round(dec_bytes / us / 1e3, 1),
            "frac_of_hbm": round(dec_bytes / us / 1e3 / PEAK_HBM_GBS, 4), "algorithmic_bytes": dec_bytes}


def _profile_roles(dispatches):
    """Label the DSA kernels of a --profile-run in dispatch order.  A layer step
    launches indexer, topk, mla, dec_indexer, dec_topk, dec_mla in that order (a
    combine after an MLA with split partials takes the MLA's role + "_combine");
    an MLA launched where a layer step would start is a config-3 decode, or the
    config-4 prefill when no combine follows it."""
    seq = ("indexer", "topk", "mla", "dec_indexer", "dec_topk", "dec_mla")

    def cat(name):
        if "combine" in name:
            return "comb"
        if "indexer" in name:
            return "idx"
        if "topk" in name:
            return "topk"
        if "mla" in name:
            return "mla"
        return None

    kind = {"indexer": "idx", "topk": "topk", "mla": "mla", "dec_indexer": "idx", "dec_topk": "topk",
            "dec_mla": "mla"}
    roles, prev, pos = [], None, 0
    for name in dispatches:
        c, role = cat(name), None
        if c == "comb":
            role = f"{prev}_combine" if prev and not prev.endswith("_combine") else None
        elif c is not None:
            if kind[seq[pos]] == c:
                role = seq[pos]
                pos = (pos + 1) % len(seq)
            elif pos == 0 and c == "mla":
                role = "config3_mla"
        roles.append(role)
        if role is not None:
            prev = role
    # an MLA outside a layer step with no combine after it is the config-4 prefill
    for i, role in enumerate(roles):
        if role == "config3_mla":
            nxt = next((r for r in roles[i + 1:] if r is not None), None)
            if nxt != "config3_mla_combine":
                roles[i] = "config4_mla"
    return roles


PROFILE_PASSES = (("GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_BUSY_CU_CYCLES", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                   "SQ_INSTS_VALU_MFMA_MOPS_F8", "SQ_INSTS_VALU_MFMA_MOPS_F6F4", "SQ_INSTS_MFMA", "SQ_WAVES"),
                  ("FETCH_SIZE",), ("WRITE_SIZE",),
                  ("SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_LDS_IDX_ACTIVE", "SQ_WAIT_INST_LDS", "SQ_INSTS_VALU",
                   "SQ_INSTS_SALU", "SQ_WAVE_CYCLES", "SQ_WAIT_ANY"))


def summarize_profile(root: str) -> str:
    """Text summary of the rocprofv3 runs of ``bench.py --profile-run`` under ``root``:
    per DSA kernel role, the median over its dispatches of the kernel-trace duration,
    the counters, the clock (GRBM_GUI_ACTIVE / 8 XCDs over the duration), the MFMA
    busy fraction (SQ_VALU_MFMA_BUSY_CYCLES over 1024 SIMDs x those cycles) and the
    HBM bytes (FETCH_SIZE and WRITE_SIZE in KiB, each scaled by what it reads for the
    run's 1 GiB device copy)."""
    import csv
    import glob
    import statistics

    counters = {}  # run dir -> list of (dispatch id, kernel, {counter: value})
    traces = []
    for path in sorted(glob.glob(os.path.join(root, "**", "*counter_collection.csv"), recursive=True)):
        per = {}
        with open(path) as fh:
            for r in csv.DictReader(fh):
                key = int(r["Dispatch_Id"])
                per.setdefault(key, [r["Kernel_Name"], {}])[1][r["Counter_Name"]] = float(r["Counter_Value"])
        counters[path] = [(k, v[0], v[1]) for k, v in sorted(per.items())]
    for path in sorted(glob.glob(os.path.join(root, "**", "*kernel_trace.csv"), recursive=True)):
        with open(path) as fh:
            traces = [(int(r["Dispatch_Id"]), r["Kernel_Name"], int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
                      for r in csv.DictReader(fh)]
        traces.sort()

    def by_role(rows, value):
        out = {}
        for role, row in zip(_profile_roles([r[1] for r in rows]), rows):
            if role is not None:
                out.setdefault(role, []).append(value(row))
        return out

    vals = {}
    calib = {}
    # the 1 GiB device copy at the start of the run is the largest copy dispatch
    # (input set-up issues smaller ones later)
    biggest = {}
    for rows in counters.values():
        for _, name, c in rows:
            if "copyBuffer" in name:
                for cname in ("FETCH_SIZE", "WRITE_SIZE"):
                    if cname in c and c[cname] > biggest.get(cname, 100000):
                        biggest[cname] = c[cname]
    for cname, v in biggest.items():
        calib[cname] = 1073741824.0 / (v * 1024.0)
    for rows in counters.values():
        for role, lst in by_role(rows, lambda r: r[2]).items():
            for c in lst:
                for cname, v in c.items():
                    vals.setdefault(role, {}).setdefault(cname, []).append(v)
    dur = by_role(traces, lambda r: r[2] / 1000.0)
    lines = [
        "# rocprofv3 summary of bench.py --profile-run (1 GiB device copy, config 5 layer step x 13 = the bench's "
        "3 warmup + 10 timed steps, config 3 decode x 3, config 4 prefill x 15)",
        "# made on one MI355X (repo root R, after cd /tmp && export TMPDIR=/tmp), one rocprofv3 run per line:",
        f"#   rocprofv3 --pmc {' '.join(PROFILE_PASSES[0])} -d R/gpurun_out/prof/p1 -o run --output-format csv "
        "-- python3 R/bench.py --profile-run",
        "#   rocprofv3 --pmc FETCH_SIZE -d R/gpurun_out/prof/p2 ... (same)",
        "#   rocprofv3 --pmc WRITE_SIZE -d R/gpurun_out/prof/p3 ... (same)",
        f"#   rocprofv3 --pmc {' '.join(PROFILE_PASSES[3])} -d R/gpurun_out/prof/p4 ... (same)",
        "#   rocprofv3 --kernel-trace --stats -d R/gpurun_out/prof/kt -o run --output-format csv -- python3 "
        "R/bench.py --profile-run",
        "#   python3 R/bench.py --summarize-profile R/gpurun_out/prof",
        f"# calibration (1 GiB device copy): FETCH_SIZE x {calib.get('FETCH_SIZE', float('nan')):.4f}, "
        f"WRITE_SIZE x {calib.get('WRITE_SIZE', float('nan')):.4f} bytes per KiB read / 1024",
        "# role: median over the role's dispatches (trace_mean/min/max_us: mean, min, max of its kernel-trace "
        "durations); mfma_busy = SQ_VALU_MFMA_BUSY_CYCLES / (1024 SIMDs x "
        "GRBM_GUI_ACTIVE / 8); clock_ghz = GRBM_GUI_ACTIVE / 8 / trace_us (the counter's clock domain: near the "
        "shader clock for the long kernels, above it for short ones, up to past the 2.4 GHz shader maximum); "
        "lds_bank_conflict_frac = SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; lds_wait_frac = SQ_WAIT_INST_LDS / "
        "SQ_WAVE_CYCLES",
    ]
    for role in ("indexer", "topk", "mla", "mla_combine", "dec_indexer", "dec_topk", "dec_mla", "dec_mla_combine",
                 "config3_mla", "config3_mla_combine", "config4_mla"):
        if role not in vals and role not in dur:
            continue
        m = {k: statistics.median(v) for k, v in vals.get(role, {}).items()}
        t = statistics.median(dur[role]) if role in dur else None
        out = {"trace_us": round(t, 2) if t else None}
        if role in dur:
            out["trace_mean_us"] = round(statistics.fmean(dur[role]), 2)
            out["trace_min_us"] = round(min(dur[role]), 2)
            out["trace_max_us"] = round(max(dur[role]), 2)
        grbm = m.get("GRBM_GUI_ACTIVE")
        if grbm and t:
            out["clock_ghz"] = round(grbm / 8 / (t * 1e3), 3)
        if grbm and "SQ_VALU_MFMA_BUSY_CYCLES" in m:
            out["mfma_busy"] = round(m["SQ_VALU_MFMA_BUSY_CYCLES"] / (1024 * grbm / 8), 4)
        for cname, label in (("SQ_INSTS_VALU_MFMA_MOPS_BF16", "mfma_flops_bf16"),
                             ("SQ_INSTS_VALU_MFMA_MOPS_F8", "mfma_flops_f8"),
                             ("SQ_INSTS_VALU_MFMA_MOPS_F6F4", "mfma_flops_f6f4")):
            if m.get(cname):
                out[label] = float(f"{m[cname] * 512:.4e}")
        if "FETCH_SIZE" in m and "FETCH_SIZE" in calib:
            out["fetch_bytes"] = float(f"{m['FETCH_SIZE'] * 1024 * calib['FETCH_SIZE']:.4e}")
        if "WRITE_SIZE" in m and "WRITE_SIZE" in calib:
            out["write_bytes"] = float(f"{m['WRITE_SIZE'] * 1024 * calib['WRITE_SIZE']:.4e}")
        if "fetch_bytes" in out and "write_bytes" in out:
            out["hbm_bytes"] = float(f"{out['fetch_bytes'] + out['write_bytes']:.4e}")
        if m.get("SQ_LDS_IDX_ACTIVE"):
            out["lds_bank_conflict_frac"] = round(m.get("SQ_LDS_BANK_CONFLICT", 0.0) / m["SQ_LDS_IDX_ACTIVE"], 4)
        if m.get("SQ_WAVE_CYCLES"):
            out["lds_wait_frac"] = round(m.get("SQ_WAIT_INST_LDS", 0.0) / m["SQ_WAVE_CYCLES"], 4)
        for cname in ("SQ_INSTS_MFMA", "SQ_WAVES", "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE", "SQ_VALU_MFMA_BUSY_CYCLES",
                      *PROFILE_PASSES[3]):
            if cname in m:
                out[cname] = float(f"{m[cname]:.5e}")
        lines.append(f"role={role} " + " ".join(f"{k}={v}" for k, v in out.items() if v is not None))
    return "\n".join(lines)


def summarize_trace(path: str, layer_steps: int) -> str:
    """Per (phase, kernel, workgroups) durations from the rocprofv3 kernel trace
    (``*kernel_trace.csv``) of a bench.py run: the first ``layer_steps`` x 7 DSA
    dispatches are the layer steps (warmup and timed; in each step the first three
    are the prefill chunk, phase "layer", and the last four the decode step, phase
    "decode"), the rest the target shapes; torch, runtime-copy and BLAS helper
    kernels are left out."""
    import csv
    import glob

    if os.path.isdir(path):
        path = glob.glob(os.path.join(path, "**", "*kernel_trace.csv"), recursive=True)[0]
    with open(path) as fh:
        rows = [r for r in csv.DictReader(fh)
                if not any(x in r["Kernel_Name"] for x in ("at::", "rocclr", "Cijk", "rocprim"))]
    rows.sort(key=lambda r: int(r["Dispatch_Id"]))
    agg = {}
    for i, r in enumerate(rows):
        name = r["Kernel_Name"].replace("void ", "").replace("(anonymous namespace)::", "").split("(")[0]
        grid = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0)
        wg = int(r.get("Workgroup_Size_X") or r.get("Workgroup_Size") or 1)
        phase = ("layer" if i % 7 < 3 else "decode") if i < 7 * layer_steps else "target"
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        agg.setdefault((phase, name, grid // max(wg, 1), wg), []).append((d, r))
    lines = [f"{'phase':6s} {'kernel':36s} {'workgroups':>10s} {'wg_size':>7s} {'calls':>5s} {'avg_us':>9s} "
             f"{'min_us':>9s} {'max_us':>9s} {'lds_B':>7s} {'vgpr':>5s} {'scratch':>7s}"]
    for (ph, k, g, w), v in agg.items():
        ds = [x[0] for x in v]
        r0 = v[0][1]
        vg = r0.get("VGPR_Count") or r0.get("Arch_VGPR_Count") or ""
        lines.append(f"{ph:6s} {k[:36]:36s} {g:10d} {w:7d} {len(ds):5d} {sum(ds) / len(ds):9.2f} {min(ds):9.2f} "
                     f"{max(ds):9.2f} {r0.get('LDS_Block_Size', ''):>7s} {vg:>5s} {r0.get('Scratch_Size', ''):>7s}")
    return "\n".join(lines)


def read_profile(path: str) -> dict:
    """role -> {key: value} from a summarize_profile text (empty if missing)."""
    out = {}
    try:
        with open(path) as fh:
            for line in fh:
                if not line.startswith("role="):
                    continue
                kv = dict(tok.split("=", 1) for tok in line.split())
                role = kv.pop("role")
                out[role] = {k: float(v) for k, v in kv.items()}
    except (OSError, ValueError):
        return {}
    return out


def prefill_config4(L, runs: int, warmup: int = 10) -> dict:
    """Config 4, sparse-MLA prefill: Sq = Skv = 16384 causal, H = 128, top-2048 (row
    i draws from [0, i], -1 padded); mean microseconds per launch after `warmup`
    launches (the shader clock under this 7.6 ms kernel settles only after about
    ten launches in a process; the first ones run up to 10 % slower)."""
    import torch

    from dsa import inputs

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    p = inputs.mla_prefill(B=1, S=16384, Skv=16384, H=H, topk=TOPK, seed=4, q_start=0, device=dev)
    S = p["q"].shape[1]
    out = torch.empty((1, S, H, DV), dtype=torch.bfloat16, device=dev)
    lse = torch.empty((1, S, H), dtype=torch.float32, device=dev)
    qs = torch.zeros((1,), dtype=torch.int32, device=dev)

    def pre():
        rc = L.dsa_sparse_mla_fwd(p["q"].data_ptr(), p["kv"].data_ptr(), p["indices"].data_ptr(), None, None,
                                  qs.data_ptr(), None, 1, S, H, DQK, DV, S, 0, 0, TOPK, DQK ** -0.5, 1, 1,
                                  out.data_ptr(), lse.data_ptr(), None, 0, st)
        if rc != 0:
            raise RuntimeError(f"prefill: {L.dsa_last_error().decode()}")

    us = _time_launches(pre, runs, warmup=warmup)
    fl = mla_flops(S)
    del p, out, lse
    return {"us": round(us, 1), "tflops": round(fl / us / 1e6, 1),
            "frac_of_bf16_peak": round(fl / us / 1e6 / PEAK_BF16_TFLOPS, 4)}


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
    res["decode_b64_64k"] = decode_config3(L, runs=steps)
    torch.cuda.empty_cache()

    # config 4: prefill, Sq = Skv = 16384, causal index ranges, top-2048
    res["prefill_16k"] = prefill_config4(L, runs=max(2, steps // 2))
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
    res["indexer_h16_128k"] = indexer_h16_config(L, steps)
    res["bench_sfa_decode"] = bench_sfa_configs(L, steps)
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


def indexer_h16_config(L, steps: int) -> dict:
    """The indexer at the reference wrapper's own precision (bf16 q and k,
    examples/deepseek_v4/lightning_indexer.py:1250-1253) at config-5 size: 4096 tail
    queries x 131072 keys, 64 heads x 128, causal, top-2048 (the full entry: the
    16-bit MFMA logits kernel with its 16-key group maxima, then the group-maxima
    top-k).  That top-k alone on the same logits and maxima is timed too; the
    indexer's share is the difference.
    FLOP = 2 * 64 * 128 per visible pair, against the 2.5 PFLOP/s 16-bit MFMA peak."""
    import torch

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    S1, S2 = 4096, 131072
    g = torch.Generator(device=dev).manual_seed(12)
    q = torch.randn((1, S1, IDX_HEADS, IDX_DIM), generator=g, device=dev).to(torch.bfloat16)
    k = torch.randn((1, S2, 1, IDX_DIM), generator=g, device=dev).to(torch.bfloat16)
    w = torch.randn((1, S1, IDX_HEADS), generator=g, device=dev) / 8
    idx = torch.empty((1, S1, 1, TOPK), dtype=torch.int32, device=dev)
    wsb = L.dsa_lightning_indexer_varlen_workspace_bytes(S1, S2)
    ws = torch.empty((wsb,), dtype=torch.uint8, device=dev)
    logits = ws[: S1 * S2 * 4].view(torch.float32)
    # the entry point's workspace: logits | row lengths | group maxima, 256-byte aligned
    rl_off = (S1 * S2 * 4 + 255) // 256 * 256
    gm_off = rl_off + (S1 * 4 + 255) // 256 * 256
    ld_g = (S2 + 15) // 16
    row_len = ws[rl_off:][: S1 * 4].view(torch.int32)
    gmax = ws[gm_off:][: S1 * ld_g * 4].view(torch.float32)
    idx2 = torch.empty((S1, TOPK), dtype=torch.int32, device=dev)

    def full():
        rc = L.dsa_lightning_indexer_h16_varlen(q.data_ptr(), k.data_ptr(), None, w.data_ptr(), None, 0, None, 0,
                                                None, 0, 0, 0, 1, S1, S2, S1, IDX_HEADS, IDX_DIM, 0, TOPK, 3,
                                                idx.data_ptr(), None, ws.data_ptr(), wsb, st)
        if rc != 0:
            raise RuntimeError(f"indexer_h16: {L.dsa_last_error().decode()}")

    def tk():
        rc = L.dsa_topk_f32_group_max(logits.data_ptr(), S1, S2, S2, row_len.data_ptr(), gmax.data_ptr(), ld_g, TOPK,
                                      1, idx2.data_ptr(), None, st)
        if rc != 0:
            raise RuntimeError(f"topk of the h16 logits: {L.dsa_last_error().decode()}")

    uf = _time_launches(full, max(2, steps // 2), warmup=3)
    ut = _time_launches(tk, max(2, steps // 2))
    fl = indexer_flops_causal(S1, S2)
    ui = uf - ut
    if not torch.equal(idx.view(S1, TOPK), idx2):
        raise RuntimeError("indexer_h16: the timed top-k differs from the entry point's")
    del q, k, w, idx, ws, logits, row_len, gmax, idx2
    torch.cuda.empty_cache()
    return {"dtype": "bf16", "indexer_topk_us": round(uf, 1), "topk_us": round(ut, 1),
            "indexer_us_derived": round(ui, 1), "indexer_tflops": round(fl / ui / 1e6, 1),
            "indexer_frac_of_bf16_peak": round(fl / ui / 1e6 / PEAK_BF16_TFLOPS, 4)}


# bench_sfa decode shapes and the times the reference publishes for them on Ascend
# (examples/sparse_flash_attention/bench_sfa/bench_sfa.py:106-153, README.md:31-34)
SFA_SHAPES = ((2560, 109.76), (6400, 109.10), (48000, 108.98))


def bench_sfa_configs(L, steps: int) -> dict:
    """The reference's only published sparse-MLA decode shapes (bench_sfa.py:106-153):
    T = 1 query, B = 1, 128 heads, D = 512 + 64 rope, top-2048 of the first
    act_kv = 2560 keys (topk of uniform noise), 128-key pages with an identity block
    table, scale 0.5, KV_S = 2560 / 6400 / 48000.  ``kernel_us``: dsa_sparse_mla_fwd
    on a joined 576-wide page cache (HIP events, inputs resident); ``wrapper_us``:
    dsa.sparse_attn_tilelang with separate rope tensors, which joins q and the key
    cache per call as the reference wrapper does (sparse_flash_attn_pa_no_cv_pipeline.py:406).
    ``ascend_tilelang_us``: the reference's published TileLang times (Ascend A2/A3)."""
    import torch

    import dsa

    dev = torch.device("cuda:0")
    st = torch.cuda.current_stream(dev).cuda_stream
    res = {}
    T, N, D, Dr, bs, act_kv, topk = 1, 128, 512, 64, 128, 2560, 2048
    for kv_s, pub in SFA_SHAPES:
        g = torch.Generator(device=dev).manual_seed(kv_s)
        query = (torch.randn((T, N, D), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        key = (torch.randn((kv_s // bs, bs, 1, D), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        qr = (torch.randn((T, N, Dr), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        kr = (torch.randn((kv_s // bs, bs, 1, Dr), generator=g, device=dev) * 0.5).to(torch.bfloat16)
        idx = torch.topk(torch.rand((T, 1, act_kv), generator=g, device=dev), topk, dim=-1).indices.int()
        bt = torch.arange(kv_s // bs, dtype=torch.int32, device=dev).view(1, -1)
        aq = torch.ones((1,), dtype=torch.int32, device=dev)
        ak = torch.full((1,), act_kv, dtype=torch.int32, device=dev)
        q576 = torch.cat((query, qr), -1).unsqueeze(0).contiguous()
        kv576 = torch.cat((key, kr), -1).contiguous()
        i4 = idx.view(1, T, 1, topk).contiguous()
        qs = ak - aq
        out = torch.empty((1, T, N, D), dtype=torch.bfloat16, device=dev)
        lse = torch.empty((1, T, N), dtype=torch.float32, device=dev)
        wsb = L.dsa_sparse_mla_workspace_bytes(1, T, N, topk, 0)
        ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)

        def kern():
            rc = L.dsa_sparse_mla_fwd(q576.data_ptr(), kv576.data_ptr(), i4.data_ptr(), bt.data_ptr(), ak.data_ptr(),
                                      qs.data_ptr(), None, 1, T, N, DQK, DV, kv576.shape[0] * bs, bs, bt.shape[1],
                                      topk, 0.5, 1, 0, out.data_ptr(), lse.data_ptr(), ws.data_ptr(), ws.numel(), st)
            if rc != 0:
                raise RuntimeError(f"bench_sfa: {L.dsa_last_error().decode()}")

        def wrap():
            dsa.sparse_attn_tilelang(query=query, key=key, value=key, sparse_indices=idx, scale_value=0.5,
                                     sparse_block_size=1, actual_seq_lengths_query=aq, actual_seq_lengths_kv=ak,
                                     query_rope=qr, key_rope=kr, layout_query="TND", layout_kv="PA_BSND",
                                     sparse_mode=0, block_table=bt, attention_mode=2)

        uk = _time_launches(kern, steps, warmup=3)
        uw = _time_launches(wrap, steps, warmup=3)
        byts = topk * DQK * 2 + N * DQK * 2 + topk * 4 + N * (DV * 2 + 4)
        res[f"kv_s_{kv_s}"] = {"kernel_us": round(uk, 2), "wrapper_us": round(uw, 2),
                               "ascend_tilelang_us": pub, "speedup_vs_ascend_kernel": round(pub / uk, 2),
                               "algorithmic_bytes": byts}
        del query, key, qr, kr, idx, q576, kv576, out, lse, ws
    torch.cuda.empty_cache()
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


def _median_time(fn, runs: int = 3, warmup: int = 1) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baseline_configs() -> dict:
    """The oracle (torch on the host cores) on configs 1-4 of the baseline: 1 warm-up
    + median of 3 for configs 1-3, one run of a stated subsample for config 4.
    Inputs are the configs' own generators (dsa.inputs, seeded) on the CPU."""
    import torch

    from dsa import inputs
    from oracle.dsa_oracle import indexer_scores, sparse_mla_fwd_gather, stable_topk

    res = {}
    # config 1: sparse MLA, B=1 S=128 Skv=4096 H=16 topk=512 (the whole config)
    c1 = inputs.mla_prefill()
    f1 = lambda: sparse_mla_fwd_gather(c1["q"], c1["kv"], c1["indices"], c1["sm_scale"],  # noqa: E731
                                       q_start_index_s=c1["q_start"], is_causal=True, p_dtype=torch.bfloat16)
    t = _median_time(f1)
    fl = 2.0 * 16 * 512 * 1088 * 128
    res["config1_mla_small"] = {"s": round(t, 4), "tflops": round(fl / t / 1e12, 4), "sample": "whole config"}
    del c1
    # config 2: indexer + top-k, 4096 x 32768, causal, K = 2048: the last 256 query
    # rows (the config's inputs, seed 2), scaled to the 4096 rows by the visible
    # (query, key) pairs
    S1c, S2c, nr = 4096, 32768, 256
    ix = inputs.indexer_fp8(B=1, S1=S1c, S2=S2c, seed=2)
    k = ix["k"][0, :, 0].float() * ix["key_scale"][0].unsqueeze(1)
    qf, w = ix["q"][0, S1c - nr:].float().contiguous(), ix["w"][0, S1c - nr:].contiguous()
    vis = torch.arange(S2c - nr + 1, S2c + 1)  # causal lengths of the sample rows

    def f2():
        sc = indexer_scores(qf, k, w, nr, S2c, 0)
        sc.masked_fill_(torch.arange(S2c)[None, :] >= vis[:, None], float("-inf"))
        stable_topk(sc, 2048, row_len=vis)

    t = _median_time(f2)
    pairs_all = sum(S2c - S1c + r + 1 for r in range(S1c))
    scaled = t * pairs_all / int(vis.sum())
    res["config2_indexer_topk_32k"] = {"s_sample": round(t, 3), "us_scaled": round(scaled * 1e6, 1),
                                       "sample": f"last {nr} of {S1c} query rows, scaled by visible pairs"}
    del ix, k, qf, w
    # config 3: decode B=64, H=128, topk=2048 over 64K paged contexts.  The oracle's
    # work is the gather of 64 x 2048 pool rows and the attention over them; the
    # pool here holds 4096 pages of 64 rows (302 MB) instead of 65536, so that the
    # baseline does not spend a minute generating 4.8 GB: the same rows are
    # gathered, from a smaller pool
    c3 = inputs.mla_decode(B=64, ctx=65536, pool_blocks=4096, seed=3)
    f3 = lambda: sparse_mla_fwd_gather(c3["q"], c3["kv"], c3["indices"], c3["sm_scale"],  # noqa: E731
                                       block_table=c3["block_table"], is_causal=False, p_dtype=torch.bfloat16)
    t = _median_time(f3)
    res["config3_decode_b64_64k"] = {"s": round(t, 4), "us": round(t * 1e6, 1),
                                     "sample": "whole batch; 4096-page pool (same gathers)"}
    del c3
    # config 4: prefill Sq = Skv = 16384, causal, topk 2048: one run over the last
    # 512 query rows (each with 2048 valid indices), scaled to the 16384 rows by
    # their valid-index counts
    # (inputs of the config's distribution drawn for the sample rows only: q and kv
    # N(0, 1) * 0.5 in bf16, row i's indices the first 2048 of a random order of [0, i])
    S, nr = 16384, 512
    g = torch.Generator().manual_seed(4)
    q4 = (torch.randn((1, nr, 128, 576), generator=g) * 0.5).to(torch.bfloat16)
    kv4 = (torch.randn((1, S, 1, 576), generator=g) * 0.5).to(torch.bfloat16)
    idx4 = torch.stack([torch.randperm(i + 1, generator=g)[:2048] for i in range(S - nr, S)]).int()
    t0 = time.perf_counter()
    sparse_mla_fwd_gather(q4, kv4, idx4.view(1, nr, 1, 2048), 576 ** -0.5, q_start_index_s=S - nr,
                          is_causal=True, p_dtype=torch.bfloat16)
    t = time.perf_counter() - t0
    valid_all = sum(min(i + 1, 2048) for i in range(S))
    scaled = t * valid_all / (nr * 2048)
    res["config4_prefill_16k"] = {"s_sample": round(t, 3), "s_scaled": round(scaled, 2),
                                  "tflops": round(2.0 * 128 * 2048 * 1088 * S / scaled / 1e12, 4),
                                  "sample": f"last {nr} of {S} rows, one run, scaled by valid indices"}
    return res


def cpu_baseline(S1: int, S2: int, budget_rows: int = 2048, mla_tokens: int = 4096) -> dict:
    """Time the CPU oracle on a bounded sample of the same workload and scale it,
    plus configs 1-4 (cpu_baseline_configs); all host cores."""
    import torch

    from dsa import inputs
    from oracle.dsa_oracle import indexer_scores, sparse_mla_fwd_gather, stable_topk

    torch.set_num_threads(os.cpu_count() or 1)
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
    del ix, k, sc, q, kv, idx
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
        "configs": cpu_baseline_configs(),
        "cpu_model": _cpu_model(),
        "os_cpu_count": os.cpu_count(),
        "torch_threads": threads,
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
    ap.add_argument("--profile", default=os.path.join(ROOT, "profiles", "pmc_dsa_layer128k.txt"),
                    help="rocprofv3 summary written by --summarize-profile (counters of the layer's kernels)")
    ap.add_argument("--profile-run", action="store_true",
                    help="for rocprofv3 (one --pmc pass or --kernel-trace per run): one 1 GiB device copy "
                         "(counter calibration), two warm-up layer steps, one layer step and one config-3 "
                         "decode (B=64, 64K paged); prints no benchmark line")
    ap.add_argument("--summarize-trace", metavar="PATH",
                    help="per-kernel durations from the rocprofv3 --kernel-trace output (a directory or its "
                         "*kernel_trace.csv) of a bench.py run with the same --steps / --warmup")
    ap.add_argument("--summarize-profile", metavar="DIR",
                    help="summarise the rocprofv3 runs of --profile-run under DIR (subdirectories holding "
                         "*counter_collection.csv or *kernel_trace.csv) and print the profile text")
    args = ap.parse_args()
    if args.summarize_trace:
        print(summarize_trace(args.summarize_trace, args.warmup + args.steps))
        return 0
    if args.summarize_profile:
        print(summarize_profile(args.summarize_profile))
        return 0
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported on this path "
              "(each GPU box has one GPU)", file=sys.stderr)
        return 2
    import torch

    layer = Layer(args.s1, args.s2, args.dec_batch)
    torch.cuda.synchronize()
    if args.profile_run:
        src = torch.ones((1 << 28,), dtype=torch.float32, device="cuda:0")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        del src, dst
        torch.cuda.synchronize()
        for _ in range(args.warmup + args.steps):
            layer.step()
        torch.cuda.synchronize()
        lib_handle = layer.L
        del layer
        torch.cuda.empty_cache()
        decode_config3(lib_handle, runs=3)
        torch.cuda.empty_cache()
        prefill_config4(lib_handle, runs=5, warmup=10)
        torch.cuda.synchronize()
        print(f"profile run: copy of 1073741824 bytes, {args.warmup + args.steps} layer steps, three config-3 "
              "decodes, fifteen config-4 prefills", flush=True)
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
    # the top-k's roofline reads every visible logit once; its group-maxima path
    # reads only the groups the indexer's maxima admit, so its bandwidth is the
    # profiled bytes over its time, and the full-row figure is a time ratio
    topk_bytes = 4.0 * sum(S2 - S1 + t + 1 for t in range(S1)) + 4.0 * S1 * TOPK
    topk_roof_us = topk_bytes / PEAK_HBM_GBS / 1e3
    topk_prof = read_profile(args.profile).get("topk", {})
    topk_gbs = (topk_prof["hbm_bytes"] / (per["topk"] * 1e-6) / 1e9) if topk_prof.get("hbm_bytes") else None

    kern = {"indexer": ("mfma", idx_tflops, PEAK_FP8_TFLOPS, "TFLOP/s"),
            "mla": ("mfma", mla_tflops, PEAK_BF16_TFLOPS, "TFLOP/s"),
            "topk": ("hbm", topk_gbs or 0.0, PEAK_HBM_GBS, "GB/s")}
    dom = max(kern, key=lambda k: per[k])
    bound, ach, peak, unit = kern[dom]
    prof = read_profile(args.profile).get(dom, {})
    traffic = prof.get("hbm_bytes")
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
        "topk_gbs_measured": round(topk_gbs, 1) if topk_gbs else None,
        "topk_full_row_roofline_us": round(topk_roof_us, 2),
        "mla_us": round(per["mla"], 2),
        "decode_us": {"indexer": round(per["dec_indexer"], 2), "topk": round(per["dec_topk"], 2),
                      "mla": round(per["dec_mla"], 2)},
        "roofline": {"kernel": dom, "bound": bound, "achieved": round(ach, 2), "peak": peak, "unit": unit,
                     "frac": round(ach / peak, 4), "traffic": traffic,
                     "traffic_source": (f"{os.path.relpath(args.profile, ROOT)} (rocprofv3 FETCH_SIZE + WRITE_SIZE "
                                        f"of bench.py --profile-run, copy-calibrated)") if traffic else None,
                     "event_us": round(per[dom], 2), "profiled_us": prof.get("trace_us"),
                     "profiled_frac": (round(ach * per[dom] / prof["trace_us"] / peak, 4)
                                       if prof.get("trace_us") else None),
                     "profiled_mfma_flops": prof.get("mfma_flops_f8") or prof.get("mfma_flops_bf16"),
                     "profiled_mfma_busy": prof.get("mfma_busy"), "profiled_clock_ghz": prof.get("clock_ghz")},
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
