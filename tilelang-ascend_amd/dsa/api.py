"""Python entry points of the MI355X DSA path, with the reference's call signatures.

Each function validates its arguments the way the reference's host wrapper does
(same conditions, ``ValueError``/``AssertionError`` where the reference raises
them), allocates outputs and workspaces with torch on the input's device (the
reference's ``out_idx`` / ``workspace_idx`` convention,
tilelang/jit/adapter/cython/cython_wrapper.pyx:102-141) and calls the HIP library
through its C ABI on the current stream.  There is no CPU path: tensors must be
on a ROCm device and the library must be built.
"""

from __future__ import annotations

from typing import Callable, Optional, Tuple

import torch

from ._lib import check, lib

INT64_MAX = (1 << 63) - 1
_FP8 = getattr(torch, "float8_e4m3fn", None)


# ---------------------------------------------------------------------------
# helpers
# ---------------------------------------------------------------------------
def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(*tensors: torch.Tensor) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise ValueError(f"expected a tensor on a ROCm device, got one on {t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors are on different devices: {dev} and {t.device}")
    return dev


def _require_contiguous(name: str, t: torch.Tensor) -> None:
    # cython_wrapper.pyx:148-150 raises for non-contiguous inputs
    if not t.is_contiguous():
        raise ValueError(f"Expected {name} to be contiguous")


def _host_lengths(t) -> torch.Tensor:
    """Per-batch lengths / prefix sums as a host int64 vector: the grid sizes derive
    from them, so the host needs their values (the reference reads them on the host
    too, examples/deepseek_v4/lightning_indexer.py:1265-1279).  One device-to-host
    copy when they live on the GPU, none when the caller passes them on the CPU."""
    return torch.as_tensor(t).reshape(-1).to(device="cpu", dtype=torch.int64)


def _int32_vec(name: str, t: Optional[torch.Tensor], n: int, device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    t = torch.as_tensor(t)
    if t.numel() != n:
        raise ValueError(f"{name} must have {n} entries, got {t.numel()}")
    return t.to(device=device, dtype=torch.int32).contiguous()


# ---------------------------------------------------------------------------
# top-k selector
# ---------------------------------------------------------------------------
def topk_selector(x: torch.Tensor, top_k: int, *, row_len: Optional[torch.Tensor] = None,
                  pad_invalid: bool = True, return_values: bool = False,
                  group_max: Optional[torch.Tensor] = None):
    """Row-wise top-k of fp32 ``x [B, N]`` -> int32 indices ``[B, top_k]``.

    Same output as the topk_selector example's reference ``torch.topk(x, k)[1]``
    (examples/topk_selector/example_topk_selector.py:57-58) with the ordering and
    tie rule of the lightning-indexer golden: descending value, equal values in
    ascending index order (examples/deepseek_v4/lightning_indexer.py:318-320).
    With ``pad_invalid`` entries whose value is <= -1e30 (masked) become -1, and
    rows shorter than ``top_k`` (``row_len``) are padded with -1 (:321-325).
    ``group_max [B, ceil(N / 16)]`` fp32 (optional): upper bounds of the maxima of
    each row's 16-element groups, as the lightning indexer emits them; long rows
    then read only the groups that can hold a selected element (same result).
    """
    if x.dim() != 2:
        raise ValueError(f"x must be 2-D [B, N], got shape {tuple(x.shape)}")
    if x.dtype != torch.float32:
        raise ValueError(f"x must be float32, got {x.dtype}")
    if not (1 <= top_k <= 8192):
        raise ValueError(f"top_k must be in [1, 8192], got {top_k}")
    dev = _require_gpu(x, row_len)
    _require_contiguous("x", x)
    B, N = x.shape
    rl = _int32_vec("row_len", row_len, B, dev)
    idx = torch.empty((B, top_k), dtype=torch.int32, device=dev)
    val = torch.empty((B, top_k), dtype=torch.float32, device=dev) if return_values else None
    if group_max is None:
        check(lib().dsa_topk_f32(_ptr(x), B, N, N, _ptr(rl), top_k, int(bool(pad_invalid)), _ptr(idx),
                                 _ptr(val), _stream(dev)), "dsa_topk_f32")
    else:
        ng = (N + 15) // 16
        if group_max.dtype != torch.float32 or tuple(group_max.shape) != (B, ng):
            raise ValueError(f"group_max must be float32 [{B}, {ng}], got {group_max.dtype} {tuple(group_max.shape)}")
        _require_gpu(x, group_max)
        _require_contiguous("group_max", group_max)
        check(lib().dsa_topk_f32_group_max(_ptr(x), B, N, N, _ptr(rl), _ptr(group_max), ng, top_k,
                                           int(bool(pad_invalid)), _ptr(idx), _ptr(val), _stream(dev)),
              "dsa_topk_f32_group_max")
    return (idx, val) if return_values else idx


def simple_topk_selector(B: int, N: int, top_k: int, block_N: int, dtype: str = "float32") -> Callable:
    """Factory with the signature of the reference's JIT kernel builder
    (examples/topk_selector/example_topk_selector.py:19): returns ``kernel(x) -> indices``.
    ``block_N`` was the reference's UB copy granularity and has no effect here."""
    if dtype != "float32":
        raise ValueError(f"simple_topk_selector supports float32 only, got {dtype}")
    del block_N

    def kernel(x: torch.Tensor) -> torch.Tensor:
        if tuple(x.shape) != (B, N):
            raise ValueError(f"expected x of shape {(B, N)}, got {tuple(x.shape)}")
        return topk_selector(x, top_k, pad_invalid=False)

    return kernel


# ---------------------------------------------------------------------------
# lightning indexer
# ---------------------------------------------------------------------------
def lightning_indexer(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor, *,
                      key_scale: Optional[torch.Tensor] = None,
                      actual_seq_lengths_query: Optional[torch.Tensor] = None,
                      actual_seq_lengths_key: Optional[torch.Tensor] = None,
                      block_table: Optional[torch.Tensor] = None,
                      layout_query: str = "BSND", layout_key: str = "BSND",
                      sparse_count: int = 2048, sparse_mode: int = 3,
                      pre_tokens: int = INT64_MAX, next_tokens: int = INT64_MAX,
                      return_value: bool = False, block_n: Optional[int] = None,
                      pp_slots: int = 2, max_cores: Optional[int] = None,
                      return_logits: bool = False):
    """Lightning indexer: per query row the ``sparse_count`` keys with the largest
    ``sum_h w[h] * ReLU(q[h] . k)`` (times ``key_scale``), causal for sparse_mode 3.

    Signature and validation of ``lightning_indexer``
    (examples/deepseek_v4/lightning_indexer.py:1202-1283); semantics of its golden
    ``cpu_lightning_indexer`` (:199-335).  q/k are the reference's fp16 / bf16
    (weights fp32 or q's dtype; a 16-bit MFMA kernel accumulating the exact
    products in fp32, ``values`` in q's dtype as there), or fp8 e4m3
    (``torch.float8_e4m3fn``, weights fp32, ``values`` fp32) for the fp8 MFMA
    kernel.  Either takes an optional per-key fp32 ``key_scale`` of shape
    ``[B, S2]`` (or ``[B, S2, 1]``) multiplying the logits.  N1 <= 64 (fewer heads
    count as zero heads; the fp8 operands are padded to 64).  ``block_n``,
    ``pp_slots`` and ``max_cores`` were Ascend tiling knobs and are accepted and
    ignored.  Layouts (N2 = 1): query BSND ``[B, S1, N1, D]`` or TND ``[T, N1, D]``
    (``actual_seq_lengths_query`` = prefix sums); key BSND ``[B, S2, 1, D]``, TND
    ``[T2, 1, D]`` (prefix sums) or PA_BSND ``[blocks, block_size, 1, D]`` with
    ``block_table [B, max_blocks]`` and per-batch ``actual_seq_lengths_key``; the
    key scale has the key's shape without D.  TND and paged keys are read in place
    by the kernel (the reference pads and gathers them on the host first).
    Returns ``(indices int32 [B, S1, 1, sparse_count] or [T, 1, sparse_count] for
    TND, values)``; ``values`` is an empty tensor unless ``return_value``.
    ``return_logits`` additionally returns the fp32 logits ``[B, S1, S2]`` (or
    ``[T, S2]``), valid for keys below the row's causal length.
    """
    del block_n, pp_slots, max_cores
    if layout_query not in ("BSND", "TND"):
        raise AssertionError(f"Unsupported query layout: {layout_query}")
    if layout_key not in ("BSND", "PA_BSND", "TND"):
        raise AssertionError(f"Unsupported key layout: {layout_key}")
    is_pa = layout_key == "PA_BSND"
    if is_pa and return_value:
        raise ValueError("PA_BSND layout does not support return_value")
    if not is_pa and layout_query != layout_key:
        raise ValueError(f"layout_query({layout_query}) must equal layout_key({layout_key}) when key is non-PA_BSND")
    if not (1 <= sparse_count <= 2048 or (sparse_count % 1024 == 0 and sparse_count <= 8192)):
        raise ValueError(f"sparse_count must be in [1,2048] or a multiple of 1024 up to 8192, got {sparse_count}")
    if sparse_mode not in (0, 3):
        raise ValueError(f"sparse_mode must be 0 (defaultMask) or 3 (rightDownCausal), got {sparse_mode}")
    if pre_tokens != INT64_MAX:
        raise ValueError(f"pre_tokens must be INT64_MAX, got {pre_tokens}")
    if next_tokens != INT64_MAX:
        raise ValueError(f"next_tokens must be INT64_MAX, got {next_tokens}")
    if query.dtype != key.dtype:
        raise ValueError(f"query dtype {query.dtype} must equal key dtype {key.dtype}")
    half = query.dtype in (torch.float16, torch.bfloat16)
    if not half and query.dtype != _FP8:
        raise ValueError(f"query/key dtype must be float16 or bfloat16 (or float8_e4m3fn), got {query.dtype}")
    if weights.dtype != torch.float32 and not (half and weights.dtype == query.dtype):
        raise ValueError(f"weights dtype {weights.dtype} must be float32 or same as query {query.dtype}")
    is_tnd = layout_query == "TND"
    is_tnd_key = layout_key == "TND"
    if is_tnd and actual_seq_lengths_query is None:
        raise AssertionError("TND layout requires actual_seq_lengths_query (prefix sums)")
    if is_pa and actual_seq_lengths_key is None:
        raise AssertionError("PA_BSND case requires actual_seq_lengths")
    if is_tnd_key and actual_seq_lengths_key is None:
        raise AssertionError("TND layout requires actual_seq_lengths_key (prefix sums)")
    if is_pa and block_table is None:
        raise ValueError("PA_BSND layout requires block_table")
    dev = _require_gpu(query, key, weights, key_scale, block_table)
    for name, t in (("query", query), ("key", key), ("weights", weights)):
        _require_contiguous(name, t)

    # ---- query rows: BSND [B, S1, N1, D] or TND [T, N1, D] with prefix-sum lengths
    if is_tnd:
        if query.dim() != 3:
            raise ValueError("TND query must be 3-D [T, N1, D]")
        if actual_seq_lengths_query is None:
            raise AssertionError("TND layout requires actual_seq_lengths_query (prefix sums)")
        q_tot, N1, D = query.shape
        cum_h = _host_lengths(actual_seq_lengths_query)
        B = cum_h.shape[0]
        if B == 0 or int(cum_h[-1]) != q_tot:
            raise ValueError(f"actual_seq_lengths_query must be prefix sums ending at T = {q_tot}")
        q_lens = torch.diff(cum_h, prepend=torch.zeros(1, dtype=torch.int64))
        if bool((q_lens < 0).any()):
            raise ValueError("actual_seq_lengths_query must be non-decreasing prefix sums")
        S1 = int(q_lens.max())
        cum_q = cum_h.to(device=dev, dtype=torch.int32)
        if tuple(weights.shape) != (q_tot, N1):
            raise ValueError(f"weights must be [T, N1] = {(q_tot, N1)}, got {tuple(weights.shape)}")
        seq_q, seq_q_cum = cum_q, 1
    else:
        if query.dim() != 4:
            raise ValueError("BSND query must be 4-D [B, S, N, D]")
        B, S1, N1, D = query.shape
        q_tot = B * S1
        if tuple(weights.shape) != (B, S1, N1):
            raise ValueError(f"weights must be [B, S1, N1] = {(B, S1, N1)}, got {tuple(weights.shape)}")
        seq_q, seq_q_cum = _int32_vec("actual_seq_lengths_query", actual_seq_lengths_query, B, dev), 0

    # ---- keys: BSND [B, S2, 1, D], TND [T2, 1, D] (prefix sums) or PA_BSND
    # [blocks, block_size, 1, D] through block_table [B, max_blocks] (per-batch lengths)
    bt, block_size, max_blocks, pool_rows = None, 0, 0, 0
    if is_pa:
        if key.dim() != 4:
            raise ValueError("PA_BSND key must be 4-D [blocks, block_size, N2, D]")
        nblk, block_size, N2, Dk = key.shape
        if actual_seq_lengths_key is None:
            raise AssertionError("PA_BSND case requires actual_seq_lengths")
        if block_table is None:
            raise ValueError("PA_BSND layout requires block_table")
        if block_size % 16 != 0 or block_size > 1024 or block_size <= 0:
            raise ValueError(f"PA block_size must be a positive multiple of 16 and <= 1024, got {block_size}")
        if block_table.dim() != 2 or block_table.shape[0] != B:
            raise ValueError(f"block_table must be [B, max_blocks], got {tuple(block_table.shape)}")
        bt = block_table.to(device=dev, dtype=torch.int32).contiguous()
        max_blocks, pool_rows = bt.shape[1], nblk * block_size
        seq_h = _host_lengths(actual_seq_lengths_key)
        if seq_h.numel() != B:
            raise ValueError(f"actual_seq_lengths_key must have B = {B} entries, got {seq_h.numel()}")
        S2 = int(seq_h.max()) if B > 0 else 0
        seq_k, seq_k_cum = seq_h.to(device=dev, dtype=torch.int32), 0
        k_tokens = pool_rows
    elif is_tnd_key:
        if key.dim() != 3:
            raise ValueError("TND key must be 3-D [T2, N2, D]")
        if actual_seq_lengths_key is None:
            raise AssertionError("TND layout requires actual_seq_lengths_key (prefix sums)")
        k_tot, N2, Dk = key.shape
        seq_h = _host_lengths(actual_seq_lengths_key)
        if seq_h.numel() != B or (B > 0 and int(seq_h[-1]) != k_tot):
            raise ValueError(f"actual_seq_lengths_key must be {B} prefix sums ending at T2 = {k_tot}")
        k_lens = torch.diff(seq_h, prepend=torch.zeros(1, dtype=torch.int64))
        if bool((k_lens < 0).any()):
            raise ValueError("actual_seq_lengths_key must be non-decreasing prefix sums")
        S2 = int(k_lens.max()) if B > 0 else 0
        seq_k, seq_k_cum = seq_h.to(device=dev, dtype=torch.int32), 1
        k_tokens = k_tot
    else:
        if key.dim() != 4:
            raise ValueError("BSND key must be 4-D [B, S, N, D]")
        Bk, S2, N2, Dk = key.shape
        if Bk != B:
            raise ValueError(f"key shape {tuple(key.shape)} does not match query batch {B}")
        seq_k, seq_k_cum = _int32_vec("actual_seq_lengths_key", actual_seq_lengths_key, B, dev), 0
        k_tokens = B * S2
    if Dk != D:
        raise ValueError(f"key head dim {Dk} does not match query head dim {D}")
    if D != 128:
        raise AssertionError(f"head dim must be 128, got {D}")
    if N2 != 1:
        raise AssertionError(f"N2 must be 1, got N2={N2}")
    if N1 > 64:
        raise ValueError(f"query head_num (N1) must be <= 64, got {N1}")
    if half:
        weights = weights.to(torch.float32).contiguous()
    elif N1 != 64:
        # the fp8 kernel holds 64 heads: zero heads (and zero weights) add nothing
        pad_q = torch.zeros((*query.shape[:-2], 64, D), dtype=torch.uint8, device=dev)
        pad_q[..., :N1, :] = query.view(torch.uint8)
        query = pad_q.view(_FP8)
        pad_w = torch.zeros((*weights.shape[:-1], 64), dtype=torch.float32, device=dev)
        pad_w[..., :N1] = weights
        weights, N1 = pad_w, 64
    ks = None
    if key_scale is not None:
        if key_scale.numel() != k_tokens:
            raise ValueError(f"key_scale must have one entry per key token ({k_tokens}), got {key_scale.numel()}")
        ks = key_scale.to(device=dev, dtype=torch.float32).contiguous()

    out_shape = (q_tot, 1, sparse_count) if is_tnd else (B, S1, 1, sparse_count)
    indices = torch.empty(out_shape, dtype=torch.int32, device=dev)
    values = torch.empty(out_shape, dtype=torch.float32, device=dev) if return_value else None
    L = lib()
    ws_bytes = L.dsa_lightning_indexer_varlen_workspace_bytes(q_tot, S2)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    if half:
        check(L.dsa_lightning_indexer_h16_varlen(_ptr(query), _ptr(key), _ptr(ks), _ptr(weights), _ptr(seq_q),
                                                 seq_q_cum, _ptr(seq_k), seq_k_cum, _ptr(bt), block_size, max_blocks,
                                                 pool_rows, B, S1, S2, q_tot, N1, D,
                                                 int(query.dtype == torch.float16), sparse_count, sparse_mode,
                                                 _ptr(indices), _ptr(values), _ptr(ws), ws_bytes, _stream(dev)),
              "dsa_lightning_indexer_h16_varlen")
    else:
        check(L.dsa_lightning_indexer_fp8_varlen(_ptr(query), _ptr(key), _ptr(ks), _ptr(weights), _ptr(seq_q),
                                                 seq_q_cum, _ptr(seq_k), seq_k_cum, _ptr(bt), block_size, max_blocks,
                                                 pool_rows, B, S1, S2, q_tot, N1, D, sparse_count, sparse_mode,
                                                 _ptr(indices), _ptr(values), _ptr(ws), ws_bytes, _stream(dev)),
              "dsa_lightning_indexer_fp8_varlen")
    out_dtype = query.dtype if half else torch.float32  # the golden's values are in q's dtype (:322)
    if values is None:
        values = torch.empty((0,), dtype=out_dtype, device=dev)
    elif half:
        values = values.to(out_dtype)
    if return_logits:
        logits = ws[: q_tot * S2 * 4].view(torch.float32).view(q_tot, S2)
        if not is_tnd:
            logits = logits.view(B, S1, S2)
        return indices, values, logits
    return indices, values


def indexer_logits(query: torch.Tensor, key: torch.Tensor, weights: torch.Tensor, *,
                   key_scale: Optional[torch.Tensor] = None,
                   actual_seq_lengths_query: Optional[torch.Tensor] = None,
                   actual_seq_lengths_key: Optional[torch.Tensor] = None,
                   sparse_mode: int = 3) -> Tuple[torch.Tensor, torch.Tensor]:
    """The logits stage alone: ``(logits fp32 [B, S1, S2], row_len int32 [B, S1])``.
    ``logits[b, t, s]`` is defined for ``s < row_len[b, t]`` (the golden's
    ``full_scores`` there, lightning_indexer.py:303-314)."""
    B, S1, N1, D = query.shape
    S2 = key.shape[1]
    if query.dtype != _FP8 or key.dtype != _FP8:
        raise ValueError("query/key must be float8_e4m3fn")
    dev = _require_gpu(query, key, weights, key_scale)
    for name, t in (("query", query), ("key", key), ("weights", weights)):
        _require_contiguous(name, t)
    ks = None if key_scale is None else key_scale.to(torch.float32).contiguous()
    aq = _int32_vec("actual_seq_lengths_query", actual_seq_lengths_query, B, dev)
    ak = _int32_vec("actual_seq_lengths_key", actual_seq_lengths_key, B, dev)
    logits = torch.empty((B, S1, S2), dtype=torch.float32, device=dev)
    row_len = torch.zeros((B, S1), dtype=torch.int32, device=dev)
    check(lib().dsa_indexer_logits_fp8(_ptr(query), _ptr(key), _ptr(ks), _ptr(weights), _ptr(aq), _ptr(ak),
                                       B, S1, S2, N1, D, sparse_mode, _ptr(logits), S2, _ptr(row_len),
                                       _stream(dev)), "dsa_indexer_logits_fp8")
    return logits, row_len


# ---------------------------------------------------------------------------
# sparse MLA forward
# ---------------------------------------------------------------------------
def sparse_mla_fwd(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor,
                   sm_scale: Optional[float] = None, *, d_v: int = 512,
                   block_table: Optional[torch.Tensor] = None,
                   seq_len_kv: Optional[torch.Tensor] = None,
                   q_start_index_s=None, is_causal: bool = True,
                   attn_sink: Optional[torch.Tensor] = None,
                   num_splits: int = 0, return_lse: bool = True):
    """Sparse MLA forward with one shared latent KV head -> ``(out, lse)``.

    q ``[B, S, H, d_qk]`` bf16 or fp16 (d_qk 576 = 512 latent + 64 rope, or 512);
    kv ``[B, Skv, 1, d_qk]`` of q's dtype, or a page pool ``[blocks, block_size, 1, d_qk]``
    with ``block_table [B, max_blocks]`` int32 (index i of batch b lives at
    ``pool[block_table[b, i // block_size], i % block_size]``,
    bench_sfa/sparse_flash_attn_pa_no_cv_pipeline.py:196-200); indices
    ``[B, S, 1, topk]`` int32.  Semantics follow ``sparse_attention_fwd`` and its
    reference (examples/sparse_flash_attention/example_sparse_flash_attn.py:18-292)
    with the gather rule of examples/deepseek_v4/sparse_attention.py:171-198:
    ``-1`` and out-of-range indices are skipped; ``is_causal`` also skips indices
    above ``q_start_index_s + s`` (per batch if a tensor; default ``seq_len_kv[b] - S``,
    or ``Skv - S`` without ``seq_len_kv``, as example_sparse_flash_attn_mask_pa.py:221).
    ``out [B, S, H, 512]`` in q's dtype and ``lse [B, S, H]`` fp32 (natural log,
    sparse_flash_mla_golden.py:147-149).  A row without a valid index gets
    out = 0 and lse = -inf.  fp16 runs fp16 MFMAs with the probabilities rounded
    to fp16 before P.V (the reference's ``p.type(v.dtype)``,
    example_sparse_flash_attn.py:288); bf16 rounds them to bf16.
    """
    if q.dtype not in (torch.bfloat16, torch.float16) or kv.dtype != q.dtype:
        raise ValueError(f"q and kv must both be bfloat16 or both float16, got {q.dtype} and {kv.dtype}")
    if indices.dtype != torch.int32:
        raise ValueError(f"indices must be int32, got {indices.dtype}")
    if q.dim() != 4 or kv.dim() != 4 or indices.dim() != 4:
        raise ValueError("q, kv and indices must be 4-D")
    B, S, H, d_qk = q.shape
    if d_v != 512:
        raise ValueError(f"d_v must be 512, got {d_v}")
    if d_qk not in (576, 512):
        raise ValueError(f"d_qk must be 576 or 512, got {d_qk}")
    if kv.shape[2] != 1 or kv.shape[3] != d_qk:
        raise ValueError(f"kv must be [*, *, 1, {d_qk}], got {tuple(kv.shape)}")
    if indices.shape[0] != B or indices.shape[1] != S or indices.shape[2] != 1:
        raise ValueError(f"indices must be [B, S, 1, topk] = [{B}, {S}, 1, topk], got {tuple(indices.shape)}")
    topk = indices.shape[3]
    dev = _require_gpu(q, kv, indices, block_table, attn_sink)
    for name, t in (("q", q), ("kv", kv), ("indices", indices)):
        _require_contiguous(name, t)
    paged = block_table is not None
    if paged:
        if block_table.dim() != 2 or block_table.shape[0] != B:
            raise ValueError(f"block_table must be [B, max_blocks], got {tuple(block_table.shape)}")
        bt = block_table.to(torch.int32).contiguous()
        block_size = kv.shape[1]
        max_blocks = bt.shape[1]
        skv = kv.shape[0] * block_size  # rows in the pool
    else:
        if kv.shape[0] != B:
            raise ValueError(f"kv batch {kv.shape[0]} != q batch {B}")
        bt = None
        block_size = max_blocks = 0
        skv = kv.shape[1]
    kvl = _int32_vec("seq_len_kv", seq_len_kv, B, dev)
    qs = None
    if q_start_index_s is not None:
        if isinstance(q_start_index_s, int):
            qs = torch.full((B,), q_start_index_s, dtype=torch.int32, device=dev)
        else:
            qs = _int32_vec("q_start_index_s", q_start_index_s, B, dev)
    sink = None
    if attn_sink is not None:
        if attn_sink.numel() != H:
            raise ValueError(f"attn_sink must have H = {H} entries")
        sink = attn_sink.to(torch.float32).contiguous()
    if sm_scale is None:
        sm_scale = d_qk ** -0.5
    out = torch.empty((B, S, H, d_v), dtype=q.dtype, device=dev)
    lse = torch.empty((B, S, H), dtype=torch.float32, device=dev)
    L = lib()
    ws_bytes = L.dsa_sparse_mla_workspace_bytes(B, S, H, topk, num_splits)
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    fn, name = ((L.dsa_sparse_mla_fwd_f16, "dsa_sparse_mla_fwd_f16") if q.dtype == torch.float16
                else (L.dsa_sparse_mla_fwd, "dsa_sparse_mla_fwd"))
    check(fn(_ptr(q), _ptr(kv), _ptr(indices), _ptr(bt), _ptr(kvl), _ptr(qs), _ptr(sink),
             B, S, H, d_qk, d_v, skv, block_size, max_blocks, topk, float(sm_scale),
             int(bool(is_causal)), int(num_splits), _ptr(out), _ptr(lse), _ptr(ws),
             ws_bytes, _stream(dev)), name)
    return (out, lse) if return_lse else out


def sparse_attention_fwd(heads: int, dim: int, tail_dim: int, topk: int, kv_stride: int,
                         kv_group: int = 1, sm_scale: Optional[float] = None, is_causal: bool = True,
                         block_I: int = 64) -> Callable:
    """Factory with the signature of the reference's ``sparse_attention_fwd``
    (examples/sparse_flash_attention/example_sparse_flash_attn.py:18-46), returning
    ``kernel(q, kv, indices) -> out``.  Asserts as the reference does; the
    out-of-range sentinel ``Skv`` used to pad its indices (:303) is skipped.

    With ``kv_stride > 1`` the KV rows are compressed positions: row n stands for
    original keys up to ``n * kv_stride + kv_stride - 1`` and query m (at original
    position ``Skv * kv_stride - S + m``) sees it when that position is at least
    ``n * kv_stride + kv_stride - 1``, the causal rule of the golden
    ``ref_sparse_attention_fwd_interface`` (:255-280); its first ``kv_stride - 1``
    rows always attend key 0, listed or not (:280: the golden sets that mask entry
    after the causal AND).  Indices that fail the rule are set to -1 on the device
    before the launch, and those rows get key 0 in one extra list column when
    their list lacks it."""
    def _pow2(x):
        return x > 0 and (x & (x - 1)) == 0
    assert _pow2(dim), f"haven't check padding correctness yet, dim={dim}"
    assert _pow2(tail_dim), f"haven't check padding correctness yet, dim={tail_dim}"
    assert is_causal, "non-casual is not supported"
    assert topk % block_I == 0, "otherwise will load some index=0 thus causing wrong kv to be loaded"
    if kv_group != 1:
        raise NotImplementedError("one latent KV head (kv_group = 1) only")
    if kv_stride < 1:
        raise ValueError(f"kv_stride must be >= 1, got {kv_stride}")
    scale = (1.0 / (dim + tail_dim)) ** 0.5 if sm_scale is None else sm_scale

    def kernel(q: torch.Tensor, kv: torch.Tensor, indices: torch.Tensor) -> torch.Tensor:
        if q.shape[2] != heads or q.shape[3] != dim + tail_dim or indices.shape[3] != topk:
            raise ValueError("q / indices shape does not match the kernel's heads, dim + tail_dim, topk")
        if kv_stride == 1:
            return sparse_mla_fwd(q, kv, indices, scale, is_causal=is_causal, return_lse=False)
        S, skv = q.shape[1], kv.shape[1]
        m = torch.arange(S, device=indices.device, dtype=torch.int64)
        last = torch.div(skv * kv_stride - S + m + 1, kv_stride, rounding_mode="floor") - 1
        last = torch.where(m < kv_stride - 1, last.clamp_min(0), last).view(1, S, 1, 1)
        idx = torch.where(indices.to(torch.int64) <= last, indices, torch.full_like(indices, -1)).to(torch.int32)
        # rows m < kv_stride - 1 see key 0 whatever their list holds: append it
        # (once) where the filtered list lacks it
        nrow = min(kv_stride - 1, S)
        extra = torch.full((*idx.shape[:3], 1), -1, dtype=torch.int32, device=idx.device)
        has0 = (idx[:, :nrow] == 0).any(dim=-1, keepdim=True)
        extra[:, :nrow] = torch.where(has0, -1, 0).to(torch.int32)
        idx = torch.cat((idx, extra), dim=-1)
        return sparse_mla_fwd(q, kv, idx.contiguous(), scale, is_causal=False, return_lse=False)

    return kernel


def sparse_attn_tilelang(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, sparse_indices: torch.Tensor,
                         scale_value: float, sparse_block_size: int, actual_seq_lengths_query: torch.Tensor,
                         actual_seq_lengths_kv: torch.Tensor, query_rope: Optional[torch.Tensor] = None,
                         key_rope: Optional[torch.Tensor] = None, layout_query: str = "BSND",
                         layout_kv: str = "BSND", sparse_mode: int = 3, block_table: Optional[torch.Tensor] = None,
                         attention_mode=None) -> torch.Tensor:
    """Paged sparse MLA with the signature of the reference's ``sparse_attn_tilelang``
    (examples/sparse_flash_attention/bench_sfa/sparse_flash_attn_pa_no_cv_pipeline.py:384-419,
    the ``npu_sparse_flash_attention`` argument list of bench_sfa.py:55-73).

    query ``[T, N, 512]`` (TND, one batch: the reference views it as ``[1, T, N, D]``),
    key ``[blocks, block_size, 1, 512]`` (PA_BSND, ``value`` is the same cache and is
    not read, as there), query_rope ``[T, N, 64]`` / key_rope ``[blocks, block_size, 1, 64]``
    or both None, sparse_indices ``[T, 1, topk]`` int32, block_table ``[1, max_blocks]``.
    Row s attends to its indices ``<= actual_seq_lengths_kv[0] - actual_seq_lengths_query[0] + s``
    (the kernel's rule, :185, applied for sparse_mode 0 and 3 alike); rows
    ``s >= actual_seq_lengths_query[0]`` are not computed there and are zero here.
    Returns ``[T, N, 512]`` in query's dtype (bf16 or fp16).  With rope parts the key cache is joined into one
    ``[blocks, block_size, 1, 576]`` copy per call, as the reference does (:406);
    callers that keep a joined cache call ``sparse_mla_fwd`` on it directly."""
    if sparse_block_size != 1:
        raise ValueError(f"sparse_block_size must be 1, got {sparse_block_size}")
    if sparse_mode not in (0, 3):
        raise ValueError(f"sparse_mode must be 0 or 3, got {sparse_mode}")
    if query.dim() != 3 or key.dim() != 4 or key.shape[2] != 1:
        raise ValueError("query must be [T, N, D] and key [blocks, block_size, 1, D]")
    if block_table is None or block_table.dim() != 2:
        raise ValueError("block_table [batch, max_blocks] is required")
    if (query_rope is None) != (key_rope is None):
        raise ValueError("query_rope and key_rope are given together or not at all")
    if block_table.shape[0] != 1 or actual_seq_lengths_query.numel() != 1 or actual_seq_lengths_kv.numel() != 1:
        raise NotImplementedError("one batch, as the reference wrapper (query.unsqueeze(0))")
    T, N, D = query.shape
    if sparse_indices.dim() != 3 or sparse_indices.shape[0] != T or sparse_indices.shape[1] != 1:
        raise ValueError(f"sparse_indices must be [{T}, 1, topk], got {tuple(sparse_indices.shape)}")
    dev = _require_gpu(query, key)
    if query_rope is not None:
        q = torch.cat((query, query_rope.to(query.dtype)), dim=-1).unsqueeze(0).contiguous()
        kv = torch.cat((key, key_rope.to(key.dtype)), dim=-1).contiguous()
    else:
        q = query.unsqueeze(0).contiguous()
        kv = key.contiguous()
    # the lengths stay on the device (no host round trip): the causal start and
    # the rows past the query length are formed there
    act_q = actual_seq_lengths_query.reshape(1).to(device=dev, dtype=torch.int32)
    act_kv = actual_seq_lengths_kv.reshape(1).to(device=dev, dtype=torch.int32)
    idx = sparse_indices.to(device=dev, dtype=torch.int32).contiguous().view(1, T, 1, -1)
    out = sparse_mla_fwd(q, kv, idx, float(scale_value), block_table=block_table, seq_len_kv=act_kv,
                         q_start_index_s=act_kv - act_q, is_causal=True, return_lse=False)[0]
    # masked_fill, not a multiply: a padded row may hold NaN / Inf, and NaN * 0 is NaN
    out.masked_fill_((torch.arange(T, device=dev, dtype=torch.int32) >= act_q).view(T, 1, 1), 0)
    return out


def sparse_attn(query_states: torch.Tensor, kv_states: torch.Tensor, attn_sink: torch.Tensor,
                topk_idxs: torch.Tensor, softmax_scale: float) -> torch.Tensor:
    """DeepSeek-V4 sparse attention with a per-head sink, on the sparse MLA core
    (examples/deepseek_v4/sparse_attention.py:171-198 for the semantics, kernel
    :27-168): q ``[b, m, h, d]`` bf16, kv ``[b, n, d]`` bf16 (K = V, d = 512),
    attn_sink ``[h]`` fp32, topk_idxs ``[b, m, topk]`` int32 -> fp32 ``[b, m, h, d]``.
    ``-1`` (and out-of-range) indices select nothing; no causal rule.  The core
    rounds P and the output to bf16 (the output is returned widened to fp32)."""
    if query_states.dim() != 4 or kv_states.dim() != 3 or topk_idxs.dim() != 3:
        raise ValueError("query_states must be [b, m, h, d], kv_states [b, n, d] and topk_idxs [b, m, topk]")
    b, m, h, d = query_states.shape
    if kv_states.shape[0] != b or kv_states.shape[2] != d:
        raise ValueError(f"kv_states must be [{b}, n, {d}], got {tuple(kv_states.shape)}")
    if tuple(topk_idxs.shape[:2]) != (b, m):
        raise ValueError(f"topk_idxs must be [{b}, {m}, topk], got {tuple(topk_idxs.shape)}")
    if d != 512:
        raise NotImplementedError(f"d = 512 only (got {d})")
    _require_gpu(query_states, kv_states, topk_idxs)
    _require_contiguous("kv_states", kv_states)
    _require_contiguous("topk_idxs", topk_idxs)
    out = sparse_mla_fwd(query_states.contiguous(), kv_states.unsqueeze(2), topk_idxs.unsqueeze(2),
                         float(softmax_scale), is_causal=False, attn_sink=attn_sink, return_lse=False)
    return out.float()


def sparse_attn_kernel(h: int, d: int, scale: Optional[float] = None) -> Callable:
    """Factory with the signature of the reference's ``sparse_attn_kernel``
    (examples/deepseek_v4/sparse_attention.py:27-34, ``out_idx=[2]``): returns
    ``kernel(q, kv, attn_sink, topk_idxs) -> output`` fp32 ``[b, m, h, d]``;
    ``scale`` defaults to ``d ** -0.5`` as there (:34)."""
    sc = (1.0 / d) ** 0.5 if scale is None else scale

    def kernel(q: torch.Tensor, kv: torch.Tensor, attn_sink: torch.Tensor, topk_idxs: torch.Tensor) -> torch.Tensor:
        if q.dim() != 4 or q.shape[2] != h or q.shape[3] != d or attn_sink.numel() != h:
            raise ValueError(f"q must be [b, m, {h}, {d}] and attn_sink [{h}]")
        return sparse_attn(q, kv, attn_sink, topk_idxs, sc)

    return kernel


# ---------------------------------------------------------------------------
# row quantisation (the producer of the indexer's fp8 operands; int8 act quant)
# ---------------------------------------------------------------------------
def _bf16_rows(name: str, x: torch.Tensor) -> torch.device:
    if x.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16, got {x.dtype}")
    dev = _require_gpu(x)
    _require_contiguous(name, x)
    if x.dim() < 1 or x.shape[-1] % 8 != 0 or x.shape[-1] == 0:
        raise ValueError(f"{name}: the last dimension must be a positive multiple of 8, got {tuple(x.shape)}")
    return dev


def act_quant(x: torch.Tensor, round_scale: bool = False) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row int8 quantisation with the outputs of ``act_quant_torch``
    (examples/deepseek_v4/act_quant.py:110-149): bf16 ``x [M, N]`` or ``[b, s, N]``
    -> ``(y int8 of x's shape, scales fp32 [M, 1] or [b, s, 1])`` with
    ``s = max(absmax, 1e-4) / 127`` (a power of two with ``round_scale``) and
    ``y = round_half_even(clamp(x / s, -127, 127))``."""
    if x.dim() not in (2, 3):
        raise ValueError(f"x must be 2-D or 3-D, got {x.dim()}-D")
    dev = _bf16_rows("x", x)
    N = x.shape[-1]
    M = x.numel() // N
    y = torch.empty(x.shape, dtype=torch.int8, device=dev)
    s = torch.empty((*x.shape[:-1], 1), dtype=torch.float32, device=dev)
    check(lib().dsa_act_quant_int8(_ptr(x), M, N, int(bool(round_scale)), _ptr(y), _ptr(s), _stream(dev)),
          "dsa_act_quant_int8")
    return y, s


def act_quant_kernel_int8_optimized(N: int, block_M: int = 32, block_N: int = 32,
                                    round_scale: bool = False) -> Callable:
    """Factory with the signature of the reference kernel
    (examples/deepseek_v4/act_quant.py:25-90), returning ``kernel(X [M, N] bf16) ->
    (Y [M, N] int8, S [M] fp32)`` as its ``out_idx=[-2, -1]`` does.  The block sizes
    only tile the reference's Ascend kernel and are accepted for compatibility;
    the scale is per whole row either way (the golden's rule, :117-149)."""
    if N % 8 != 0 or N <= 0:
        raise ValueError(f"N must be a positive multiple of 8, got {N}")

    def kernel(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        if x.dim() != 2 or x.shape[1] != N:
            raise ValueError(f"X must be [M, {N}], got {tuple(x.shape)}")
        y, s = act_quant(x, round_scale)
        return y, s.view(-1)

    return kernel


def quant_fp8(x: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-row fp8 quantisation over the last dim: bf16 ``x [..., D]`` ->
    ``(y float8_e4m3fn [..., D], scale fp32 [...])`` with
    ``scale = max(absmax / 448, FLT_MIN)`` and ``y = e4m3fn(x / scale)`` (nearest
    even).  Keys quantised this way are the indexer's ``key`` / ``key_scale``."""
    dev = _bf16_rows("x", x)
    if _FP8 is None:
        raise RuntimeError("this torch build has no float8_e4m3fn dtype")
    D = x.shape[-1]
    y = torch.empty(x.shape, dtype=_FP8, device=dev)
    s = torch.empty(x.shape[:-1], dtype=torch.float32, device=dev)
    check(lib().dsa_quant_fp8_rows(_ptr(x), x.numel() // D, D, _ptr(y), _ptr(s), _stream(dev)),
          "dsa_quant_fp8_rows")
    return y, s


def paged_slots(block_table: torch.Tensor, batch: torch.Tensor, positions: torch.Tensor,
                block_size: int) -> torch.Tensor:
    """Pool rows of key positions in a paged cache: ``block_table[b, p // block_size]
    * block_size + p % block_size`` (the PA_BSND addressing of
    examples/deepseek_v4/lightning_indexer.py:271-292); ``-1`` where the table has
    no page.  int64, on the table's device."""
    b = batch.to(device=block_table.device, dtype=torch.int64)
    p = positions.to(device=block_table.device, dtype=torch.int64)
    blk = p // block_size
    ok = (blk < block_table.shape[1]) & (p >= 0)
    page = block_table.long()[b, torch.where(ok, blk, 0)]
    return torch.where(ok & (page >= 0), page * block_size + p % block_size, -1)


def indexer_k_append_fp8(key: torch.Tensor, pool: torch.Tensor, pool_scale: torch.Tensor,
                         slots: torch.Tensor) -> None:
    """Quantise-on-append into a paged fp8 key cache: bf16 ``key [T, D]`` (or
    ``[T, 1, D]``) is quantised as :func:`quant_fp8` does and written, with its
    scale, to ``pool [blocks, block_size, 1, D]`` / ``pool_scale [blocks,
    block_size]`` at pool rows ``slots [T]`` (see :func:`paged_slots`; ``-1`` and
    rows past the pool are dropped).  The pool is the indexer's PA_BSND key."""
    if pool.dtype != _FP8 or pool_scale.dtype != torch.float32:
        raise ValueError("pool must be float8_e4m3fn and pool_scale float32")
    dev = _bf16_rows("key", key)
    _require_gpu(key, pool, pool_scale, slots)
    D = key.shape[-1]
    T = key.numel() // D
    if pool.dim() != 4 or pool.shape[2] != 1 or pool.shape[3] != D:
        raise ValueError(f"pool must be [blocks, block_size, 1, {D}], got {tuple(pool.shape)}")
    if tuple(pool_scale.shape) != tuple(pool.shape[:2]):
        raise ValueError(f"pool_scale must be {tuple(pool.shape[:2])}, got {tuple(pool_scale.shape)}")
    _require_contiguous("pool", pool)
    _require_contiguous("pool_scale", pool_scale)
    if slots.numel() != T:
        raise ValueError(f"slots must have T = {T} entries, got {slots.numel()}")
    sl = slots.to(device=dev, dtype=torch.int64).contiguous()
    rows = pool.shape[0] * pool.shape[1]
    check(lib().dsa_indexer_k_append_fp8(_ptr(key), T, D, _ptr(sl), rows, _ptr(pool), _ptr(pool_scale),
                                         _stream(dev)), "dsa_indexer_k_append_fp8")


def indexer_q_quant_fp8(query: torch.Tensor, weights: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Indexer query producer: bf16 ``query [..., N1, D]`` -> fp8 ``q8`` with one scale
    per (token, head) folded into fp32 ``weights [..., N1]``: returns ``(q8,
    weights * scale)``, the operands :func:`lightning_indexer` takes."""
    dev = _bf16_rows("query", query)
    _require_gpu(query, weights)
    if query.dim() < 2 or tuple(weights.shape) != tuple(query.shape[:-1]):
        raise ValueError(f"weights must be query.shape[:-1] = {tuple(query.shape[:-1])}, got {tuple(weights.shape)}")
    N1, D = query.shape[-2], query.shape[-1]
    T = query.numel() // (N1 * D)
    w = weights.to(torch.float32).contiguous()
    q8 = torch.empty(query.shape, dtype=_FP8, device=dev)
    wo = torch.empty(w.shape, dtype=torch.float32, device=dev)
    check(lib().dsa_indexer_q_quant_fp8(_ptr(query), _ptr(w), T, N1, D, _ptr(q8), _ptr(wo), _stream(dev)),
          "dsa_indexer_q_quant_fp8")
    return q8, wo


# ---------------------------------------------------------------------------
# DeepSeek-V4 sparse flash MLA (sliding window + compressed KV, sinks)
# ---------------------------------------------------------------------------
def sparse_flash_mla(q: torch.Tensor, *, ori_kv: torch.Tensor, cmp_kv: Optional[torch.Tensor] = None,
                     cmp_sparse_indices: Optional[torch.Tensor] = None, ori_block_table: torch.Tensor,
                     cmp_block_table: Optional[torch.Tensor] = None, cu_seqlens_q: Optional[torch.Tensor] = None,
                     seqused_q: Optional[torch.Tensor] = None, seqused_kv: torch.Tensor, sinks: torch.Tensor,
                     softmax_scale: float, cmp_ratio: Optional[int] = None, ori_mask_mode: int = 4,
                     cmp_mask_mode: int = 3, ori_win_left: int = 127, ori_win_right: int = 0,
                     layout_q: str = "TND", layout_kv: str = "PA_ND", return_softmax_lse: bool = False,
                     core_num: Optional[int] = None, topk_cmp: Optional[int] = None):
    """DeepSeek-V4 sparse flash MLA with the signature, checks and outputs of
    ``sparse_flash_mla`` (examples/deepseek_v4/sparse_flash_mla/sparse_flash_mla_api.py:94-253):
    scenario 1 (``cmp_kv`` None) attends to a window of ``ori_win_left + 1`` original
    keys, scenario 2 (``cmp_kv`` without ``cmp_sparse_indices``) also to every visible
    compressed key, scenario 3 to the listed compressed keys; sinks in the softmax
    denominator, K = V.  Semantics of sparse_flash_mla_golden.py:56-153.  ``core_num``
    and ``seqused_q`` are accepted and unused, as in the reference."""
    del seqused_q, core_num
    assert ori_mask_mode == 4, "only ori_mask_mode=4 supported"
    assert cmp_mask_mode == 3 or cmp_kv is None, "only cmp_mask_mode=3 supported"
    assert ori_win_right == 0, "only ori_win_right=0 supported"
    assert layout_kv == "PA_ND", "only layout_kv=PA_ND supported"
    assert layout_q in ("TND", "BSND"), f"unsupported layout_q={layout_q!r}"
    if q.dtype not in (torch.bfloat16, torch.float16):  # sparse_flash_mla_api.py:16-21
        raise ValueError(f"unsupported torch dtype {q.dtype}")
    scenario = 1 if cmp_kv is None else (2 if cmp_sparse_indices is None else 3)
    # the small tensors (tables, lengths, sinks, lists) may live anywhere: they are
    # moved to q's device, as sparse_flash_mla_api.py:186-214 does
    dev = _require_gpu(q, ori_kv, cmp_kv)
    # query lengths and row offsets are formed on the device (no host round trip)
    if layout_q == "TND":
        assert cu_seqlens_q is not None, "cu_seqlens_q is required for TND"
        cu = cu_seqlens_q.reshape(-1).to(device=dev, dtype=torch.int32)
        B = cu.numel() - 1
        T, N1, D = q.shape
        act_q = (cu[1:] - cu[:-1]).contiguous()
        q_prefix = cu[:-1].contiguous()
        S_max = None
    else:
        B, S_max, N1, D = q.shape
        T = B * S_max
        q_prefix = torch.arange(B, dtype=torch.int32, device=dev) * S_max
        act_q = torch.full((B,), S_max, dtype=torch.int32, device=dev)
        if cu_seqlens_q is not None:
            cu = cu_seqlens_q.reshape(-1).to(device=dev, dtype=torch.int32)
            act_q = (cu[1:] - cu[:-1]).contiguous()
    N2 = ori_kv.shape[2]
    if scenario == 3:
        ci = cmp_sparse_indices.to(torch.int32)
        N2 = ci.shape[-2]
        K = topk_cmp if topk_cmp is not None else ci.shape[-1]
        assert ci.shape[-1] == K, "topk_cmp does not match cmp_sparse_indices last dim"
        cmp_idx = ci.reshape(T, N2, K)[:, 0, :].contiguous().to(dev)
        n_cmp = K
    elif scenario == 2:
        N2 = cmp_kv.shape[2]
        cmp_idx, K = None, 0
        n_cmp = int(_host_lengths(seqused_kv).max()) // cmp_ratio
    else:
        cmp_idx, K, n_cmp = None, 0, 0
    if N1 != 64 or N2 != 1 or D != 512:
        raise ValueError(f"only N1=64, N2=1, D=512 supported (got N1={N1}, N2={N2}, D={D})")
    for name, t in (("q", q), ("ori_kv", ori_kv)) + ((("cmp_kv", cmp_kv),) if cmp_kv is not None else ()):
        if t.dtype != q.dtype:
            raise ValueError(f"{name} must have q's dtype {q.dtype}, got {t.dtype}")
        _require_contiguous(name, t)
    ori_bt = ori_block_table.to(device=dev, dtype=torch.int32).contiguous()
    cmp_bt = cmp_block_table.to(device=dev, dtype=torch.int32).contiguous() if cmp_kv is not None else None
    qp = q_prefix
    kvl = seqused_kv.to(device=dev, dtype=torch.int32).contiguous()
    sk = sinks.to(device=dev, dtype=torch.float32).contiguous()
    out = torch.empty((T, N1, D), dtype=q.dtype, device=dev)
    lse = torch.empty((T, N1), dtype=torch.float32, device=dev)
    L = lib()
    wsb = L.dsa_sparse_flash_mla_workspace_bytes(T, N1, ori_win_left, n_cmp)
    ws = torch.empty((max(wsb, 1),), dtype=torch.uint8, device=dev)
    cb, cbs, ctl = (cmp_kv.shape[0], cmp_kv.shape[1], cmp_bt.shape[1]) if cmp_kv is not None else (0, 0, 0)
    fn, name = ((L.dsa_sparse_flash_mla_f16, "dsa_sparse_flash_mla_f16") if q.dtype == torch.float16
                else (L.dsa_sparse_flash_mla, "dsa_sparse_flash_mla"))
    check(fn(_ptr(q), T, N1, D, _ptr(qp), _ptr(act_q), _ptr(kvl), B, _ptr(ori_kv),
             ori_kv.shape[0], ori_kv.shape[1], _ptr(ori_bt), ori_bt.shape[1], _ptr(cmp_kv), cb,
             cbs, _ptr(cmp_bt), ctl, _ptr(cmp_idx), K, n_cmp,
             int(cmp_ratio) if cmp_ratio is not None else 0, _ptr(sk), float(softmax_scale),
             ori_win_left, _ptr(out), _ptr(lse), _ptr(ws), wsb, _stream(dev)), name)
    if layout_q == "BSND":
        out = out.view(B, S_max, N1, D)
        lse = lse.view(B, S_max, N1)
    return (out, lse) if return_softmax_lse else out


# ---------------------------------------------------------------------------
# block-sparse indexer logits (HISA second stage)
# ---------------------------------------------------------------------------
def block_sparse_indexer_logits(q: torch.Tensor, kv_cache: torch.Tensor, topk_block_indices: torch.Tensor,
                                weights: torch.Tensor, context_lens: torch.Tensor,
                                block_tables: torch.Tensor) -> torch.Tensor:
    """Indexer logits of every key in each token's top-k logical key blocks:
    q ``[T, heads, 128]`` (fp16 or bf16), kv_cache ``[blocks, block_size, 1, 128]``,
    topk_block_indices ``[T, topk]``, weights ``[T, heads]``, context_lens ``[batch]``,
    block_tables ``[batch, max_blocks]`` (T = batch * seq_len, token t in batch
    t // seq_len) -> fp32 ``[T, topk, block_size]``, ``sum_h w_h ReLU(q_h . k)`` and
    -inf at positions past the context (examples/HISA/paged_block_sparse_mqa_attn_expert.py:425-468)."""
    if q.dim() != 3 or kv_cache.dim() != 4 or kv_cache.shape[2] != 1:
        raise ValueError("q must be [T, heads, dim] and kv_cache [blocks, block_size, 1, dim]")
    if q.dtype not in (torch.float16, torch.bfloat16) or kv_cache.dtype != q.dtype:
        raise ValueError(f"q and kv_cache must both be float16 or bfloat16, got {q.dtype} and {kv_cache.dtype}")
    T, H, D = q.shape
    B = context_lens.numel()
    if B == 0 or T % B != 0:
        raise ValueError(f"{T} tokens do not split evenly over {B} batches")
    topk = topk_block_indices.shape[-1]
    dev = _require_gpu(q, kv_cache)
    for name, t in (("q", q), ("kv_cache", kv_cache)):
        _require_contiguous(name, t)
    w = weights.to(device=dev, dtype=q.dtype).contiguous()
    if tuple(w.shape) != (T, H):
        raise ValueError(f"weights must be [T, heads] = {(T, H)}, got {tuple(w.shape)}")
    blk = topk_block_indices.to(device=dev, dtype=torch.int32).contiguous().view(T, topk)
    ctx = context_lens.to(device=dev, dtype=torch.int32).contiguous()
    bt = block_tables.to(device=dev, dtype=torch.int32).contiguous()
    bs = kv_cache.shape[1]
    out = torch.empty((T, topk, bs), dtype=torch.float32, device=dev)
    check(lib().dsa_block_sparse_indexer_logits(_ptr(q), _ptr(kv_cache), _ptr(blk), _ptr(w), _ptr(ctx), _ptr(bt), B,
                                                T // B, H, D, topk, kv_cache.shape[0], bs, bt.shape[1],
                                                int(q.dtype == torch.bfloat16), _ptr(out), _stream(dev)),
          "dsa_block_sparse_indexer_logits")
    return out


def paged_block_sparse_mqa_attn_return_logits(batch: int, seq_len: int, num_phys_blocks: int, kv_block_size: int,
                                              topk: int, heads: int, index_dim: int, max_blocks: int,
                                              num_stages: int = 2, threads: int = 2) -> Callable:
    """Factory with the signature of the reference's JIT kernel
    (examples/HISA/paged_block_sparse_mqa_attn_expert.py:54-66): returns
    ``kernel(q [T, heads, dim], kv_cache, topk_block_indices [T, topk], weights [T, heads],
    context_lens, block_tables) -> logits [T, topk, kv_block_size]`` (its ``out_idx=[3]``)."""
    del num_stages, threads
    assert topk % 4 == 0, "topk must be divisible by 4"

    def kernel(q, kv_cache, topk_block_indices, weights, context_lens, block_tables):
        if q.shape != (batch * seq_len, heads, index_dim) or kv_cache.shape[:2] != (num_phys_blocks, kv_block_size):
            raise ValueError("inputs do not match the kernel's batch, seq_len, heads, index_dim or cache shape")
        if topk_block_indices.shape[-1] != topk or block_tables.shape[-1] != max_blocks:
            raise ValueError("topk_block_indices / block_tables do not match topk / max_blocks")
        return block_sparse_indexer_logits(q, kv_cache, topk_block_indices, weights, context_lens, block_tables)

    return kernel
