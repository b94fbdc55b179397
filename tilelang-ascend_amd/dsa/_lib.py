"""ctypes binding of libdsa_mi355x.so (declarations: include/dsa_mi355x.h).

The library is built ahead of time (``dsa.build``) and must exist: there is no
fallback path.  ``lib()`` raises ``RuntimeError`` when it is missing.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libdsa_mi355x.so"

c_i32, c_i64, c_f32, c_vp, c_sz = ctypes.c_int32, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p, ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/dsa_mi355x.h
SIGNATURES = {
    "dsa_last_error": (ctypes.c_char_p, []),
    "dsa_clear_error": (None, []),
    "dsa_abi_version": (c_i32, []),
    "dsa_topk_f32": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "dsa_topk_f32_group_max": (c_i32, [c_vp, c_i64, c_i64, c_i64, c_vp, c_vp, c_i64, c_i32, c_i32, c_vp,
                                       c_vp, c_vp]),
    "dsa_indexer_logits_fp8": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                       c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp]),
    "dsa_indexer_logits_fp8_group_max": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                                 c_i32, c_i32, c_i32, c_vp, c_i64, c_vp, c_vp, c_i64, c_vp]),
    "dsa_lightning_indexer_workspace_bytes": (c_sz, [c_i64, c_i64, c_i64]),
    "dsa_lightning_indexer_fp8": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64,
                                          c_i32, c_i32, c_i32, c_i32, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_indexer_logits_fp8_varlen": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,
                                              c_i32, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32, c_vp,
                                              c_i64, c_vp, c_vp]),
    "dsa_lightning_indexer_varlen_workspace_bytes": (c_sz, [c_i64, c_i64]),
    "dsa_lightning_indexer_fp8_varlen": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,
                                                 c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32,
                                                 c_i32, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_lightning_indexer_h16_varlen": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i32, c_vp, c_i32, c_vp, c_i32,
                                                 c_i32, c_i64, c_i64, c_i64, c_i64, c_i64, c_i32, c_i32, c_i32,
                                                 c_i32, c_i32, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_sparse_mla_workspace_bytes": (c_sz, [c_i64, c_i64, c_i32, c_i32, c_i32]),
    "dsa_sparse_mla_fwd": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i32,
                                   c_i32, c_i32, c_i64, c_i32, c_i32, c_i32, c_f32, c_i32, c_i32,
                                   c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_sparse_mla_fwd_f16": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i32,
                                       c_i32, c_i32, c_i64, c_i32, c_i32, c_i32, c_f32, c_i32, c_i32,
                                       c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_sparse_mla_fwd_noalloc": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i32,
                                           c_i32, c_i32, c_i64, c_i32, c_i32, c_i32, c_f32, c_i32, c_i32,
                                           c_vp, c_vp, c_vp]),
    "dsa_sparse_flash_mla_workspace_bytes": (c_sz, [c_i64, c_i32, c_i32, c_i32]),
    "dsa_sparse_flash_mla": (c_i32, [c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i32, c_vp,
                                     c_i32, c_vp, c_i64, c_i32, c_vp, c_i32, c_vp, c_i32, c_i32, c_i32, c_vp, c_f32,
                                     c_i32, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_sparse_flash_mla_f16": (c_i32, [c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp, c_i64, c_vp, c_i64, c_i32,
                                         c_vp, c_i32, c_vp, c_i64, c_i32, c_vp, c_i32, c_vp, c_i32, c_i32, c_i32,
                                         c_vp, c_f32, c_i32, c_vp, c_vp, c_vp, c_sz, c_vp]),
    "dsa_block_sparse_indexer_logits": (c_i32, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i32, c_i32, c_i32,
                                                c_i64, c_i32, c_i32, c_i32, c_vp, c_vp]),
    "dsa_act_quant_int8": (c_i32, [c_vp, c_i64, c_i64, c_i32, c_vp, c_vp, c_vp]),
    "dsa_quant_fp8_rows": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "dsa_indexer_k_append_fp8": (c_i32, [c_vp, c_i64, c_i32, c_vp, c_i64, c_vp, c_vp, c_vp]),
    "dsa_indexer_q_quant_fp8": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
    "dsa_quant_fp8_rows_f16": (c_i32, [c_vp, c_i64, c_i64, c_vp, c_vp, c_vp]),
    "dsa_indexer_q_quant_fp8_f16": (c_i32, [c_vp, c_vp, c_i64, c_i32, c_i32, c_vp, c_vp, c_vp]),
}

_lock = threading.Lock()
_lib = None


class DSAError(RuntimeError):
    """A C-ABI call returned a non-zero status."""


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build the HIP library first "
                    "(python -c 'import __graft_entry__ as g; g.build()' or python -m dsa.build)")
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().dsa_last_error().decode(errors="replace")
        raise DSAError(f"{what} failed with status {rc}: {msg}")
