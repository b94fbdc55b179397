"""The C ABI without a GPU: the library loads, exports every function that
include/dsa_mi355x.h declares with the argument counts the ctypes layer uses,
and its host-side checks and size queries behave as documented.  Nothing here
launches a kernel.  Also the Python layer's argument checks, which mirror the
reference wrapper's (examples/deepseek_v4/lightning_indexer.py:1229-1255,1280-1288)."""

import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_mi355x.h")


def _declared():
    """name -> number of parameters, for every function declared in the header."""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for m in re.finditer(r"\b(dsa_\w+)\s*\(([^;{]*?)\)\s*;", text, flags=re.S):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


@pytest.fixture(scope="module")
def L():
    from dsa import _lib
    if not _lib.LIB_PATH.exists():
        from dsa import build
        build.build()
    return _lib.lib()


def test_header_declares_the_entry_points():
    names = set(_declared())
    assert {"dsa_topk_f32", "dsa_indexer_logits_fp8", "dsa_lightning_indexer_fp8",
            "dsa_lightning_indexer_workspace_bytes", "dsa_sparse_mla_fwd",
            "dsa_sparse_mla_workspace_bytes", "dsa_last_error", "dsa_clear_error",
            "dsa_abi_version"} <= names


def test_library_exports_every_declared_symbol(L):
    from dsa._lib import SIGNATURES
    decl = _declared()
    for name, nparams in decl.items():
        assert hasattr(L, name), f"{name} declared in the header but not exported"
        assert name in SIGNATURES, f"{name} has no ctypes signature"
        assert len(SIGNATURES[name][1]) == nparams, f"{name}: header has {nparams} params"


def test_version_and_error_channel(L):
    assert L.dsa_abi_version() == 1
    L.dsa_clear_error()
    assert L.dsa_last_error() == b""
    # a negative k is rejected on the host, before any HIP call
    rc = L.dsa_topk_f32(None, 4, 16, 16, None, -1, 1, None, None, None)
    assert rc == 1
    assert b"dsa_topk_f32" in L.dsa_last_error()
    L.dsa_clear_error()
    assert L.dsa_last_error() == b""


def test_host_side_rejections(L):
    # k above the supported maximum
    assert L.dsa_topk_f32(ctypes.c_void_p(16), 1, 16, 16, None, 8193, 1, ctypes.c_void_p(16), None, None) == 3
    # ld < cols
    assert L.dsa_topk_f32(ctypes.c_void_p(16), 1, 16, 8, None, 4, 1, ctypes.c_void_p(16), None, None) == 1
    # indexer: only 64 heads x 128 dims are built
    assert L.dsa_indexer_logits_fp8(None, None, None, None, None, None, 1, 1, 1, 32, 128, 3,
                                    None, 1, None, None) == 3
    assert L.dsa_indexer_logits_fp8(None, None, None, None, None, None, 1, 1, 1, 64, 128, 1,
                                    None, 1, None, None) == 1
    # lightning indexer: workspace too small
    assert L.dsa_lightning_indexer_fp8(None, None, None, None, None, None, 1, 4, 64, 64, 128, 16, 3,
                                       None, None, None, 0, None) == 2
    assert L.dsa_lightning_indexer_fp8(None, None, None, None, None, None, 1, 4, 64, 64, 128, 0, 3,
                                       None, None, None, 0, None) == 1
    # sparse MLA: d_v, d_qk and sm_scale checks
    args = [None] * 7 + [1, 1, 16, 576, 512, 64, 0, 0, 8, 0.1, 1, 0, None, None, None, 0, None]
    bad_dv = list(args); bad_dv[11] = 256
    assert L.dsa_sparse_mla_fwd(*bad_dv) == 3
    bad_dqk = list(args); bad_dqk[10] = 640
    assert L.dsa_sparse_mla_fwd(*bad_dqk) == 3
    bad_scale = list(args); bad_scale[16] = 0.0
    assert L.dsa_sparse_mla_fwd(*bad_scale) == 1
    bad_page = list(args); bad_page[3] = ctypes.c_void_p(16); bad_page[13] = 0
    assert L.dsa_sparse_mla_fwd(*bad_page) == 1
    # an empty problem is a no-op that succeeds
    empty = list(args); empty[7] = 0
    assert L.dsa_sparse_mla_fwd(*empty) == 0
    # row quantisers: cols must be a multiple of 8; null slot map / weights; empty is a no-op
    assert L.dsa_quant_fp8_rows(None, 4, 12, None, None, None) == 1
    assert L.dsa_quant_fp8_rows(None, 4, 16, None, None, None) == 1
    assert L.dsa_act_quant_int8(None, 0, 16, 0, None, None, None) == 0
    assert L.dsa_indexer_k_append_fp8(None, 2, 128, None, 10, None, None, None) == 1
    assert L.dsa_indexer_q_quant_fp8(None, None, 1, 64, 128, None, None, None) == 1
    assert L.dsa_indexer_q_quant_fp8(None, None, 1, 0, 128, None, None, None) == 1


def test_workspace_queries(L):
    rows, S2 = 4096, 32768
    up = lambda x: (x + 255) // 256 * 256  # noqa: E731
    # logits | row lengths | maxima of 16-key groups
    want = up(rows * S2 * 4) + up(rows * 4) + rows * (S2 // 16) * 4
    assert L.dsa_lightning_indexer_workspace_bytes(1, rows, S2) == want
    assert L.dsa_lightning_indexer_varlen_workspace_bytes(rows, S2) == want
    assert L.dsa_lightning_indexer_workspace_bytes(0, rows, S2) == 0
    # prefill (many tokens): no split, no workspace
    assert L.dsa_sparse_mla_workspace_bytes(1, 4096, 128, 2048, 0) == 0
    # decode (64 tokens x 2048 keys): the index list is split, partial out + lse per split
    ws = L.dsa_sparse_mla_workspace_bytes(64, 1, 128, 2048, 0)
    unit = 64 * 128 * (512 * 2 + 8)  # fp16 partial outputs + lse + scale per (token, head)
    assert ws > 0 and ws % unit == 0 and ws // unit >= 2
    assert L.dsa_sparse_mla_workspace_bytes(64, 1, 128, 2048, 3) == 3 * unit


# ------------------------------------------------------------- Python layer checks (no GPU)
def test_python_layer_rejects_bad_arguments():
    import dsa
    with pytest.raises(ValueError, match="ROCm device"):
        dsa.topk_selector(torch.zeros(2, 8), 4)
    with pytest.raises(ValueError, match="2-D"):
        dsa.topk_selector(torch.zeros(8), 4)
    with pytest.raises(ValueError, match="float32"):
        dsa.topk_selector(torch.zeros(2, 8, dtype=torch.float16), 4)
    with pytest.raises(ValueError, match="top_k"):
        dsa.topk_selector(torch.zeros(2, 8), 0)
    f8 = torch.float8_e4m3fn
    q = torch.zeros(1, 4, 64, 128).to(f8)
    k = torch.zeros(1, 16, 1, 128).to(f8)
    w = torch.zeros(1, 4, 64)
    with pytest.raises(ValueError, match="sparse_mode"):
        dsa.lightning_indexer(q, k, w, sparse_mode=1)
    with pytest.raises(ValueError, match="sparse_count"):
        dsa.lightning_indexer(q, k, w, sparse_count=3000)
    with pytest.raises(AssertionError, match="layout"):
        dsa.lightning_indexer(q, k, w, layout_query="XYZ")
    with pytest.raises(AssertionError, match="actual_seq_lengths_query"):
        dsa.lightning_indexer(q.view(4, 64, 128), k.view(16, 1, 128), w.view(4, 64),
                              layout_query="TND", layout_key="TND")
    with pytest.raises(ValueError, match="block_table"):
        dsa.lightning_indexer(q, k.view(1, 16, 1, 128), w, layout_key="PA_BSND",
                              actual_seq_lengths_key=torch.tensor([16]))
    with pytest.raises(ValueError, match="layout_query"):
        dsa.lightning_indexer(q, k.view(16, 1, 128), w, layout_key="TND")
    with pytest.raises(ValueError, match="dtype"):
        dsa.lightning_indexer(q.float(), k.float(), w)
    bf = torch.bfloat16
    with pytest.raises(ValueError, match="bfloat16"):
        dsa.sparse_mla_fwd(torch.zeros(1, 2, 16, 576), torch.zeros(1, 8, 1, 576, dtype=bf),
                           torch.zeros(1, 2, 1, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="int32"):
        dsa.sparse_mla_fwd(torch.zeros(1, 2, 16, 576, dtype=bf), torch.zeros(1, 8, 1, 576, dtype=bf),
                           torch.zeros(1, 2, 1, 4, dtype=torch.int64))
    with pytest.raises(ValueError, match="d_qk"):
        dsa.sparse_mla_fwd(torch.zeros(1, 2, 16, 640, dtype=bf), torch.zeros(1, 8, 1, 640, dtype=bf),
                           torch.zeros(1, 2, 1, 4, dtype=torch.int32))
    with pytest.raises(ValueError, match="kv_states"):
        dsa.sparse_attn(torch.zeros(1, 2, 16, 512, dtype=bf), torch.zeros(1, 8, 256, dtype=bf),
                        torch.zeros(16), torch.zeros(1, 2, 4, dtype=torch.int32), 0.1)
    with pytest.raises(ValueError, match="attn_sink"):
        dsa.sparse_attn_kernel(h=16, d=512)(torch.zeros(1, 2, 16, 512, dtype=bf), torch.zeros(1, 8, 512, dtype=bf),
                                            torch.zeros(8), torch.zeros(1, 2, 4, dtype=torch.int32))
    with pytest.raises(NotImplementedError, match="d = 512"):
        dsa.sparse_attn(torch.zeros(1, 2, 16, 256, dtype=bf), torch.zeros(1, 8, 256, dtype=bf),
                        torch.zeros(16), torch.zeros(1, 2, 4, dtype=torch.int32), 0.1)
    q3 = torch.zeros(2, 128, 512, dtype=bf)
    key = torch.zeros(4, 64, 1, 512, dtype=bf)
    idx = torch.zeros(2, 1, 16, dtype=torch.int32)
    one = torch.ones(1, dtype=torch.int32)
    bt = torch.zeros(1, 4, dtype=torch.int32)
    with pytest.raises(ValueError, match="sparse_block_size"):
        dsa.sparse_attn_tilelang(q3, key, key, idx, 0.5, 2, one, one, block_table=bt)
    with pytest.raises(ValueError, match="sparse_mode"):
        dsa.sparse_attn_tilelang(q3, key, key, idx, 0.5, 1, one, one, sparse_mode=1, block_table=bt)
    with pytest.raises(ValueError, match="block_table"):
        dsa.sparse_attn_tilelang(q3, key, key, idx, 0.5, 1, one, one)
    with pytest.raises(ValueError, match="query_rope and key_rope"):
        dsa.sparse_attn_tilelang(q3, key, key, idx, 0.5, 1, one, one, query_rope=torch.zeros(2, 128, 64, dtype=bf),
                                 block_table=bt)
    with pytest.raises(NotImplementedError, match="one batch"):
        dsa.sparse_attn_tilelang(q3, key, key, idx, 0.5, 1, torch.ones(2, dtype=torch.int32),
                                 torch.ones(2, dtype=torch.int32), block_table=torch.zeros(2, 4, dtype=torch.int32))
