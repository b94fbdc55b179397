"""MI355X-native DeepSeek Sparse Attention path: lightning indexer (fp8 MFMA),
top-k selector (radix select) and sparse MLA forward (bf16 MFMA), hand-written
HIP kernels for gfx950 behind the C ABI in include/dsa_mi355x.h."""

from .api import (  # noqa: F401
    indexer_logits,
    lightning_indexer,
    simple_topk_selector,
    sparse_attention_fwd,
    sparse_mla_fwd,
    topk_selector,
)
from ._lib import DSAError, LIB_PATH, lib  # noqa: F401

__all__ = [
    "lightning_indexer", "indexer_logits", "topk_selector", "simple_topk_selector",
    "sparse_mla_fwd", "sparse_attention_fwd", "DSAError", "LIB_PATH", "lib",
]
