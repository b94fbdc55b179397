"""MI355X-native DeepSeek Sparse Attention path: lightning indexer (fp8 MFMA),
top-k selector (radix select), sparse MLA forward (bf16 MFMA) and the fp8 / int8
row quantisers that produce the indexer's operands, hand-written
HIP kernels for gfx950 behind the C ABI in include/dsa_mi355x.h."""

from .api import (  # noqa: F401
    act_quant,
    act_quant_kernel_int8_optimized,
    block_sparse_indexer_logits,
    indexer_k_append_fp8,
    indexer_logits,
    indexer_q_quant_fp8,
    lightning_indexer,
    paged_block_sparse_mqa_attn_return_logits,
    paged_slots,
    quant_fp8,
    simple_topk_selector,
    sparse_attention_fwd,
    sparse_attn,
    sparse_attn_tilelang,
    sparse_attn_kernel,
    sparse_flash_mla,
    sparse_mla_fwd,
    topk_selector,
)
from ._lib import DSAError, LIB_PATH, lib  # noqa: F401

__all__ = [
    "lightning_indexer", "indexer_logits", "topk_selector", "simple_topk_selector",
    "sparse_mla_fwd", "sparse_attention_fwd", "sparse_attn", "sparse_attn_kernel", "sparse_attn_tilelang", "act_quant", "act_quant_kernel_int8_optimized",
    "sparse_flash_mla", "block_sparse_indexer_logits", "paged_block_sparse_mqa_attn_return_logits", "quant_fp8", "paged_slots", "indexer_k_append_fp8", "indexer_q_quant_fp8",
    "DSAError", "LIB_PATH", "lib",
]
