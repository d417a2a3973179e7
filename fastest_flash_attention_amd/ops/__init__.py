"""Ops layer: the forward and backward entry points, the autograd wrapper, block-sparse masks and
the KV caches."""

from .attention_backward import fastest_flash_attn_backward
from .attention_forward import fastest_flash_attn_forward
from .attention_func import FastestFlashAttnFunc, fastest_flash_attn_func
from .block_sparse import (
    combine_block_masks,
    create_causal_block_mask,
    create_local_block_mask,
    create_sliding_window_block_mask,
)
from .kv_cache import ContinuousKVCache, PagedKVCache, fastest_flash_paged_decode
from .mla_decode import MLALatentCache, fastest_flash_mla_decode

__all__ = [
    "fastest_flash_attn_forward",
    "fastest_flash_attn_backward",
    "FastestFlashAttnFunc",
    "fastest_flash_attn_func",
    "ContinuousKVCache",
    "PagedKVCache",
    "fastest_flash_paged_decode",
    "MLALatentCache",
    "fastest_flash_mla_decode",
    "create_causal_block_mask",
    "create_sliding_window_block_mask",
    "create_local_block_mask",
    "combine_block_masks",
]
