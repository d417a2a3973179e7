"""Ops layer: the forward entry point, the autograd wrapper and the paged KV cache."""

from .attention_forward import fastest_flash_attn_forward
from .attention_func import FastestFlashAttnFunc, fastest_flash_attn_func
from .kv_cache import PagedKVCache, fastest_flash_paged_decode

__all__ = [
    "fastest_flash_attn_forward",
    "FastestFlashAttnFunc",
    "fastest_flash_attn_func",
    "PagedKVCache",
    "fastest_flash_paged_decode",
]
