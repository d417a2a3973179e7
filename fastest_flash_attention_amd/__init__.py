"""fastest_flash_attention_amd — MI355X-native attention.

Drop-in for the attention hot path of MindIntels/fastest_flash_attention
(reference __init__.py:40-88): the same functional entry points (forward, backward,
autograd function), modules, config and paged KV cache, with the GPU work done by
hand-written gfx950 HIP kernels in libffa.so (C ABI: include/ffa.h).
"""

from .config import AttentionConfig
from .modules import FastestFlashGQA, FastestFlashMHA, FastestFlashMLA
from .ops import (
    ContinuousKVCache,
    FastestFlashAttnFunc,
    MLALatentCache,
    PagedKVCache,
    combine_block_masks,
    create_causal_block_mask,
    create_local_block_mask,
    create_sliding_window_block_mask,
    fastest_flash_attn_backward,
    fastest_flash_attn_forward,
    fastest_flash_attn_func,
    fastest_flash_mla_decode,
    fastest_flash_paged_decode,
)
from .utils import auto_select_block_size, check_hip_available, check_triton_available

__version__ = "1.0.0"  # the reference package's version (its __init__.py:59): a drop-in

__all__ = [
    "AttentionConfig",
    "fastest_flash_attn_forward",
    "fastest_flash_attn_backward",
    "fastest_flash_attn_func",
    "FastestFlashAttnFunc",
    "fastest_flash_paged_decode",
    "fastest_flash_mla_decode",
    "MLALatentCache",
    "FastestFlashMHA",
    "FastestFlashGQA",
    "FastestFlashMLA",
    "PagedKVCache",
    "ContinuousKVCache",
    "create_causal_block_mask",
    "create_sliding_window_block_mask",
    "create_local_block_mask",
    "combine_block_masks",
    "auto_select_block_size",
    "check_hip_available",
    "check_triton_available",
]
