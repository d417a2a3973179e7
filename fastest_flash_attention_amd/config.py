"""Attention configuration — the same dataclass as the reference (config.py:14-81).

Fields read on the forward path: causal, sliding_window, softcap, num_kv_heads,
compute_dtype, two_pass, return_lse, block_size_q/kv. When a config is passed to
``fastest_flash_attn_forward`` its causal/softcap/sliding_window/two_pass/
compute_dtype/num_kv_heads/return_lse override the keyword arguments, and its block
sizes apply only when ``block_size`` is None (reference ops/attention_forward.py:66-73,
102-105). use_triton, pipeline_stages, dropout_p, deterministic, max_seqlen_q/kv and
page_size are kept for interface compatibility and, as in the reference, read nowhere.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional, Tuple

import torch


@dataclass
class AttentionConfig:
    block_size_q: int = 0
    block_size_kv: int = 0
    causal: bool = False
    sliding_window: Optional[int] = None
    softcap: Optional[float] = None
    num_kv_heads: Optional[int] = None
    compute_dtype: Optional[torch.dtype] = None
    use_triton: bool = True
    two_pass: bool = False
    pipeline_stages: int = 2
    return_lse: bool = False
    dropout_p: float = 0.0
    deterministic: bool = False
    max_seqlen_q: int = 0
    max_seqlen_kv: int = 0
    page_size: int = 64

    def resolve_block_sizes(self, S_q: int, S_kv: int, D: int) -> Tuple[int, int]:
        """(block_q, block_kv); a zero field is auto-selected (reference config.py:75-81)."""
        from .utils import auto_select_block_size

        bq = self.block_size_q or auto_select_block_size(S_q, S_kv, D)
        bkv = self.block_size_kv or auto_select_block_size(S_q, S_kv, D)
        return bq, bkv
