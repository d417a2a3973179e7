"""FastestFlashGQA — grouped-query attention module (reference modules/flash_gqa.py:22-139).

Same interface and outputs as the reference. The reference materialises
``repeat_kv`` before calling the op (:102-103); here the KV heads are handed over
unrepeated with ``num_kv_heads`` and the HIP kernel maps q head h to kv head
``h // (num_heads // num_kv_heads)`` — the identical head map without the copy.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from ..ops.attention_forward import fastest_flash_attn_forward
from ..ops.attention_func import fastest_flash_attn_func


class FastestFlashGQA(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        num_kv_heads: int,
        head_dim: Optional[int] = None,
        bias: bool = False,
        causal: bool = False,
        block_size: int = 0,
        softcap: Optional[float] = None,
        sliding_window: Optional[int] = None,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim or hidden_size // num_heads
        self.default_causal = causal
        self.block_size = block_size
        self.softcap = softcap
        self.sliding_window = sliding_window
        assert num_heads % num_kv_heads == 0, "num_heads must be divisible by num_kv_heads"
        self.q_proj = nn.Linear(hidden_size, num_heads * self.head_dim, bias=bias)
        self.k_proj = nn.Linear(hidden_size, num_kv_heads * self.head_dim, bias=bias)
        self.v_proj = nn.Linear(hidden_size, num_kv_heads * self.head_dim, bias=bias)
        self.o_proj = nn.Linear(num_heads * self.head_dim, hidden_size, bias=bias)
        self.scale = 1.0 / math.sqrt(self.head_dim)

    def forward(
        self,
        x: torch.Tensor,
        causal: Optional[bool] = None,
        block_size: Optional[int] = None,
        kv_cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
        return_lse: bool = False,
    ) -> torch.Tensor | Tuple[torch.Tensor, torch.Tensor]:
        """x: [B, S, hidden] -> [B, S, hidden]. A kv_cache holds num_kv_heads heads."""
        B, S, _ = x.shape
        use_causal = self.default_causal if causal is None else causal
        bs = block_size or self.block_size or None
        q = self.q_proj(x).view(B, S, self.num_heads, self.head_dim).transpose(1, 2)
        k = self.k_proj(x).view(B, S, self.num_kv_heads, self.head_dim).transpose(1, 2)
        v = self.v_proj(x).view(B, S, self.num_kv_heads, self.head_dim).transpose(1, 2)
        if self.training and not return_lse and kv_cache is None:
            attn = fastest_flash_attn_func(
                q, k, v, scale=self.scale, causal=use_causal, block_size=bs or 64,
                softcap=self.softcap, sliding_window=self.sliding_window,
                num_kv_heads=self.num_kv_heads,
            )
            lse = None
        else:
            attn, lse = fastest_flash_attn_forward(
                q, k, v, scale=self.scale, causal=use_causal, block_size=bs,
                softcap=self.softcap, sliding_window=self.sliding_window,
                num_kv_heads=self.num_kv_heads, kv_cache=kv_cache, return_lse=return_lse,
            )
        out = self.o_proj(attn.transpose(1, 2).contiguous().view(B, S, -1))
        if return_lse:
            return out, lse
        return out

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_size}, q_heads={self.num_heads}, "
            f"kv_heads={self.num_kv_heads}, head_dim={self.head_dim}, "
            f"causal={self.default_causal}, softcap={self.softcap}"
        )
