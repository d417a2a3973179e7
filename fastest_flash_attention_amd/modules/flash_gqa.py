"""FastestFlashGQA — grouped-query attention module (reference modules/flash_gqa.py:22-139).

Same interface and outputs as the reference. The reference materialises
``repeat_kv`` before calling the op (:102-103); here the KV heads are handed over
unrepeated with ``num_kv_heads`` and the HIP kernel maps q head h to kv head
``h // (num_heads // num_kv_heads)`` — the identical head map without the copy.

A ``kv_cache`` in the reference's layout holds ``num_heads`` heads (the reference
concatenates it with the repeated K/V, :102-103,121-125 -> ops/attention_forward.py:82-89):
then the S new K/V rows are repeated to ``num_heads`` as the reference repeats them and
the op runs with one KV head per q head. A cache of ``num_kv_heads`` heads is accepted
too (an extension: it is what the unrepeated path concatenates with, and it is
``num_heads // num_kv_heads`` times smaller).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from ..ops.attention_forward import fastest_flash_attn_forward
from ..ops.attention_func import fastest_flash_attn_func
from ..utils import repeat_kv


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
        """x: [B, S, hidden] -> [B, S, hidden] (or (out, lse) with return_lse).

        ``kv_cache = (K_c, V_c)`` is ``[B, num_heads, S_c, head_dim]`` as in the
        reference, or ``[B, num_kv_heads, S_c, head_dim]``."""
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
            kv_heads = self.num_kv_heads
            if kv_cache is not None and self._cache_heads(kv_cache) == self.num_heads != kv_heads:
                # the reference layout: its K/V are repeated before the concatenation
                k = repeat_kv(k, self.num_heads, kv_heads)
                v = repeat_kv(v, self.num_heads, kv_heads)
                kv_heads = None
            attn, lse = fastest_flash_attn_forward(
                q, k, v, scale=self.scale, causal=use_causal, block_size=bs,
                softcap=self.softcap, sliding_window=self.sliding_window,
                num_kv_heads=kv_heads, kv_cache=kv_cache, return_lse=return_lse,
            )
        out = self.o_proj(attn.transpose(1, 2).contiguous().view(B, S, -1))
        if return_lse:
            return out, lse
        return out

    @staticmethod
    def _cache_heads(kv_cache) -> int:
        k_cache = kv_cache[0]
        return 1 if k_cache.dim() == 3 else k_cache.size(1)

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_size}, q_heads={self.num_heads}, "
            f"kv_heads={self.num_kv_heads}, head_dim={self.head_dim}, "
            f"causal={self.default_causal}, softcap={self.softcap}"
        )
