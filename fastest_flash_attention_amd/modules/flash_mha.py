"""FastestFlashMHA — multi-head attention module (reference modules/flash_mha.py:20-158).

Same constructor, weights, forward signature and outputs as the reference; the
attention core is the HIP forward. q/k/v are passed as the strided
``[B, H, S, D]`` views of the projections (no copies: the kernel takes any strides).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn

from ..ops.attention_forward import fastest_flash_attn_forward
from ..ops.attention_func import fastest_flash_attn_func


class FastestFlashMHA(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        head_dim: Optional[int] = None,
        dropout: float = 0.0,
        bias: bool = False,
        causal: bool = False,
        block_size: int = 0,
        softcap: Optional[float] = None,
        sliding_window: Optional[int] = None,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim or hidden_size // num_heads
        assert self.head_dim * num_heads == hidden_size, (
            "hidden_size must equal num_heads * head_dim"
        )
        self.default_causal = causal
        self.block_size = block_size
        self.softcap = softcap
        self.sliding_window = sliding_window
        self.q_proj = nn.Linear(hidden_size, hidden_size, bias=bias)
        self.k_proj = nn.Linear(hidden_size, hidden_size, bias=bias)
        self.v_proj = nn.Linear(hidden_size, hidden_size, bias=bias)
        self.o_proj = nn.Linear(hidden_size, hidden_size, bias=bias)
        self.scale = 1.0 / math.sqrt(self.head_dim)

    def load_weights(self, w_q: torch.Tensor, w_k: torch.Tensor, w_v: torch.Tensor,
                     w_o: torch.Tensor):
        """Copy in the four projection weight matrices (reference :75-86)."""
        self.q_proj.weight.data.copy_(w_q)
        self.k_proj.weight.data.copy_(w_k)
        self.v_proj.weight.data.copy_(w_v)
        self.o_proj.weight.data.copy_(w_o)

    def _heads(self, t: torch.Tensor, B: int, S: int) -> torch.Tensor:
        return t.view(B, S, self.num_heads, self.head_dim).transpose(1, 2)

    def forward(
        self,
        x: torch.Tensor,
        causal: Optional[bool] = None,
        block_size: Optional[int] = None,
        kv_cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
        return_lse: bool = False,
    ) -> torch.Tensor | Tuple[torch.Tensor, torch.Tensor]:
        """x: [B, S, hidden] -> [B, S, hidden] (or (out, lse) with return_lse)."""
        B, S, _ = x.shape
        use_causal = self.default_causal if causal is None else causal
        bs = block_size or self.block_size or None
        q = self._heads(self.q_proj(x), B, S)
        k = self._heads(self.k_proj(x), B, S)
        v = self._heads(self.v_proj(x), B, S)
        if self.training and not return_lse and kv_cache is None:
            attn = fastest_flash_attn_func(
                q, k, v, scale=self.scale, causal=use_causal, block_size=bs or 64,
                softcap=self.softcap, sliding_window=self.sliding_window,
            )
            lse = None
        else:
            attn, lse = fastest_flash_attn_forward(
                q, k, v, scale=self.scale, causal=use_causal, block_size=bs,
                softcap=self.softcap, sliding_window=self.sliding_window,
                kv_cache=kv_cache, return_lse=return_lse,
            )
        out = self.o_proj(attn.transpose(1, 2).contiguous().view(B, S, -1))
        if return_lse:
            return out, lse
        return out

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_size}, heads={self.num_heads}, "
            f"head_dim={self.head_dim}, block_size={self.block_size}, "
            f"causal={self.default_causal}, softcap={self.softcap}, "
            f"window={self.sliding_window}"
        )
