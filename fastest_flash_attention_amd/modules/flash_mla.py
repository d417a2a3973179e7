"""FastestFlashMLA — multi-latent attention module (reference modules/flash_mla.py:29-179).

Same architecture and outputs as the reference: latent KV down/up projection,
decoupled RoPE on a rope_dim slice of q and of a shared k_rope, attention with
D = head_dim + rope_dim over V zero-padded to D, output projection from
num_heads * D. The attention core is the HIP forward.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from ..ops.attention_forward import fastest_flash_attn_forward
from ..ops.attention_func import fastest_flash_attn_func


class RotaryEmbedding(nn.Module):
    """Rotate-half RoPE over the last dim (reference modules/flash_mla.py:29-52).
    Positions are built in the input dtype, as in the reference. The result is cast
    back to the input dtype: the reference lets fp32 frequencies promote bf16/fp16
    inputs to fp32, which would leave q/k and v in different dtypes."""

    def __init__(self, dim: int, max_len: int = 8192, base: float = 10000.0):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        self.register_buffer("inv_freq", inv_freq)
        self.max_len = max_len

    def forward(self, x: torch.Tensor, offset: int = 0) -> torch.Tensor:
        S = x.size(2)
        pos = torch.arange(offset, offset + S, device=x.device, dtype=x.dtype)
        freqs = torch.outer(pos, self.inv_freq.to(x.device))
        emb = torch.cat([freqs, freqs], dim=-1)
        half = x.size(-1) // 2
        cos = emb.cos()[None, None, :, :half]
        sin = emb.sin()[None, None, :, :half]
        x1 = x[..., :half]
        x2 = x[..., half:]
        return torch.cat([x1 * cos - x2 * sin, x2 * cos + x1 * sin], dim=-1).to(x.dtype)


class FastestFlashMLA(nn.Module):
    def __init__(
        self,
        hidden_size: int,
        num_heads: int,
        head_dim: int = 128,
        latent_dim: int = 512,
        rope_dim: int = 64,
        causal: bool = True,
        block_size: int = 0,
    ):
        super().__init__()
        self.hidden_size = hidden_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.latent_dim = latent_dim
        self.rope_dim = rope_dim
        self.default_causal = causal
        self.block_size = block_size
        self.attn_dim = head_dim + rope_dim
        self.scale = 1.0 / math.sqrt(self.attn_dim)
        self.q_proj = nn.Linear(hidden_size, num_heads * head_dim, bias=False)
        self.q_rope_proj = nn.Linear(hidden_size, num_heads * rope_dim, bias=False)
        self.kv_down_proj = nn.Linear(hidden_size, latent_dim, bias=False)
        self.kv_up_proj = nn.Linear(latent_dim, num_heads * (head_dim + head_dim), bias=False)
        self.k_rope_proj = nn.Linear(hidden_size, rope_dim, bias=False)
        self.rope = RotaryEmbedding(rope_dim)
        self.o_proj = nn.Linear(num_heads * (head_dim + rope_dim), hidden_size, bias=False)

    def project_qkv(self, x: torch.Tensor):
        """q, k, v_padded ``[B, H, S, head_dim + rope_dim]`` as the reference builds
        them (:129-152)."""
        B, S, _ = x.shape
        H = self.num_heads
        q_nope = self.q_proj(x).view(B, S, H, self.head_dim).transpose(1, 2)
        q_rope = self.rope(self.q_rope_proj(x).view(B, S, H, self.rope_dim).transpose(1, 2))
        q = torch.cat([q_nope, q_rope], dim=-1)
        kv = self.kv_up_proj(self.kv_down_proj(x)).view(B, S, H, 2 * self.head_dim).transpose(1, 2)
        k_nope = kv[..., : self.head_dim]
        v = kv[..., self.head_dim:]
        k_rope = self.k_rope_proj(x).unsqueeze(1).expand(-1, H, -1, -1)
        k_rope = self.rope(k_rope)
        k = torch.cat([k_nope, k_rope], dim=-1)
        v_padded = torch.nn.functional.pad(v, (0, self.rope_dim))
        return q, k, v_padded

    def forward(self, x: torch.Tensor, causal: Optional[bool] = None,
                block_size: Optional[int] = None) -> torch.Tensor:
        """x: [B, S, hidden] -> [B, S, hidden]."""
        B, S, _ = x.shape
        use_causal = self.default_causal if causal is None else causal
        bs = block_size or self.block_size or None
        q, k, v_padded = self.project_qkv(x)
        if self.training:
            attn = fastest_flash_attn_func(q, k, v_padded, scale=self.scale, causal=use_causal,
                                           block_size=bs or 64)
        else:
            attn, _ = fastest_flash_attn_forward(q, k, v_padded, scale=self.scale,
                                                 causal=use_causal, block_size=bs)
        return self.o_proj(attn.transpose(1, 2).contiguous().view(B, S, -1))

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_size}, heads={self.num_heads}, "
            f"head_dim={self.head_dim}, latent={self.latent_dim}, "
            f"rope_dim={self.rope_dim}"
        )
