"""FastestFlashMLA — multi-latent attention module (reference modules/flash_mla.py:29-179).

Same architecture and outputs as the reference: latent KV down/up projection,
decoupled RoPE on a rope_dim slice of q and of a shared k_rope, attention with
D = head_dim + rope_dim over V zero-padded to D, output projection from
num_heads * D. The attention core is the HIP forward.
"""

from __future__ import annotations

import math
from typing import Optional, Sequence

import torch
import torch.nn as nn

from ..ops.attention_forward import fastest_flash_attn_forward
from ..ops.attention_func import fastest_flash_attn_func
from ..ops.mla_decode import MLALatentCache


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

    def rotate_at(self, x: torch.Tensor, positions: Sequence[int]) -> torch.Tensor:
        """RoPE of one token per batch row: x ``[B, ..., D_rope]``, token of row b at
        ``positions[b]``. Bitwise the rotation ``forward`` applies at that position
        (positions in the input dtype, fp32 angles)."""
        pos = torch.tensor(list(positions), dtype=x.dtype, device=x.device)
        freqs = pos.float()[:, None] * self.inv_freq.to(x.device)[None, :]
        emb = torch.cat([freqs, freqs], dim=-1)
        half = x.size(-1) // 2
        shape = (x.size(0),) + (1,) * (x.dim() - 2) + (half,)
        cos = emb.cos()[:, :half].reshape(shape)
        sin = emb.sin()[:, :half].reshape(shape)
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

    def project_qkv(self, x: torch.Tensor, pad_v: bool = True):
        """q, k, v_padded ``[B, H, S, head_dim + rope_dim]`` as the reference builds
        them (:129-152); with ``pad_v=False`` V stays ``[B, H, S, head_dim]`` (a view of
        the up-projection's output)."""
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
        if not pad_v:
            return q, k, v
        v_padded = torch.nn.functional.pad(v, (0, self.rope_dim))
        return q, k, v_padded

    def forward(self, x: torch.Tensor, causal: Optional[bool] = None,
                block_size: Optional[int] = None) -> torch.Tensor:
        """x: [B, S, hidden] -> [B, S, hidden]."""
        B, S, _ = x.shape
        use_causal = self.default_causal if causal is None else causal
        bs = block_size or self.block_size or None
        # V at its own head_dim: the forward and the backward take a narrower V as
        # zero-padded (the same O as with v_padded, its rope_dim tail 0; dV on V's dims)
        # and skip the P V / dO V^T / dV work on the pad
        q, k, v = self.project_qkv(x, pad_v=False)
        if self.training:
            attn = fastest_flash_attn_func(q, k, v, scale=self.scale, causal=use_causal,
                                           block_size=bs or 64)
        else:
            attn, _ = fastest_flash_attn_forward(q, k, v, scale=self.scale,
                                                 causal=use_causal, block_size=bs)
        return self.o_proj(attn.transpose(1, 2).contiguous().view(B, S, -1))

    # ---- decode over the compressed latent cache (no counterpart in the reference) ----

    def absorbed_weights(self):
        """Per-head ``(W_uk, W_uv)``, each ``[H, head_dim, latent_dim]``: the K_nope and V
        rows of kv_up_proj (reference :102-104, :141-144 split its output per head as
        [K_nope | V])."""
        w = self.kv_up_proj.weight.view(self.num_heads, 2 * self.head_dim, self.latent_dim)
        return w[:, : self.head_dim], w[:, self.head_dim:]

    def new_latent_cache(self, max_pages: int, page_size: int = 64) -> MLALatentCache:
        w = self.kv_up_proj.weight
        return MLALatentCache(max_pages=max_pages, page_size=page_size,
                              latent_dim=self.latent_dim, rope_dim=self.rope_dim,
                              dtype=w.dtype, device=w.device)

    def prefill_with_cache(self, x: torch.Tensor, cache: MLALatentCache,
                           seq_ids: Sequence[int]) -> torch.Tensor:
        """``forward(x)`` (causal prompt of new sequences ``seq_ids``, positions 0..S-1)
        that also stores every token's latent row ``[c_t | r_t]`` in ``cache``."""
        if any(cache.seq_len(s) != 0 for s in seq_ids):
            raise ValueError("prefill_with_cache starts new sequences (positions 0..S-1)")
        B, S, _ = x.shape
        out = self.forward(x, causal=True)
        latent = self.kv_down_proj(x)                               # [B, S, latent]
        k_rope = self.rope(self.k_rope_proj(x).unsqueeze(1))[:, 0]  # [B, S, rope]
        for i, sid in enumerate(seq_ids):
            cache.append(sid, latent[i], k_rope[i])
        return out

    def decode_step(self, x: torch.Tensor, cache: MLALatentCache, seq_ids: Sequence[int],
                    return_attention: bool = False):
        """One new token per sequence: x ``[B, 1, hidden]`` -> ``[B, 1, hidden]``.

        The token's latent row is appended at position ``len(seq)``, then every head
        attends over the sequence's cached rows through ``ffa_mla_decode_fwd`` with the
        absorbed query ``[W_uk^T q_nope, q_rope]``; the latent output is up-projected by
        W_uv and zero-padded over the rope dims as the reference pads V (:152). The
        result is the reference forward of the whole sequence at its last position.
        With ``return_attention`` also the attention output ``[B, H, head_dim + rope]``.
        """
        B = x.size(0)
        H, hd, R, lat = self.num_heads, self.head_dim, self.rope_dim, self.latent_dim
        if x.dim() != 3 or x.size(1) != 1 or len(seq_ids) != B:
            raise ValueError("decode_step takes x [B, 1, hidden] and one seq id per row")
        pos = [cache.seq_len(s) for s in seq_ids]
        q_nope = self.q_proj(x).view(B, H, hd)
        q_rope = self.rope.rotate_at(self.q_rope_proj(x).view(B, H, R), pos)
        latent = self.kv_down_proj(x).view(B, lat)
        k_rope = self.rope.rotate_at(self.k_rope_proj(x).view(B, R), pos)
        for i, sid in enumerate(seq_ids):
            cache.append(sid, latent[i:i + 1], k_rope[i:i + 1])
        w_uk, w_uv = self.absorbed_weights()
        # batched products over heads, operands contiguous (no transposed views)
        q_lat = torch.bmm(q_nope.transpose(0, 1).contiguous(), w_uk.contiguous())  # [H, B, lat]
        q_abs = torch.cat([q_lat.transpose(0, 1), q_rope], dim=-1).contiguous()
        o_lat, _ = cache.decode(q_abs, seq_ids, scale=self.scale)                 # [B, H, lat]
        o = torch.bmm(o_lat.transpose(0, 1).contiguous(),
                      w_uv.transpose(1, 2).contiguous()).transpose(0, 1)          # [B, H, hd]
        attn = torch.cat([o, o.new_zeros(B, H, R)], dim=-1)
        out = self.o_proj(attn.reshape(B, 1, H * (hd + R)))
        return (out, attn) if return_attention else out

    def extra_repr(self) -> str:
        return (
            f"hidden={self.hidden_size}, heads={self.num_heads}, "
            f"head_dim={self.head_dim}, latent={self.latent_dim}, "
            f"rope_dim={self.rope_dim}"
        )
