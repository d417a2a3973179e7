"""Autograd wrapper around the HIP forward and backward (reference
ops/attention_func.py:20-125).

The forward is ``fastest_flash_attn_forward`` with ``return_lse=True``; q, k, v, O and
the LSE are saved (not the attention matrix) and the backward is
``fastest_flash_attn_backward``, which recomputes P from them on the GPU. With
``num_kv_heads`` (GQA) the saved K/V keep their own head count and the backward sums
dK/dV over each head group.
"""

from __future__ import annotations

from typing import Optional

import torch
from torch.autograd import Function

from .attention_backward import fastest_flash_attn_backward
from .attention_forward import fastest_flash_attn_forward


class FastestFlashAttnFunc(Function):
    @staticmethod
    def forward(ctx, q, k, v, scale, causal, block_size, softcap, sliding_window, two_pass,
                num_kv_heads=None):
        output, lse = fastest_flash_attn_forward(
            q, k, v,
            scale=scale, causal=causal, block_size=block_size, softcap=softcap,
            sliding_window=sliding_window, two_pass=two_pass, num_kv_heads=num_kv_heads,
            return_lse=True,
        )
        ctx.save_for_backward(q, k, v, output, lse)
        ctx.scale = scale
        ctx.causal = causal
        ctx.block_size = block_size
        ctx.softcap = softcap
        ctx.sliding_window = sliding_window
        return output

    @staticmethod
    def backward(ctx, grad_output):
        q, k, v, output, lse = ctx.saved_tensors
        dq, dk, dv = fastest_flash_attn_backward(
            grad_output.contiguous(), q, k, v, output, lse,
            scale=ctx.scale, causal=ctx.causal, block_size=ctx.block_size,
            softcap=ctx.softcap, sliding_window=ctx.sliding_window,
        )
        return dq, dk, dv, None, None, None, None, None, None, None


def fastest_flash_attn_func(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    scale: Optional[float] = None,
    causal: bool = False,
    block_size: int = 64,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    two_pass: bool = False,
    num_kv_heads: Optional[int] = None,
) -> torch.Tensor:
    """Differentiable-API forward (reference ops/attention_func.py:93-125). The extra
    trailing ``num_kv_heads`` lets GQA callers skip materialising repeated KV heads."""
    # a v narrower than q / k is taken as zero-padded by the forward and the backward
    # (dV has v's dims)
    return FastestFlashAttnFunc.apply(
        q, k, v, scale, causal, block_size, softcap, sliding_window, two_pass, num_kv_heads,
    )
