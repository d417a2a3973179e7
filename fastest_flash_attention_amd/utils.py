"""Helpers on the forward path (reference utils.py).

``auto_select_block_size`` and ``repeat_kv`` keep the reference's semantics exactly
(utils.py:36-67, 111-130). On the GPU path the block size is a hint only: it fixes
the reference tiling that defines the LSE of rows with no visible key, while the HIP
kernel uses its own tile shapes (results are otherwise tile-size invariant).
"""

from __future__ import annotations

import math
from typing import Tuple

import torch


def check_hip_available() -> bool:
    """True when libffa.so loads and a ROCm GPU is visible (replaces utils.py:20-29)."""
    from .kernels import _lib

    return _lib.is_available()


def check_triton_available() -> bool:
    """Name kept for drop-in compatibility: reports the HIP kernel library probe.

    This package contains no Triton; the GPU path is libffa.so.
    """
    return check_hip_available()


def auto_select_block_size(
    S_q: int,
    S_kv: int,
    D: int,
    max_block: int = 256,
    min_block: int = 16,
) -> int:
    """Power-of-two tile size: ``4096 // D`` clamped to [min_block, max_block], halved
    while fewer than 4 KV tiles would remain (reference utils.py:36-67)."""
    bs = max(min_block, min(4096 // max(D, 1), max_block))
    while bs > min_block and math.ceil(S_kv / bs) < 4:
        bs //= 2
    if bs > 0:
        bs = 1 << (bs.bit_length() - 1)
    return max(min_block, min(bs, max_block))


def maybe_unsqueeze_head(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, bool]:
    """[B, S, D] -> [B, 1, S, D] (reference utils.py:98-108)."""
    if q.dim() == 3:
        return q.unsqueeze(1), k.unsqueeze(1), v.unsqueeze(1), True
    return q, k, v, False


def repeat_kv(kv: torch.Tensor, num_q_heads: int, num_kv_heads: int) -> torch.Tensor:
    """Materialise GQA/MQA KV heads: q head h uses kv head h // (Hq // Hkv)
    (reference utils.py:111-130). The HIP kernels apply this map by index instead."""
    if num_q_heads == num_kv_heads:
        return kv
    ratio = num_q_heads // num_kv_heads
    B, H_kv, S, D = kv.shape
    return kv[:, :, None, :, :].expand(B, H_kv, ratio, S, D).reshape(B, num_q_heads, S, D)
