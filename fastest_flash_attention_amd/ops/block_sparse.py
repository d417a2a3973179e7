"""Block-sparse tile masks for ``block_mask=`` (reference ops/block_sparse.py:17-132).

A mask is a ``[n_br, n_bc]`` bool tensor over (query tile, key tile) pairs of the
``block_q x block_kv`` tiling; ``True`` keeps the tile, ``False`` drops its keys for
the tile's query rows. The HIP prefill applies it per key (see
``attention_forward._expand_block_mask``). These generators are host-side and return
CPU tensors, as the reference's do; each is written as one vectorised comparison.
"""

from __future__ import annotations

import math

import torch


def _tiles(S: int, block: int) -> torch.Tensor:
    return torch.arange(math.ceil(S / block), dtype=torch.int64)


def create_causal_block_mask(S_q: int, S_kv: int, block_q: int, block_kv: int,
                             q_offset: int = 0) -> torch.Tensor:
    """Tile (i, j) is kept when its last query row reaches the tile's first key
    (reference ops/block_sparse.py:17-45)."""
    i = _tiles(S_q, block_q)
    j = _tiles(S_kv, block_kv)
    q_last = q_offset + torch.clamp((i + 1) * block_q, max=S_q) - 1
    return q_last[:, None] >= (j * block_kv)[None, :]


def create_sliding_window_block_mask(S_q: int, S_kv: int, block_q: int, block_kv: int,
                                     window_size: int, q_offset: int = 0) -> torch.Tensor:
    """Tile (i, j) is kept when some key of it lies in [q - window + 1, q] for some
    query row of tile i (reference ops/block_sparse.py:48-81)."""
    i = _tiles(S_q, block_q)
    j = _tiles(S_kv, block_kv)
    q_first = q_offset + i * block_q
    q_last = q_offset + torch.clamp((i + 1) * block_q, max=S_q) - 1
    k_first = j * block_kv
    k_last = torch.clamp((j + 1) * block_kv, max=S_kv) - 1
    return ((k_last[None, :] >= (q_first - window_size + 1)[:, None])
            & (k_first[None, :] <= q_last[:, None]))


def create_local_block_mask(S_q: int, S_kv: int, block_q: int, block_kv: int,
                            local_radius: int) -> torch.Tensor:
    """Tile (i, j) is kept when the tile centres are within
    ``local_radius + max(block_q, block_kv)`` (reference ops/block_sparse.py:84-110)."""
    q_center = _tiles(S_q, block_q) * block_q + block_q // 2
    k_center = _tiles(S_kv, block_kv) * block_kv + block_kv // 2
    reach = local_radius + max(block_q, block_kv)
    return (q_center[:, None] - k_center[None, :]).abs() <= reach


def combine_block_masks(*masks: torch.Tensor, mode: str = "and") -> torch.Tensor:
    """Intersection (``"and"``) or union (``"or"``) of same-shape masks
    (reference ops/block_sparse.py:113-132)."""
    if not masks:
        raise ValueError("combine_block_masks needs at least one mask")
    if mode not in ("and", "or"):
        raise ValueError(f"Unknown mode: {mode!r}")
    out = masks[0]
    for m in masks[1:]:
        out = (out & m) if mode == "and" else (out | m)
    return out
