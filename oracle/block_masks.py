"""Loop restatements of the reference's block-sparse helpers — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module. Each function follows the reference loop it cites
statement by statement (plain Python over numpy bool arrays), so the vectorised
generators and the block-mask expansion of the product can be checked against it.

  causal_block_mask          ops/block_sparse.py:17-45
  sliding_window_block_mask  ops/block_sparse.py:48-81
  local_block_mask           ops/block_sparse.py:84-110
  visited_tiles              kernels/cpu_reference.py:215-231 (tile skip rules)

Pinned by tests/test_host_ext.py against the reference's own generator tests
(tests/test_fastest_flash.py:648-667) and brute-force element-level definitions
(a tile is kept iff some (q, k) pair inside it satisfies the pattern).
"""

from __future__ import annotations

import math

import numpy as np


def causal_block_mask(S_q, S_kv, block_q, block_kv, q_offset=0):
    n_br, n_bc = math.ceil(S_q / block_q), math.ceil(S_kv / block_kv)
    mask = np.zeros((n_br, n_bc), dtype=bool)
    for i in range(n_br):
        q_end = q_offset + min((i + 1) * block_q, S_q) - 1
        for j in range(n_bc):
            if q_end >= j * block_kv:
                mask[i, j] = True
            else:
                break
    return mask


def sliding_window_block_mask(S_q, S_kv, block_q, block_kv, window_size, q_offset=0):
    n_br, n_bc = math.ceil(S_q / block_q), math.ceil(S_kv / block_kv)
    mask = np.zeros((n_br, n_bc), dtype=bool)
    for i in range(n_br):
        q_start = q_offset + i * block_q
        q_end = q_offset + min((i + 1) * block_q, S_q) - 1
        for j in range(n_bc):
            k_start = j * block_kv
            k_end = min((j + 1) * block_kv, S_kv) - 1
            if k_end >= q_start - window_size + 1 and k_start <= q_end:
                mask[i, j] = True
    return mask


def local_block_mask(S_q, S_kv, block_q, block_kv, local_radius):
    n_br, n_bc = math.ceil(S_q / block_q), math.ceil(S_kv / block_kv)
    mask = np.zeros((n_br, n_bc), dtype=bool)
    for i in range(n_br):
        q_center = i * block_q + block_q // 2
        for j in range(n_bc):
            k_center = j * block_kv + block_kv // 2
            if abs(q_center - k_center) <= local_radius + max(block_q, block_kv):
                mask[i, j] = True
    return mask


def visited_tiles(S_q, S_kv, block_q, block_kv, causal=False, sliding_window=None,
                  q_offset=0, block_mask=None):
    """Number of kv tiles the reference forward loop processes for each query tile
    (the tiles that add log(1e-30) to a row with no visible key)."""
    n_br, n_bc = math.ceil(S_q / block_q), math.ceil(S_kv / block_kv)
    out = np.zeros(n_br, dtype=np.int64)
    for i in range(n_br):
        qs = i * block_q
        qe = min(qs + block_q, S_q)
        q_abs_s, q_abs_e = q_offset + qs, q_offset + qe
        for j in range(n_bc):
            ks = j * block_kv
            ke = min(ks + block_kv, S_kv)
            if block_mask is not None and not block_mask[i, j]:
                continue
            if causal and ks > (q_abs_e - 1):
                break
            if sliding_window is not None and ke - 1 < q_abs_s - sliding_window + 1:
                continue
            out[i] += 1
    return out
