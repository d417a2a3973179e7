"""Brute-force masked scaled-dot-product attention in float64.

TEST INFRASTRUCTURE ONLY (pins the oracle; never used by the product).

The textbook form of the reference test-suite oracle ``_naive_sdpa``
(reference tests/test_fastest_flash.py:55-88): full score matrix, softcap, causal
triangle, window mask, max-subtracted softmax with NaN rows -> 0, P @ V. Extended
with the absolute query offset of the kv_cache path (ops/attention_forward.py:82-89)
and the row logsumexp (tests/test_fastest_flash.py:806-810).
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np


def visible_mask(S_q: int, S_kv: int, causal: bool, window: Optional[int],
                 q_offset: int = 0) -> np.ndarray:
    """[S_q, S_kv] bool, True where query row i may attend to key j."""
    rows = q_offset + np.arange(S_q)[:, None]
    cols = np.arange(S_kv)[None, :]
    vis = np.ones((S_q, S_kv), dtype=bool)
    if causal:
        vis &= cols <= rows
    if window is not None:
        vis &= cols >= rows - window + 1
    return vis


def naive_sdpa(q, k, v, scale: Optional[float] = None, causal: bool = False,
               softcap: Optional[float] = None, window: Optional[int] = None,
               q_offset: int = 0) -> Tuple[np.ndarray, np.ndarray]:
    """(O, LSE) in float64; q [.., S_q, D], k/v [.., S_kv, D] broadcastable."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    D = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    s = np.matmul(q, np.swapaxes(k, -1, -2)) * scale
    if softcap is not None:
        s = softcap * np.tanh(s / softcap)
    vis = visible_mask(q.shape[-2], k.shape[-2], causal, window, q_offset)
    s = np.where(vis, s, -np.inf)
    with np.errstate(invalid="ignore", divide="ignore"):
        m = np.max(s, axis=-1, keepdims=True)
        e = np.exp(s - m)
        w = e / np.sum(e, axis=-1, keepdims=True)
        w = np.nan_to_num(w, nan=0.0)
        lse = m + np.log(np.sum(e, axis=-1, keepdims=True))
    lse = np.where(np.isnan(lse), -np.inf, lse)
    return np.matmul(w, v), lse
