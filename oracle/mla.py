"""CPU restatement of MLA decode attention, in both forms.

TEST INFRASTRUCTURE ONLY (the checker of ffa_mla_decode_fwd and of
FastestFlashMLA.decode_step).

* up_projected_decode  the reference's attention for one new token of an MLA layer
                       (modules/flash_mla.py:129-168): per head, K = [c W_uk^T | r] and
                       V = [c W_uv^T | 0] (V zero-padded over the rope dims, :152),
                       scores scaled by 1/sqrt(head_dim + rope_dim) (:96-97), the new
                       token attending to every cached token (the kv_cache path of
                       ops/attention_forward.py:82-96 with S_q = 1).
* absorbed_decode      the same result from the latent rows [c_t | r_t] and the
                       absorbed query [W_uk^T q_nope | q_rope], as ffa_mla_decode_fwd
                       computes it; returns the latent output sum_t p_t c_t and the LSE.
* paged_rows           gather a sequence's rows from a [pages, page_size, dim] pool by
                       the PagedKVCache index law (ops/kv_cache.py:194-203).

Pinned by tests/test_oracle_mla.py: absorbed == up-projected in fp64 (the algebraic
identity the kernel relies on), single-token and identical-key closed forms, and
planted mistakes (W_uv used for the absorption, rope dims dropped, V not padded).
"""

from __future__ import annotations

from typing import Sequence, Tuple

import numpy as np


def _softmax_lse(s: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Row softmax and natural-log LSE of scores [..., L] (L >= 1)."""
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    tot = e.sum(axis=-1, keepdims=True)
    return e / tot, (m + np.log(tot))[..., 0]


def up_projected_decode(q_nope: np.ndarray, q_rope: np.ndarray, latent: np.ndarray,
                        k_rope: np.ndarray, w_uk: np.ndarray, w_uv: np.ndarray,
                        scale: float) -> Tuple[np.ndarray, np.ndarray]:
    """q_nope [H, hd], q_rope [H, R], latent [L, lat], k_rope [L, R] (rotated),
    w_uk / w_uv [H, hd, lat]. Returns (attention output [H, hd + R], lse [H])."""
    H, hd = q_nope.shape
    R = q_rope.shape[1]
    L = latent.shape[0]
    out = np.zeros((H, hd + R))
    lse = np.full(H, -np.inf)
    if L == 0:
        return out, lse
    for h in range(H):
        k = np.concatenate([latent @ w_uk[h].T, k_rope], axis=1)          # [L, hd + R]
        v = np.concatenate([latent @ w_uv[h].T, np.zeros((L, R))], axis=1)
        q = np.concatenate([q_nope[h], q_rope[h]])
        p, lse[h] = _softmax_lse((k @ q) * scale)
        out[h] = p @ v
    return out, lse


def absorbed_query(q_nope: np.ndarray, q_rope: np.ndarray, w_uk: np.ndarray) -> np.ndarray:
    """[W_uk_h^T q_nope_h | q_rope_h] per head: [H, lat + R]."""
    q_lat = np.einsum("hd,hdl->hl", q_nope, w_uk)
    return np.concatenate([q_lat, q_rope], axis=1)


def absorbed_decode(q_abs: np.ndarray, rows: np.ndarray, dim_v: int,
                    scale: float) -> Tuple[np.ndarray, np.ndarray]:
    """q_abs [H, dim_v + R], rows [L, dim_v + R]. Returns (o_lat [H, dim_v], lse [H]);
    L == 0 gives o_lat = 0 and lse = -inf."""
    H = q_abs.shape[0]
    if rows.shape[0] == 0:
        return np.zeros((H, dim_v)), np.full(H, -np.inf)
    p, lse = _softmax_lse((q_abs @ rows.T) * scale)
    return p @ rows[:, :dim_v], lse


def up_project(o_lat: np.ndarray, w_uv: np.ndarray, rope_dim: int) -> np.ndarray:
    """Attention output [H, hd + R] from the latent output: W_uv_h o_lat_h, then zeros."""
    o = np.einsum("hl,hdl->hd", o_lat, w_uv)
    return np.concatenate([o, np.zeros((o.shape[0], rope_dim))], axis=1)


def paged_rows(pages: np.ndarray, page_table: Sequence[int], length: int) -> np.ndarray:
    """Rows 0..length-1 of a sequence: token t at (page_table[t // P], t % P)."""
    P = pages.shape[1]
    t = np.arange(length)
    return pages[np.asarray(page_table, dtype=np.int64)[t // P], t % P] if length else \
        np.zeros((0, pages.shape[2]), dtype=pages.dtype)


def paged_absorbed_decode(q_abs: np.ndarray, pages: np.ndarray, block_tables: np.ndarray,
                          lens: Sequence[int], dim_v: int,
                          scale: float) -> Tuple[np.ndarray, np.ndarray]:
    """Batched absorbed decode: q_abs [B, H, dim_v + R] over each sequence's paged
    rows. Returns (o_lat [B, H, dim_v], lse [B, H]) in float64."""
    B, H, _ = q_abs.shape
    o = np.zeros((B, H, dim_v))
    lse = np.zeros((B, H))
    for b in range(B):
        rows = paged_rows(pages, block_tables[b], int(lens[b])).astype(np.float64)
        o[b], lse[b] = absorbed_decode(q_abs[b].astype(np.float64), rows, dim_v, scale)
    return o, lse
