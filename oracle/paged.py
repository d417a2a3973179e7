"""CPU restatement of the paged KV cache and of decode attention over it.

TEST INFRASTRUCTURE ONLY (the checker of ffa_paged_gather / ffa_paged_decode_fwd).

* PagedPool           PagedKVCache bookkeeping and index law (ops/kv_cache.py:110-240):
                      pool [max_pages, H, page_size, D], free list popped from the front
                      (:157-161), freed pages appended to the tail (:163-168), token t at
                      (page_table[t // page_size], t % page_size) (:192-204).
* gather_sequence     get_kv (:208-232): contiguous [H, L, D], bit-exact.
* paged_decode        get_kv per sequence, then the reference forward with the new token
                      as the query at absolute position L-1 (kv_cache path,
                      ops/attention_forward.py:82-96; GQA by repeat_kv :94-96).
"""

from __future__ import annotations

import math
from typing import Optional, Sequence, Tuple

import numpy as np

from .reference_forward import flash_attn_cpu_forward, repeat_kv


class PagedPool:
    def __init__(self, max_pages: int, page_size: int, num_heads: int, head_dim: int,
                 dtype=np.float32):
        self.max_pages = max_pages
        self.page_size = page_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.k_pages = np.zeros((max_pages, num_heads, page_size, head_dim), dtype=dtype)
        self.v_pages = np.zeros_like(self.k_pages)
        self.free_pages = list(range(max_pages))
        self.sequences: dict = {}

    def allocate_page(self) -> int:
        if not self.free_pages:
            raise RuntimeError("PagedKVCache: out of physical pages")
        return self.free_pages.pop(0)

    def free_sequence(self, seq_id: int) -> None:
        if seq_id in self.sequences:
            for page in self.sequences[seq_id]["page_table"]:
                self.free_pages.append(page)
            del self.sequences[seq_id]

    def append_tokens(self, seq_id: int, k_tokens: np.ndarray, v_tokens: np.ndarray) -> int:
        """The reference per-token loop, literally (:186-206)."""
        seq = self.sequences.setdefault(seq_id, {"page_table": [], "len": 0})
        for t in range(k_tokens.shape[1]):
            cur = seq["len"]
            page_idx, offset = cur // self.page_size, cur % self.page_size
            while len(seq["page_table"]) <= page_idx:
                seq["page_table"].append(self.allocate_page())
            phys = seq["page_table"][page_idx]
            self.k_pages[phys, :, offset, :] = k_tokens[:, t, :]
            self.v_pages[phys, :, offset, :] = v_tokens[:, t, :]
            seq["len"] += 1
        return seq["len"]

    def get_kv(self, seq_id: int):
        if seq_id not in self.sequences or self.sequences[seq_id]["len"] == 0:
            return None, None
        seq = self.sequences[seq_id]
        return gather_sequence(self.k_pages, self.v_pages, seq["page_table"], seq["len"])


def token_location(page_table: Sequence[int], t: int, page_size: int) -> Tuple[int, int]:
    """Index law: (physical page, slot) of token t."""
    return page_table[t // page_size], t % page_size


def gather_sequence(k_pages, v_pages, page_table: Sequence[int], length: int):
    """get_kv: copy pages in page-table order, truncating the last page (:225-230)."""
    H, P, D = k_pages.shape[1], k_pages.shape[2], k_pages.shape[3]
    k_out = np.empty((H, length, D), dtype=k_pages.dtype)
    v_out = np.empty_like(k_out)
    pos = 0
    for page in page_table:
        n = min(P, length - pos)
        if n <= 0:
            break
        k_out[:, pos:pos + n] = k_pages[page, :, :n]
        v_out[:, pos:pos + n] = v_pages[page, :, :n]
        pos += n
    return k_out, v_out


def paged_decode(q: np.ndarray, k_pages: np.ndarray, v_pages: np.ndarray,
                 block_tables: np.ndarray, context_lens: Sequence[int],
                 scale: Optional[float] = None, softcap: Optional[float] = None,
                 sliding_window: Optional[int] = None,
                 block_size: Optional[int] = 256) -> Tuple[np.ndarray, np.ndarray]:
    """Decode oracle. q [B, Hq, D] -> (O fp32 [B, Hq, D], LSE fp32 [B, Hq]).

    Sequence b: K, V = get_kv(b) ([Hkv, L, D]); the query is the last token, at
    absolute position L-1, attending to all L cached keys (the reference call with
    kv_cache = first L-1 tokens: q_offset = L-1). A sequence with L = 0 has no
    reference result; it is defined here as O = 0, LSE = -inf.
    """
    B, Hq, D = q.shape
    Hkv = k_pages.shape[1]
    out = np.zeros((B, Hq, D), dtype=np.float32)
    lse = np.full((B, Hq), -np.inf, dtype=np.float32)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    for b in range(B):
        L = int(context_lens[b])
        if L == 0:
            continue
        kb, vb = gather_sequence(k_pages, v_pages, list(block_tables[b]), L)
        kb = repeat_kv(kb[None].astype(np.float32), Hq, Hkv)
        vb = repeat_kv(vb[None].astype(np.float32), Hq, Hkv)
        bs = block_size or 64
        o, l = flash_attn_cpu_forward(q[b][None, :, None, :].astype(np.float32), kb, vb,
                                      scale=scale, causal=False, block_q=bs, block_kv=bs,
                                      softcap=softcap, sliding_window=sliding_window,
                                      q_offset=L - 1, return_lse=True)
        out[b] = o[0, :, 0, :]
        lse[b] = l[0, :, 0, 0]
    return out, lse
