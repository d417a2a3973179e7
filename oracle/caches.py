"""Restatement of the reference ContinuousKVCache — TEST INFRASTRUCTURE ONLY.

Only tests/ may import this module. Follows ops/kv_cache.py:18-107 line by line
(per-batch slice writes, AssertionError on overflow after the earlier entries were
written) on numpy arrays, as the checker for the product's vectorised cache. Pinned
by tests/test_host_ext.py through the index law: row t of entry b after appends of
sizes n_1, n_2, ... is the (t - sum of earlier sizes)-th row of the block that
covered position t.
"""

from __future__ import annotations

import numpy as np


class ContinuousCache:
    def __init__(self, max_batch, max_seq_len, num_heads, head_dim):
        self.max_seq_len = max_seq_len
        self.k = np.zeros((max_batch, num_heads, max_seq_len, head_dim), dtype=np.float32)
        self.v = np.zeros_like(self.k)
        self.lens = np.zeros(max_batch, dtype=np.int64)

    def append(self, k_new, v_new):
        B, H, S_new, D = k_new.shape
        for b in range(B):
            start = int(self.lens[b])
            end = start + S_new
            if end > self.max_seq_len:
                raise AssertionError(f"KV-cache overflow: {end} > {self.max_seq_len}")
            self.k[b, :, start:end, :] = k_new[b]
            self.v[b, :, start:end, :] = v_new[b]
            self.lens[b] = end
        max_len = int(self.lens[:B].max())
        return self.k[:B, :, :max_len, :], self.v[:B, :, :max_len, :]
