"""Host-side checks of the block-sparse, compute-dtype and cache extensions (no GPU)."""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest
import torch

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))

import fastest_flash_attention_amd as ffa  # noqa: E402
from fastest_flash_attention_amd.ops.attention_forward import (  # noqa: E402
    _expand_block_mask,
    resolve_forward_args,
)
from oracle import block_masks as obm  # noqa: E402
from oracle import caches as oc  # noqa: E402
from oracle import reference_forward as rf  # noqa: E402

RNG = np.random.default_rng(7)
SIZES = [(int(RNG.integers(1, 90)), int(RNG.integers(1, 90)), int(RNG.choice([1, 3, 4, 8, 16])),
          int(RNG.choice([1, 2, 5, 8, 16])), int(RNG.integers(0, 20)), int(RNG.integers(1, 40)))
         for _ in range(40)]


def _brute(S_q, S_kv, bq, bkv, pred):
    n_br, n_bc = math.ceil(S_q / bq), math.ceil(S_kv / bkv)
    out = np.zeros((n_br, n_bc), dtype=bool)
    for i in range(n_br):
        for j in range(n_bc):
            out[i, j] = any(pred(q, k) for q in range(i * bq, min((i + 1) * bq, S_q))
                            for k in range(j * bkv, min((j + 1) * bkv, S_kv)))
    return out


@pytest.mark.parametrize("S_q,S_kv,bq,bkv,off,w", SIZES[:12])
def test_oracle_masks_pinned_by_brute_force(S_q, S_kv, bq, bkv, off, w):
    """A tile is kept iff some (q, k) pair in it satisfies the element pattern."""
    want_c = _brute(S_q, S_kv, bq, bkv, lambda q, k: q + off >= k)
    assert np.array_equal(obm.causal_block_mask(S_q, S_kv, bq, bkv, off), want_c)
    want_w = _brute(S_q, S_kv, bq, bkv, lambda q, k: q + off - w + 1 <= k <= q + off)
    assert np.array_equal(obm.sliding_window_block_mask(S_q, S_kv, bq, bkv, w, off), want_w)


@pytest.mark.parametrize("S_q,S_kv,bq,bkv,off,w", SIZES)
def test_generators_match_reference_loops(S_q, S_kv, bq, bkv, off, w):
    assert np.array_equal(ffa.create_causal_block_mask(S_q, S_kv, bq, bkv, off).numpy(),
                          obm.causal_block_mask(S_q, S_kv, bq, bkv, off))
    assert np.array_equal(
        ffa.create_sliding_window_block_mask(S_q, S_kv, bq, bkv, w, off).numpy(),
        obm.sliding_window_block_mask(S_q, S_kv, bq, bkv, w, off))
    assert np.array_equal(ffa.create_local_block_mask(S_q, S_kv, bq, bkv, w).numpy(),
                          obm.local_block_mask(S_q, S_kv, bq, bkv, w))


def test_reference_generator_tests():
    """tests/test_fastest_flash.py:648-667 of the reference."""
    m = ffa.create_causal_block_mask(32, 32, 8, 8)
    assert m.shape == (4, 4) and m.dtype == torch.bool
    assert m[0, 0].item() is True and m[-1, -1].item() is True
    m = ffa.create_sliding_window_block_mask(32, 32, 8, 8, window_size=8)
    assert m.shape == (4, 4) and all(m[i, i].item() is True for i in range(4))
    m = ffa.create_local_block_mask(32, 32, 8, 8, local_radius=8)
    assert m.shape == (4, 4) and m[0, 0].item() is True
    a, b = torch.tensor([[True, False]]), torch.tensor([[True, True]])
    assert ffa.combine_block_masks(a, b).tolist() == [[True, False]]
    assert ffa.combine_block_masks(a, b, mode="or").tolist() == [[True, True]]
    with pytest.raises(ValueError):
        ffa.combine_block_masks(a, b, mode="xor")


@pytest.mark.parametrize("causal,window,q_off", [(False, None, 0), (True, None, 0),
                                                 (False, 5, 0), (True, 7, 0), (True, None, 6)])
@pytest.mark.parametrize("bs", [4, 8, 16])
def test_block_mask_expansion(causal, window, q_off, bs):
    S_q, S_kv, D = 37, 37 + q_off, 16
    g = torch.Generator().manual_seed(bs)
    q = torch.randn(1, 1, S_q, D, generator=g)
    k = torch.randn(1, 1, S_kv - q_off, D, generator=g)
    kw = {}
    if q_off:
        kw["kv_cache"] = (torch.randn(1, 1, q_off, D), torch.randn(1, 1, q_off, D))
    n_br, n_bc = math.ceil(S_q / bs), math.ceil(S_kv / bs)
    bm = torch.rand(n_br, n_bc, generator=g) < 0.6
    r = resolve_forward_args(q, k, k, causal=causal, sliding_window=window, block_size=bs,
                             block_mask=bm, **kw)
    packed, words, visited = _expand_block_mask(bm, r, torch.device("cpu"))
    assert words == math.ceil(S_kv / 64) and packed.shape == (n_br, words)
    bits = ((packed.numpy().astype(np.uint64)[:, :, None] >> np.arange(64, dtype=np.uint64))
            & np.uint64(1)).reshape(n_br, -1).astype(bool)
    for i in range(n_br):
        for key in range(words * 64):
            assert bits[i, key] == (key < S_kv and bool(bm[i, key // bs])), (i, key)
    want = obm.visited_tiles(S_q, S_kv, bs, bs, causal, window, q_off, bm.numpy())
    assert np.array_equal(visited.numpy(), want)


def test_visited_tiles_fix_the_sentinel():
    """The oracle forward's LSE of a fully masked row is log(n * 1e-30) with n the
    tiles visited_tiles counts for its query tile."""
    g = np.random.default_rng(3)
    q = g.standard_normal((1, 1, 16, 8)).astype(np.float32)
    k = g.standard_normal((1, 1, 16, 8)).astype(np.float32)
    bm = np.ones((4, 4), dtype=bool)
    bm[1, :] = [False, False, True, True]   # tile row 1 only sees keys 8..15
    _, lse = rf.forward(q, k, k, causal=True, block_size=4, block_mask=bm, return_lse=True)
    n = obm.visited_tiles(16, 16, 4, 4, causal=True, block_mask=bm)
    assert n[1] == 0  # keys 8..15 are past the causal bound of rows 4..7: nothing visited
    assert np.all(np.isneginf(lse[0, 0, 4:8, 0]))
    bm[1, :] = [False, True, True, True]
    _, lse = rf.forward(q, k, k, causal=True, block_size=4, block_mask=bm, return_lse=True)
    assert np.isfinite(lse[0, 0, 4:8, 0]).all()


def test_compute_dtype_round_trip_is_exact():
    """bf16 -> fp16 -> bf16 keeps every in-range bf16 value; fp16 -> bf16 -> fp16 is the
    bf16 rounding the reference applies (cpu_reference.py:28-32, 260-262)."""
    x = (torch.randn(4096) * 8).to(torch.bfloat16)
    assert torch.equal(x.to(torch.float16).to(torch.bfloat16), x)
    y = (torch.randn(4096) * 8).to(torch.float16)
    assert torch.equal(y.to(torch.bfloat16).to(torch.float16).float(),
                       y.to(torch.bfloat16).float())


def test_continuous_cache_matches_reference_restatement():
    g = torch.Generator().manual_seed(11)
    cache = ffa.ContinuousKVCache(max_batch=3, max_seq_len=10, num_heads=2, head_dim=4,
                                  dtype=torch.float32)
    ref = oc.ContinuousCache(3, 10, 2, 4)
    for n in (3, 1, 4):
        kn = torch.randn(3, 2, n, 4, generator=g)
        vn = torch.randn(3, 2, n, 4, generator=g)
        kf, vf = cache.append(kn, vn)
        rk, rv = ref.append(kn.numpy(), vn.numpy())
        assert np.array_equal(kf.numpy(), rk) and np.array_equal(vf.numpy(), rv)
    assert cache.seq_lens.tolist() == [8, 8, 8]
    kc, vc = cache.get_cache(2)
    assert kc.shape == (2, 2, 8, 4)
    # overflow: first entry at 8 + 3 > 10 fails before anything is written
    with pytest.raises(AssertionError, match="overflow"):
        cache.append(torch.randn(3, 2, 3, 4), torch.randn(3, 2, 3, 4))
    assert cache.seq_lens.tolist() == [8, 8, 8]
    cache.reset(torch.tensor([1]))
    assert cache.seq_lens.tolist() == [8, 0, 8]
    cache.reset()
    assert cache.get_cache(3) == (None, None)


def test_continuous_cache_partial_overflow_like_reference():
    cache = ffa.ContinuousKVCache(max_batch=2, max_seq_len=4, num_heads=1, head_dim=2,
                                  dtype=torch.float32)
    ref = oc.ContinuousCache(2, 4, 1, 2)
    cache.seq_lens[1] = 3  # entry 1 already near the end
    ref.lens[1] = 3
    kn = torch.ones(2, 1, 2, 2)
    with pytest.raises(AssertionError):
        cache.append(kn, kn)
    with pytest.raises(AssertionError):
        ref.append(kn.numpy(), kn.numpy())
    assert cache.seq_lens.tolist() == ref.lens.tolist() == [2, 3]
    assert np.array_equal(cache.k_cache.numpy(), ref.k)
