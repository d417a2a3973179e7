"""Pins oracle/mla.py (the checker of the MLA latent-cache decode) on the CPU.

1. The absorbed form equals the reference's up-projected MLA attention
   (modules/flash_mla.py:129-168) in fp64 for random weights, lengths and heads: the
   algebraic identity the kernel relies on.
2. Closed forms: one cached token gives O = its up-projected V; identical rows give the
   same O for every softmax; L = 0 gives O = 0, LSE = -inf.
3. Planted mistakes (W_uv used for the absorption, rope dims dropped from the score,
   V not zero-padded) make check 1 fail.
4. The paged gather follows the PagedKVCache index law, and MLALatentCache keeps the
   PagedKVCache bookkeeping (CPU pool).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import mla


def _case(seed, H=4, hd=16, lat=32, R=8, L=23):
    rng = np.random.default_rng(seed)
    return dict(
        q_nope=rng.standard_normal((H, hd)), q_rope=rng.standard_normal((H, R)),
        latent=rng.standard_normal((L, lat)), k_rope=rng.standard_normal((L, R)),
        w_uk=rng.standard_normal((H, hd, lat)) * 0.2, w_uv=rng.standard_normal((H, hd, lat)) * 0.2,
        scale=1.0 / np.sqrt(hd + R))


def _absorbed_full(c):
    q_abs = mla.absorbed_query(c["q_nope"], c["q_rope"], c["w_uk"])
    rows = np.concatenate([c["latent"], c["k_rope"]], axis=1)
    o_lat, lse = mla.absorbed_decode(q_abs, rows, c["latent"].shape[1], c["scale"])
    return mla.up_project(o_lat, c["w_uv"], c["q_rope"].shape[1]), lse


@pytest.mark.parametrize("seed,L,H", [(0, 23, 4), (1, 1, 2), (2, 200, 8), (3, 64, 1)])
def test_absorbed_equals_up_projected(seed, L, H):
    c = _case(seed, H=H, L=L)
    ref, ref_lse = mla.up_projected_decode(**c)
    got, lse = _absorbed_full(c)
    assert np.allclose(got, ref, atol=1e-12, rtol=1e-10)
    assert np.allclose(lse, ref_lse, atol=1e-12)
    assert np.all(got[:, c["q_nope"].shape[1]:] == 0.0)  # padded V dims stay zero


def test_closed_forms():
    c = _case(5, L=1)
    out, _ = mla.up_projected_decode(**c)
    v = c["latent"][0] @ np.transpose(c["w_uv"], (0, 2, 1))  # [H, hd]: O = V of the only token
    assert np.allclose(out[:, :16], v, atol=1e-12)
    c = _case(6, L=7)
    c["latent"][:] = c["latent"][0]
    c["k_rope"][:] = c["k_rope"][0]
    out, lse = mla.up_projected_decode(**c)
    one, lse1 = mla.up_projected_decode(**{**c, "latent": c["latent"][:1], "k_rope": c["k_rope"][:1]})
    assert np.allclose(out, one, atol=1e-12) and np.allclose(lse, lse1 + np.log(7), atol=1e-12)
    o_lat, lse0 = mla.absorbed_decode(np.ones((3, 40)), np.zeros((0, 40)), 32, 1.0)
    assert np.all(o_lat == 0) and np.all(np.isneginf(lse0))


def test_planted_mistakes_fail():
    c = _case(7, L=31)
    ref, _ = mla.up_projected_decode(**c)
    # absorbing W_uv instead of W_uk
    bad = mla.up_projected_decode(**{**c, "w_uk": c["w_uv"]})[0]
    assert not np.allclose(bad, ref, atol=1e-3)
    # rope dims dropped from the score
    bad, _ = mla.up_projected_decode(**{**c, "q_rope": np.zeros_like(c["q_rope"])})
    assert not np.allclose(bad, ref, atol=1e-3)
    # absorbed form with the wrong up-projection for O
    q_abs = mla.absorbed_query(c["q_nope"], c["q_rope"], c["w_uk"])
    rows = np.concatenate([c["latent"], c["k_rope"]], axis=1)
    o_lat, _ = mla.absorbed_decode(q_abs, rows, 32, c["scale"])
    assert not np.allclose(mla.up_project(o_lat, c["w_uk"], 8), ref, atol=1e-3)


def test_paged_rows_index_law():
    pages = np.arange(6 * 4 * 3, dtype=np.float64).reshape(6, 4, 3)
    rows = mla.paged_rows(pages, [5, 0, 2], 10)
    want = np.concatenate([pages[5], pages[0], pages[2][:2]])
    assert np.array_equal(rows, want)


def test_latent_cache_bookkeeping_cpu():
    cache = ffa.MLALatentCache(max_pages=5, page_size=4, latent_dim=8, rope_dim=4,
                               dtype=torch.float32, device="cpu")
    g = torch.Generator().manual_seed(0)
    lat = [torch.randn(n, 8, generator=g) for n in (6, 3, 5)]
    rop = [torch.randn(n, 4, generator=g) for n in (6, 3, 5)]
    assert cache.append(0, lat[0], rop[0]) == 6
    assert cache.append(1, lat[1], rop[1]) == 3
    assert cache.sequences[0]["page_table"] == [0, 1] and cache.sequences[1]["page_table"] == [2]
    cache.free_sequence(1)
    assert cache.free_pages == [3, 4, 2]
    # out of pages: the rows that fit are written, then RuntimeError
    with pytest.raises(RuntimeError):
        cache.append(2, torch.cat([lat[2], lat[2], lat[2]]), torch.cat([rop[2]] * 3))
    assert cache.sequences[2]["len"] == 12 and cache.sequences[2]["page_table"] == [3, 4, 2]
    rows = mla.paged_rows(cache.pages.numpy(), cache.sequences[0]["page_table"], 6)
    assert np.array_equal(rows, torch.cat([lat[0], rop[0]], dim=1).numpy())
    bt, lens = cache.block_tables([0, 2, 9])
    assert bt.tolist() == [[0, 1, 0], [3, 4, 2], [0, 0, 0]] and lens.tolist() == [6, 12, 0]
