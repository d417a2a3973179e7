"""GPU parity of the paged read path: ffa_paged_gather (get_kv, bit-exact) and the
split-K decode kernel ffa_paged_decode_fwd against oracle/paged.py."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import paged as opaged
from tests.gpu_util import assert_parity, np32, require_gpu, say, seeded

pytestmark = pytest.mark.gpu

BF16, F16 = torch.bfloat16, torch.float16


@pytest.mark.parametrize("dtype,page_size,D", [(BF16, 16, 128), (F16, 4, 64),
                                               (torch.float32, 64, 8), (BF16, 12, 20)])
def test_get_kv_bit_exact(dtype, page_size, D):
    require_gpu()
    g = torch.Generator().manual_seed(1)
    cache = ffa.PagedKVCache(max_pages=64, page_size=page_size, num_heads=2, head_dim=D,
                             dtype=dtype, device="cuda")
    pool = opaged.PagedPool(max_pages=64, page_size=page_size, num_heads=2, head_dim=D)
    say(f"get_kv {dtype} page {page_size} D {D}")
    for sid, n in [(0, 7), (1, 33), (0, 20), (2, 1), (1, 5)]:
        k = torch.randn(2, n, D, generator=g).to(dtype)
        v = torch.randn(2, n, D, generator=g).to(dtype)
        cache.append_tokens(sid, k.cuda(), v.cuda())
        pool.append_tokens(sid, np32(k), np32(v))
    cache.free_sequence(2)
    pool.free_sequence(2)
    cache.append_tokens(3, *(torch.randn(2, 9, D, generator=g).to(dtype) for _ in range(2)))
    for sid in (0, 1):
        ko, vo = cache.get_kv(sid)
        kr, vr = pool.get_kv(sid)
        assert np.array_equal(np32(ko), kr) and np.array_equal(np32(vo), vr)
    assert cache.get_kv(2) == (None, None)


def _build_pool(lens, Hkv, D, P, dtype, seed, poison=True):
    """Random page permutation pool (BASELINE cfg4 recipe); unused slots are NaN."""
    g = torch.Generator().manual_seed(seed)
    pages = [max(1, math.ceil(L / P)) for L in lens]
    total = sum(pages) + 5
    perm = torch.randperm(total, generator=g)
    k_pages = torch.randn(total, Hkv, P, D, generator=g).to(dtype)
    v_pages = torch.randn(total, Hkv, P, D, generator=g).to(dtype)
    bt = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    off = 0
    used = torch.zeros(total, P, dtype=torch.bool)
    for b, (L, n) in enumerate(zip(lens, pages)):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        for t in range(L):
            used[bt[b, t // P], t % P] = True
        off += n
    if poison:
        mask = ~used
        k_pages[mask.nonzero(as_tuple=True)[0], :, mask.nonzero(as_tuple=True)[1]] = float("nan")
        v_pages[mask.nonzero(as_tuple=True)[0], :, mask.nonzero(as_tuple=True)[1]] = float("nan")
    return k_pages, v_pages, bt


DECODE = [
    # name, lens, Hq, Hkv, D, page, kwargs, tokens_per_split
    ("gqa4_p16", [1, 15, 16, 17, 100, 1000, 2049], 8, 2, 128, 16, {}, None),
    ("small_splits", [33, 64, 65, 700], 8, 2, 128, 16, {}, 32),
    ("window", [5, 300, 1000], 8, 2, 128, 16, {"sliding_window": 100}, 64),
    ("softcap", [200, 513], 4, 1, 64, 16, {"softcap": 30.0}, None),
    ("mha_d192", [129, 700], 4, 4, 192, 16, {}, 128),
    ("page_nonpow2", [50, 97], 8, 2, 128, 12, {}, 64),
    ("page4_d64", [3, 40], 2, 2, 64, 4, {}, 32),
    ("g32_colgroups", [70, 300], 32, 1, 128, 16, {}, 64),
    # a last column group narrower than 16 query heads (20 = 16 + 4, 24 = 16 + 8)
    ("g20_partial_group", [70, 300, 2049], 40, 2, 128, 16, {}, 64),
    ("g24_d64_softcap", [40, 513], 24, 1, 64, 16, {"softcap": 20.0}, None),
    ("g6_d256", [100, 700], 12, 2, 256, 16, {}, 128),
    ("fp16", [100, 400], 8, 2, 128, 16, {"softcap": 50.0}, None),
    ("empty_seq", [0, 50], 4, 2, 64, 16, {}, None),
    ("negative_scale", [50, 300], 8, 2, 128, 16, {"scale": -0.1}, None),
]


@pytest.mark.parametrize("case", DECODE, ids=[c[0] for c in DECODE])
def test_decode_parity(case):
    require_gpu()
    name, lens, Hq, Hkv, D, P, kw, tps = case
    dtype = F16 if name == "fp16" else BF16
    k_pages, v_pages, bt = _build_pool(lens, Hkv, D, P, dtype, seed=3)
    q = seeded((len(lens), Hq, D), dtype, 4)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    say(f"decode {name} lens={lens} Hq{Hq} Hkv{Hkv} D{D} page{P} {kw} tps={tps}")
    o, lse = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(), bt.cuda(),
                                            lens_t.cuda(), return_lse=True, tokens_per_split=tps,
                                            **kw)
    torch.cuda.synchronize()
    ro, rl = opaged.paged_decode(np32(q), np32(k_pages), np32(v_pages), bt.numpy(), lens, **kw)
    assert_parity(o, ro, lse, rl, name)
    for b, L in enumerate(lens):
        if L == 0:
            assert torch.all(o[b] == 0) and torch.all(torch.isneginf(lse[b]))


def test_decode_permutation_invariance():
    """Relabelling physical pages (pool and block tables together) is bit-identical."""
    require_gpu()
    lens = [300, 1000, 77]
    k_pages, v_pages, bt = _build_pool(lens, 2, 128, 16, BF16, seed=5, poison=False)
    q = seeded((3, 8, 128), BF16, 6)
    perm = torch.randperm(k_pages.size(0), generator=torch.Generator().manual_seed(7))
    inv = torch.argsort(perm)
    say("decode permutation invariance")
    o1, l1 = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(), bt.cuda(),
                                            torch.tensor(lens, dtype=torch.int32).cuda(),
                                            return_lse=True)
    o2, l2 = ffa.fastest_flash_paged_decode(q.cuda(), k_pages[perm].cuda(), v_pages[perm].cuda(),
                                            inv[bt.long()].to(torch.int32).cuda(),
                                            torch.tensor(lens, dtype=torch.int32).cuda(),
                                            return_lse=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_cache_decode_matches_prefill_with_kv_cache():
    """PagedKVCache.decode == fastest_flash_attn_forward(kv_cache=get_kv) for the new
    token (two HIP paths) and == the oracle."""
    require_gpu()
    Hq, Hkv, D = 8, 2, 128
    cache = ffa.PagedKVCache(max_pages=256, page_size=16, num_heads=Hkv, head_dim=D,
                             dtype=BF16, device="cuda")
    g = torch.Generator().manual_seed(8)
    lens = [40, 257, 600]
    for sid, L in enumerate(lens):
        cache.append_tokens(sid, torch.randn(Hkv, L, D, generator=g).to(BF16).cuda(),
                            torch.randn(Hkv, L, D, generator=g).to(BF16).cuda())
    q = seeded((3, Hq, D), BF16, 9).cuda()
    say("cache.decode vs prefill kv_cache")
    o, lse = cache.decode(q, [0, 1, 2], return_lse=True)
    for sid, L in enumerate(lens):
        kf, vf = cache.get_kv(sid)
        op, lp = ffa.fastest_flash_attn_forward(
            q[sid][None, :, None, :], kf[None, :, L - 1:], vf[None, :, L - 1:],
            kv_cache=(kf[None, :, :L - 1], vf[None, :, :L - 1]), num_kv_heads=Hkv,
            return_lse=True)
        assert (o[sid].float() - op[0, :, 0].float()).abs().max().item() < 2e-2
        assert (lse[sid] - lp[0, :, 0, 0]).abs().max().item() < 1e-3


def test_cfg4_full_size_sampled():
    """BASELINE cfg4: B=64, Hq 32 / Hkv 8, D 128, page 16, L ~ U[512, 32768], random
    page permutation; the kernel runs the whole batch, the oracle checks 3 sequences."""
    require_gpu()
    g = torch.Generator().manual_seed(0)
    B, Hq, Hkv, D, P = 64, 32, 8, 128, 16
    lens = torch.randint(512, 32769, (B,), generator=g)
    pages = (lens + P - 1) // P
    total = int(pages.sum())
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.zeros(B, int(pages.max()), dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(pages[b])
        bt[b, :n] = perm[off:off + n]
        off += n
    gd = torch.Generator(device="cuda").manual_seed(1)
    k_pages = torch.randn(total, Hkv, P, D, generator=gd, device="cuda").to(BF16)
    v_pages = torch.randn(total, Hkv, P, D, generator=gd, device="cuda").to(BF16)
    q = torch.randn(B, Hq, D, generator=gd, device="cuda").to(BF16)
    say("decode cfg4 full size")
    o, lse = ffa.fastest_flash_paged_decode(q, k_pages, v_pages, bt.cuda(),
                                            lens.to(torch.int32).cuda(), return_lse=True,
                                            max_context_len=int(lens.max()))
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    for b in [int(lens.argmax()), int(lens.argmin()), 17]:
        n = int(pages[b])
        ids = bt[b, :n].long().cuda()
        kp = np32(k_pages[ids])
        vp = np32(v_pages[ids])
        sub_bt = np.arange(n, dtype=np.int32)[None]
        ro, rl = opaged.paged_decode(np32(q[b:b + 1]), kp, vp, sub_bt, [int(lens[b])])
        assert_parity(o[b:b + 1], ro, lse[b:b + 1], rl, f"cfg4 seq {b}")
