"""A seeded sweep of mixed shapes through the public API, forward and backward, against
the oracle: head_dim 16-256 (padded widths included), bf16 / fp16 / fp32, GQA ratios,
square and ragged lengths, kv_cache offsets (including more queries than keys, which
leaves fully masked rows), causal / window / softcap in every combination. The cases
are drawn once from a fixed seed, so every run checks the same list; they complement
the hand-picked cases of the other files with combinations nobody chose."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import reference_backward as rb
from oracle import reference_forward as rf
from tests.gpu_util import assert_parity, np32, require_gpu, say, seeded
from tests.test_gpu_backward import _check, _oracle_forward

pytestmark = pytest.mark.gpu

DTYPES = (torch.bfloat16, torch.float16, torch.float32)
DIMS = (16, 24, 40, 64, 72, 96, 128, 136, 160, 192, 256)


def _draw(n: int, seed: int, with_cache: bool):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice(DIMS))
        dt = DTYPES[int(rng.integers(len(DTYPES)))]
        Hkv = int(rng.choice((1, 2, 4)))
        Hq = Hkv * int(rng.choice((1, 2, 4)))
        B = int(rng.integers(1, 3))
        Sq = int(rng.integers(1, 260))
        Skv = Sq if rng.random() < 0.5 else int(rng.integers(1, 300))
        cache = int(rng.integers(1, 200)) if with_cache and rng.random() < 0.35 else 0
        causal = bool(rng.random() < 0.6)
        window = int(rng.integers(1, 150)) if rng.random() < 0.35 else None
        softcap = float(rng.choice((10.0, 30.0, 50.0))) if rng.random() < 0.3 else None
        name = (f"{i}_B{B}_H{Hq}-{Hkv}_S{Sq}x{Skv}+{cache}_D{D}_{str(dt)[6:]}"
                f"_c{int(causal)}_w{window}_cap{softcap}")
        cases.append((name, B, Hq, Hkv, Sq, Skv, cache, D, dt, causal, window, softcap))
    return cases


FWD_CASES = _draw(48, 20261202, with_cache=True)
BWD_CASES = _draw(32, 20261203, with_cache=False)


@pytest.mark.parametrize("case", FWD_CASES, ids=[c[0] for c in FWD_CASES])
def test_forward_sweep(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, cache, D, dt, causal, window, softcap = case
    seed = 7 + 13 * int(name.split("_")[0])
    q = seeded((B, Hq, Sq, D), dt, seed)
    k = seeded((B, Hkv, Skv, D), dt, seed + 1)
    v = seeded((B, Hkv, Skv, D), dt, seed + 2)
    kw = dict(causal=causal, sliding_window=window, softcap=softcap, return_lse=True)
    if Hq != Hkv:
        kw["num_kv_heads"] = Hkv
    kv_cache = None
    if cache:
        kv_cache = (seeded((B, Hkv, cache, D), dt, seed + 3), seeded((B, Hkv, cache, D), dt, seed + 4))
    say(f"forward sweep {name}")
    o, lse = ffa.fastest_flash_attn_forward(
        q.cuda(), k.cuda(), v.cuda(),
        kv_cache=None if kv_cache is None else (kv_cache[0].cuda(), kv_cache[1].cuda()), **kw)
    torch.cuda.synchronize()
    assert o.dtype == dt and o.shape == q.shape
    ro, rl = rf.forward(np32(q), np32(k), np32(v),
                        kv_cache=None if kv_cache is None else (np32(kv_cache[0]), np32(kv_cache[1])),
                        **kw)
    max_abs, _ = assert_parity(o, ro, lse, rl, name)
    if dt == torch.float32:
        assert max_abs < 1e-4, f"{name}: fp32 max-abs {max_abs:.2e}"


def _draw_long(n: int, seed: int):
    """Sweeps long enough that interior tiles run the kernels' fast step (its own max,
    rescale and softcap code), with scales whose scores span a wide range: the running
    max moves often and, with softcap, tanh spans most of [-1, 1]."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D, Dv = [(64, 64), (128, 128), (192, 128), (192, 192), (256, 256)][int(rng.integers(5))]
        dt = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
        Hkv = int(rng.choice((1, 2)))
        Hq = Hkv * int(rng.choice((1, 2)))
        Sq = int(rng.integers(600, 1300))
        Skv = Sq if rng.random() < 0.6 else int(rng.integers(600, 1300))
        causal = bool(rng.random() < 0.5)
        window = int(rng.integers(200, 700)) if rng.random() < 0.3 else None
        softcap = float(rng.choice((20.0, 50.0))) if rng.random() < 0.5 else None
        scale = float(rng.choice((-3.0, -0.5, 0.05, 0.5, 3.0)))
        name = (f"{i}_H{Hq}-{Hkv}_S{Sq}x{Skv}_D{D}v{Dv}_{str(dt)[6:]}_c{int(causal)}_w{window}"
                f"_cap{softcap}_s{scale}")
        cases.append((name, Hq, Hkv, Sq, Skv, D, Dv, dt, causal, window, softcap, scale))
    return cases


LONG_CASES = _draw_long(24, 20261205)


@pytest.mark.parametrize("case", LONG_CASES, ids=[c[0] for c in LONG_CASES])
def test_forward_sweep_long_wide_range(case):
    require_gpu()
    name, Hq, Hkv, Sq, Skv, D, Dv, dt, causal, window, softcap, scale = case
    seed = 11 + 17 * int(name.split("_")[0])
    q = seeded((1, Hq, Sq, D), dt, seed)
    k = seeded((1, Hkv, Skv, D), dt, seed + 1)
    v = seeded((1, Hkv, Skv, Dv), dt, seed + 2)
    kw = dict(causal=causal, sliding_window=window, softcap=softcap, scale=scale, return_lse=True)
    if Hq != Hkv:
        kw["num_kv_heads"] = Hkv
    say(f"forward sweep long {name}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all(), f"{name}: non-finite output"
    vp = torch.nn.functional.pad(v, (0, D - Dv))
    ro, rl = rf.forward(np32(q), np32(k), np32(vp), **kw)
    assert_parity(o, ro, lse, rl, name)


@pytest.mark.parametrize("case", BWD_CASES, ids=[c[0] for c in BWD_CASES])
def test_backward_sweep(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, _, D, dt, causal, window, softcap = case
    seed = 11 + 17 * int(name.split("_")[0])
    q = seeded((B, Hq, Sq, D), dt, seed)
    k = seeded((B, Hkv, Skv, D), dt, seed + 1)
    v = seeded((B, Hkv, Skv, D), dt, seed + 2)
    do = seeded((B, Hq, Sq, D), dt, seed + 3)
    scale = 1.0 / math.sqrt(D)
    o32, lse = _oracle_forward(q, k, v, scale=scale, causal=causal, window=window,
                               softcap=softcap, q_offset=0)
    o = torch.from_numpy(o32).to(dt)
    say(f"backward sweep {name}")
    dq, dk, dv = ffa.fastest_flash_attn_backward(
        do.cuda(), q.cuda(), k.cuda(), v.cuda(), o.cuda(), torch.from_numpy(lse).cuda(),
        scale=scale, causal=causal, softcap=softcap, sliding_window=window)
    torch.cuda.synchronize()
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(v), np32(o), lse, scale=scale,
                             causal=causal, softcap=softcap, sliding_window=window)
    _check(dq, rq, dt, f"{name} dq")
    _check(dk, rk, dt, f"{name} dk")
    _check(dv, rv, dt, f"{name} dv")


def _draw_bwd_long(n: int, seed: int):
    """Backward sweeps long enough for the kernels' interior tiles, with wide scales."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice((64, 128, 192, 256)))
        dt = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
        Hkv = int(rng.choice((1, 2)))
        Hq = Hkv * int(rng.choice((1, 2)))
        Sq = int(rng.integers(500, 1000))
        Skv = Sq if rng.random() < 0.6 else int(rng.integers(500, 1000))
        causal = bool(rng.random() < 0.6)
        window = int(rng.integers(100, 500)) if rng.random() < 0.3 else None
        softcap = float(rng.choice((20.0, 50.0))) if rng.random() < 0.4 else None
        scale = float(rng.choice((-1.0, -1.0 / math.sqrt(D), 1.0 / math.sqrt(D), 1.0)))
        name = (f"{i}_H{Hq}-{Hkv}_S{Sq}x{Skv}_D{D}_{str(dt)[6:]}_c{int(causal)}_w{window}"
                f"_cap{softcap}_s{scale:.3g}")
        cases.append((name, Hq, Hkv, Sq, Skv, D, dt, causal, window, softcap, scale))
    return cases


BWD_LONG_CASES = _draw_bwd_long(12, 20261206)


@pytest.mark.parametrize("case", BWD_LONG_CASES, ids=[c[0] for c in BWD_LONG_CASES])
def test_backward_sweep_long(case):
    require_gpu()
    name, Hq, Hkv, Sq, Skv, D, dt, causal, window, softcap, scale = case
    seed = 19 + 23 * int(name.split("_")[0])
    q = seeded((1, Hq, Sq, D), dt, seed)
    k = seeded((1, Hkv, Skv, D), dt, seed + 1)
    v = seeded((1, Hkv, Skv, D), dt, seed + 2)
    do = seeded((1, Hq, Sq, D), dt, seed + 3)
    o32, lse = _oracle_forward(q, k, v, scale=scale, causal=causal, window=window,
                               softcap=softcap, q_offset=0)
    o = torch.from_numpy(o32).to(dt)
    say(f"backward sweep long {name}")
    dq, dk, dv = ffa.fastest_flash_attn_backward(
        do.cuda(), q.cuda(), k.cuda(), v.cuda(), o.cuda(), torch.from_numpy(lse).cuda(),
        scale=scale, causal=causal, softcap=softcap, sliding_window=window)
    torch.cuda.synchronize()
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(v), np32(o), lse, scale=scale,
                             causal=causal, softcap=softcap, sliding_window=window)
    _check(dq, rq, dt, f"{name} dq")
    _check(dk, rk, dt, f"{name} dk")
    _check(dv, rv, dt, f"{name} dv")


def _draw_decode(n: int, seed: int):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice((32, 64, 96, 128, 192, 256)))
        dt = (torch.bfloat16, torch.float16)[int(rng.integers(2))]
        Hkv = int(rng.choice((1, 2, 4, 8)))
        Hq = Hkv * int(rng.choice((1, 2, 4, 8)))
        P = int(rng.choice((4, 8, 12, 16, 32, 64)))
        nseq = int(rng.integers(1, 6))
        lens = [int(x) for x in rng.integers(0, 1500, size=nseq)]
        window = int(rng.integers(1, 400)) if rng.random() < 0.3 else None
        softcap = float(rng.choice((20.0, 50.0))) if rng.random() < 0.3 else None
        tps = int(rng.choice((0, 32, 64, 256, 1024)))
        name = (f"{i}_L{'-'.join(map(str, lens))}_H{Hq}-{Hkv}_D{D}_P{P}_{str(dt)[6:]}"
                f"_w{window}_cap{softcap}_tps{tps}")
        cases.append((name, lens, Hq, Hkv, D, P, dt, window, softcap, tps or None))
    return cases


DEC_CASES = _draw_decode(24, 20261204)


@pytest.mark.parametrize("case", DEC_CASES, ids=[c[0] for c in DEC_CASES])
def test_paged_decode_sweep(case):
    require_gpu()
    from oracle import paged as opaged
    from tests.test_gpu_decode import _build_pool

    name, lens, Hq, Hkv, D, P, dt, window, softcap, tps = case
    idx = int(name.split("_")[0])
    k_pages, v_pages, bt = _build_pool(lens, Hkv, D, P, dt, seed=100 + idx)
    q = seeded((len(lens), Hq, D), dt, 200 + idx)
    kw = dict(sliding_window=window, softcap=softcap)
    say(f"decode sweep {name}")
    o, lse = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(), bt.cuda(),
                                            torch.tensor(lens, dtype=torch.int32).cuda(),
                                            return_lse=True, tokens_per_split=tps, **kw)
    torch.cuda.synchronize()
    ro, rl = opaged.paged_decode(np32(q), np32(k_pages), np32(v_pages), bt.numpy(), lens, **kw)
    assert_parity(o, ro, lse, rl, name)
    for b, L in enumerate(lens):
        if L == 0:
            assert torch.all(o[b] == 0) and torch.all(torch.isneginf(lse[b]))


DEC_WIDE_CASES = [
    # (name, lens, Hq, Hkv, D, P, dtype, window, softcap, tps, scale): scores spanning a
    # wide range, so the split kernel's running max moves and rescales often
    ("neg3", [900, 37, 1400], 8, 2, 128, 16, torch.bfloat16, None, None, 256, -3.0),
    ("pos3_softcap", [1200, 600], 8, 8, 64, 16, torch.float16, None, 50.0, 0, 3.0),
    ("neg3_softcap_window", [1500, 800], 16, 2, 128, 12, torch.bfloat16, 300, 50.0, 64, -3.0),
    ("pos1_d256", [700, 1300], 4, 1, 256, 32, torch.bfloat16, None, None, 0, 1.0),
]


@pytest.mark.parametrize("case", DEC_WIDE_CASES, ids=[c[0] for c in DEC_WIDE_CASES])
def test_paged_decode_wide_scores(case):
    require_gpu()
    from oracle import paged as opaged
    from tests.test_gpu_decode import _build_pool

    name, lens, Hq, Hkv, D, P, dt, window, softcap, tps, scale = case
    k_pages, v_pages, bt = _build_pool(lens, Hkv, D, P, dt, seed=300 + len(name))
    q = seeded((len(lens), Hq, D), dt, 400 + len(name))
    kw = dict(sliding_window=window, softcap=softcap, scale=scale)
    say(f"decode wide scores {name}")
    o, lse = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(), bt.cuda(),
                                            torch.tensor(lens, dtype=torch.int32).cuda(),
                                            return_lse=True, tokens_per_split=tps or None, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all()
    ro, rl = opaged.paged_decode(np32(q), np32(k_pages), np32(v_pages), bt.numpy(), lens, **kw)
    assert_parity(o, ro, lse, rl, name)


def _draw_narrow(n: int, seed: int):
    """V narrower than q / k (taken as zero-padded to D): the narrow-V kernels for
    16-bit inputs at head_dim 129..192 with V dims <= 128 and a multiple of 8, the
    host zero-pad elsewhere (fp32, other widths)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = int(rng.choice((136, 144, 160, 176, 192)))
        Dv = int(rng.choice((8, 32, 64, 96, 120, 128, 100, 129))) if D > 129 else 64
        Dv = min(Dv, D - 8)
        dt = DTYPES[int(rng.choice((0, 0, 1, 2)))]
        Hkv = int(rng.choice((1, 2, 4)))
        Hq = Hkv * int(rng.choice((1, 2, 4)))
        B = int(rng.integers(1, 3))
        Sq = int(rng.integers(1, 260))
        Skv = Sq if rng.random() < 0.5 else int(rng.integers(1, 300))
        cache = int(rng.integers(1, 200)) if rng.random() < 0.3 else 0
        causal = bool(rng.random() < 0.6)
        window = int(rng.integers(1, 150)) if rng.random() < 0.35 else None
        softcap = float(rng.choice((10.0, 30.0, 50.0))) if rng.random() < 0.3 else None
        name = (f"{i}_B{B}_H{Hq}-{Hkv}_S{Sq}x{Skv}+{cache}_D{D}v{Dv}_{str(dt)[6:]}"
                f"_c{int(causal)}_w{window}_cap{softcap}")
        cases.append((name, B, Hq, Hkv, Sq, Skv, cache, D, Dv, dt, causal, window, softcap))
    return cases


NARROW_CASES = _draw_narrow(20, 20261204)


@pytest.mark.parametrize("case", NARROW_CASES, ids=[c[0] for c in NARROW_CASES])
def test_forward_sweep_narrow_v(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, cache, D, Dv, dt, causal, window, softcap = case
    seed = 5 + 19 * int(name.split("_")[0])
    q = seeded((B, Hq, Sq, D), dt, seed)
    k = seeded((B, Hkv, Skv, D), dt, seed + 1)
    v = seeded((B, Hkv, Skv, Dv), dt, seed + 2)
    kw = dict(causal=causal, sliding_window=window, softcap=softcap, return_lse=True)
    if Hq != Hkv:
        kw["num_kv_heads"] = Hkv
    kv_cache = None
    if cache:
        kv_cache = (seeded((B, Hkv, cache, D), dt, seed + 3), seeded((B, Hkv, cache, Dv), dt, seed + 4))
    say(f"forward sweep narrow v {name}")
    o, lse = ffa.fastest_flash_attn_forward(
        q.cuda(), k.cuda(), v.cuda(),
        kv_cache=None if kv_cache is None else (kv_cache[0].cuda(), kv_cache[1].cuda()), **kw)
    torch.cuda.synchronize()
    assert o.dtype == dt and o.shape == q.shape
    assert torch.all(o[..., Dv:] == 0), f"{name}: O dims past v's must be 0"
    pad = lambda t: np.pad(np32(t), [(0, 0)] * 3 + [(0, D - Dv)])
    ro, rl = rf.forward(np32(q), np32(k), pad(v),
                        kv_cache=None if kv_cache is None else (np32(kv_cache[0]), pad(kv_cache[1])),
                        **kw)
    max_abs, _ = assert_parity(o, ro, lse, rl, name)
    if dt == torch.float32:
        assert max_abs < 1e-4, f"{name}: fp32 max-abs {max_abs:.2e}"
