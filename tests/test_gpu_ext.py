"""GPU parity of the block-sparse and compute-dtype prefill options, the HIP paged
append (ffa_paged_append) and ContinuousKVCache on the device."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import reference_forward as rf
from tests.gpu_util import assert_parity, np32, require_gpu, say, seeded

pytestmark = pytest.mark.gpu

BF16, F16 = torch.bfloat16, torch.float16

# (name, B, Hq, Hkv, Sq, Skv, D, block, keep-prob, kwargs, dtype)
BM_CASES = [
    ("dense_mask", 1, 2, 2, 96, 96, 64, 16, 1.0, {}, BF16),
    ("sparse", 2, 2, 2, 130, 130, 64, 16, 0.6, {}, BF16),
    ("sparse_causal", 1, 4, 4, 200, 200, 128, 32, 0.7, {"causal": True}, BF16),
    ("sparse_window_softcap", 1, 2, 2, 160, 160, 128, 16, 0.7,
     {"causal": True, "sliding_window": 40, "softcap": 20.0}, BF16),
    ("sparse_gqa_d192", 1, 4, 2, 100, 100, 192, 8, 0.5, {"num_kv_heads": 2}, BF16),
    ("sparse_fp16_small_blocks", 1, 2, 2, 40, 40, 32, 4, 0.5, {"causal": True}, F16),
    ("sparse_rect", 1, 2, 2, 48, 150, 64, 16, 0.6, {}, BF16),
    # fp32 inputs (the split fp32 kernel at these grid sizes)
    ("sparse_fp32_causal", 1, 4, 4, 200, 200, 64, 16, 0.6, {"causal": True}, torch.float32),
    ("sparse_fp32_gqa_window_softcap", 1, 4, 2, 150, 170, 128, 32, 0.7,
     {"sliding_window": 60, "softcap": 25.0, "num_kv_heads": 2}, torch.float32),
]


@pytest.mark.parametrize("case", BM_CASES, ids=[c[0] for c in BM_CASES])
def test_block_mask_parity(case):
    """Masked tiles contribute nothing; rows whose visible keys all sit in masked tiles
    carry the reference's sentinel LSE (log(n * 1e-30) or -inf)."""
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, bs, keep, kw, dt = case
    q = seeded((B, Hq, Sq, D), dt, 21)
    k = seeded((B, Hkv, Skv, D), dt, 22)
    v = seeded((B, Hkv, Skv, D), dt, 23)
    g = torch.Generator().manual_seed(24)
    bm = torch.rand(math.ceil(Sq / bs), math.ceil(Skv / bs), generator=g) < keep
    if keep < 1.0:
        bm[0, :] = False   # one query tile fully masked: sentinel rows
    say(f"block_mask {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} bs{bs} {kw} {dt}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), block_size=bs,
                                            block_mask=bm, return_lse=True, **kw)
    torch.cuda.synchronize()
    ro, rl = rf.forward(np32(q), np32(k), np32(v), block_size=bs, block_mask=bm.numpy(),
                        return_lse=True, **kw)
    assert_parity(o, ro, lse, rl, name)
    if keep < 1.0:
        assert np.all(np32(o)[:, :, :bs] == 0)


@pytest.mark.parametrize("S,bs,H", [(230, 32, 4), (4200, 64, 1)])
def test_block_mask_narrow_v(S, bs, H):
    """A block mask on the narrow-V kernel (head_dim 192 over a 128-dim V taken as
    zero-padded): its live-tile list sits in dynamic LDS beside the K/V buffers. At
    4200 rows the eight-wave (256-row) workgroups build the list."""
    require_gpu()
    B, D, Dv = 1, 192, 128
    q = seeded((B, H, S, D), BF16, 31)
    k = seeded((B, H, S, D), BF16, 32)
    v = seeded((B, H, S, Dv), BF16, 33)
    g = torch.Generator().manual_seed(34)
    bm = torch.rand(math.ceil(S / bs), math.ceil(S / bs), generator=g) < 0.6
    bm[0, :] = False
    say(f"block_mask narrow v B{B} H{H} S{S} D{D} Dv{Dv} bs{bs}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), block_size=bs,
                                            block_mask=bm, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.all(o[..., Dv:] == 0)
    vp = torch.nn.functional.pad(v, (0, D - Dv))
    ro, rl = rf.forward(np32(q), np32(k), np32(vp), block_size=bs, block_mask=bm.numpy(),
                        causal=True, return_lse=True)
    assert_parity(o, ro, lse, rl, "block_mask narrow v")


# Masks that leave whole 64-key tiles of a workgroup's rows empty, so the kernel's
# live-tile list skips them: (name, Sq, Skv, D, block, mask kind, kwargs)
SKIP_CASES = [
    ("local_b64", 1024, 1024, 128, 64, "local", {"causal": True}),
    ("local_b128_noncausal", 768, 1024, 64, 128, "local", {}),
    ("local_b32_d192_window", 640, 640, 192, 32, "local", {"causal": True, "sliding_window": 300}),
    ("stripes_b64", 512, 1024, 128, 64, "stripes", {}),
]


@pytest.mark.parametrize("case", SKIP_CASES, ids=[c[0] for c in SKIP_CASES])
def test_block_mask_tile_skipping_parity(case):
    """Sparse block masks whose masked tiles the kernel never loads or computes: same O
    and LSE as the reference loop, which skips them too (cpu_reference.py:220-222)."""
    require_gpu()
    name, Sq, Skv, D, bs, kind, kw = case
    q = seeded((1, 2, Sq, D), BF16, 41)
    k = seeded((1, 2, Skv, D), BF16, 42)
    v = seeded((1, 2, Skv, D), BF16, 43)
    n_br, n_bc = math.ceil(Sq / bs), math.ceil(Skv / bs)
    if kind == "local":
        bm = ffa.create_local_block_mask(Sq, Skv, bs, bs, local_radius=2 * bs).cpu()
    else:
        bm = torch.zeros(n_br, n_bc, dtype=torch.bool)
        bm[:, ::3] = True   # every third key block
    say(f"block_mask skip {name} Sq{Sq} Skv{Skv} D{D} bs{bs} {kind} {kw}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), block_size=bs,
                                            block_mask=bm, return_lse=True, **kw)
    torch.cuda.synchronize()
    ro, rl = rf.forward(np32(q), np32(k), np32(v), block_size=bs, block_mask=bm.numpy(),
                        return_lse=True, **kw)
    assert_parity(o, ro, lse, rl, name)


def test_block_mask_long_sweep_visits_every_tile():
    """A sweep longer than the live-tile list (2048 tiles of 64 keys) visits every tile;
    an all-true mask there still equals the unmasked result bit for bit."""
    require_gpu()
    Skv = 2048 * 64 + 1000
    q = seeded((1, 1, 48, 64), BF16, 51).cuda()
    k = seeded((1, 1, Skv, 64), BF16, 52).cuda()
    v = seeded((1, 1, Skv, 64), BF16, 53).cuda()
    say(f"block_mask long sweep Skv{Skv}")
    dense, dl = ffa.fastest_flash_attn_forward(q, k, v, block_size=64, return_lse=True)
    full = torch.ones(1, math.ceil(Skv / 64), dtype=torch.bool)
    masked, ml = ffa.fastest_flash_attn_forward(q, k, v, block_size=64, block_mask=full,
                                                return_lse=True)
    assert torch.equal(dense, masked) and torch.equal(dl, ml)


def test_block_mask_all_ones_equals_dense():
    """The reference's own check (tests/test_fastest_flash.py:240-258): an all-True
    mask gives the unmasked result."""
    require_gpu()
    q, k, v = (seeded((1, 2, 64, 64), BF16, s).cuda() for s in (31, 32, 33))
    say("block_mask all-true vs dense")
    dense, dl = ffa.fastest_flash_attn_forward(q, k, v, block_size=16, return_lse=True)
    full = torch.ones(4, 4, dtype=torch.bool)
    masked, ml = ffa.fastest_flash_attn_forward(q, k, v, block_size=16, block_mask=full,
                                                return_lse=True)
    assert torch.equal(dense, masked) and torch.equal(dl, ml)


@pytest.mark.parametrize("dt,cd", [(BF16, F16), (F16, BF16), (BF16, torch.float32),
                                   (F16, F16)])
def test_compute_dtype_parity(dt, cd):
    require_gpu()
    q = seeded((1, 2, 96, 64), dt, 41, scale=3.0)
    k = seeded((1, 2, 96, 64), dt, 42, scale=3.0)
    v = seeded((1, 2, 96, 64), dt, 43)
    say(f"compute_dtype {dt} -> {cd}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), causal=True,
                                            compute_dtype=cd, return_lse=True)
    torch.cuda.synchronize()
    np_cd = {BF16: "bfloat16", F16: "float16", torch.float32: None}[cd]
    ro, rl = rf.forward(np32(q), np32(k), np32(v), causal=True, compute_dtype=np_cd,
                        return_lse=True)
    assert_parity(o, ro, lse, rl, f"compute_dtype {dt}->{cd}")


@pytest.mark.parametrize("dt,P,D,H", [(F16, 16, 64, 2), (BF16, 5, 128, 4),
                                      (torch.float32, 8, 32, 2), (BF16, 3, 40, 1)])
def test_paged_append_bit_exact(dt, P, D, H):
    """ffa_paged_append on a device pool writes exactly what the reference's per-token
    loop writes (restated by the CPU-pool path): same pages, slots and bytes, across
    page boundaries, strided inputs and the out-of-pages path."""
    require_gpu()
    gpu = ffa.PagedKVCache(max_pages=9, page_size=P, num_heads=H, head_dim=D, dtype=dt,
                           device="cuda")
    cpu = ffa.PagedKVCache(max_pages=9, page_size=P, num_heads=H, head_dim=D, dtype=dt,
                           device="cpu")
    g = torch.Generator().manual_seed(P * D)
    steps = [(0, 7), (1, P + 2), (0, 1), (2, 3), (1, 2 * P)]
    for seq, n in steps:
        # tokens arrive as a transposed view ([S, H, D] -> [H, S, D]), as from a projection
        kt = torch.randn(n, H, D, generator=g).to(dt).transpose(0, 1)
        vt = torch.randn(n, H, D, generator=g).to(dt).transpose(0, 1)
        say(f"paged append seq {seq} n {n} P{P} D{D} H{H} {dt}")
        for cache, dev in ((gpu, "cuda"), (cpu, "cpu")):
            try:
                cache.append_tokens(seq, kt.to(dev), vt.to(dev))
            except RuntimeError as e:
                assert "out of physical pages" in str(e)
    torch.cuda.synchronize()
    assert gpu.free_pages == cpu.free_pages
    assert {s: dict(v) for s, v in gpu.sequences.items()} == \
           {s: dict(v) for s, v in cpu.sequences.items()}
    assert torch.equal(gpu.k_pages.cpu(), cpu.k_pages)
    assert torch.equal(gpu.v_pages.cpu(), cpu.v_pages)


def test_continuous_cache_on_device():
    require_gpu()
    gpu = ffa.ContinuousKVCache(max_batch=4, max_seq_len=40, num_heads=2, head_dim=64,
                                dtype=BF16, device="cuda")
    cpu = ffa.ContinuousKVCache(max_batch=4, max_seq_len=40, num_heads=2, head_dim=64,
                                dtype=BF16, device="cpu")
    g = torch.Generator().manual_seed(5)
    say("continuous cache on device")
    for n in (5, 1, 9):
        kn = torch.randn(3, 2, n, 64, generator=g).to(BF16)
        vn = torch.randn(3, 2, n, 64, generator=g).to(BF16)
        kg, vg = gpu.append(kn.cuda(), vn.cuda())
        kc, vc = cpu.append(kn, vn)
        assert torch.equal(kg.cpu(), kc) and torch.equal(vg.cpu(), vc)
    # the cache feeds the forward's kv_cache argument (bottom-right causal alignment)
    kk, vv = gpu.get_cache(3)
    q = seeded((3, 2, 2, 64), BF16, 6).cuda()
    kn = seeded((3, 2, 2, 64), BF16, 7).cuda()
    vn = seeded((3, 2, 2, 64), BF16, 8).cuda()
    o, lse = ffa.fastest_flash_attn_forward(q, kn, vn, kv_cache=(kk, vv), causal=True,
                                            return_lse=True)
    ro, rl = rf.forward(np32(q), np32(kn), np32(vn), kv_cache=(np32(kk), np32(vv)),
                        causal=True, return_lse=True)
    assert_parity(o, ro, lse, rl, "continuous cache -> forward")
