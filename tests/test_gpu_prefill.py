"""GPU parity of the prefill kernel (ffa_prefill_fwd through fastest_flash_attn_forward)
against the CPU oracle (oracle/reference_forward.py) on identical seeded inputs."""

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

# (name, B, Hq, Hkv, Sq, Skv, D, kwargs, dtype)
CASES = [
    ("plain", 2, 4, 4, 128, 128, 64, {}, BF16),
    ("causal_tail", 1, 3, 3, 200, 200, 128, {"causal": True}, BF16),
    ("causal_window", 1, 2, 2, 300, 300, 128, {"causal": True, "sliding_window": 37}, BF16),
    ("softcap_causal", 2, 2, 2, 150, 150, 64, {"causal": True, "softcap": 10.0}, BF16),
    ("gqa", 1, 8, 2, 256, 256, 128, {"causal": True, "num_kv_heads": 2}, BF16),
    ("mqa_broadcast", 1, 4, 1, 96, 96, 64, {}, BF16),
    ("d192_mla", 1, 2, 2, 256, 256, 192, {"causal": True}, BF16),
    ("d256", 1, 2, 2, 130, 130, 256, {"causal": True}, BF16),
    ("d96", 1, 2, 2, 77, 77, 96, {"causal": True}, BF16),
    ("d16", 2, 2, 2, 40, 40, 16, {}, BF16),
    ("d8_scalar", 1, 2, 2, 17, 17, 8, {"causal": True}, BF16),
    ("d4_scalar", 1, 1, 1, 8, 8, 4, {}, BF16),
    ("fp16", 1, 4, 4, 200, 200, 128, {"causal": True, "softcap": 30.0}, F16),
    ("sq_ne_skv", 1, 2, 2, 64, 300, 64, {}, BF16),
    ("causal_sq_lt_skv", 1, 2, 2, 64, 300, 64, {"causal": True}, BF16),
    ("window_noncausal_masked_rows", 1, 2, 2, 32, 8, 16, {"sliding_window": 4,
                                                          "block_size": 4}, BF16),
    ("single", 1, 2, 2, 1, 1, 64, {}, BF16),
    ("gqa_window_softcap", 2, 8, 2, 333, 333, 128, {"causal": True, "sliding_window": 100,
                                                    "softcap": 50.0, "num_kv_heads": 2}, BF16),
    # the kernels need scale > 0; the host maps these exactly (negated q / 1e-30)
    ("negative_scale", 1, 2, 2, 150, 150, 64, {"causal": True, "scale": -0.2}, BF16),
    ("negative_scale_softcap", 1, 2, 2, 90, 90, 128, {"softcap": 5.0, "scale": -0.3}, BF16),
    ("zero_scale", 1, 2, 2, 70, 70, 64, {"causal": True, "scale": 0.0}, BF16),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_prefill_parity(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, kw, dt = case
    q = seeded((B, Hq, Sq, D), dt, 1)
    k = seeded((B, Hkv, Skv, D), dt, 2)
    v = seeded((B, Hkv, Skv, D), dt, 3)
    say(f"prefill {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} {kw} {dt}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), return_lse=True, **kw)
    torch.cuda.synchronize()
    assert o.dtype == dt and o.shape == q.shape and lse.shape == (B, Hq, Sq, 1)
    ro, rl = rf.forward(np32(q), np32(k), np32(v), return_lse=True, **kw)
    assert_parity(o, ro, lse, rl, name)


# (name, B, Hq, Hkv, Sq, Skv, D, Dv, kwargs, dtype): v narrower than q / k, which the
# forward takes as zero-padded to D (the MLA module passes its 128-dim V this way).
# head_dim 129..192 with Dv <= 128 (a multiple of 8) runs the narrow-V kernels; the
# last two shapes are zero-padded on the host.
NARROW_V = [
    ("mla_causal", 1, 4, 4, 300, 300, 192, 128, {"causal": True}, BF16),
    ("mla_gqa_window_softcap", 2, 8, 2, 333, 333, 192, 128,
     {"causal": True, "sliding_window": 100, "softcap": 50.0, "num_kv_heads": 2}, BF16),
    ("mla_noncausal_ragged", 1, 2, 2, 77, 203, 192, 128, {}, BF16),
    ("d136_dv64_fp16", 1, 2, 2, 100, 100, 136, 64, {"causal": True}, F16),
    ("d160_dv120_window", 1, 2, 2, 260, 260, 160, 120, {"sliding_window": 50}, BF16),
    ("mla_negative_scale", 1, 2, 2, 140, 140, 192, 128, {"causal": True, "scale": -0.1}, BF16),
    # from 4096 query rows on the narrow-V kernels run 256-row (eight-wave) workgroups
    ("mla_wide_causal_ragged", 1, 1, 1, 4100, 4100, 192, 128, {"causal": True}, BF16),
    ("mla_wide_gqa_window_softcap", 1, 2, 1, 4096, 4400, 192, 128,
     {"sliding_window": 700, "softcap": 30.0, "num_kv_heads": 1}, BF16),
    ("wide_d160_dv120_fp16", 1, 1, 1, 4096, 4096, 160, 120, {"causal": True}, F16),
    ("host_padded_d128_dv64", 1, 2, 2, 90, 90, 128, 64, {"causal": True}, BF16),
    ("host_padded_dv100", 1, 2, 2, 90, 90, 192, 100, {"causal": True}, BF16),
]


@pytest.mark.parametrize("case", NARROW_V, ids=[c[0] for c in NARROW_V])
def test_prefill_narrow_v(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, Dv, kw, dt = case
    q = seeded((B, Hq, Sq, D), dt, 11)
    k = seeded((B, Hkv, Skv, D), dt, 12)
    v = seeded((B, Hkv, Skv, Dv), dt, 13)
    say(f"prefill narrow v {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} Dv{Dv} {kw} {dt}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), return_lse=True, **kw)
    torch.cuda.synchronize()
    assert o.shape == q.shape and o.dtype == dt
    assert torch.all(o[..., Dv:] == 0), "O dims past v's must be 0"
    vp = torch.nn.functional.pad(v, (0, D - Dv))
    ro, rl = rf.forward(np32(q), np32(k), np32(vp), return_lse=True, **kw)
    assert_parity(o, ro, lse, rl, name)


@pytest.mark.parametrize("dtype,D,block_mask", [(BF16, 64, False), (BF16, 192, False),
                                               (torch.float32, 64, False), (BF16, 128, True)])
def test_reference_tile_floor(dtype, D, block_mask):
    """Every visited reference tile in which a row sees no key adds 1e-30 to that row's
    softmax sum (the reference's clamp(min=1e-30) per tile). With every logit near -100
    that floor, not the row's own keys, sets O and the LSE of most rows: the kernels must
    add it for rows that see keys too, not only for fully masked rows."""
    require_gpu()
    B, H, S, bs = 1, 2, 300, 32
    u = seeded((1, 1, 1, D), torch.float32, 61)
    u = u / u.norm()
    q = (-10.0 * u).expand(B, H, S, D) + 0.01 * seeded((B, H, S, D), torch.float32, 62)
    k = (10.0 * u).expand(B, H, S, D) + 0.01 * seeded((B, H, S, D), torch.float32, 63)
    q, k = q.to(dtype), k.to(dtype)
    v = seeded((B, H, S, D), dtype, 64)
    kw = dict(causal=True, sliding_window=40, scale=1.0, block_size=bs, return_lse=True)
    if block_mask:
        g = torch.Generator().manual_seed(65)
        bm = torch.rand(math.ceil(S / bs), math.ceil(S / bs), generator=g) < 0.7
        kw["block_mask"] = bm
    say(f"reference tile floor {dtype} D{D} block_mask={block_mask}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), **kw)
    torch.cuda.synchronize()
    okw = dict(kw)
    if block_mask:
        okw["block_mask"] = kw["block_mask"].numpy()
    ro, rl = rf.forward(np32(q), np32(k), np32(v), **okw)
    # the floor sets the LSE of many rows (log(k 1e-30), about -69, instead of about -96)
    assert np.sum(np.abs(rl - np.log(1e-30)) < 1.0) > 50 and np.nanmin(rl) < -90
    assert_parity(o, ro, lse, rl, f"tile floor {dtype} D{D}")


def test_kv_cache_offset():
    require_gpu()
    B, H, D = 2, 4, 128
    q = seeded((B, H, 70, D), BF16, 4)
    kn = seeded((B, H, 70, D), BF16, 5)
    vn = seeded((B, H, 70, D), BF16, 6)
    kc = seeded((B, H, 200, D), BF16, 7)
    vc = seeded((B, H, 200, D), BF16, 8)
    for causal in (False, True):
        say(f"prefill kv_cache causal={causal}")
        o, lse = ffa.fastest_flash_attn_forward(q.cuda(), kn.cuda(), vn.cuda(), causal=causal,
                                                kv_cache=(kc.cuda(), vc.cuda()),
                                                return_lse=True)
        ro, rl = rf.forward(np32(q), np32(kn), np32(vn), causal=causal,
                            kv_cache=(np32(kc), np32(vc)), return_lse=True)
        assert_parity(o, ro, lse, rl, f"kv_cache causal={causal}")


def test_negative_offset_masked_rows():
    """q longer than the concatenated keys: q_offset < 0, early causal rows see no key
    and must carry the reference sentinel LSE."""
    require_gpu()
    q = seeded((1, 2, 40, 64), BF16, 9)
    kn = seeded((1, 2, 6, 64), BF16, 10)
    kc = seeded((1, 2, 10, 64), BF16, 11)
    say("prefill negative q_offset")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), kn.cuda(), kn.cuda(), causal=True,
                                            kv_cache=(kc.cuda(), kc.cuda()), block_size=8,
                                            return_lse=True)
    ro, rl = rf.forward(np32(q), np32(kn), np32(kn), causal=True, kv_cache=(np32(kc), np32(kc)),
                        block_size=8, return_lse=True)
    assert np.isneginf(rl).any() or (rl < -60).any()
    assert_parity(o, ro, lse, rl, "negative offset")


def test_two_pass_sentinel():
    require_gpu()
    q = seeded((1, 2, 32, 16), BF16, 12)
    k = seeded((1, 2, 8, 16), BF16, 13)
    say("prefill two_pass masked rows")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), k.cuda(), sliding_window=4,
                                            block_size=4, two_pass=True, return_lse=True)
    _, rl = rf.forward(np32(q), np32(k), np32(k), sliding_window=4, block_size=4,
                       two_pass=True, return_lse=True)
    lse_c = np32(lse)
    assert np.array_equal(np.isneginf(lse_c), np.isneginf(rl))
    assert np.all(np32(o)[0, :, 11:] == 0)


def test_module_layout_views_and_3d():
    """Strided [B,H,S,D] views of [B,S,H*D] projections (the modules' layout) and 3D input."""
    require_gpu()
    B, S, H, D = 2, 100, 4, 64
    x = seeded((B, S, 3 * H * D), BF16, 14).cuda()
    q, k, v = (t.view(B, S, H, D).transpose(1, 2) for t in x.split(H * D, dim=-1))
    say("prefill strided views")
    o, lse = ffa.fastest_flash_attn_forward(q, k, v, causal=True, return_lse=True)
    ro, rl = rf.forward(np32(q), np32(k), np32(v), causal=True, return_lse=True)
    assert_parity(o, ro, lse, rl, "strided views")
    q3 = seeded((3, 50, 32), BF16, 15)
    say("prefill 3d")
    o3, l3 = ffa.fastest_flash_attn_forward(q3.cuda(), q3.cuda(), q3.cuda(), causal=True,
                                            return_lse=True)
    assert o3.shape == (3, 50, 32) and l3.shape == (3, 50, 1)
    ro3, rl3 = rf.forward(np32(q3), np32(q3), np32(q3), causal=True, return_lse=True)
    assert_parity(o3, ro3, l3, rl3, "3d")


def test_batch_broadcast_kv():
    require_gpu()
    q = seeded((3, 2, 64, 64), BF16, 16)
    k = seeded((1, 2, 64, 64), BF16, 17)
    say("prefill batch-broadcast kv")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), k.cuda(), return_lse=True)
    ro, rl = rf.forward(np32(q), np32(k), np32(k), return_lse=True)
    assert_parity(o, ro, lse, rl, "batch broadcast")


def test_special_values():
    """Closed forms on the device: one key -> O = V; zero q -> mean(V)."""
    require_gpu()
    v = seeded((1, 2, 1, 64), BF16, 18)
    q = seeded((1, 2, 9, 64), BF16, 19)
    o, _ = ffa.fastest_flash_attn_forward(q.cuda(), v.cuda(), v.cuda())
    assert torch.equal(o.cpu(), v.expand_as(o))
    qz = torch.zeros(1, 1, 16, 64, dtype=BF16)
    kv = seeded((1, 1, 48, 64), BF16, 20)
    o, _ = ffa.fastest_flash_attn_forward(qz.cuda(), kv.cuda(), kv.cuda())
    assert np.abs(np32(o) - np32(kv).mean(axis=2, keepdims=True)).max() < 1e-2


def test_constant_v_and_large_softcap():
    """Closed forms: rows of V all equal -> O = that row for any q and mask (P is a
    convex combination; its bf16 rounding moves O by < 2^-8 relative). A softcap far
    above every score (1000 against |s| < 10) leaves the result within tolerance of no
    softcap (c tanh(s/c) - s ~ s^3 / 3c^2)."""
    require_gpu()
    q = seeded((1, 2, 200, 128), BF16, 71)
    k = seeded((1, 2, 200, 128), BF16, 72)
    row = seeded((1, 2, 1, 128), BF16, 73)
    v = row.expand(1, 2, 200, 128).contiguous()
    for causal, window in ((False, None), (True, None), (True, 64)):
        say(f"constant V causal={causal} window={window}")
        o, _ = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), causal=causal,
                                              sliding_window=window)
        assert np.abs(np32(o) - np32(v)).max() <= 1e-2 * np.abs(np32(row)).max()
    v2 = seeded((1, 2, 200, 128), BF16, 74)
    say("softcap 1000 vs none")
    o1, l1 = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v2.cuda(), causal=True,
                                            softcap=1000.0, return_lse=True)
    o0, l0 = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v2.cuda(), causal=True,
                                            return_lse=True)
    assert np.abs(np32(o1) - np32(o0)).max() < 2e-2
    assert np.abs(np32(l1) - np32(l0)).max() < 1e-3


def test_empty_inputs():
    """Degenerate shapes as the reference loop leaves them: no keys -> O = 0 and
    LSE = -inf (no tile visited); no queries or no batch -> empty outputs."""
    require_gpu()
    q = seeded((1, 2, 5, 64), BF16, 61).cuda()
    none = torch.zeros(1, 2, 0, 64, dtype=BF16, device="cuda")
    say("empty: S_kv = 0")
    o, lse = ffa.fastest_flash_attn_forward(q, none, none, return_lse=True)
    ro, rl = rf.forward(np32(q), np32(none), np32(none), return_lse=True)
    assert o.shape == ro.shape and not o.abs().any()
    assert torch.isneginf(lse).all() and np.isneginf(rl).all()
    say("empty: S_q = 0")
    kv = seeded((1, 2, 7, 64), BF16, 62).cuda()
    o, lse = ffa.fastest_flash_attn_forward(q[:, :, :0], kv, kv, causal=True, return_lse=True)
    assert o.shape == (1, 2, 0, 64) and lse.shape == (1, 2, 0, 1)
    say("empty: B = 0")
    z = torch.zeros(0, 2, 9, 64, dtype=BF16, device="cuda")
    o, lse = ffa.fastest_flash_attn_forward(z, z, z, causal=True, return_lse=True)
    assert o.shape == z.shape and lse.shape == (0, 2, 9, 1)


def test_rejects_unsupported():
    require_gpu()
    q = torch.randn(1, 1, 8, 16, device="cuda")
    with pytest.raises(TypeError):
        qd = q.double()
        ffa.fastest_flash_attn_forward(qd, qd, qd)
    qb = q.to(BF16)
    with pytest.raises(ValueError, match="does not cover"):
        # 8 rows / block 4 = 2 query tiles: a 1x1 mask is too small
        ffa.fastest_flash_attn_forward(qb, qb, qb, block_size=4,
                                       block_mask=torch.ones(1, 1, dtype=torch.bool))
    with pytest.raises(TypeError, match="compute_dtype"):
        ffa.fastest_flash_attn_forward(qb, qb, qb, compute_dtype=torch.int8)


# ---------------------------------------------------------------------------------
# BASELINE configs at full size: the kernel runs the whole batch, the oracle checks
# sampled (batch, head) pairs exactly (rows are independent), plus global invariants.
# ---------------------------------------------------------------------------------

FULL = [
    ("cfg2_mha", 4, 32, 32, 4096, 128, {"causal": True}, [(0, 0), (3, 31)]),
    ("north_star", 4, 32, 32, 8192, 128, {"causal": True}, [(1, 5)]),
    ("cfg3_gqa", 2, 32, 8, 8192, 128, {"causal": True, "sliding_window": 4096,
                                        "softcap": 50.0, "num_kv_heads": 8}, [(0, 0), (1, 31)]),
    ("cfg5_mla_d192", 2, 32, 32, 4096, 192, {"causal": True}, [(1, 17)]),
]


@pytest.mark.parametrize("cfg", FULL, ids=[c[0] for c in FULL])
def test_full_size_sampled_heads(cfg):
    require_gpu()
    name, B, Hq, Hkv, S, D, kw, samples = cfg
    g = torch.Generator(device="cuda").manual_seed(0)
    q = torch.randn(B, Hq, S, D, generator=g, device="cuda").to(BF16)
    k = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(BF16)
    v = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(BF16)
    say(f"prefill full {name}")
    o, lse = ffa.fastest_flash_attn_forward(q, k, v, return_lse=True, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    ratio = Hq // Hkv
    okw = {kk: vv for kk, vv in kw.items() if kk != "num_kv_heads"}
    for b, h in samples:
        hk = h // ratio
        ro, rl = rf.flash_attn_cpu_forward(
            np32(q[b:b + 1, h:h + 1]), np32(k[b:b + 1, hk:hk + 1]), np32(v[b:b + 1, hk:hk + 1]),
            scale=1 / math.sqrt(D), block_q=256, block_kv=256, return_lse=True,
            causal=okw.get("causal", False), sliding_window=okw.get("sliding_window"),
            softcap=okw.get("softcap"))
        assert_parity(o[b:b + 1, h:h + 1], ro, lse[b:b + 1, h:h + 1], rl, f"{name} b{b} h{h}")
    # size-independent property: LSE >= max visible score and the first row attends only
    # to key 0 under causal masking -> O[:, :, 0] == V[:, kv(h), 0]
    o0 = o[:, :, 0].float()
    v0 = v[:, torch.arange(Hq, device="cuda") // ratio, 0].float()
    assert (o0 - v0).abs().max().item() < 1e-2


# fp32 inputs: computed in fp32 (fp32 MFMA), as the reference computes them; the
# tolerance is the north-star one, the fp32 path lands far inside it. Grids of fewer
# than 2048 128-row workgroups (all but the two "classic" cases, which have exactly
# 2048, and head_dim > 128) run the split kernel, whose four waves share a row block's
# keys; "long_kv" gives each wave many tiles, "few_tiles" leaves some waves none.
F32_CASES = [
    ("cfg1_mha_fp32", 2, 8, 8, 1024, 1024, 64, {"causal": True, "block_size": 64}),
    ("fp32_classic_grid_causal", 2, 32, 32, 4096, 4096, 32, {"causal": True}),
    ("fp32_classic_grid_gqa_window", 1, 64, 16, 4096, 4096, 32,
     {"causal": True, "sliding_window": 300, "num_kv_heads": 16}),
    ("fp32_split_grid_512_gqa_window", 1, 32, 8, 2048, 2048, 64,
     {"causal": True, "sliding_window": 300, "num_kv_heads": 8}),
    ("fp32_split_long_kv", 1, 4, 4, 5, 3000, 64, {}),
    ("fp32_split_long_kv_causal_topleft", 1, 2, 2, 70, 2500, 128, {"causal": True}),
    ("fp32_split_few_tiles", 2, 3, 3, 40, 40, 64, {"causal": True}),
    ("fp32_window_softcap_gqa", 1, 4, 2, 200, 200, 128, {"causal": True, "sliding_window": 50,
                                                         "softcap": 30.0, "num_kv_heads": 2}),
    ("fp32_d32_noncausal_rect", 2, 2, 2, 70, 130, 32, {}),
    ("fp32_d192_masked_rows", 1, 2, 2, 40, 12, 192, {"sliding_window": 5, "block_size": 8}),
    ("fp32_d256", 1, 2, 2, 66, 66, 256, {"causal": True}),
]


@pytest.mark.parametrize("case", F32_CASES, ids=[c[0] for c in F32_CASES])
def test_prefill_fp32_parity(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, kw = case
    q = seeded((B, Hq, Sq, D), torch.float32, 51)
    k = seeded((B, Hkv, Skv, D), torch.float32, 52)
    v = seeded((B, Hkv, Skv, D), torch.float32, 53)
    say(f"prefill fp32 {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} {kw}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), return_lse=True, **kw)
    torch.cuda.synchronize()
    assert o.dtype == torch.float32 and o.shape == q.shape
    ro, rl = rf.forward(np32(q), np32(k), np32(v), return_lse=True, **kw)
    max_abs, _ = assert_parity(o, ro, lse, rl, name)
    assert max_abs < 1e-4, f"{name}: fp32 path max-abs {max_abs:.2e}"
