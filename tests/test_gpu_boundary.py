"""GPU tests of the C-ABI contracts at the drop-in boundary, called through ctypes:

* any finite scale (negative, zero, denormal) is applied by the library itself, for
  the 16-bit and fp32 prefill kernels, with and without softcap;
* out-of-range page ids exclude the tokens they would hold in both decode kernels
  (and raise IndexError on request, as the reference's page indexing does);
* fp32 page pools decode (gather + fp32 prefill kernel) and the reference's own
  PagedKVCache flow runs on a ROCm pool;
* every output element of a full-size launch is written: outputs pre-filled with NaN
  come back finite, and one (batch, head) per XCD matches the oracle.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from fastest_flash_attention_amd.kernels import _lib
from fastest_flash_attention_amd.ops import attention_forward as af
from oracle import mla as omla
from oracle import paged as opaged
from oracle import reference_forward as rf
from tests.gpu_util import assert_parity, np32, require_gpu, say, seeded

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16

SCALES = [
    ("neg", BF16, -0.2, None, True),
    ("neg_softcap", BF16, -0.3, 5.0, False),
    ("zero", BF16, 0.0, None, True),
    ("zero_softcap", BF16, 0.0, 7.0, True),
    ("denormal", BF16, 1e-41, None, False),
    ("neg_fp16", torch.float16, -0.15, None, True),
    ("neg_fp32", torch.float32, -0.2, None, True),
    ("zero_fp32", torch.float32, 0.0, None, False),
    ("neg_fp32_softcap", torch.float32, -0.25, 6.0, True),
]
# Longer sweeps whose interior tiles run the kernels' fast step (its softcap transform
# and running max are its own code): a negative scale with a large cap and scores that
# span most of tanh's range, where a max taken in the wrong direction overflows the
# exponentials (cap * log2(e) * 2 > 128).
SCALES_LONG = [
    ("neg_softcap_long_d128", BF16, -3.0, 50.0, False, 128),
    ("neg_softcap_long_d64", BF16, -3.0, 50.0, True, 64),
    ("pos_softcap_long_d128", BF16, 3.0, 50.0, True, 128),
    ("neg_softcap_narrow_range", BF16, -0.3, 50.0, False, 128),
]


@pytest.mark.parametrize("name,dtype,scale,softcap,causal", SCALES, ids=[s[0] for s in SCALES])
def test_abi_scale_contract(name, dtype, scale, softcap, causal):
    """ffa_prefill_fwd called directly through ctypes with the raw scale."""
    require_gpu()
    B, H, S, D = 1, 3, 150, 64
    q, k, v = (seeded((B, H, S, D), dtype, s) for s in (31, 32, 33))
    say(f"abi scale {name} {dtype} scale={scale} softcap={softcap} causal={causal}")
    call = af.prepare_prefill(q.cuda(), k.cuda(), v.cuda(), scale=scale, causal=causal,
                              softcap=softcap, return_lse=True)
    assert call.args.scale == np.float32(scale)  # the Python layer passes it unchanged
    lib = _lib.load()
    stream = _lib.current_stream_handle(call.q.device)
    rc = lib.ffa_prefill_fwd(ctypes.byref(call.args), ctypes.c_void_p(stream))
    assert rc == 0, _lib.strerror(rc)
    torch.cuda.synchronize()
    ro, rl = rf.forward(np32(q), np32(k), np32(v), scale=scale, causal=causal, softcap=softcap,
                        return_lse=True)
    assert_parity(call.out, ro, call.lse, rl, name)
    if scale == 0.0 or abs(scale) < 1e-30:
        # uniform softmax over the visible keys: lse = log(n)
        n = np.arange(1, S + 1) if causal else np.full(S, S)
        assert np.allclose(np32(call.lse)[0, :, :, 0], np.log(n)[None, :], atol=1e-5)


@pytest.mark.parametrize("name,dtype,scale,softcap,causal,D", SCALES_LONG,
                         ids=[s[0] for s in SCALES_LONG])
def test_scale_softcap_fast_step(name, dtype, scale, softcap, causal, D):
    require_gpu()
    B, H, S = 1, 2, 1024
    q, k, v = (seeded((B, H, S, D), dtype, s) for s in (41, 42, 43))
    say(f"scale {name} {dtype} scale={scale} softcap={softcap} causal={causal} D{D}")
    o, lse = ffa.fastest_flash_attn_forward(q.cuda(), k.cuda(), v.cuda(), scale=scale,
                                            causal=causal, softcap=softcap, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    ro, rl = rf.forward(np32(q), np32(k), np32(v), scale=scale, causal=causal, softcap=softcap,
                        return_lse=True)
    assert_parity(o, ro, lse, rl, name)


def _masked_oracle(q, k_pages, v_pages, bt, lens, num_pages, scale):
    """Decode with the tokens of out-of-range pages excluded (no window: every other
    cached key is visible, so attention is over the kept keys only)."""
    B, Hq, D = q.shape
    Hkv, P = k_pages.shape[1], k_pages.shape[2]
    out = np.zeros((B, Hq, D), np.float32)
    lse = np.full((B, Hq), -np.inf, np.float32)
    for b, L in enumerate(lens):
        keep = [t for t in range(L) if 0 <= bt[b, t // P] < num_pages]
        if not keep:
            continue
        kk = np.stack([k_pages[bt[b, t // P], :, t % P] for t in keep], axis=1)[None]
        vv = np.stack([v_pages[bt[b, t // P], :, t % P] for t in keep], axis=1)[None]
        kk = rf.repeat_kv(kk.astype(np.float32), Hq, Hkv)
        vv = rf.repeat_kv(vv.astype(np.float32), Hq, Hkv)
        o, l = rf.flash_attn_cpu_forward(q[b][None, :, None, :].astype(np.float32), kk, vv,
                                         scale=scale, causal=False, block_q=64, block_kv=64,
                                         return_lse=True)
        out[b], lse[b] = o[0, :, 0, :], l[0, :, 0, 0]
    return out, lse


def test_decode_invalid_pages_are_excluded():
    require_gpu()
    g = torch.Generator().manual_seed(41)
    Hq, Hkv, D, P, num_pages = 8, 2, 128, 16, 40
    lens = [100, 37, 16, 300]
    k_pages = torch.randn(num_pages, Hkv, P, D, generator=g).to(BF16)
    v_pages = torch.randn(num_pages, Hkv, P, D, generator=g).to(BF16)
    bt = torch.randint(0, num_pages, (4, 20), generator=g, dtype=torch.int32)
    bt[0, 2] = num_pages          # one past the pool
    bt[1, 0] = -5                 # negative
    bt[2, 0] = 1 << 30            # the sequence's only page: no key left
    bt[3, 1:4] = torch.tensor([-1, 999, num_pages + 7], dtype=torch.int32)
    q = seeded((4, Hq, D), BF16, 42)
    lens_t = torch.tensor(lens, dtype=torch.int32)
    scale = 1 / math.sqrt(D)
    ro, rl = _masked_oracle(np32(q), np32(k_pages), np32(v_pages), bt.numpy(), lens, num_pages,
                            scale)
    for tps in (32, None):
        say(f"decode invalid pages tps={tps}")
        o, lse = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(),
                                                bt.cuda(), lens_t.cuda(), return_lse=True,
                                                tokens_per_split=tps)
        torch.cuda.synchronize()
        assert_parity(o, ro, lse, rl, f"invalid pages tps={tps}")
        assert torch.all(o[2] == 0) and torch.isneginf(lse[2]).all()
    with pytest.raises(IndexError, match="outside the pool"):
        ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(), bt.cuda(),
                                       lens_t.cuda(), check_block_tables=True)
    # valid tables pass the check and give the unmasked result
    bt_ok = torch.remainder(bt, num_pages)
    o1, _ = ffa.fastest_flash_paged_decode(q.cuda(), k_pages.cuda(), v_pages.cuda(),
                                           bt_ok.cuda(), lens_t.cuda(), check_block_tables=True)
    ro1, _ = opaged.paged_decode(np32(q), np32(k_pages), np32(v_pages), bt_ok.numpy(), lens)
    assert_parity(o1, ro1, what="valid tables")


@pytest.mark.parametrize("dim_v,P", [(512, 16), (512, 64), (256, 32)])
def test_mla_decode_invalid_pages_are_excluded(dim_v, P):
    """Page sizes that are multiples of 32 take the kernel's whole-tile page path (one
    page id per 32-token tile); 16 takes the per-row path. Both exclude the tokens of
    out-of-range ids."""
    require_gpu()
    g = torch.Generator().manual_seed(43)
    H, num_pages = 32, 30
    lens = [200, 100, 5]
    pool = torch.randn(num_pages, P, dim_v + 64, generator=g).to(BF16)
    bt = torch.randint(0, num_pages, (3, 13), generator=g, dtype=torch.int32)
    bt[0, 3] = -2
    bt[1, 1] = num_pages
    bt[2, 0] = 12345
    q = torch.randn(3, H, dim_v + 64, generator=g).to(BF16)
    scale = 1 / math.sqrt(dim_v + 64)
    say(f"mla decode invalid pages dim_v {dim_v} page {P}")
    o, lse = ffa.fastest_flash_mla_decode(q.cuda(), pool.cuda(), bt.cuda(),
                                          torch.tensor(lens, dtype=torch.int32).cuda(),
                                          dim_v=dim_v, scale=scale, return_lse=True,
                                          tokens_per_split=64)
    torch.cuda.synchronize()
    pool64 = np32(pool).astype(np.float64)
    for b, L in enumerate(lens):
        keep = [t for t in range(L) if 0 <= bt[b, t // P] < num_pages]
        rows = pool64[[int(bt[b, t // P]) for t in keep], [t % P for t in keep]]
        ro, rl = omla.absorbed_decode(np32(q[b]).astype(np.float64), rows, dim_v, scale)
        assert_parity(o[b], ro, lse[b], rl, f"mla invalid pages b{b}")
    assert torch.all(o[2] == 0) and torch.isneginf(lse[2]).all()
    with pytest.raises(IndexError):
        ffa.fastest_flash_mla_decode(q.cuda(), pool.cuda(), bt.cuda(),
                                     torch.tensor(lens, dtype=torch.int32).cuda(), dim_v=dim_v,
                                     scale=scale, check_block_tables=True)


def test_fp32_pool_decode_and_reference_paged_flow():
    """The reference's test_paged_basic on a ROCm fp32 pool, then decode over it (fp32
    pools: gather + the fp32 MFMA prefill kernel per sequence) against the oracle."""
    require_gpu()
    g = torch.Generator().manual_seed(44)
    cache = ffa.PagedKVCache(max_pages=64, page_size=4, num_heads=2, head_dim=8,
                             dtype=torch.float32, device="cuda")
    k = torch.randn(2, 6, 8, generator=g)
    v = torch.randn(2, 6, 8, generator=g)
    assert cache.append_tokens(0, k.cuda(), v.cuda()) == 6
    k_out, v_out = cache.get_kv(0)
    assert k_out.shape == (2, 6, 8) and torch.equal(k_out.cpu(), k) and torch.equal(v_out.cpu(), v)
    for sid, n in ((1, 33), (2, 1), (0, 9)):
        cache.append_tokens(sid, torch.randn(2, n, 8, generator=g).cuda(),
                            torch.randn(2, n, 8, generator=g).cuda())
    q = torch.randn(3, 4, 8, generator=g)
    for kw in ({}, {"sliding_window": 5, "softcap": 3.0}, {"scale": -0.4}):
        say(f"fp32 pool decode {kw}")
        o, lse = cache.decode(q.cuda(), [0, 1, 2], return_lse=True, **kw)
        torch.cuda.synchronize()
        bt, lens = cache.block_tables([0, 1, 2])
        ro, rl = opaged.paged_decode(np32(q), np32(cache.k_pages), np32(cache.v_pages),
                                     bt.cpu().numpy(), lens.cpu().tolist(), **kw)
        max_abs, _ = assert_parity(o, ro, lse, rl, f"fp32 pool {kw}")
        assert o.dtype == torch.float32 and max_abs < 1e-4


# Full-size launches with NaN-filled outputs: every element must be written. One
# (batch, head) on each XCD is compared with the oracle on three row blocks (the first,
# a middle and the last 128 rows: rows are independent, so q rows are sliced with
# their absolute offset).
NAN_FILL = [
    ("north_star", 4, 32, 32, 8192, 128, {"causal": True}),
    ("cfg2_mha", 4, 32, 32, 4096, 128, {"causal": True}),
    ("cfg3_gqa", 2, 32, 8, 8192, 128, {"causal": True, "sliding_window": 4096,
                                        "softcap": 50.0, "num_kv_heads": 8}),
    ("cfg5_mla_d192", 2, 32, 32, 4096, 192, {"causal": True}),
]


@pytest.mark.parametrize("cfg", NAN_FILL, ids=[c[0] for c in NAN_FILL])
def test_full_size_every_element_written(cfg):
    require_gpu()
    name, B, Hq, Hkv, S, D, kw = cfg
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(B, Hq, S, D, generator=g, device="cuda").to(BF16)
    k = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(BF16)
    v = torch.randn(B, Hkv, S, D, generator=g, device="cuda").to(BF16)
    out = torch.full((B, Hq, S, D), float("nan"), dtype=BF16, device="cuda")
    call = af.prepare_prefill(q, k, v, out=out, return_lse=True, **kw)
    assert call.out.data_ptr() == out.data_ptr()
    call.lse.fill_(float("nan"))
    say(f"nan-filled full-size prefill {name}")
    af.launch_prefill(call)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all(), f"{name}: unwritten output elements"
    assert torch.isfinite(call.lse).all(), f"{name}: unwritten LSE elements"
    ratio = Hq // Hkv
    okw = {kk: vv for kk, vv in kw.items() if kk != "num_kv_heads"}
    units = B * Hq
    for x in range(8):  # the prefill grid keeps units [x U/8, (x+1) U/8) on XCD x
        u = x * (units // 8) + (x * 5) % (units // 8)
        b, h = divmod(u, Hq)
        hk = h // ratio
        for r0 in (0, (S // 2 // 128) * 128, S - 128):
            ro, rl = rf.flash_attn_cpu_forward(
                np32(q[b:b + 1, h:h + 1, r0:r0 + 128]), np32(k[b:b + 1, hk:hk + 1, :r0 + 128]),
                np32(v[b:b + 1, hk:hk + 1, :r0 + 128]), scale=1 / math.sqrt(D), block_q=128,
                block_kv=512, return_lse=True, q_offset=r0, causal=okw.get("causal", False),
                sliding_window=okw.get("sliding_window"), softcap=okw.get("softcap"))
            assert_parity(out[b:b + 1, h:h + 1, r0:r0 + 128], ro,
                          call.lse[b:b + 1, h:h + 1, r0:r0 + 128], rl, f"{name} b{b} h{h} r{r0}")
