"""GPU parity of the MLA latent-cache decode (ffa_mla_decode_fwd) against oracle/mla.py,
and of FastestFlashMLA.decode_step against the module's own full forward."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import mla as omla
from tests.gpu_util import assert_parity, np32, require_gpu, say

pytestmark = pytest.mark.gpu

BF16, F16 = torch.bfloat16, torch.float16


def _paged_case(seed, lens, page_size, dim_v, H, dtype, poison=True):
    """Sequences of `lens` tokens in a randomly permuted page pool; slots past each
    length hold NaN (they must never be read)."""
    g = torch.Generator().manual_seed(seed)
    dqk = dim_v + 64
    pages_per = [max(1, math.ceil(n / page_size)) for n in lens]
    total = sum(pages_per) + 3
    perm = torch.randperm(total, generator=g).tolist()
    pool = torch.randn(total, page_size, dqk, generator=g)
    width = max(pages_per)
    bt = torch.zeros(len(lens), width, dtype=torch.int32)
    off = 0
    for b, (n, np_) in enumerate(zip(lens, pages_per)):
        ids = perm[off:off + np_]
        off += np_
        bt[b, :np_] = torch.tensor(ids, dtype=torch.int32)
        if poison:
            for t in range(n, np_ * page_size):
                pool[ids[t // page_size], t % page_size] = float("nan")
    q = torch.randn(len(lens), H, dqk, generator=g)
    return q.to(dtype), pool.to(dtype), bt, torch.tensor(lens, dtype=torch.int32)


MLA_CASES = [
    # dtype, dim_v, heads, page_size, lens, tokens_per_split
    (BF16, 512, 32, 16, [4096, 1, 31, 32, 33, 0, 700], None),
    (BF16, 512, 40, 64, [1000, 2049], 256),
    (F16, 256, 16, 12, [130, 77, 5], 64),
    (BF16, 512, 8, 16, [1024, 3], 1024),
    (BF16, 256, 1, 1, [45, 9], 32),
    (BF16, 256, 32, 32, [700, 64, 33, 1], None),  # whole-tile page path at dim_v 256
    # one-token pages with the largest split: a split spans 1024 pages, every entry of
    # the kernel's staged block table
    (BF16, 512, 16, 1, [2053, 1030], 1024),
]


@pytest.mark.parametrize("dtype,dim_v,H,page_size,lens,tps", MLA_CASES)
def test_mla_decode_parity(dtype, dim_v, H, page_size, lens, tps):
    require_gpu()
    q, pool, bt, lens_t = _paged_case(11, lens, page_size, dim_v, H, dtype)
    scale = 1.0 / math.sqrt(dim_v + 64)
    say(f"mla decode {dtype} dim_v {dim_v} H {H} page {page_size} lens {lens} tps {tps}")
    o, lse = ffa.fastest_flash_mla_decode(q.cuda(), pool.cuda(), bt.cuda(), lens_t.cuda(),
                                          dim_v=dim_v, scale=scale, return_lse=True,
                                          tokens_per_split=tps)
    torch.cuda.synchronize()
    ro, rl = omla.paged_absorbed_decode(np32(q), np32(pool), bt.numpy(), lens, dim_v, scale)
    assert_parity(o, ro, lse, rl, f"mla {lens}")
    zero = [i for i, n in enumerate(lens) if n == 0]
    for i in zero:
        assert torch.all(o[i] == 0) and torch.all(torch.isneginf(lse[i]))


def test_mla_decode_negative_scale():
    require_gpu()
    lens = [200, 31]
    q, pool, bt, lens_t = _paged_case(8, lens, 16, 512, 32, BF16)
    say("mla decode negative scale")
    o, lse = ffa.fastest_flash_mla_decode(q.cuda(), pool.cuda(), bt.cuda(), lens_t.cuda(),
                                          dim_v=512, scale=-0.05, return_lse=True)
    ro, rl = omla.paged_absorbed_decode(np32(q), np32(pool), bt.numpy(), lens, 512, -0.05)
    assert_parity(o, ro, lse, rl, "mla negative scale")


def test_mla_decode_page_permutation_invariance():
    require_gpu()
    lens = [300, 17]
    q, pool, bt, lens_t = _paged_case(3, lens, 16, 512, 32, BF16, poison=False)
    say("mla decode permutation invariance")
    o1, l1 = ffa.fastest_flash_mla_decode(q.cuda(), pool.cuda(), bt.cuda(), lens_t.cuda(),
                                          dim_v=512, scale=0.05, return_lse=True)
    perm = torch.randperm(pool.size(0), generator=torch.Generator().manual_seed(4))
    inv = torch.empty_like(perm)
    inv[perm] = torch.arange(perm.numel())
    pool2 = pool[perm]               # physical page p moves to slot inv[p]
    bt2 = inv[bt.long()].to(torch.int32)
    o2, l2 = ffa.fastest_flash_mla_decode(q.cuda(), pool2.cuda(), bt2.cuda(), lens_t.cuda(),
                                          dim_v=512, scale=0.05, return_lse=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_latent_cache_append_bit_exact():
    require_gpu()
    g = torch.Generator().manual_seed(5)
    dev = ffa.MLALatentCache(max_pages=12, page_size=16, latent_dim=512, dtype=BF16, device="cuda")
    cpu = ffa.MLALatentCache(max_pages=12, page_size=16, latent_dim=512, dtype=BF16, device="cpu")
    say("mla latent cache append")
    for sid, n in [(0, 20), (1, 7), (0, 13), (2, 40), (1, 1)]:
        lat = torch.randn(n, 512, generator=g).to(BF16)
        rop = torch.randn(n, 64, generator=g).to(BF16)
        assert dev.append(sid, lat.cuda(), rop.cuda()) == cpu.append(sid, lat, rop)
    torch.cuda.synchronize()
    assert torch.equal(dev.pages.cpu(), cpu.pages)


def _mla_module(seed, dtype=BF16):
    torch.manual_seed(seed)
    m = ffa.FastestFlashMLA(hidden_size=512, num_heads=8, head_dim=128, latent_dim=512,
                            rope_dim=64)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0.0, 0.02)
    return m.to(device="cuda", dtype=dtype).eval()


def test_module_decode_step_matches_forward():
    """prefill_with_cache on S0 tokens, then decode steps: each step's attention output
    and module output equal the full causal forward at that position."""
    require_gpu()
    m = _mla_module(0)
    B, S0, S = 2, 37, 41
    g = torch.Generator().manual_seed(1)
    x = torch.randn(B, S, 512, generator=g).to(BF16).cuda()
    say("mla module decode_step vs forward")
    with torch.no_grad():
        q, k, v = m.project_qkv(x)
        attn_full, _ = ffa.fastest_flash_attn_forward(q, k, v, scale=m.scale, causal=True)
        out_full = m(x)
        cache = m.new_latent_cache(max_pages=16, page_size=16)
        out_pre = m.prefill_with_cache(x[:, :S0], cache, [0, 1])
        # the same causal rows through GEMMs of another shape: equal up to rounding
        pre_diff = (out_pre.float() - out_full[:, :S0].float()).abs()
        assert pre_diff.max().item() < 2e-2 and pre_diff.mean().item() < 2e-3
        for t in range(S0, S):
            out_t, attn_t = m.decode_step(x[:, t:t + 1], cache, [0, 1], return_attention=True)
            assert_parity(attn_t, np32(attn_full[:, :, t]), None, None, f"decode attn t={t}")
            diff = (out_t[:, 0].float() - out_full[:, t].float()).abs()
            assert diff.max().item() < 2e-2 and diff.mean().item() < 2e-3, (t, diff.max().item())
    assert cache.seq_len(0) == S and cache.seq_len(1) == S


def test_mla_decode_rejects_bad_shapes():
    require_gpu()
    q = torch.zeros(1, 4, 128 + 64, dtype=BF16, device="cuda")
    pool = torch.zeros(2, 16, 128 + 64, dtype=BF16, device="cuda")
    bt = torch.zeros(1, 2, dtype=torch.int32, device="cuda")
    lens = torch.ones(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError):
        ffa.fastest_flash_mla_decode(q, pool, bt, lens, dim_v=128, scale=0.1)
    with pytest.raises(RuntimeError):  # a CPU query: there is no CPU path
        ffa.fastest_flash_mla_decode(torch.zeros(1, 4, 576, dtype=BF16),
                                     pool.new_zeros(2, 16, 576), bt, lens, dim_v=512, scale=0.1)


def test_prepared_mla_call_matches_one_shot():
    """prepare_mla_decode once + launch_mla_decode per step (the serving loop form) gives
    the one-shot call's result, also after q is refilled in place."""
    require_gpu()
    from fastest_flash_attention_amd.ops.mla_decode import launch_mla_decode, prepare_mla_decode
    lens = [300, 45, 1]
    q, pool, bt, lens_t = _paged_case(21, lens, 16, 512, 32, BF16)
    q, pool, bt, lens_t = q.cuda(), pool.cuda(), bt.cuda(), lens_t.cuda()
    say("mla decode prepared call")
    with pytest.raises(ValueError, match="max_context_len"):
        prepare_mla_decode(q, pool, bt, lens_t, dim_v=512, scale=0.06)
    call = prepare_mla_decode(q, pool, bt, lens_t, dim_v=512, scale=0.06, return_lse=True,
                              max_context_len=300)
    for seed in (0, 1):
        if seed:
            q.copy_(torch.randn(q.shape, generator=torch.Generator().manual_seed(seed)).to(BF16))
        launch_mla_decode(call)
        o, lse = ffa.fastest_flash_mla_decode(q, pool, bt, lens_t, dim_v=512, scale=0.06,
                                              return_lse=True)
        torch.cuda.synchronize()
        assert torch.equal(call.out, o) and torch.equal(call.lse, lse)
    # lengths refilled past the prepared bound: the documented limit, the first
    # max_context_len tokens of the longer sequence
    lens_t.copy_(torch.tensor([310, 45, 1], dtype=torch.int32))
    launch_mla_decode(call)
    torch.cuda.synchronize()
    lens_t.copy_(torch.tensor([300, 45, 1], dtype=torch.int32))
    o, lse = ffa.fastest_flash_mla_decode(q, pool, bt, lens_t, dim_v=512, scale=0.06,
                                          return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(call.out, o) and torch.equal(call.lse, lse)
