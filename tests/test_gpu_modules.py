"""The unchanged callers (MHA / GQA / MLA modules) on the GPU path."""

from __future__ import annotations

import copy
import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from fastest_flash_attention_amd.utils import repeat_kv
from oracle import reference_forward as rf
from tests.gpu_util import np32, require_gpu, say

pytestmark = pytest.mark.gpu


def test_mha_module_matches_manual_composition():
    require_gpu()
    torch.manual_seed(0)
    m = ffa.FastestFlashMHA(hidden_size=256, num_heads=4, causal=True).cuda().to(torch.bfloat16)
    m.eval()
    x = torch.randn(2, 77, 256, device="cuda").to(torch.bfloat16)
    say("module MHA")
    out, lse = m(x, return_lse=True)
    q = m.q_proj(x).view(2, 77, 4, 64).transpose(1, 2)
    k = m.k_proj(x).view(2, 77, 4, 64).transpose(1, 2)
    v = m.v_proj(x).view(2, 77, 4, 64).transpose(1, 2)
    a, l2 = ffa.fastest_flash_attn_forward(q.contiguous(), k.contiguous(), v.contiguous(),
                                           causal=True, return_lse=True)
    ref = m.o_proj(a.transpose(1, 2).reshape(2, 77, 256))
    assert torch.equal(out, ref) and torch.equal(lse, l2)


def test_gqa_module_index_map_equals_repeat_kv():
    """The module passes unrepeated KV heads; the result must equal the reference's
    materialised repeat_kv path bit for bit."""
    require_gpu()
    torch.manual_seed(1)
    m = ffa.FastestFlashGQA(hidden_size=256, num_heads=8, num_kv_heads=2, causal=True,
                            softcap=30.0, sliding_window=40).cuda().to(torch.bfloat16)
    m.eval()
    x = torch.randn(2, 90, 256, device="cuda").to(torch.bfloat16)
    say("module GQA")
    out = m(x)
    q = m.q_proj(x).view(2, 90, 8, 32).transpose(1, 2)
    k = repeat_kv(m.k_proj(x).view(2, 90, 2, 32).transpose(1, 2), 8, 2)
    v = repeat_kv(m.v_proj(x).view(2, 90, 2, 32).transpose(1, 2), 8, 2)
    a, _ = ffa.fastest_flash_attn_forward(q, k, v, causal=True, softcap=30.0,
                                          sliding_window=40)
    ref = m.o_proj(a.transpose(1, 2).reshape(2, 90, 256))
    assert torch.equal(out, ref)


def test_mla_module_d192():
    require_gpu()
    torch.manual_seed(2)
    m = ffa.FastestFlashMLA(hidden_size=512, num_heads=4, head_dim=128, latent_dim=64,
                            rope_dim=64).cuda().to(torch.bfloat16)
    m.eval()
    x = torch.randn(1, 130, 512, device="cuda").to(torch.bfloat16)
    say("module MLA")
    out = m(x)
    # eval mode passes V at its 128 dims (taken as zero-padded to 192)
    q, k, v = m.project_qkv(x, pad_v=False)
    assert q.shape[-1] == 192 and v.shape[-1] == 128 and q.dtype == torch.bfloat16
    a, _ = ffa.fastest_flash_attn_forward(q, k, v, scale=m.scale, causal=True)
    assert torch.equal(out, m.o_proj(a.transpose(1, 2).reshape(1, 130, -1)))
    assert torch.isfinite(out).all()
    # the same as the reference's zero-padded V, up to rounding
    _, _, vp = m.project_qkv(x)
    ap, _ = ffa.fastest_flash_attn_forward(q, k, vp, scale=m.scale, causal=True)
    d = (a.float() - ap.float()).abs()
    assert torch.all(a[..., 128:] == 0) and d.max().item() < 2e-2 and d.mean().item() < 2e-3


def _mha_reference_fp32(m, x):
    """The module's training forward restated in plain fp32 torch on the CPU (same bf16
    weights and input, upcast): projections, causal softmax attention, output projection."""
    W = {n: p.detach().float().cpu().requires_grad_() for n, p in m.named_parameters()}
    xr = x.detach().float().cpu().requires_grad_()
    B, S, Hd = xr.shape
    H, D = m.num_heads, m.head_dim

    def heads(t):
        return t.view(B, S, H, D).transpose(1, 2)

    q = heads(xr @ W["q_proj.weight"].t())
    k = heads(xr @ W["k_proj.weight"].t())
    v = heads(xr @ W["v_proj.weight"].t())
    s = (q @ k.transpose(-1, -2)) * m.scale
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), diagonal=1)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1)
    a = (p @ v).transpose(1, 2).reshape(B, S, Hd)
    return a @ W["o_proj.weight"].t(), xr, W


def test_training_mode_forward_and_backward():
    """Training mode routes through the autograd function: gradients reach the input and
    every projection weight and match the fp32 CPU restatement of the module."""
    require_gpu()
    torch.manual_seed(3)
    m = ffa.FastestFlashMHA(hidden_size=128, num_heads=2, causal=True).cuda().to(torch.bfloat16)
    m.train()
    x = torch.randn(1, 40, 128, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    g = torch.randn(1, 40, 128, dtype=torch.bfloat16)
    say("module training-mode forward + backward")
    out = m(x)
    assert out.shape == (1, 40, 128)
    out.backward(g.cuda())
    ref, xr, W = _mha_reference_fp32(m, x)
    ref.backward(g.float())
    pairs = [(out, ref), (x.grad, xr.grad)]
    pairs += [(p.grad, W[n].grad) for n, p in m.named_parameters()]
    for got, want in pairs:
        assert got is not None and want is not None
        got = got.detach().float().cpu()
        want = want.detach()
        err = (got - want).abs()
        assert err.max() <= 5e-2 * want.abs().max(), (err.max(), want.abs().max())
        assert err.mean() <= 2e-2 * want.abs().mean(), (err.mean(), want.abs().mean())


def test_mla_training_mode_backward_d192():
    """The MLA module trains through the HIP backward at D = head_dim + rope_dim = 192:
    the loss gradient reaches the input and every projection weight and matches a fp32
    CPU restatement (the module's own projections and RoPE on an fp32 copy of its
    weights, textbook causal softmax attention over the zero-padded V)."""
    require_gpu()
    torch.manual_seed(4)
    m = ffa.FastestFlashMLA(hidden_size=256, num_heads=2, head_dim=128, latent_dim=64,
                            rope_dim=64).cuda().to(torch.bfloat16)
    m.train()
    B, S = 2, 70
    x = torch.randn(B, S, 256, device="cuda", dtype=torch.bfloat16, requires_grad=True)
    g = torch.randn(B, S, 256, dtype=torch.bfloat16)
    say("module MLA training-mode forward + backward (D = 192)")
    out = m(x)
    assert out.shape == (B, S, 256)
    out.backward(g.cuda())
    torch.cuda.synchronize()

    mr = copy.deepcopy(m).float().cpu()
    mr.zero_grad(set_to_none=True)
    xr = x.detach().float().cpu().requires_grad_()
    q, k, vp = mr.project_qkv(xr)
    assert q.shape[-1] == 192
    s = (q @ k.transpose(-1, -2)) * mr.scale
    mask = torch.triu(torch.ones(S, S, dtype=torch.bool), diagonal=1)
    p = torch.softmax(s.masked_fill(mask, float("-inf")), dim=-1)
    a = (p @ vp).transpose(1, 2).reshape(B, S, -1)
    ref = mr.o_proj(a)
    ref.backward(g.float())
    grads = dict(mr.named_parameters())
    pairs = [("out", out, ref), ("x", x.grad, xr.grad)]
    pairs += [(n, p_.grad, grads[n].grad) for n, p_ in m.named_parameters()]
    for name, got, want in pairs:
        assert got is not None and want is not None, name
        got = got.detach().float().cpu()
        want = want.detach()
        err = (got - want).abs()
        print(f"  {name}: max err {err.max():.3e} (ref max {want.abs().max():.3e})", flush=True)
        assert err.max() <= 5e-2 * want.abs().max(), (name, err.max(), want.abs().max())
        assert err.mean() <= 2e-2 * want.abs().mean(), (name, err.mean(), want.abs().mean())


def _close(name, got, want):
    got = got.detach().float().cpu()
    want = want.detach().float()
    err = (got - want).abs()
    print(f"  {name}: max err {err.max():.3e} (ref max {want.abs().max():.3e})", flush=True)
    assert err.max() <= 5e-2 * want.abs().max(), (name, err.max(), want.abs().max())
    assert err.mean() <= 2e-2 * want.abs().mean(), (name, err.mean(), want.abs().mean())


def test_eval_modules_match_fp32_restatement():
    """Eval mode of the three modules against an fp32 CPU restatement that shares no GPU
    code: the module's own projections (and RoPE) on an fp32 copy of its weights, the
    attention through the oracle (the reference dispatcher and CPU kernel, with its
    softcap / window / GQA semantics), the output projection."""
    require_gpu()
    torch.manual_seed(5)
    B, S = 2, 77
    cases = [
        ("MHA", ffa.FastestFlashMHA(hidden_size=256, num_heads=4, causal=True), {"causal": True}),
        ("GQA", ffa.FastestFlashGQA(hidden_size=256, num_heads=8, num_kv_heads=2, causal=True,
                                    softcap=30.0, sliding_window=40),
         {"causal": True, "softcap": 30.0, "sliding_window": 40, "num_kv_heads": 2}),
        ("MLA", ffa.FastestFlashMLA(hidden_size=256, num_heads=2, head_dim=128, latent_dim=64,
                                    rope_dim=64), {"causal": True}),
    ]
    for name, m, kw in cases:
        m = m.cuda().to(torch.bfloat16).eval()
        x = torch.randn(B, S, 256, device="cuda").to(torch.bfloat16)
        say(f"module {name} eval vs fp32 restatement")
        with torch.no_grad():
            out = m(x)
            mr = copy.deepcopy(m).float().cpu()
            xr = x.float().cpu()
            if name == "MLA":
                q, k, v = mr.project_qkv(xr)  # V zero-padded, as the reference builds it
                scale = mr.scale
            else:
                Hkv = kw.get("num_kv_heads", mr.num_heads)
                q = mr.q_proj(xr).view(B, S, mr.num_heads, mr.head_dim).transpose(1, 2)
                k = mr.k_proj(xr).view(B, S, Hkv, mr.head_dim).transpose(1, 2)
                v = mr.v_proj(xr).view(B, S, Hkv, mr.head_dim).transpose(1, 2)
                scale = getattr(mr, "scale", 1.0 / math.sqrt(mr.head_dim))
            a, _ = rf.forward(np32(q), np32(k), np32(v), scale=scale, return_lse=True, **kw)
            ref = mr.o_proj(torch.from_numpy(np.ascontiguousarray(a)).transpose(1, 2).reshape(B, S, -1))
        torch.cuda.synchronize()
        _close(f"{name} out", out, ref)


@pytest.mark.parametrize("name", ["MHA", "GQA-ref-layout", "GQA-kv-heads"])
def test_modules_with_kv_cache_match_oracle(name):
    """Eval-mode MHA / GQA modules with a kv_cache (decode-style: a few new tokens after
    a cached prefix) against the oracle's forward(..., kv_cache=...) fed the module's own
    fp32 projections. The GQA module takes the reference's cache layout, num_heads heads
    (ref modules/flash_gqa.py:101-125), and the num_kv_heads-head cache extension."""
    require_gpu()
    torch.manual_seed(12)
    B, S, Sc, H, Hkv, D = 2, 3, 150, 8, 2, 64
    hidden = H * D
    if name == "MHA":
        m = ffa.FastestFlashMHA(hidden_size=hidden, num_heads=H, causal=True)
        Hc, kw = H, {}
    else:
        m = ffa.FastestFlashGQA(hidden_size=hidden, num_heads=H, num_kv_heads=Hkv, causal=True,
                                softcap=30.0, sliding_window=100)
        Hc = H if name == "GQA-ref-layout" else Hkv
        kw = {"softcap": 30.0, "sliding_window": 100}
    m = m.cuda().to(torch.bfloat16).eval()
    x = torch.randn(B, S, hidden).to(torch.bfloat16)
    kc = torch.randn(B, Hc, Sc, D).to(torch.bfloat16)
    vc = torch.randn(B, Hc, Sc, D).to(torch.bfloat16)
    say(f"module {name} with kv_cache")
    with torch.no_grad():
        out, lse = m(x.cuda(), kv_cache=(kc.cuda(), vc.cuda()), return_lse=True)
        torch.cuda.synchronize()
        mr = copy.deepcopy(m).float().cpu()
        xr = x.float()
        q = mr.q_proj(xr).view(B, S, H, D).transpose(1, 2)
        hk = H if name == "MHA" else Hkv
        k = mr.k_proj(xr).view(B, S, hk, D).transpose(1, 2)
        v = mr.v_proj(xr).view(B, S, hk, D).transpose(1, 2)
        if name == "GQA-ref-layout":  # the reference module repeats, then the op concatenates
            k, v = repeat_kv(k, H, Hkv), repeat_kv(v, H, Hkv)
        okw = dict(kw)
        if name == "GQA-kv-heads":
            okw["num_kv_heads"] = Hkv
        a, l_ref = rf.forward(np32(q), np32(k), np32(v), scale=mr.scale, causal=True,
                              kv_cache=(np32(kc), np32(vc)), return_lse=True, **okw)
        ref = mr.o_proj(torch.from_numpy(np.ascontiguousarray(a)).transpose(1, 2).reshape(B, S, -1))
    _close(f"{name} out", out, ref)
    assert np.abs(np32(lse) - l_ref).max() <= 1e-2, np.abs(np32(lse) - l_ref).max()
