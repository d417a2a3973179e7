"""GPU parity of the attention backward (ffa_attn_bwd through fastest_flash_attn_backward
and FastestFlashAttnFunc.backward) against the CPU oracle
(oracle/reference_backward.py, itself pinned by fp64 autograd) on identical inputs:
the same 16-bit q, k, v, dO and the same O (rounded to the input dtype) and LSE.

Tolerance (the gradients have no tolerance of their own in the task statement; these
bars are stated here, per tensor, relative to the oracle's magnitude): P and dS are
rounded to the input's 16-bit type for the matrix products and the results are
stored in it, so
    max |got - ref| <= 2e-2 * max |ref|   and   mean |got - ref| <= 1e-2 * mean |ref|
for bf16 (8-bit mantissa), a quarter of that for fp16 (11-bit). The fp32 kernels keep
every product and the stored gradients in fp32, so their bar is a hundredth of bf16's:
    max |got - ref| <= 2e-4 * max |ref|   and   mean |got - ref| <= 1e-4 * mean |ref|
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import reference_backward as rb
from oracle import reference_forward as rf
from tests.gpu_util import np32, require_gpu, say, seeded

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _oracle_forward(q, k, v, *, scale, causal, window, softcap, q_offset, two_pass=False):
    """O (fp32) and LSE of the reference forward, K/V repeated to q's heads."""
    ratio = q.shape[1] // k.shape[1]
    kr, vr = np.repeat(np32(k), ratio, axis=1), np.repeat(np32(v), ratio, axis=1)
    return rf.flash_attn_cpu_forward(np32(q), kr, vr, scale=scale, causal=causal,
                                     softcap=softcap, sliding_window=window,
                                     two_pass=two_pass, q_offset=q_offset, return_lse=True)


def _check(got: torch.Tensor, ref: np.ndarray, dtype, what: str):
    g = np32(got).astype(np.float64)
    r = np.asarray(ref, dtype=np.float64)
    assert g.shape == r.shape, (what, g.shape, r.shape)
    assert np.isfinite(g).all(), f"{what}: non-finite gradient"
    rel = {BF16: 1.0, F16: 0.25, F32: 0.01}[dtype]
    err = np.abs(g - r)
    if r.size == 0:
        return
    max_ref, mean_ref = float(np.abs(r).max()), float(np.abs(r).mean())
    print(f"  {what}: max err {err.max():.3e} (ref max {max_ref:.3e}), "
          f"mean err {err.mean():.3e} (ref mean {mean_ref:.3e})", flush=True)
    # absolute floors: a gradient that is zero in exact arithmetic (one visible key gives
    # dS = dP - D_i = 0) is left with fp32 cancellation residue of dO . v (about 1e-6)
    assert err.max() <= 2e-2 * rel * max_ref + 1e-5, f"{what}: max err {err.max():.3e}"
    assert err.mean() <= 1e-2 * rel * mean_ref + 2e-6, f"{what}: mean err {err.mean():.3e}"


# (name, B, Hq, Hkv, Sq, Skv, D, q_offset, kwargs, dtype)
CASES = [
    ("plain", 2, 4, 4, 128, 128, 64, 0, {}, BF16),
    ("causal_ragged", 1, 3, 3, 257, 257, 128, 0, {"causal": True}, BF16),
    ("noncausal_ragged", 1, 2, 2, 200, 333, 128, 0, {}, BF16),
    ("causal_window", 1, 2, 2, 300, 300, 128, 0, {"causal": True, "sliding_window": 37}, BF16),
    ("window_noncausal", 1, 2, 2, 180, 180, 64, 0, {"sliding_window": 50}, BF16),
    ("softcap_causal", 2, 2, 2, 150, 150, 64, 0, {"causal": True, "softcap": 10.0}, BF16),
    ("gqa", 1, 8, 2, 256, 256, 128, 0, {"causal": True}, BF16),
    ("mqa", 1, 4, 1, 96, 96, 64, 0, {}, BF16),
    ("q_offset_causal", 1, 2, 2, 70, 300, 128, 230, {"causal": True}, BF16),
    ("q_offset_window_softcap", 1, 4, 2, 45, 200, 64, 155,
     {"causal": True, "sliding_window": 60, "softcap": 20.0}, BF16),
    ("d40_padded", 1, 2, 2, 100, 100, 40, 0, {"causal": True}, BF16),
    ("d96", 1, 2, 2, 77, 77, 96, 0, {"causal": True}, BF16),
    ("d16", 2, 2, 2, 40, 40, 16, 0, {}, BF16),
    ("fp16_softcap", 1, 4, 4, 200, 200, 128, 0, {"causal": True, "softcap": 30.0}, F16),
    ("fp16_gqa_window", 2, 4, 2, 160, 160, 64, 0, {"causal": True, "sliding_window": 33}, F16),
    ("single", 1, 2, 2, 1, 1, 64, 0, {}, BF16),
    ("negative_scale", 1, 2, 2, 150, 150, 64, 0, {"causal": True, "scale": -0.2}, BF16),
    ("zero_scale", 1, 2, 2, 70, 70, 64, 0, {"causal": True, "scale": 0.0}, BF16),
    ("gqa_window_softcap", 2, 8, 2, 333, 333, 128, 0,
     {"causal": True, "sliding_window": 100, "softcap": 50.0}, BF16),
    # head_dim 192 (the MLA module's head_dim + rope_dim) and 256
    ("d192_causal", 1, 4, 4, 300, 300, 192, 0, {"causal": True}, BF16),
    ("d192_gqa_window_softcap", 2, 4, 2, 257, 257, 192, 0,
     {"causal": True, "sliding_window": 90, "softcap": 30.0}, BF16),
    ("d192_noncausal_ragged", 1, 2, 2, 150, 211, 192, 0, {}, BF16),
    ("d256_causal", 1, 2, 2, 200, 200, 256, 0, {"causal": True}, BF16),
    ("d176_fp16_qoffset", 1, 2, 1, 60, 190, 176, 130, {"causal": True}, F16),
    ("d256_fp16_window", 1, 2, 2, 130, 130, 256, 0, {"sliding_window": 41}, F16),
    # fp32 (the reference's default training dtype)
    ("fp32_cfg1_shape", 2, 8, 8, 1024, 1024, 64, 0, {"causal": True}, F32),
    ("fp32_d128_noncausal", 1, 2, 2, 133, 170, 128, 0, {}, F32),
    ("fp32_d40", 1, 2, 2, 100, 100, 40, 0, {}, F32),
    ("fp32_d192_gqa_window_softcap", 1, 4, 2, 160, 160, 192, 0,
     {"causal": True, "sliding_window": 50, "softcap": 20.0}, F32),
    ("fp32_d256_causal", 1, 2, 2, 97, 97, 256, 0, {"causal": True}, F32),
    ("fp32_q_offset", 1, 2, 2, 40, 180, 64, 140, {"causal": True, "softcap": 15.0}, F32),
    ("fp32_single", 1, 1, 1, 1, 1, 64, 0, {}, F32),
    # fp32 MFMA kernels (head_dim <= 128): GQA + window + softcap over many tiles per
    # wave, ragged ends, q_offset with a window, negative scale, MQA at head_dim 128
    ("fp32_d64_gqa_window_softcap", 2, 8, 2, 300, 300, 64, 0,
     {"causal": True, "sliding_window": 100, "softcap": 30.0}, F32),
    ("fp32_d128_causal_ragged", 1, 3, 3, 289, 289, 128, 0, {"causal": True}, F32),
    ("fp32_d96_qoffset_window", 1, 2, 1, 70, 250, 96, 180,
     {"causal": True, "sliding_window": 64}, F32),
    ("fp32_d128_mqa_window_noncausal", 1, 4, 1, 150, 203, 128, 0, {"sliding_window": 45}, F32),
    ("fp32_negative_scale", 1, 2, 2, 150, 150, 64, 0, {"causal": True, "scale": -0.2}, F32),
    ("fp32_d16_noncausal", 2, 2, 2, 40, 67, 16, 0, {}, F32),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_backward_parity(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, off, kw, dt = case
    q = seeded((B, Hq, Sq, D), dt, 1)
    k = seeded((B, Hkv, Skv, D), dt, 2)
    v = seeded((B, Hkv, Skv, D), dt, 3)
    do = seeded((B, Hq, Sq, D), dt, 4)
    scale = kw.get("scale", 1.0 / math.sqrt(D))
    causal = kw.get("causal", False)
    window = kw.get("sliding_window")
    softcap = kw.get("softcap")
    o32, lse = _oracle_forward(q, k, v, scale=scale, causal=causal, window=window,
                               softcap=softcap, q_offset=off)
    o = torch.from_numpy(o32).to(dt)
    say(f"backward {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} off{off} {kw} {dt}")
    dq, dk, dv = ffa.fastest_flash_attn_backward(
        do.cuda(), q.cuda(), k.cuda(), v.cuda(), o.cuda(), torch.from_numpy(lse).cuda(),
        scale=scale, causal=causal, softcap=softcap, sliding_window=window, q_offset=off)
    torch.cuda.synchronize()
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    assert dq.dtype == dk.dtype == dv.dtype == dt
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(v), np32(o), lse, scale=scale,
                             causal=causal, softcap=softcap, sliding_window=window,
                             q_offset=off)
    _check(dq, rq, dt, f"{name} dq")
    _check(dk, rk, dt, f"{name} dk")
    _check(dv, rv, dt, f"{name} dv")


# (name, B, Hq, Hkv, Sq, Skv, D, Dv, q_offset, kwargs, dtype): v narrower than q / k,
# taken as zero-padded (the MLA module's V); head_dim 129..192 with Dv <= 128 (a
# multiple of 8) runs the narrow-V kernels, the last two are zero-padded on the host
NARROW_V = [
    ("mla_causal", 1, 4, 4, 300, 300, 192, 128, 0, {"causal": True}, BF16),
    ("mla_gqa_window_softcap", 2, 4, 2, 257, 257, 192, 128, 0,
     {"causal": True, "sliding_window": 90, "softcap": 30.0}, BF16),
    ("mla_noncausal_ragged", 1, 2, 2, 150, 211, 192, 128, 0, {}, BF16),
    ("d136_dv64_fp16_qoffset", 1, 2, 1, 60, 190, 136, 64, 130, {"causal": True}, F16),
    ("d160_dv120_window", 1, 2, 2, 140, 140, 160, 120, 0, {"sliding_window": 41}, BF16),
    ("host_padded_d128_dv64", 1, 2, 2, 90, 90, 128, 64, 0, {"causal": True}, BF16),
    ("host_padded_fp32", 1, 2, 2, 90, 90, 192, 128, 0, {"causal": True}, F32),
]


@pytest.mark.parametrize("case", NARROW_V, ids=[c[0] for c in NARROW_V])
def test_backward_narrow_v(case):
    require_gpu()
    name, B, Hq, Hkv, Sq, Skv, D, Dv, off, kw, dt = case
    q = seeded((B, Hq, Sq, D), dt, 61)
    k = seeded((B, Hkv, Skv, D), dt, 62)
    v = seeded((B, Hkv, Skv, Dv), dt, 63)
    do = seeded((B, Hq, Sq, D), dt, 64)
    vp = torch.nn.functional.pad(v, (0, D - Dv))
    scale = 1.0 / math.sqrt(D)
    causal = kw.get("causal", False)
    window = kw.get("sliding_window")
    softcap = kw.get("softcap")
    o32, lse = _oracle_forward(q, k, vp, scale=scale, causal=causal, window=window,
                               softcap=softcap, q_offset=off)
    o = torch.from_numpy(o32).to(dt)
    say(f"backward narrow v {name} B{B} Hq{Hq} Hkv{Hkv} Sq{Sq} Skv{Skv} D{D} Dv{Dv} off{off} {kw} {dt}")
    dq, dk, dv = ffa.fastest_flash_attn_backward(
        do.cuda(), q.cuda(), k.cuda(), v.cuda(), o.cuda(), torch.from_numpy(lse).cuda(),
        scale=scale, causal=causal, softcap=softcap, sliding_window=window, q_offset=off)
    torch.cuda.synchronize()
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(vp), np32(o), lse, scale=scale,
                             causal=causal, softcap=softcap, sliding_window=window,
                             q_offset=off)
    _check(dq, rq, dt, f"{name} dq")
    _check(dk, rk, dt, f"{name} dk")
    _check(dv, rv[..., :Dv], dt, f"{name} dv")


@pytest.mark.parametrize("dt", [BF16, F32], ids=["bf16", "fp32"])
def test_backward_deterministic(dt):
    """No atomics: two calls give bit-identical gradients (fp32: the four waves' partial
    sums of a block meet in a fixed order)."""
    require_gpu()
    B, H, S, D = 2, 4, 300, 128
    q, k, v, do = (seeded((B, H, S, D), dt, s).cuda() for s in (11, 12, 13, 14))
    say(f"backward determinism {dt}")
    o, lse = ffa.fastest_flash_attn_forward(q, k, v, causal=True, return_lse=True)
    a = ffa.fastest_flash_attn_backward(do, q, k, v, o, lse, causal=True)
    b = ffa.fastest_flash_attn_backward(do, q, k, v, o, lse, causal=True)
    torch.cuda.synchronize()
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_autograd_func_matches_oracle():
    """fastest_flash_attn_func forward + .backward() (the training entry point), 3D
    inputs, against the oracle fed the HIP forward's own O and LSE."""
    require_gpu()
    B, S, D = 2, 190, 64
    q, k, v = (seeded((B, S, D), BF16, s).cuda().requires_grad_() for s in (21, 22, 23))
    do = seeded((B, S, D), BF16, 24).cuda()
    say("autograd func 3D causal softcap")
    out = ffa.fastest_flash_attn_func(q, k, v, causal=True, softcap=15.0)
    out.backward(do)
    torch.cuda.synchronize()
    o, lse = ffa.fastest_flash_attn_forward(q.detach(), k.detach(), v.detach(), causal=True,
                                            softcap=15.0, return_lse=True)
    assert torch.equal(o, out.detach())
    rq, rk, rv = rb.backward(np32(do)[:, None], np32(q)[:, None], np32(k)[:, None],
                             np32(v)[:, None], np32(o)[:, None], np32(lse)[:, None],
                             causal=True, softcap=15.0)
    _check(q.grad, rq[:, 0], BF16, "func dq")
    _check(k.grad, rk[:, 0], BF16, "func dk")
    _check(v.grad, rv[:, 0], BF16, "func dv")


def test_autograd_func_gqa_matches_oracle():
    require_gpu()
    B, Hq, Hkv, S, D = 1, 8, 2, 256, 128
    q = seeded((B, Hq, S, D), BF16, 31).cuda().requires_grad_()
    k = seeded((B, Hkv, S, D), BF16, 32).cuda().requires_grad_()
    v = seeded((B, Hkv, S, D), BF16, 33).cuda().requires_grad_()
    do = seeded((B, Hq, S, D), BF16, 34).cuda()
    say("autograd func GQA")
    out = ffa.fastest_flash_attn_func(q, k, v, causal=True, num_kv_heads=Hkv)
    out.backward(do)
    o, lse = ffa.fastest_flash_attn_forward(q.detach(), k.detach(), v.detach(), causal=True,
                                            num_kv_heads=Hkv, return_lse=True)
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(v), np32(o), np32(lse),
                             causal=True)
    _check(q.grad, rq, BF16, "gqa dq")
    _check(k.grad, rk, BF16, "gqa dk")
    _check(v.grad, rv, BF16, "gqa dv")


def test_autograd_func_narrow_v():
    """fastest_flash_attn_func with V narrower than q / k (the MLA shape: 192 / 128)
    against the same call on the zero-padded V: the output and dQ / dK agree to the
    kernels' rounding (other key tiles), and dV is the padded call's dV on V's dims."""
    require_gpu()
    B, H, S, D, Dv = 1, 4, 200, 192, 128
    q = seeded((B, H, S, D), BF16, 41).cuda()
    k = seeded((B, H, S, D), BF16, 42).cuda()
    v = seeded((B, H, S, Dv), BF16, 43).cuda()
    do = seeded((B, H, S, D), BF16, 44).cuda()
    say("autograd func narrow v")
    grads = []
    for vv in (v, torch.nn.functional.pad(v, (0, D - Dv))):
        qa, ka, va = (t.clone().requires_grad_() for t in (q, k, vv))
        out = ffa.fastest_flash_attn_func(qa, ka, va, causal=True)
        out.backward(do)
        grads.append((out.detach(), qa.grad, ka.grad, va.grad))
    torch.cuda.synchronize()
    (o1, dq1, dk1, dv1), (o2, dq2, dk2, dv2) = grads
    assert dv1.shape == v.shape and torch.all(o1[..., Dv:] == 0)
    for what, x, y in (("O", o1, o2), ("dQ", dq1, dq2), ("dK", dk1, dk2),
                       ("dV", dv1, dv2[..., :Dv])):
        d = (x.float() - y.float()).abs()
        ref = y.float().abs().max().item()
        assert d.max().item() <= 2e-2 * max(ref, 1.0), (what, d.max().item(), ref)


def test_autograd_func_fp32_matches_oracle():
    """Training in fp32 (the reference's default dtype): fp32 forward + fp32 backward
    through fastest_flash_attn_func, GQA with a window, against the oracle fed the HIP
    forward's own O and LSE."""
    require_gpu()
    B, Hq, Hkv, S, D = 2, 4, 2, 230, 64
    q = seeded((B, Hq, S, D), F32, 51).cuda().requires_grad_()
    k = seeded((B, Hkv, S, D), F32, 52).cuda().requires_grad_()
    v = seeded((B, Hkv, S, D), F32, 53).cuda().requires_grad_()
    do = seeded((B, Hq, S, D), F32, 54).cuda()
    say("autograd func fp32 GQA window")
    out = ffa.fastest_flash_attn_func(q, k, v, causal=True, num_kv_heads=Hkv,
                                      sliding_window=70)
    out.backward(do)
    torch.cuda.synchronize()
    o, lse = ffa.fastest_flash_attn_forward(q.detach(), k.detach(), v.detach(), causal=True,
                                            num_kv_heads=Hkv, sliding_window=70,
                                            return_lse=True)
    assert out.dtype == q.grad.dtype == k.grad.dtype == F32
    rq, rk, rv = rb.backward(np32(do), np32(q), np32(k), np32(v), np32(o), np32(lse),
                             causal=True, sliding_window=70)
    _check(q.grad, rq, F32, "fp32 func dq")
    _check(k.grad, rk, F32, "fp32 func dk")
    _check(v.grad, rv, F32, "fp32 func dv")


def test_empty_inputs():
    """No keys: dq = 0 and empty dk/dv; no queries or no batch: empty gradients."""
    require_gpu()
    from fastest_flash_attention_amd.ops.attention_backward import fastest_flash_attn_backward
    q = seeded((1, 2, 6, 64), BF16, 71).cuda()
    none = torch.zeros(1, 2, 0, 64, dtype=BF16, device="cuda")
    say("backward empty: S_kv = 0")
    o, lse = ffa.fastest_flash_attn_forward(q, none, none, return_lse=True)
    dq, dk, dv = fastest_flash_attn_backward(seeded((1, 2, 6, 64), BF16, 72).cuda(), q, none,
                                             none, o, lse)
    assert dq.shape == q.shape and not dq.abs().any()
    assert dk.shape == none.shape and dv.shape == none.shape
    say("backward empty: S_q = 0, B = 0")
    for shape in ((1, 2, 0, 64), (0, 2, 5, 64)):
        z = torch.zeros(*shape, dtype=BF16, device="cuda")
        lz = torch.zeros(*shape[:3], 1, dtype=torch.float32, device="cuda")
        kv = z if shape[0] == 0 else seeded((1, 2, 5, 64), BF16, 73).cuda()
        dq, dk, dv = fastest_flash_attn_backward(z, z, kv, kv, z, lz)
        assert dq.shape == z.shape and dk.shape == kv.shape and not dk.abs().any()


def test_rows_without_keys_get_zero_gradient():
    """A two-pass forward gives rows with no visible key lse = -inf; their P is 0 (the
    reference's exp(-inf - (-inf)) would be NaN), so they add nothing to dK / dV and
    get dq = 0. Here the window leaves rows 0..q_offset-window-… empty: q_offset < 0."""
    require_gpu()
    B, H, Sq, Skv, D = 1, 2, 64, 64, 64
    q, k, v, do = (seeded((B, H, n, D), BF16, s) for n, s in ((Sq, 41), (Skv, 42), (Skv, 43),
                                                               (Sq, 44)))
    off = -20  # rows 0..19 sit before key 0: causal leaves them no key
    o32, lse = _oracle_forward(q, k, v, scale=0.125, causal=True, window=None, softcap=None,
                               q_offset=off, two_pass=True)
    assert np.isneginf(lse[:, :, :20]).all() and np.isfinite(lse[:, :, 20:]).all()
    o = torch.from_numpy(np.nan_to_num(o32)).to(BF16)
    say("backward rows without keys")
    dq, dk, dv = ffa.fastest_flash_attn_backward(
        do.cuda(), q.cuda(), k.cuda(), v.cuda(), o.cuda(), torch.from_numpy(lse).cuda(),
        scale=0.125, causal=True, q_offset=off)
    torch.cuda.synchronize()
    assert torch.all(dq[:, :, :20] == 0)
    # the live rows alone give the oracle's dK / dV
    live = slice(20, None)
    rq, rk, rv = rb.backward(np32(do)[:, :, live], np32(q)[:, :, live], np32(k), np32(v),
                             np32(o)[:, :, live], lse[:, :, live], scale=0.125, causal=True,
                             q_offset=off + 20)
    _check(dq[:, :, live], rq, BF16, "live dq")
    _check(dk, rk, BF16, "live dk")
    _check(dv, rv, BF16, "live dv")


def test_backward_rejects_unsupported():
    require_gpu()
    x = torch.zeros(1, 2, 8, 264, dtype=BF16, device="cuda")
    lse = torch.zeros(1, 2, 8, 1, device="cuda")
    with pytest.raises(ValueError):
        ffa.fastest_flash_attn_backward(x, x, x, x, x, lse)
    y = torch.zeros(1, 2, 8, 64, dtype=torch.float64, device="cuda")
    with pytest.raises(TypeError):
        ffa.fastest_flash_attn_backward(y, y, y, y, y, lse)
