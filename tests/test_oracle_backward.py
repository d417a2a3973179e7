"""Pins oracle/reference_backward.py (the restated reference backward) on the CPU.

1. torch.autograd in fp64 through the textbook attention (scores * scale, softcap
   c * tanh(s / c), causal / one-sided window relative to q_offset, softmax, P V)
   gives the same dq, dk, dv on small shapes, with O and LSE from the oracle forward.
2. Block-size invariance of the tiled recompute.
3. GQA: the group sum equals the gradient through an explicit repeat_kv.
4. Planted mistakes (softcap derivative dropped, D_i dropped, scale missing on dK)
   fail check 1.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import reference_backward as rb
from oracle import reference_forward as rf


def _autograd(q, k, v, do, scale, causal, window, softcap, q_offset):
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    s = qt @ kt.transpose(-1, -2) * scale
    if softcap is not None:
        s = softcap * torch.tanh(s / softcap)
    S_q, S_kv = q.shape[2], k.shape[2]
    row = torch.arange(S_q)[:, None] + q_offset
    col = torch.arange(S_kv)[None, :]
    masked = torch.zeros(S_q, S_kv, dtype=torch.bool)
    if causal:
        masked |= col > row
    if window is not None:
        masked |= col < row - window + 1
    s = s.masked_fill(masked, -math.inf)
    o = torch.softmax(s, dim=-1) @ vt
    o.backward(torch.tensor(do, dtype=torch.float64))
    return qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


CASES = [
    # B, H, S_q, S_kv, D, causal, window, softcap, q_offset, block
    (1, 2, 13, 13, 8, False, None, None, 0, 4),
    (2, 1, 17, 17, 16, True, None, None, 0, 8),
    (1, 2, 20, 20, 8, True, 5, None, 0, 4),
    (1, 1, 15, 15, 8, True, None, 3.0, 0, 8),
    (1, 2, 6, 19, 8, True, 7, 2.0, 13, 4),
    (1, 1, 11, 9, 16, False, 4, None, 0, 4),
]


def _inputs(seed, B, H, S_q, S_kv, D):
    rng = np.random.default_rng(seed)
    f = lambda *s: rng.standard_normal(s).astype(np.float32)  # noqa: E731
    return f(B, H, S_q, D), f(B, H, S_kv, D), f(B, H, S_kv, D), f(B, H, S_q, D)


@pytest.mark.parametrize("case", CASES)
def test_backward_matches_autograd(case):
    B, H, S_q, S_kv, D, causal, window, softcap, off, bs = case
    q, k, v, do = _inputs(1, B, H, S_q, S_kv, D)
    scale = 1.0 / math.sqrt(D)
    o, lse = rf.flash_attn_cpu_forward(q, k, v, scale=scale, causal=causal, block_q=bs,
                                       block_kv=bs, softcap=softcap, sliding_window=window,
                                       q_offset=off, return_lse=True)
    dq, dk, dv = rb.flash_attn_cpu_backward(do, q, k, v, o, lse, scale=scale, causal=causal,
                                            block_q=bs, block_kv=bs, softcap=softcap,
                                            sliding_window=window, q_offset=off)
    gq, gk, gv = _autograd(q, k, v, do, scale, causal, window, softcap, off)
    for got, want in ((dq, gq), (dk, gk), (dv, gv)):
        assert np.allclose(got, want, atol=2e-5, rtol=1e-4)


def test_block_size_invariance():
    q, k, v, do = _inputs(2, 1, 2, 37, 37, 16)
    o, lse = rf.flash_attn_cpu_forward(q, k, v, causal=True, block_q=16, block_kv=16,
                                       return_lse=True)
    a = rb.flash_attn_cpu_backward(do, q, k, v, o, lse, causal=True, block_q=4, block_kv=16)
    b = rb.flash_attn_cpu_backward(do, q, k, v, o, lse, causal=True, block_q=32, block_kv=8)
    for x, y in zip(a, b):
        assert np.allclose(x, y, atol=1e-5)


def test_gqa_sum_equals_explicit_repeat():
    rng = np.random.default_rng(3)
    q = rng.standard_normal((1, 4, 21, 8)).astype(np.float32)
    k = rng.standard_normal((1, 2, 21, 8)).astype(np.float32)
    v = rng.standard_normal((1, 2, 21, 8)).astype(np.float32)
    do = rng.standard_normal((1, 4, 21, 8)).astype(np.float32)
    o, lse = rf.forward(q, k, v, causal=True, num_kv_heads=2, return_lse=True)
    dq, dk, dv = rb.backward(do, q, k, v, o, lse, causal=True, block_size=8)
    kr, vr = np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1)
    gq, gk, gv = _autograd(q, kr, vr, do, 1 / math.sqrt(8), True, None, None, 0)
    assert np.allclose(dq, gq, atol=2e-5)
    assert np.allclose(dk, gk.reshape(1, 2, 2, 21, 8).sum(2), atol=2e-5)
    assert np.allclose(dv, gv.reshape(1, 2, 2, 21, 8).sum(2), atol=2e-5)


def test_planted_mistakes_fail(monkeypatch):
    B, H, S_q, S_kv, D, causal, window, softcap, off, bs = CASES[3]
    q, k, v, do = _inputs(1, B, H, S_q, S_kv, D)
    scale = 1.0 / math.sqrt(D)
    o, lse = rf.flash_attn_cpu_forward(q, k, v, scale=scale, causal=causal, block_q=bs,
                                       block_kv=bs, softcap=softcap, return_lse=True)
    gq, gk, _ = _autograd(q, k, v, do, scale, causal, window, softcap, off)
    # softcap derivative dropped: tanh' = 1 everywhere
    monkeypatch.setattr(rb.np, "tanh", lambda x: np.zeros_like(x))
    dq, _, _ = rb.flash_attn_cpu_backward(do, q, k, v, o, lse, scale=scale, causal=causal,
                                          block_q=bs, block_kv=bs, softcap=softcap)
    monkeypatch.undo()
    assert not np.allclose(dq, gq, atol=1e-3)
    # D_i dropped (dS = P * dP)
    dq, _, _ = rb.flash_attn_cpu_backward(do, q, k, v, np.zeros_like(o), lse, scale=scale,
                                          causal=causal, block_q=bs, block_kv=bs,
                                          softcap=softcap)
    assert not np.allclose(dq, gq, atol=1e-3)
    # scale missing on dK (scale applied twice elsewhere is the same class of error)
    _, dk, _ = rb.flash_attn_cpu_backward(do, q, k, v, o, lse, scale=scale, causal=causal,
                                          block_q=bs, block_kv=bs, softcap=softcap)
    assert not np.allclose(dk / scale, gk, atol=1e-3)
