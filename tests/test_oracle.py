"""Pins the CPU oracle (oracle/) before it is trusted as the parity checker.

1. The reference's own test suite (reference tests/test_fastest_flash.py), run on the
   oracle with the same seeded inputs (torch.manual_seed + torch.randn) against the
   reference's test oracle _naive_sdpa restated in fp64 (oracle/naive.py), at the
   reference tolerances.
2. Independent library routines: scipy.special.logsumexp / softmax, torch's bf16 and
   fp16 rounding.
3. Closed forms: a single key gives O = V, identical keys give mean(V), constant V
   gives O = V, fully-masked rows give the sentinel derived by hand below.
4. Invariants: block-size invariance, GQA == explicit repetition, two-pass == one-pass.
5. Planted mistakes in the oracle's helpers must make these checks fail.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import scipy.special
import torch

from oracle import naive
from oracle import paged as opaged
from oracle import reference_forward as rf


def randn(*shape):
    return torch.randn(*shape).numpy()


def close(a, b, atol):
    return np.allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), atol=atol, rtol=0)


def ref_naive(q, k, v, scale, causal=False, softcap=None, window_size=None):
    """_naive_sdpa of the reference tests (tests/test_fastest_flash.py:55-88)."""
    o, _ = naive.naive_sdpa(q, k, v, scale, causal=causal, softcap=softcap, window=window_size)
    return o


# ---------------------------------------------------------------------------------
# 1. The reference test suite, on the oracle
# ---------------------------------------------------------------------------------

class TestReferenceSuiteOnOracle:
    @pytest.mark.parametrize("block_size", [4, 8, 16, 32])
    def test_3d_various_blocks(self, block_size):
        torch.manual_seed(42)
        B, S, D = 2, 32, 16
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, S, D), randn(B, S, D), randn(B, S, D)
        ref = ref_naive(q, k, v, scale)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=block_size)
        assert close(ref, out, 1e-5)

    def test_4d_input(self):
        torch.manual_seed(0)
        B, H, S, D = 2, 4, 24, 16
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=8)
        assert close(ref_naive(q, k, v, scale), out, 1e-5)

    def test_non_divisible_seq_len(self):
        torch.manual_seed(1)
        B, H, S, D = 1, 2, 17, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=8)
        assert close(ref_naive(q, k, v, scale), out, 1e-5)

    @pytest.mark.parametrize("block_size", [4, 8, 16])
    def test_causal_matches_naive(self, block_size):
        torch.manual_seed(10)
        B, H, S, D = 2, 4, 32, 16
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, block_size=block_size)
        assert close(ref_naive(q, k, v, scale, causal=True), out, 1e-5)

    def test_causal_3d(self):
        torch.manual_seed(11)
        B, S, D = 2, 20, 16
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, S, D), randn(B, S, D), randn(B, S, D)
        ref = ref_naive(q[:, None], k[:, None], v[:, None], scale, causal=True)[:, 0]
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, block_size=8)
        assert close(ref, out, 1e-5)

    @pytest.mark.parametrize("window", [4, 8, 16])
    def test_sliding_window(self, window):
        torch.manual_seed(20)
        B, H, S, D = 1, 2, 24, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, sliding_window=window,
                            block_size=4)
        assert close(ref_naive(q, k, v, scale, causal=True, window_size=window), out, 1e-5)

    @pytest.mark.parametrize("cap", [5.0, 10.0, 30.0])
    def test_softcap_matches_naive(self, cap):
        torch.manual_seed(30)
        B, H, S, D = 2, 2, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, softcap=cap, block_size=4)
        assert close(ref_naive(q, k, v, scale, softcap=cap), out, 1e-4)

    def test_softcap_causal(self):
        torch.manual_seed(31)
        B, H, S, D = 1, 2, 20, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, softcap=15.0, block_size=8)
        assert close(ref_naive(q, k, v, scale, causal=True, softcap=15.0), out, 1e-4)

    def test_block_mask_full_equals_dense(self):
        torch.manual_seed(40)
        B, H, S, D = 1, 1, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        full = np.ones((4, 4), dtype=bool)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4, block_mask=full)
        assert close(ref_naive(q, k, v, scale), out, 1e-5)

    def test_sparse_mask_differs(self):
        torch.manual_seed(41)
        B, H, S, D = 1, 1, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        full, _ = rf.forward(q, k, v, scale=scale, block_size=4)
        mask = np.ones((4, 4), dtype=bool)
        mask[0, -1] = False
        sparse, _ = rf.forward(q, k, v, scale=scale, block_size=4, block_mask=mask)
        assert not close(full, sparse, 1e-6)
        # rows of q tile 0 equal attention over keys 0..11 only (closed form)
        ref0 = ref_naive(q[:, :, :4], k[:, :, :12], v[:, :, :12], scale)
        assert close(sparse[:, :, :4], ref0, 1e-5)

    def test_two_pass_matches_one_pass(self):
        torch.manual_seed(50)
        B, H, S, D = 2, 2, 24, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        ref = ref_naive(q, k, v, scale)
        o1, _ = rf.forward(q, k, v, scale=scale, block_size=8, two_pass=False)
        o2, _ = rf.forward(q, k, v, scale=scale, block_size=8, two_pass=True)
        assert close(ref, o1, 1e-5) and close(ref, o2, 1e-5)

    def test_two_pass_causal(self):
        torch.manual_seed(51)
        B, H, S, D = 1, 2, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, block_size=4, two_pass=True)
        assert close(ref_naive(q, k, v, scale, causal=True), out, 1e-5)

    def test_fp16_compute(self):
        torch.manual_seed(60)
        B, H, S, D = 2, 2, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4, compute_dtype="float16")
        assert close(ref_naive(q, k, v, scale), out, 1e-3)
        # exact statement: the scores use q, k rounded to fp16 (numpy's own cast)
        ref16 = ref_naive(q.astype(np.float16), k.astype(np.float16), v, scale)
        assert close(ref16, out, 1e-5)

    def test_kv_cache_with_attention(self):
        torch.manual_seed(70)
        B, H, D = 1, 2, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, 6, D), randn(B, H, 6, D), randn(B, H, 6, D)
        out, _ = rf.forward(q, k[:, :, 4:], v[:, :, 4:], scale=scale, block_size=4,
                            kv_cache=(k[:, :, :4], v[:, :, :4]))
        assert close(ref_naive(q, k, v, scale), out, 1e-5)

    def test_gqa_and_mqa(self):
        torch.manual_seed(80)
        B, S, D = 2, 16, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, 4, S, D), randn(B, 2, S, D), randn(B, 2, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4, num_kv_heads=2)
        # closed form: q head h uses kv head h // 2 (no repeat helper involved)
        for h in range(4):
            ref_h = ref_naive(q[:, h], k[:, h // 2], v[:, h // 2], scale)
            assert close(ref_h, out[:, h], 1e-5)
        torch.manual_seed(81)
        q, k, v = randn(1, 4, 12, D), randn(1, 1, 12, D), randn(1, 1, 12, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4, num_kv_heads=1)
        for h in range(4):
            assert close(ref_naive(q[:, h], k[:, 0], v[:, 0], scale), out[:, h], 1e-5)

    def test_combined(self):
        torch.manual_seed(130)
        B, H, S, D = 1, 2, 24, 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(B, H, S, D), randn(B, H, S, D), randn(B, H, S, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, sliding_window=8, block_size=4)
        assert close(ref_naive(q, k, v, scale, causal=True, window_size=8), out, 1e-5)
        torch.manual_seed(131)
        q, k, v = randn(1, 2, 16, D), randn(1, 2, 16, D), randn(1, 2, 16, D)
        out, _ = rf.forward(q, k, v, scale=scale, causal=True, softcap=10.0, sliding_window=8,
                            block_size=4)
        ref = ref_naive(q, k, v, scale, causal=True, softcap=10.0, window_size=8)
        assert close(ref, out, 1e-4)

    def test_edge_cases(self):
        torch.manual_seed(140)
        D = 8
        scale = 1.0 / math.sqrt(D)
        q, k, v = randn(1, 2, 1, D), randn(1, 2, 1, D), randn(1, 2, 1, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4)
        assert close(ref_naive(q, k, v, scale), out, 1e-5)
        torch.manual_seed(141)
        q, k, v = randn(1, 2, 8, D), randn(1, 2, 16, D), randn(1, 2, 16, D)
        out, _ = rf.forward(q, k, v, scale=scale, block_size=4)
        assert close(ref_naive(q, k, v, scale), out, 1e-5)
        torch.manual_seed(142)
        D = 128
        q, k, v = randn(1, 1, 8, D), randn(1, 1, 8, D), randn(1, 1, 8, D)
        out, _ = rf.forward(q, k, v, scale=1 / math.sqrt(D), block_size=4)
        assert close(ref_naive(q, k, v, 1 / math.sqrt(D)), out, 1e-5)

    def test_lse(self):
        torch.manual_seed(150)
        q, k, v = randn(2, 2, 16, 8), randn(2, 2, 16, 8), randn(2, 2, 16, 8)
        _, lse = rf.forward(q, k, v, block_size=4, return_lse=True)
        assert lse.shape == (2, 2, 16, 1)
        torch.manual_seed(151)
        q, k, v = randn(1, 1, 8, 4), randn(1, 1, 8, 4), randn(1, 1, 8, 4)
        scale = 0.5
        _, lse = rf.forward(q, k, v, scale=scale, block_size=4, return_lse=True)
        ref = scipy.special.logsumexp(np.matmul(q, k.swapaxes(-1, -2)) * scale, axis=-1,
                                      keepdims=True)
        assert close(lse, ref, 1e-4)

    def test_numerical_stability(self):
        torch.manual_seed(160)
        q, k, v = randn(1, 1, 8, 4) * 100, randn(1, 1, 8, 4) * 100, randn(1, 1, 8, 4)
        out, _ = rf.forward(q, k, v, block_size=4)
        assert np.isfinite(out).all()
        q = np.zeros((1, 1, 4, 4), np.float32)
        k, v = randn(1, 1, 4, 4), randn(1, 1, 4, 4)
        out, _ = rf.forward(q, k, v, block_size=4)
        assert close(out, np.broadcast_to(v.mean(axis=2, keepdims=True), out.shape), 1e-6)

    def test_config(self):
        class Cfg:  # attributes of AttentionConfig (reference config.py:58-73)
            block_size_q = 4
            block_size_kv = 4
            causal = True
            sliding_window = None
            softcap = None
            num_kv_heads = None
            compute_dtype = None
            two_pass = False
            return_lse = False

        torch.manual_seed(170)
        q, k, v = randn(2, 2, 16, 8), randn(2, 2, 16, 8), randn(2, 2, 16, 8)
        out, _ = rf.forward(q, k, v, config=Cfg(), causal=False)  # config wins
        assert close(ref_naive(q, k, v, 1 / math.sqrt(8), causal=True), out, 1e-5)


# ---------------------------------------------------------------------------------
# 2-4. Independent routines, closed forms, invariants
# ---------------------------------------------------------------------------------

@pytest.mark.parametrize("causal,window,softcap,q_offset", [
    (False, None, None, 0), (True, None, None, 0), (True, 24, None, 0), (False, 7, None, 0),
    (True, None, 20.0, 0), (True, 16, 30.0, 0), (True, None, None, 40), (False, 9, 5.0, 33),
])
def test_lse_and_output_vs_scipy(causal, window, softcap, q_offset):
    rng = np.random.default_rng(7)
    B, H, Sq, Skv, D = 1, 2, 37, 77, 32
    q = rng.standard_normal((B, H, Sq, D)).astype(np.float32)
    k = rng.standard_normal((B, H, Skv, D)).astype(np.float32)
    v = rng.standard_normal((B, H, Skv, D)).astype(np.float32)
    scale = 1 / math.sqrt(D)
    out, lse = rf.flash_attn_cpu_forward(q, k, v, scale=scale, causal=causal, block_q=16,
                                         block_kv=16, softcap=softcap, sliding_window=window,
                                         q_offset=q_offset, return_lse=True)
    s = np.matmul(q.astype(np.float64), k.astype(np.float64).swapaxes(-1, -2)) * scale
    if softcap is not None:
        s = softcap * np.tanh(s / softcap)
    rows = q_offset + np.arange(Sq)[:, None]
    cols = np.arange(Skv)[None, :]
    vis = np.ones((Sq, Skv), bool)
    if causal:
        vis &= cols <= rows
    if window is not None:
        vis &= cols >= rows - window + 1
    has = vis.any(axis=1)
    s = np.where(vis, s, -np.inf)
    ref_lse = scipy.special.logsumexp(s[..., has, :], axis=-1)
    assert np.abs(lse[..., has, 0] - ref_lse).max() < 2e-5
    w = scipy.special.softmax(s[..., has, :], axis=-1)
    assert np.abs(out[..., has, :] - w @ v).max() < 2e-5


def test_closed_forms():
    rng = np.random.default_rng(3)
    D = 16
    q = rng.standard_normal((1, 2, 9, D)).astype(np.float32)
    v1 = rng.standard_normal((1, 2, 1, D)).astype(np.float32)
    k1 = rng.standard_normal((1, 2, 1, D)).astype(np.float32)
    out, _ = rf.flash_attn_cpu_forward(q, k1, v1, block_q=4, block_kv=4)
    assert close(out, np.broadcast_to(v1, out.shape), 1e-6)          # one key: O = V
    kk = np.broadcast_to(k1, (1, 2, 12, D)).copy()
    vv = rng.standard_normal((1, 2, 12, D)).astype(np.float32)
    out, _ = rf.flash_attn_cpu_forward(q, kk, vv, block_q=4, block_kv=8)
    assert close(out, np.broadcast_to(vv.mean(axis=2, keepdims=True), out.shape), 1e-5)
    vc = np.broadcast_to(vv[:, :, :1], vv.shape).copy()
    kr = rng.standard_normal((1, 2, 12, D)).astype(np.float32)
    out, _ = rf.flash_attn_cpu_forward(q, kr, vc, causal=True, block_q=4, block_kv=4)
    assert close(out, np.broadcast_to(vc[:, :, :1], out.shape), 1e-5)  # constant V
    # softcap -> infinity equals no softcap
    o1, l1 = rf.flash_attn_cpu_forward(q, kr, vv, softcap=1e6, block_q=4, block_kv=4,
                                       return_lse=True)
    o2, l2 = rf.flash_attn_cpu_forward(q, kr, vv, block_q=4, block_kv=4, return_lse=True)
    assert close(o1, o2, 1e-5) and close(l1, l2, 1e-5)


def test_fully_masked_row_sentinel():
    """Non-causal window 4, S_q=32, S_kv=8, block 4 (derived by hand from the loop
    conditions of cpu_reference.py:215-231): KV tile j (keys 4j..4j+3) is skipped for q
    tile i when 4j+3 < 4i-3. Rows 0..10 see keys; row 11 (q tile 2) visits only KV tile 1
    -> one logaddexp of log(1e-30); rows 12..31 (q tiles 3..7) visit nothing -> -inf."""
    rng = np.random.default_rng(11)
    q = rng.standard_normal((1, 1, 32, 8)).astype(np.float32)
    k = rng.standard_normal((1, 1, 8, 8)).astype(np.float32)
    v = rng.standard_normal((1, 1, 8, 8)).astype(np.float32)
    out, lse = rf.flash_attn_cpu_forward(q, k, v, block_q=4, block_kv=4, sliding_window=4,
                                         return_lse=True)
    assert np.all(out[0, 0, 11:] == 0)
    assert abs(lse[0, 0, 11, 0] - math.log(np.float32(1e-30))) < 1e-4
    assert np.all(np.isneginf(lse[0, 0, 12:, 0]))
    ref_o, ref_l = naive.naive_sdpa(q[:, :, :11], k, v, window=4)
    assert close(out[:, :, :11], ref_o, 1e-5) and close(lse[:, :, :11], ref_l, 1e-5)
    # with block 8 the same row 11 sits in q tile 1 (rows 8..15, q_abs_s=8): KV tile 0
    # (keys 0..7) is kept since 7 >= 8-4+1 -> n=1 for rows 11..15; rows 16+ -> -inf
    _, lse8 = rf.flash_attn_cpu_forward(q, k, v, block_q=8, block_kv=8, sliding_window=4,
                                        return_lse=True)
    assert np.allclose(lse8[0, 0, 11:16, 0], math.log(np.float32(1e-30)), atol=1e-4)
    assert np.all(np.isneginf(lse8[0, 0, 16:, 0]))
    # two tiles visited, both fully masked for the row: log(2 * 1e-30)
    q2 = rng.standard_normal((1, 1, 8, 8)).astype(np.float32)
    k2 = rng.standard_normal((1, 1, 8, 8)).astype(np.float32)
    _, l2 = rf.flash_attn_cpu_forward(q2, k2, k2, causal=True, block_q=8, block_kv=4,
                                      q_offset=-5, return_lse=True)
    # q_offset=-5: row r sits at -5+r; rows 0..4 see no key (key 0 > row); q tile [−5, 2]
    # reaches key tiles with ks <= 2 -> only tile 0 -> n = 1
    assert np.allclose(l2[0, 0, :5, 0], math.log(np.float32(1e-30)), atol=1e-4)


@pytest.mark.parametrize("bs", [16, 32, 64, 128])
def test_block_size_invariance(bs):
    rng = np.random.default_rng(5)
    q = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    k = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    v = rng.standard_normal((1, 2, 150, 64)).astype(np.float32)
    o_ref, l_ref = naive.naive_sdpa(q, k, v, causal=True, window=50)
    o, l = rf.flash_attn_cpu_forward(q, k, v, causal=True, sliding_window=50, block_q=bs,
                                     block_kv=bs, return_lse=True)
    assert close(o, o_ref, 2e-5) and close(l, l_ref, 2e-5)


def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(5000).astype(np.float32) * 10,
                        np.array([0.0, -0.0, 1.0, 1.00390625, 1.01171875, 3.4e38, -3.4e38,
                                  1e-40, np.inf, -np.inf], np.float32)])
    mine = rf.round_to_bf16(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(mine.view(np.uint32), theirs.view(np.uint32))


def test_auto_block_size_table():
    # reference utils.py:36-67 evaluated by hand for the configs
    assert rf.auto_select_block_size(1024, 1024, 64) == 64
    assert rf.auto_select_block_size(4096, 4096, 128) == 32
    assert rf.auto_select_block_size(4096, 4096, 192) == 16
    assert rf.auto_select_block_size(8, 8, 16) == 16
    assert rf.auto_select_block_size(24, 24, 8) == 16


# ---------------------------------------------------------------------------------
# 5. Planted mistakes must be caught by the pins above
# ---------------------------------------------------------------------------------

def _pin_suite_passes() -> bool:
    try:
        for args in [(True, 24, None, 0), (False, 7, None, 0), (True, None, 20.0, 0),
                     (True, None, None, 40)]:
            test_lse_and_output_vs_scipy(*args)
        test_fully_masked_row_sentinel()
        test_bf16_rounding_matches_torch()
    except AssertionError:
        return False
    return True


@pytest.mark.parametrize("mutant", ["softcap_no_tanh", "window_off_by_one", "causal_diag",
                                    "logaddexp_max", "bf16_truncate"])
def test_planted_mistakes_fail(monkeypatch, mutant):
    assert _pin_suite_passes()
    if mutant == "softcap_no_tanh":
        monkeypatch.setattr(rf, "apply_softcap", lambda s, c: s)
    elif mutant == "window_off_by_one":
        monkeypatch.setattr(rf, "window_mask", lambda qs, qe, ks, ke, w: (
            np.arange(ks, ke)[None, :] < (np.arange(qs, qe)[:, None] - w)))
    elif mutant == "causal_diag":
        monkeypatch.setattr(rf, "causal_mask", lambda qs, qe, ks, ke: (
            np.arange(qs, qe)[:, None] <= np.arange(ks, ke)[None, :]))
    elif mutant == "logaddexp_max":
        monkeypatch.setattr(rf, "_logaddexp", lambda a, b: np.maximum(a, b).astype(np.float32))
    elif mutant == "bf16_truncate":
        monkeypatch.setattr(rf, "round_to_bf16", lambda x: (
            np.ascontiguousarray(x, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32))
    assert not _pin_suite_passes()


# ---------------------------------------------------------------------------------
# Paged oracle
# ---------------------------------------------------------------------------------

def test_paged_pool_round_trip_and_index_law():
    rng = np.random.default_rng(1)
    pool = opaged.PagedPool(max_pages=16, page_size=4, num_heads=2, head_dim=8)
    k0 = rng.standard_normal((2, 6, 8)).astype(np.float32)
    v0 = rng.standard_normal((2, 6, 8)).astype(np.float32)
    assert pool.append_tokens(0, k0, v0) == 6
    k1 = rng.standard_normal((2, 3, 8)).astype(np.float32)
    pool.append_tokens(1, k1, k1)
    k0b = rng.standard_normal((2, 5, 8)).astype(np.float32)
    pool.append_tokens(0, k0b, k0b)
    ko, vo = pool.get_kv(0)
    assert np.array_equal(ko, np.concatenate([k0, k0b], axis=1))
    assert np.array_equal(vo[:, :6], v0)
    table = pool.sequences[0]["page_table"]
    assert table == [0, 1, 3]  # seq 1 took page 2 between the two appends of seq 0
    for t in range(11):
        page, slot = opaged.token_location(table, t, 4)
        assert np.array_equal(pool.k_pages[page, :, slot], ko[:, t])
    pool.free_sequence(0)
    assert pool.free_pages[-3:] == [0, 1, 3]
    with pytest.raises(RuntimeError, match="out of physical pages"):
        small = opaged.PagedPool(max_pages=1, page_size=4, num_heads=1, head_dim=2)
        small.append_tokens(0, np.zeros((1, 5, 2), np.float32), np.zeros((1, 5, 2), np.float32))


def test_paged_decode_oracle_vs_naive():
    rng = np.random.default_rng(2)
    B, Hq, Hkv, D, P = 3, 8, 2, 32, 4
    lens = [1, 9, 17]
    pages_needed = [math.ceil(L / P) for L in lens]
    n_pages = sum(pages_needed) + 3
    perm = rng.permutation(n_pages)
    k_pages = rng.standard_normal((n_pages, Hkv, P, D)).astype(np.float32)
    v_pages = rng.standard_normal((n_pages, Hkv, P, D)).astype(np.float32)
    bt = np.zeros((B, max(pages_needed)), np.int32)
    off = 0
    for b, n in enumerate(pages_needed):
        bt[b, :n] = perm[off:off + n]
        off += n
    q = rng.standard_normal((B, Hq, D)).astype(np.float32)
    for window, cap in [(None, None), (5, None), (None, 7.0)]:
        o, lse = opaged.paged_decode(q, k_pages, v_pages, bt, lens, sliding_window=window,
                                     softcap=cap, block_size=4)
        for b, L in enumerate(lens):
            kb, vb = opaged.gather_sequence(k_pages, v_pages, list(bt[b]), L)
            for h in range(Hq):
                ro, rl = naive.naive_sdpa(q[b, h][None], kb[h // 4], vb[h // 4], softcap=cap,
                                          window=window, q_offset=L - 1)
                assert close(o[b, h], ro[0], 1e-5)
                assert abs(lse[b, h] - rl[0, 0]) < 1e-5
