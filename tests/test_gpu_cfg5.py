"""The MLA module at its BASELINE size: FastestFlashMLA(hidden 4096, 32 heads,
head_dim 128, latent 512, rope 64), weights ~ N(0, 0.02), inputs ~ N(0, 1), bf16.

* prefill: B = 2, S = 4096, causal, D = head_dim + rope = 192 through the HIP prefill;
  the attention output and LSE of sampled (batch, head) pairs and row blocks (start,
  middle, end of the causal triangle) against the oracle forward
  (oracle/reference_forward.py), the module output against o_proj of that attention.
* decode: 32 sequences of 4095 cached latent rows (prefill_with_cache), then one
  decode_step each (context 4096) through ffa_mla_decode_fwd; the per-head attention
  output of sampled sequences against the reference's up-projected attention
  (oracle/mla.py up_projected_decode: K = [c W_uk^T | r], V = [c W_uv^T | 0]) on the
  cached rows, and the module output against o_proj of that attention.

Tolerances: the north-star bars (O max-abs 2e-2, mean-abs 2e-3, LSE 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from oracle import mla as omla
from oracle import reference_forward as rf
from tests.gpu_util import assert_parity, np32, require_gpu, say

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16
HIDDEN, HEADS, HEAD_DIM, LATENT, ROPE = 4096, 32, 128, 512, 64


def _cfg5_module(seed: int) -> ffa.FastestFlashMLA:
    torch.manual_seed(seed)
    m = ffa.FastestFlashMLA(HIDDEN, HEADS, HEAD_DIM, LATENT, ROPE)
    with torch.no_grad():
        for p in m.parameters():
            p.normal_(0.0, 0.02)
    return m.to(device="cuda", dtype=BF16).eval()


def _randn(shape, seed):
    g = torch.Generator(device="cuda").manual_seed(seed)
    return torch.randn(*shape, generator=g, device="cuda").to(BF16)


def test_cfg5_prefill_full_size():
    require_gpu()
    m = _cfg5_module(0)
    B, S = 2, 4096
    x = _randn((B, S, HIDDEN), 1)
    say("cfg5 prefill B2 S4096 hidden 4096 H32 D192")
    with torch.no_grad():
        # the module's own call: V at its 128 dims, taken as zero-padded to 192
        q, k, v = m.project_qkv(x, pad_v=False)
        assert q.shape == (B, HEADS, S, HEAD_DIM + ROPE) and v.shape[-1] == HEAD_DIM
        attn, lse = ffa.fastest_flash_attn_forward(q, k, v, scale=m.scale, causal=True,
                                                   return_lse=True)
        out = m(x)
        torch.cuda.synchronize()
        assert torch.isfinite(attn).all() and torch.isfinite(lse).all()
        assert torch.equal(out, m.o_proj(attn.transpose(1, 2).reshape(B, S, -1)))
        assert torch.all(attn[..., HEAD_DIM:] == 0)
        # the reference's zero-padded V through the 192-dim kernel: the same O up to
        # rounding (other key tiles), the same LSE
        vp = torch.nn.functional.pad(v, (0, ROPE))
        attn_p, lse_p = ffa.fastest_flash_attn_forward(q, k, vp, scale=m.scale, causal=True,
                                                       return_lse=True)
        d = (attn.float() - attn_p.float()).abs()
        assert d.max().item() < 2e-2 and d.mean().item() < 2e-3, d.max().item()
        assert (lse - lse_p).abs().max().item() < 1e-3
    # sampled (batch, head) pairs over both batches and the head range
    for b, h in ((0, 0), (0, 13), (1, 7), (1, 31)):
        for r0 in (0, 2048 - 64, S - 128):
            r1 = r0 + 128
            qs = np32(q[b:b + 1, h:h + 1, r0:r1])
            ks, vs = np32(k[b:b + 1, h:h + 1, :r1]), np32(vp[b:b + 1, h:h + 1, :r1])
            ro, rl = rf.flash_attn_cpu_forward(qs, ks, vs, scale=m.scale, causal=True,
                                               q_offset=r0, return_lse=True)
            assert_parity(attn[b:b + 1, h:h + 1, r0:r1], ro, lse[b:b + 1, h:h + 1, r0:r1],
                          rl, f"cfg5 prefill b{b} h{h} rows {r0}..{r1}")


def test_cfg5_decode_step_full_size():
    require_gpu()
    m = _cfg5_module(2)
    B, ctx, chunk = 32, 4096, 8
    cache = m.new_latent_cache(max_pages=B * ctx // 64 + 8, page_size=64)
    ids = list(range(B))
    say(f"cfg5 prefill_with_cache {B} x {ctx - 1} tokens")
    with torch.no_grad():
        for c0 in range(0, B, chunk):
            m.prefill_with_cache(_randn((chunk, ctx - 1, HIDDEN), 100 + c0), cache,
                                 ids[c0:c0 + chunk])
        assert all(cache.seq_len(s) == ctx - 1 for s in ids)
        xt = _randn((B, 1, HIDDEN), 3)
        say(f"cfg5 decode_step batch {B} context {ctx}")
        out, attn = m.decode_step(xt, cache, ids, return_attention=True)
        torch.cuda.synchronize()
        assert all(cache.seq_len(s) == ctx for s in ids)
        assert out.shape == (B, 1, HIDDEN) and attn.shape == (B, HEADS, HEAD_DIM + ROPE)
        assert torch.isfinite(out).all()
        assert torch.equal(out, m.o_proj(attn.reshape(B, 1, -1)))
        # the decode's own bf16 query projections (same GEMMs as decode_step)
        q_nope = m.q_proj(xt).view(B, HEADS, HEAD_DIM)
        q_rope = m.rope.rotate_at(m.q_rope_proj(xt).view(B, HEADS, ROPE), [ctx - 1] * B)
        w_uk, w_uv = (np32(w).astype(np.float64) for w in m.absorbed_weights())
    bt, lens = cache.block_tables(ids, device="cpu")
    pages = np32(cache.pages)
    heads = [0, 5, 11, 18, 24, 31]
    for b in (0, 13, 31):
        rows = omla.paged_rows(pages, bt[b].tolist(), int(lens[b])).astype(np.float64)
        assert rows.shape == (ctx, LATENT + ROPE)
        ro, _ = omla.up_projected_decode(np32(q_nope[b, heads]).astype(np.float64),
                                         np32(q_rope[b, heads]).astype(np.float64),
                                         rows[:, :LATENT], rows[:, LATENT:],
                                         w_uk[heads], w_uv[heads], m.scale)
        assert_parity(attn[b, heads], ro, None, None, f"cfg5 decode seq {b} heads {heads}")
