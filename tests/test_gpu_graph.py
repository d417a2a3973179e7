"""HIP graph capture of the prepared C-ABI calls (the serving-loop form): the prefill
and the MLA latent decode are captured once into a torch.cuda.CUDAGraph and replayed
several times, with the inputs refilled in place and eager work between replays, and
every replay must equal the eager call on the same inputs bit for bit. The library
records no memset and allocates nothing inside these calls, so a capture holds only
their kernels."""

from __future__ import annotations

import pytest
import torch

import fastest_flash_attention_amd as ffa
from fastest_flash_attention_amd.ops.attention_forward import launch_prefill, prepare_prefill
from fastest_flash_attention_amd.ops.mla_decode import launch_mla_decode, prepare_mla_decode
from tests.gpu_util import require_gpu, say, seeded

pytestmark = pytest.mark.gpu

BF16 = torch.bfloat16


def test_prefill_graph_replays_match_eager():
    require_gpu()
    B, H, Hk, S, D = 2, 8, 2, 300, 128
    q = seeded((B, H, S, D), BF16, 61).cuda()
    k = seeded((B, Hk, S, D), BF16, 62).cuda()
    v = seeded((B, Hk, S, D), BF16, 63).cuda()
    kw = dict(causal=True, sliding_window=100, softcap=30.0, num_kv_heads=Hk, return_lse=True)
    say("prefill graph capture")
    call = prepare_prefill(q, k, v, **kw)
    assert call.q.data_ptr() == q.data_ptr()  # the launch reads q in place
    launch_prefill(call)  # eager once before capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_prefill(call)
    for rep in range(3):
        gen = torch.Generator().manual_seed(100 + rep)
        q.copy_(torch.randn(q.shape, generator=gen).to(BF16))
        call.out.fill_(float("nan"))
        call.lse.fill_(float("nan"))
        graph.replay()
        o_ref, lse_ref = ffa.fastest_flash_attn_forward(q, k, v, **kw)  # eager, same inputs
        torch.cuda.synchronize()
        assert torch.equal(call.out.reshape(o_ref.shape), o_ref), f"replay {rep}: O differs from eager"
        assert torch.equal(call.lse.reshape(lse_ref.shape), lse_ref), f"replay {rep}: LSE differs"


def test_prefill_graph_narrow_v_block_mask():
    """A captured narrow-V prefill (head_dim 192 over a 128-dim V) with a block mask: the
    launch carries dynamic LDS for the mask's tile list; replays equal eager calls."""
    require_gpu()
    B, H, S, D, Dv, bs = 1, 4, 260, 192, 128, 32
    q = seeded((B, H, S, D), BF16, 81).cuda()
    k = seeded((B, H, S, D), BF16, 82).cuda()
    v = seeded((B, H, S, Dv), BF16, 83).cuda()
    gen = torch.Generator().manual_seed(84)
    n = (S + bs - 1) // bs
    bm = torch.rand(n, n, generator=gen) < 0.6
    kw = dict(causal=True, block_size=bs, block_mask=bm, return_lse=True)
    say("prefill graph capture, narrow v + block mask")
    call = prepare_prefill(q, k, v, **kw)
    assert call.args.v_head_dim == Dv and call.args.block_key_mask
    launch_prefill(call)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_prefill(call)
    for rep in range(3):
        g2 = torch.Generator().manual_seed(200 + rep)
        q.copy_(torch.randn(q.shape, generator=g2).to(BF16))
        call.out.fill_(float("nan"))
        call.lse.fill_(float("nan"))
        graph.replay()
        o_ref, lse_ref = ffa.fastest_flash_attn_forward(q, k, v, **kw)
        torch.cuda.synchronize()
        assert torch.equal(call.out.reshape(o_ref.shape), o_ref), f"replay {rep}: O differs from eager"
        assert torch.equal(call.lse.reshape(lse_ref.shape), lse_ref), f"replay {rep}: LSE differs"


def test_mla_decode_graph_replays_match_eager():
    require_gpu()
    B, H, L, lat, R, P = 5, 32, 700, 512, 64, 64
    n_pages = B * ((L + P - 1) // P)
    gen = torch.Generator().manual_seed(71)
    pool = torch.randn(n_pages, P, lat + R, generator=gen).to(BF16).cuda()
    bt = torch.randperm(n_pages, generator=gen).to(torch.int32).view(B, -1).contiguous().cuda()
    lens = torch.tensor([700, 1, 333, 64, 650], dtype=torch.int32).cuda()
    q = torch.randn(B, H, lat + R, generator=gen).to(BF16).cuda()
    say("mla decode graph capture")
    call = prepare_mla_decode(q, pool, bt, lens, dim_v=lat, scale=0.07, return_lse=True,
                              max_context_len=L)
    assert call.q.data_ptr() == q.data_ptr()  # the launch reads q in place
    launch_mla_decode(call)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch_mla_decode(call)
    for rep in range(3):
        g2 = torch.Generator().manual_seed(200 + rep)
        q.copy_(torch.randn(q.shape, generator=g2).to(BF16))
        call.out.fill_(float("nan"))
        call.lse.fill_(float("nan"))
        graph.replay()
        o_ref, lse_ref = ffa.fastest_flash_mla_decode(q, pool, bt, lens, dim_v=lat, scale=0.07,
                                                      return_lse=True, max_context_len=L)
        torch.cuda.synchronize()
        assert torch.equal(call.out, o_ref), f"replay {rep}: O differs from eager"
        assert torch.equal(call.lse, lse_ref), f"replay {rep}: LSE differs from eager"
