"""ffa_paged_decode_fwd_noalloc (the allocation-free paged decode) against
ffa_paged_decode_fwd (the same kernels with a caller workspace), through the C ABI.

Two calls in a row on one GPU, the second with a smaller problem, must each equal the
workspace entry point's result bit for bit: the shared scratch array keeps the first
call's partials, and the second call must read only what it wrote. The scratch limit
is checked on the host, before any device work.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from fastest_flash_attention_amd.kernels import _lib
from tests.gpu_util import require_gpu, say

BF16 = torch.bfloat16


def _problem(seed, lens, Hq, Hkv, D, P):
    g = torch.Generator().manual_seed(seed)
    pages = [max(1, math.ceil(n / P)) for n in lens]
    total = sum(pages) + 2
    perm = torch.randperm(total, generator=g)
    bt = torch.zeros(len(lens), max(pages), dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[off:off + n].to(torch.int32)
        off += n
    k_pages = torch.randn(total, Hkv, P, D, generator=g).to(BF16)
    v_pages = torch.randn(total, Hkv, P, D, generator=g).to(BF16)
    q = torch.randn(len(lens), Hq, D, generator=g).to(BF16)
    dev = "cuda"
    return (q.to(dev), k_pages.to(dev), v_pages.to(dev), bt.to(dev),
            torch.tensor(lens, dtype=torch.int32, device=dev))


def _args(q, k_pages, v_pages, bt, lens_t, out, lse, max_len, tps, workspace=None):
    a = _lib.PagedDecodeArgs()
    a.q, a.k_pages, a.v_pages = q.data_ptr(), k_pages.data_ptr(), v_pages.data_ptr()
    a.o, a.lse = out.data_ptr(), lse.data_ptr()
    a.block_tables, a.context_lens = bt.data_ptr(), lens_t.data_ptr()
    if workspace is not None:
        a.workspace = workspace.data_ptr()
        a.workspace_bytes = workspace.numel()
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.o_stride[:] = [out.stride(0), out.stride(1)]
    a.lse_stride[:] = [lse.stride(0), lse.stride(1)]
    a.block_table_stride = bt.size(1)
    a.batch, a.heads_q, a.heads_kv, a.head_dim = q.size(0), q.size(1), k_pages.size(1), q.size(2)
    a.page_size, a.num_pages = k_pages.size(2), k_pages.size(0)
    a.max_context_len, a.tokens_per_split = max_len, tps
    a.scale, a.dtype = 1.0 / math.sqrt(q.size(2)), _lib.FFA_DTYPE_BF16
    return a


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode():
    require_gpu()
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    # the second problem is smaller: fewer sequences, shorter contexts, other splits
    for lens, Hq, Hkv, D, P, tps in (([700, 33, 2049, 1, 0, 300], 8, 2, 128, 16, 64),
                                     ([129, 5], 4, 1, 64, 16, 32)):
        q, kp, vp, bt, lens_t = _problem(len(lens), lens, Hq, Hkv, D, P)
        max_len = max(lens)
        need = lib.ffa_paged_decode_workspace_bytes(len(lens), Hq, D, max_len, tps)
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
        o_ref = torch.empty_like(q)
        l_ref = torch.empty(len(lens), Hq, dtype=torch.float32, device="cuda")
        say(f"no-alloc decode: workspace entry point, lens {lens}")
        a = _args(q, kp, vp, bt, lens_t, o_ref, l_ref, max_len, tps, workspace=ws)
        assert lib.ffa_paged_decode_fwd(ctypes.byref(a), stream) == 0
        o = torch.full_like(q, float("nan"))
        lse = torch.full((len(lens), Hq), float("nan"), dtype=torch.float32, device="cuda")
        say(f"no-alloc decode: allocation-free entry point, lens {lens}")
        b = _args(q, kp, vp, bt, lens_t, o, lse, max_len, tps)  # no workspace given
        rc = lib.ffa_paged_decode_fwd_noalloc(ctypes.byref(b), stream)
        assert rc == 0, _lib.strerror(rc)
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), (o.float() - o_ref.float()).abs().max()
        assert torch.equal(lse, l_ref)


def test_noalloc_scratch_limit_is_checked_on_the_host():
    """A call whose partials exceed the static array is refused before any device work
    (fake, aligned pointers: nothing is dereferenced)."""
    lib = _lib.load()
    a = _lib.PagedDecodeArgs()
    a.q = a.o = a.k_pages = a.v_pages = a.block_tables = a.context_lens = 16
    a.batch, a.heads_q, a.heads_kv, a.head_dim, a.page_size, a.num_pages = 256, 64, 8, 128, 16, 4
    a.max_context_len, a.block_table_stride, a.tokens_per_split = 1 << 16, 4096, 256
    a.scale, a.dtype = 0.1, _lib.FFA_DTYPE_BF16
    need = lib.ffa_paged_decode_workspace_bytes(256, 64, 128, 1 << 16, 256)
    assert need > _lib.FFA_NOALLOC_SCRATCH_BYTES
    assert lib.ffa_paged_decode_fwd_noalloc(ctypes.byref(a), None) == -10
    assert b"static scratch" in lib.ffa_strerror(-10)


@pytest.mark.gpu
def test_noalloc_decode_graph_replays_match_eager():
    """The allocation-free decode captured into a HIP graph (after one eager call on the
    device, which resolves the scratch array's address) and replayed three times with q
    refilled in place and eager work between replays: every replay equals the workspace
    entry point on the same inputs bit for bit."""
    require_gpu()
    lib = _lib.load()
    lens, Hq, Hkv, D, P, tps = [515, 17, 1030, 64], 8, 2, 128, 16, 128
    q, kp, vp, bt, lens_t = _problem(7, lens, Hq, Hkv, D, P)
    max_len = max(lens)
    need = lib.ffa_paged_decode_workspace_bytes(len(lens), Hq, D, max_len, tps)
    ws = torch.empty(max(need, 16), dtype=torch.uint8, device="cuda")
    o_ref = torch.empty_like(q)
    l_ref = torch.empty(len(lens), Hq, dtype=torch.float32, device="cuda")
    o = torch.empty_like(q)
    lse = torch.empty(len(lens), Hq, dtype=torch.float32, device="cuda")
    a_ref = _args(q, kp, vp, bt, lens_t, o_ref, l_ref, max_len, tps, workspace=ws)
    a = _args(q, kp, vp, bt, lens_t, o, lse, max_len, tps)
    say("no-alloc decode: graph capture")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert lib.ffa_paged_decode_fwd_noalloc(ctypes.byref(a), stream) == 0  # eager first
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cap = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.ffa_paged_decode_fwd_noalloc(ctypes.byref(a), cap) == 0
    for rep in range(3):
        gen = torch.Generator().manual_seed(200 + rep)
        q.copy_(torch.randn(q.shape, generator=gen).to(BF16))
        o.fill_(float("nan"))
        lse.fill_(float("nan"))
        graph.replay()
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert lib.ffa_paged_decode_fwd(ctypes.byref(a_ref), stream) == 0
        torch.cuda.synchronize()
        assert torch.equal(o, o_ref), f"replay {rep}: O differs"
        assert torch.equal(lse, l_ref), f"replay {rep}: LSE differs"
