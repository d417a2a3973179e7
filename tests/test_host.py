"""Host-side tests (no GPU): argument resolution of the drop-in boundary, the C ABI
(struct layout against the header compiled by gcc, exported symbols, validation
error codes), and PagedKVCache bookkeeping against the oracle's restatement."""

from __future__ import annotations

import ctypes
import math
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest
import torch

import fastest_flash_attention_amd as ffa
from fastest_flash_attention_amd.kernels import _lib
from fastest_flash_attention_amd.ops import attention_forward as af
from oracle import paged as opaged

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "ffa.h")


@pytest.fixture(scope="session")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from fastest_flash_attention_amd.kernels.hip import build

        build.build(verbose=False)
    return _lib.load()


# ---------------------------------------------------------------------------------
# Argument resolution (reference ops/attention_forward.py:65-109)
# ---------------------------------------------------------------------------------

def test_config_overrides_kwargs():
    q = torch.randn(2, 2, 16, 8)
    cfg = ffa.AttentionConfig(causal=True, softcap=3.0, sliding_window=5, return_lse=True,
                              block_size_q=4, block_size_kv=8)
    r = af.resolve_forward_args(q, q, q, cfg, causal=False, softcap=None, return_lse=False)
    assert r.causal and r.softcap == 3.0 and r.sliding_window == 5 and r.return_lse
    assert (r.block_q, r.block_kv) == (4, 8)
    r = af.resolve_forward_args(q, q, q, cfg, block_size=16)
    assert (r.block_q, r.block_kv) == (16, 16)  # explicit block_size beats config


def test_auto_block_size_and_scale():
    q = torch.randn(1, 2, 4096, 128)
    r = af.resolve_forward_args(q, q, q)
    assert r.block_q == r.block_kv == 32 and math.isclose(r.scale, 1 / math.sqrt(128))
    assert ffa.auto_select_block_size(1024, 1024, 64) == 64
    assert ffa.auto_select_block_size(4096, 4096, 192) == 16


def test_kv_cache_offset_and_3d():
    q = torch.randn(2, 5, 8)
    kc = torch.randn(2, 7, 8)
    r = af.resolve_forward_args(q, q, q, kv_cache=(kc, kc))
    assert r.squeezed and r.q.shape == (2, 1, 5, 8)
    assert r.S_kv == 12 and r.q_offset == 7


def test_gqa_rules():
    q = torch.randn(1, 8, 4, 16)
    k = torch.randn(1, 2, 4, 16)
    r = af.resolve_forward_args(q, k, k, num_kv_heads=2)
    assert (r.H_q, r.H_kv) == (8, 2)
    with pytest.raises(ValueError, match="num_kv_heads"):
        af.resolve_forward_args(q, k, k)
    k1 = torch.randn(1, 1, 4, 16)  # MQA broadcasts without num_kv_heads, as torch.matmul does
    assert af.resolve_forward_args(q, k1, k1).H_kv == 1
    with pytest.raises(ValueError):
        af.resolve_forward_args(q, torch.randn(1, 3, 4, 16), torch.randn(1, 3, 4, 16),
                                num_kv_heads=3)


def test_build_args_strides_of_module_views():
    B, S, H, D = 2, 10, 4, 16
    x = torch.randn(B, S, H * D)
    q = x.view(B, S, H, D).transpose(1, 2)  # the modules' strided view
    k = torch.randn(1, H, S, D)              # batch-broadcast K
    r = af.resolve_forward_args(q, k, k, causal=True, sliding_window=3, softcap=2.0,
                                two_pass=True, block_size=8)
    out = torch.empty(B, H, S, D)
    lse = torch.empty(B, H, S, 1)
    a = af.build_prefill_args(r, out, lse, _lib.FFA_DTYPE_BF16)
    assert list(a.q_stride) == [S * H * D, D, H * D, 1]
    assert list(a.k_stride) == [0, S * D, D, 1]
    assert list(a.lse_stride) == [H * S, S, 1]
    assert (a.causal, a.window, a.softcap, a.masked_lse_mode) == (1, 3, 2.0, 1)
    assert (a.ref_block_q, a.ref_block_kv, a.q_offset) == (8, 8, 0)
    assert a.q == q.data_ptr() and a.o == out.data_ptr()


def test_product_path_refuses_cpu_and_unsupported():
    q = torch.randn(1, 1, 8, 16, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        ffa.fastest_flash_attn_forward(q, q, q)
    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        af.prepare_prefill(q, q, q, block_mask=torch.ones(1, 1, dtype=torch.bool))
    with pytest.raises(RuntimeError, match="ROCm GPU tensors only"):
        af.prepare_prefill(q, q, q, compute_dtype=torch.float16)
    # a host pool is read by get_kv (a copy), but decode attention needs the GPU
    cache = ffa.PagedKVCache(max_pages=4, page_size=4, num_heads=1, head_dim=8)
    cache.append_tokens(0, torch.randn(1, 3, 8), torch.randn(1, 3, 8))
    assert cache.get_kv(0)[0].shape == (1, 3, 8)
    with pytest.raises(RuntimeError, match="ROCm"):
        cache.decode(torch.randn(1, 1, 8, dtype=torch.float16), [0])


# ---------------------------------------------------------------------------------
# C ABI
# ---------------------------------------------------------------------------------

def _header_functions() -> list[str]:
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w\s\*]+?\b(ffa_\w+)\s*\(", text, re.M)))


def test_library_exports_every_header_symbol(lib):
    names = _header_functions()
    assert set(names) == set(_lib.EXPORTS), names
    for name in names:
        assert hasattr(lib, name)
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    for name in names:
        assert re.search(rf"\bT {name}$", out, re.M), name


def _c_layout(struct: str, fields: list[str]) -> dict:
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(){"]
    src.append(f'printf("sizeof %zu\\n", sizeof({struct}));')
    for f in fields:
        src.append(f'printf("{f} %zu\\n", offsetof({struct}, {f}));')
    src.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        exe = os.path.join(d, "l")
        open(c, "w").write("\n".join(src))
        subprocess.run(["gcc", "-std=c11", c, "-o", exe], check=True)
        text = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return {k: int(v) for k, v in (ln.split() for ln in text.splitlines())}


@pytest.mark.parametrize("cls,cname", [
    (_lib.PrefillArgs, "ffa_prefill_args"),
    (_lib.PagedGatherArgs, "ffa_paged_gather_args"),
    (_lib.PagedDecodeArgs, "ffa_paged_decode_args"),
    (_lib.PagedAppendArgs, "ffa_paged_append_args"),
    (_lib.MlaDecodeArgs, "ffa_mla_decode_args"),
    (_lib.AttnBwdArgs, "ffa_attn_bwd_args"),
])
def test_ctypes_struct_matches_header(cls, cname):
    fields = [f for f, _ in cls._fields_]
    c = _c_layout(cname, fields)
    assert c["sizeof"] == ctypes.sizeof(cls)
    for f in fields:
        assert c[f] == getattr(cls, f).offset, f


def test_abi_version_and_strerror(lib):
    assert lib.ffa_abi_version() == _lib.FFA_ABI_VERSION
    for rc in range(0, -10, -1):
        assert lib.ffa_strerror(rc).decode().strip()
    assert b"unknown" in lib.ffa_strerror(-99)


def test_validation_errors_without_device(lib):
    a = _lib.PrefillArgs()
    assert lib.ffa_prefill_fwd(None, None) == -1
    a.dtype, a.head_dim, a.batch, a.heads_q, a.heads_kv = 0, 0, 1, 1, 1
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -3
    a.head_dim, a.dtype = 64, 7
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -2
    a.dtype, a.heads_q, a.heads_kv = 0, 3, 2
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -5
    a.heads_q, a.heads_kv, a.batch, a.seqlen_q = 2, 2, 0, 4
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == 0  # empty: nothing launched
    a.batch = 1
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -1  # null pointers
    d = _lib.PagedDecodeArgs()
    d.dtype, d.head_dim, d.batch, d.heads_q, d.heads_kv, d.page_size = 0, 128, 2, 8, 2, 16
    d.max_context_len, d.block_table_stride, d.num_pages = 64, 4, 8
    d.q = d.o = d.k_pages = d.v_pages = d.block_tables = d.context_lens = 16
    d.workspace, d.workspace_bytes = 16, 8
    assert lib.ffa_paged_decode_fwd(ctypes.byref(d), None) == -6
    d.block_table_stride = 3
    assert lib.ffa_paged_decode_fwd(ctypes.byref(d), None) == -1
    g = _lib.PagedGatherArgs()
    g.elem_bytes = 3
    assert lib.ffa_paged_gather(ctypes.byref(g), None) == -2
    ap = _lib.PagedAppendArgs()
    ap.elem_bytes, ap.heads_kv, ap.page_size, ap.head_dim, ap.n_tokens, ap.num_pages = 2, 1, 16, 576, 3, 4
    ap.k_pages = ap.k_new = ap.page_table = 16
    ap.v_new = 16  # V given without its pool: K-only appends pass neither
    assert lib.ffa_paged_append(ctypes.byref(ap), None) == -1
    m = _lib.MlaDecodeArgs()
    assert lib.ffa_mla_decode_fwd(None, None) == -1
    m.dtype, m.dim_v, m.dim_rope, m.batch, m.heads_q, m.page_size = 0, 512, 32, 2, 32, 16
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -3  # rope dims must be 64
    m.dim_rope, m.dim_v = 64, 128
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -3  # latent 256 or 512
    m.dim_v, m.dtype = 512, 2
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -2  # no fp32 MLA kernel
    m.dtype, m.max_context_len, m.block_table_stride, m.num_pages = 0, 64, 4, 8
    m.q = m.o = m.kv_pages = m.block_tables = m.context_lens = 16
    m.workspace, m.workspace_bytes = 16, 8
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -6
    m.q = 24
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -4  # q not 16-byte aligned
    m.q, m.block_table_stride = 16, 3
    assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -1
    bw = _lib.AttnBwdArgs()
    assert lib.ffa_attn_bwd(None, None) == -1
    bw.dtype, bw.head_dim, bw.batch, bw.heads_q, bw.heads_kv = 3, 64, 1, 4, 2
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -2  # bf16 / fp16 / fp32 only
    bw.dtype, bw.head_dim = 0, 264
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -3  # head_dim <= 256
    bw.head_dim, bw.heads_q = 64, 3
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -5
    bw.heads_q, bw.seqlen_q, bw.seqlen_kv = 4, 100, 100
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -1  # null pointers
    bw.dout = bw.q = bw.k = bw.v = bw.o = bw.lse = bw.dq = bw.dk = bw.dv = 16
    for name in ("do_stride", "q_stride", "k_stride", "v_stride", "o_stride", "dq_stride",
                 "dk_stride", "dv_stride"):
        getattr(bw, name)[:] = [4 * 100 * 64, 100 * 64, 64, 1]
    bw.workspace, bw.workspace_bytes = 16, 8
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -6
    bw.workspace_bytes = lib.ffa_attn_bwd_workspace_bytes(1, 4, 100)
    bw.q_stride[2] = 68
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -4  # row stride not 8-aligned
    bw.q_stride[2], bw.scale = 64, float("nan")
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -1


def test_workspace_sizing(lib):
    # [B][Hq][splits][Dpad] O partials + [B][Hq][splits] lse, fp32
    assert lib.ffa_paged_decode_num_splits(32768, 512) == 64
    assert lib.ffa_paged_decode_num_splits(1000, 0) == 1  # default split 1024
    assert lib.ffa_paged_decode_num_splits(5000, 4096) == 3  # split clamped to 2048
    assert lib.ffa_paged_decode_num_splits(100, 40) == 3  # 40 rounds up to 48 (16-token tiles)
    assert lib.ffa_paged_decode_workspace_bytes(64, 32, 128, 32768, 512) == 64 * 32 * 64 * 129 * 4
    assert lib.ffa_paged_decode_workspace_bytes(2, 4, 100, 100, 64) == 2 * 4 * 2 * 129 * 4
    # MLA: 32-token tiles, default split 512, capped at 1024; dim_v-wide 16-bit O partials
    # plus one fp32 lse per (sequence, head, split)
    assert lib.ffa_mla_decode_workspace_bytes(32, 32, 512, 4096, 512) == 32 * 32 * 8 * (1024 + 4)
    assert lib.ffa_mla_decode_workspace_bytes(2, 8, 256, 1000, 0) == 2 * 8 * 2 * (512 + 4)
    assert lib.ffa_mla_decode_workspace_bytes(1, 1, 512, 5000, 4096) == 5 * (1024 + 4)
    assert lib.ffa_mla_decode_workspace_bytes(1, 1, 512, 100, 40) == 2 * (1024 + 4)  # 40 -> 64
    # backward: lse2 and D_i, fp32, rows padded to 128 per (batch, q head)
    assert lib.ffa_attn_bwd_workspace_bytes(2, 3, 100) == 2 * 2 * 3 * 128 * 4
    assert lib.ffa_attn_bwd_workspace_bytes(1, 1, 256) == 2 * 256 * 4


# ---------------------------------------------------------------------------------
# PagedKVCache bookkeeping (write path) vs the oracle restatement
# ---------------------------------------------------------------------------------

def test_paged_cache_matches_oracle_bookkeeping():
    gen = torch.Generator().manual_seed(0)
    cache = ffa.PagedKVCache(max_pages=12, page_size=4, num_heads=2, head_dim=8,
                             dtype=torch.float32)
    pool = opaged.PagedPool(max_pages=12, page_size=4, num_heads=2, head_dim=8)
    ops = [("a", 0, 6), ("a", 1, 3), ("a", 0, 5), ("f", 1, 0), ("a", 2, 9), ("a", 0, 1),
           ("a", 2, 0)]
    for op, sid, n in ops:
        if op == "a":
            k = torch.randn(2, n, 8, generator=gen)
            v = torch.randn(2, n, 8, generator=gen)
            assert cache.append_tokens(sid, k, v) == pool.append_tokens(sid, k.numpy(),
                                                                      v.numpy())
        else:
            cache.free_sequence(sid)
            pool.free_sequence(sid)
        assert cache.free_pages == pool.free_pages
        assert cache.sequences == pool.sequences
    assert np.array_equal(cache.k_pages.numpy(), pool.k_pages)
    assert np.array_equal(cache.v_pages.numpy(), pool.v_pages)
    assert cache.num_free_pages == len(pool.free_pages)
    assert cache.total_capacity == 48
    bt, lens = cache.block_tables([2, 0, 7])
    assert lens.tolist() == [9, 12, 0]
    assert bt.dtype == torch.int32 and bt.shape == (3, 3)
    assert bt[0].tolist() == pool.sequences[2]["page_table"]


def test_paged_cache_out_of_pages_matches_reference_state():
    cache = ffa.PagedKVCache(max_pages=1, page_size=4, num_heads=1, head_dim=2,
                             dtype=torch.float32)
    pool = opaged.PagedPool(max_pages=1, page_size=4, num_heads=1, head_dim=2)
    k = torch.arange(10, dtype=torch.float32).view(1, 5, 2)
    with pytest.raises(RuntimeError, match="out of physical pages"):
        cache.append_tokens(0, k, k)
    with pytest.raises(RuntimeError, match="out of physical pages"):
        pool.append_tokens(0, k.numpy(), k.numpy())
    assert cache.sequences == pool.sequences and cache.free_pages == pool.free_pages
    assert np.array_equal(cache.k_pages.numpy(), pool.k_pages)


def test_auto_tokens_per_split():
    from fastest_flash_attention_amd.ops.kv_cache import _auto_tokens_per_split

    assert _auto_tokens_per_split(64, 8, 32768) == 2048  # long-context batch: longest split
    assert _auto_tokens_per_split(2, 8, 32768) == 2048   # 2*8*16 = 256 workgroups
    assert _auto_tokens_per_split(4, 8, 8192) == 1024    # 4*8*8 = 256 workgroups
    assert _auto_tokens_per_split(1, 8, 4096) == 128     # 1*8*32 = 256 workgroups
    assert _auto_tokens_per_split(1, 1, 100) == 64       # tiny problem: shortest split


def _valid_prefill_args(scale, softcap=0.0):
    """Sizes, strides and (fake, aligned) pointers that pass every host check up to the
    scale, so the returned code is decided by scale / softcap alone."""
    a = _lib.PrefillArgs()
    a.q = a.k = a.v = a.o = 16
    st = [4 * 64 * 64, 64 * 64, 64, 1]
    a.q_stride[:] = a.k_stride[:] = a.v_stride[:] = a.o_stride[:] = st
    a.batch, a.heads_q, a.heads_kv, a.seqlen_q, a.seqlen_kv, a.head_dim = 1, 4, 4, 64, 64, 64
    a.dtype, a.scale, a.softcap = _lib.FFA_DTYPE_BF16, scale, softcap
    return a


@pytest.mark.parametrize("scale,softcap", [
    (float("inf"), 0.0), (float("-inf"), 0.0), (float("nan"), 0.0),
    (0.125, float("nan")), (0.125, float("inf")),
])
def test_abi_rejects_non_finite_scale(lib, scale, softcap):
    """The C ABI takes any finite scale (negative and zero included: the library applies
    them, see the GPU tests) and rejects non-finite ones before any HIP call."""
    a = _valid_prefill_args(scale, softcap)
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -1
    d = _lib.PagedDecodeArgs()
    d.dtype, d.head_dim, d.batch, d.heads_q, d.heads_kv, d.page_size = 0, 128, 2, 8, 2, 16
    d.max_context_len, d.block_table_stride, d.num_pages = 64, 4, 8
    d.q = d.o = d.k_pages = d.v_pages = d.block_tables = d.context_lens = 16
    d.scale, d.softcap = scale, softcap
    assert lib.ffa_paged_decode_fwd(ctypes.byref(d), None) == -1
    if softcap == 0.0:
        m = _lib.MlaDecodeArgs()
        m.dtype, m.dim_v, m.dim_rope, m.batch, m.heads_q, m.page_size = 0, 512, 64, 2, 32, 16
        m.max_context_len, m.block_table_stride, m.num_pages = 64, 4, 8
        m.q = m.o = m.kv_pages = m.block_tables = m.context_lens = 16
        m.scale = scale
        assert lib.ffa_mla_decode_fwd(ctypes.byref(m), None) == -1


def test_host_layer_passes_scale_unchanged():
    """Negative and zero scales reach the ABI struct as given: the library, not the
    Python layer, owns their meaning (ops/attention_forward.py:98-99 passes any value)."""
    q = torch.randn(1, 2, 8, 16)
    for s in (-0.25, 0.0, 0.5):
        r = af.resolve_forward_args(q, q, q, scale=s)
        out = torch.empty(1, 2, 8, 16)
        a = af.build_prefill_args(r, out, None, _lib.FFA_DTYPE_BF16)
        assert a.scale == s and a.q == q.data_ptr()


# ---------------------------------------------------------------------------------
# PagedKVCache read path of a host pool (the constructor's default device)
# ---------------------------------------------------------------------------------

def test_reference_paged_basic_flow():
    """The reference's own test_paged_basic (tests/test_fastest_flash.py:398-411): an fp32
    pool on the default device, append then get_kv."""
    cache = ffa.PagedKVCache(max_pages=16, page_size=4, num_heads=2, head_dim=8,
                             dtype=torch.float32)
    k = torch.randn(2, 6, 8)
    v = torch.randn(2, 6, 8)
    assert cache.append_tokens(0, k, v) == 6
    k_out, v_out = cache.get_kv(0)
    assert k_out.shape == (2, 6, 8)
    assert torch.allclose(k_out, k) and torch.allclose(v_out, v)
    assert cache.get_kv(1) == (None, None)


def test_host_get_kv_matches_reference_page_copies():
    """get_kv on a host pool equals the reference's per-page slice copies
    (ops/kv_cache.py:224-230, restated by oracle.paged.gather_sequence) bit for bit,
    across sequences that interleave their pages and a freed-and-reused page."""
    gen = torch.Generator().manual_seed(3)
    cache = ffa.PagedKVCache(max_pages=10, page_size=3, num_heads=3, head_dim=5,
                             dtype=torch.float16)
    pool = opaged.PagedPool(max_pages=10, page_size=3, num_heads=3, head_dim=5,
                            dtype=np.float16)
    for sid, n in ((0, 4), (1, 2), (0, 5), (2, 7)):
        k = torch.randn(3, n, 5, generator=gen).half()
        v = torch.randn(3, n, 5, generator=gen).half()
        cache.append_tokens(sid, k, v)
        pool.append_tokens(sid, k.numpy(), v.numpy())
    cache.free_sequence(1)
    pool.free_sequence(1)
    k = torch.randn(3, 4, 5, generator=gen).half()
    cache.append_tokens(3, k, k)
    pool.append_tokens(3, k.numpy(), k.numpy())
    for sid in (0, 2, 3):
        ko, vo = cache.get_kv(sid)
        seq = pool.sequences[sid]
        rk, rv = opaged.gather_sequence(pool.k_pages, pool.v_pages, seq["page_table"], seq["len"])
        assert ko.dtype == torch.float16 and ko.is_contiguous()
        assert np.array_equal(ko.numpy(), rk) and np.array_equal(vo.numpy(), rv)


def test_check_page_ids():
    from fastest_flash_attention_amd.ops.kv_cache import check_page_ids

    # pool of 8 pages, 4 tokens per page: entry j of a row is used while 4 j < length
    bt = torch.tensor([[3, 1, 7], [2, 9, -1]], dtype=torch.int32)
    check_page_ids(bt, torch.tensor([9, 4], dtype=torch.int32), 4, 8, 9)  # unused 9, -1 pass
    with pytest.raises(IndexError, match=r"block_tables\[1, 1\] = 9"):
        check_page_ids(bt, torch.tensor([9, 5], dtype=torch.int32), 4, 8, 9)
    check_page_ids(bt, torch.tensor([9, 5], dtype=torch.int32), 4, 8, 4)  # clamped length
    with pytest.raises(IndexError, match=r"block_tables\[1, 2\] = -1"):
        check_page_ids(torch.tensor([[3, 1, 7], [2, 5, -1]], dtype=torch.int32),
                       torch.tensor([0, 12], dtype=torch.int32), 4, 8, 12)
    with pytest.raises(IndexError):
        check_page_ids(bt, torch.tensor([9, 0], dtype=torch.int32), 4, 7, 9)  # 7 >= 7 pages


@pytest.mark.parametrize("field,value", [
    ("q_offset", -(1 << 29)),          # |q_offset| > 2^29 - 1
    ("q_offset", (1 << 29) - 64),      # q_offset + seqlen_q > 2^29 - 1
    ("seqlen_kv", 1 << 29),
])
def test_abi_rejects_positions_beyond_int32_range(lib, field, value):
    """Positions and window bounds are int32 in the kernels: the prefill rejects position
    ranges beyond 2^29 - 1 before any HIP call (FFA_ERR_TOO_LARGE)."""
    a = _valid_prefill_args(0.125)
    setattr(a, field, value)
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == -9


@pytest.mark.parametrize("head_dim,v_head_dim,dtype,code", [
    (192, 128, _lib.FFA_DTYPE_FP32, -3),   # narrow V: 16-bit inputs only
    (128, 64, _lib.FFA_DTYPE_BF16, -3),    # only head_dim 129..192
    (256, 128, _lib.FFA_DTYPE_BF16, -3),
    (192, 136, _lib.FFA_DTYPE_BF16, -3),   # v_head_dim <= 128
    (192, 100, _lib.FFA_DTYPE_BF16, -4),   # a multiple of 8
])
def test_abi_narrow_v_contract(lib, head_dim, v_head_dim, dtype, code):
    """A V narrower than head_dim (taken as zero-padded) is accepted only where the
    library has kernels for it; everything else is rejected before any HIP call."""
    a = _valid_prefill_args(0.125)
    a.head_dim, a.v_head_dim, a.dtype = head_dim, v_head_dim, dtype
    assert lib.ffa_prefill_fwd(ctypes.byref(a), None) == code


def test_host_layer_narrow_v():
    """The op keeps a narrower V unpadded where the kernels take it (16-bit, head_dim
    129..192, v dims <= 128 and a multiple of 8) and zero-pads it elsewhere."""
    q = torch.zeros(1, 2, 8, 192, dtype=torch.bfloat16)
    v = torch.zeros(1, 2, 8, 128, dtype=torch.bfloat16)
    r = af.resolve_forward_args(q, q, v)
    assert (r.D, r.Dv) == (192, 128)
    out = torch.empty_like(q)
    a = af.build_prefill_args(r, out, None, _lib.FFA_DTYPE_BF16)
    assert a.v_head_dim == 128 and a.head_dim == 192
    r = af.resolve_forward_args(q, q, q)
    assert af.build_prefill_args(r, out, None, _lib.FFA_DTYPE_BF16).v_head_dim == 0
    with pytest.raises(ValueError):
        af.resolve_forward_args(q[..., :64], q[..., :64], v)  # v wider than q


def test_abi_bwd_narrow_v_contract(lib):
    """The backward takes a narrower V under the forward's rule, checked before any
    HIP call."""
    bw = _lib.AttnBwdArgs()
    bw.dtype, bw.head_dim, bw.batch, bw.heads_q, bw.heads_kv = 0, 128, 1, 4, 2
    bw.v_head_dim = 64
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -3  # only head_dim 129..192
    bw.head_dim, bw.v_head_dim = 192, 100
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -4  # a multiple of 8
    bw.v_head_dim, bw.dtype = 128, 2
    assert lib.ffa_attn_bwd(ctypes.byref(bw), None) == -3  # 16-bit inputs only


# ---------------------------------------------------------------------------------
# Module kv_cache contract (reference modules/flash_gqa.py:101-125,
# ops/attention_forward.py:82-96): the op is replaced by the oracle on the CPU so that
# only the module's own argument plumbing is under test
# ---------------------------------------------------------------------------------

def _oracle_op(q, k, v, **kw):
    from oracle import reference_forward as rf

    kc = kw.pop("kv_cache", None)
    if kc is not None:
        kc = tuple(t.detach().float().numpy() for t in kc)
    o, lse = rf.forward(q.detach().float().numpy(), k.detach().float().numpy(),
                        v.detach().float().numpy(), kv_cache=kc, **kw)
    return torch.from_numpy(np.ascontiguousarray(o)), (
        None if lse is None else torch.from_numpy(np.ascontiguousarray(lse)))


@pytest.mark.parametrize("cache_heads", ["num_heads", "num_kv_heads"])
def test_gqa_module_kv_cache_layouts(monkeypatch, cache_heads):
    from fastest_flash_attention_amd.modules import flash_gqa
    from oracle import reference_forward as rf

    monkeypatch.setattr(flash_gqa, "fastest_flash_attn_forward", _oracle_op)
    torch.manual_seed(11)
    B, S, Sc, H, Hkv, D = 2, 5, 23, 8, 2, 16
    m = ffa.FastestFlashGQA(hidden_size=H * D, num_heads=H, num_kv_heads=Hkv, causal=True,
                            softcap=20.0, sliding_window=12).eval()
    x = torch.randn(B, S, H * D)
    hc = H if cache_heads == "num_heads" else Hkv
    kc, vc = torch.randn(B, hc, Sc, D), torch.randn(B, hc, Sc, D)
    with torch.no_grad():
        out, lse = m(x, kv_cache=(kc, vc), return_lse=True)
        # the reference module's statements: repeat the new K/V, concatenate the cache
        q = m.q_proj(x).view(B, S, H, D).transpose(1, 2)
        k = m.k_proj(x).view(B, S, Hkv, D).transpose(1, 2)
        v = m.v_proj(x).view(B, S, Hkv, D).transpose(1, 2)
        if cache_heads == "num_heads":
            k = torch.repeat_interleave(k, H // Hkv, dim=1)
            v = torch.repeat_interleave(v, H // Hkv, dim=1)
        else:  # the extension: the cache holds the unrepeated heads
            kc = torch.repeat_interleave(kc, H // Hkv, dim=1)
            vc = torch.repeat_interleave(vc, H // Hkv, dim=1)
            k = torch.repeat_interleave(k, H // Hkv, dim=1)
            v = torch.repeat_interleave(v, H // Hkv, dim=1)
        a, l_ref = rf.forward(q.numpy(), k.numpy(), v.numpy(), scale=m.scale, causal=True,
                              softcap=20.0, sliding_window=12,
                              kv_cache=(kc.numpy(), vc.numpy()), return_lse=True)
        ref = m.o_proj(torch.from_numpy(np.ascontiguousarray(a)).transpose(1, 2).reshape(B, S, -1))
    assert torch.allclose(out, ref, atol=1e-5, rtol=1e-5)
    assert np.allclose(lse.numpy(), l_ref, atol=1e-6)


def test_gqa_module_rejects_other_cache_head_counts(monkeypatch):
    from fastest_flash_attention_amd.modules import flash_gqa

    monkeypatch.setattr(flash_gqa, "fastest_flash_attn_forward", _oracle_op)
    m = ffa.FastestFlashGQA(hidden_size=64, num_heads=4, num_kv_heads=2).eval()
    kc = torch.randn(1, 3, 7, 16)
    with torch.no_grad(), pytest.raises((RuntimeError, ValueError)):
        m(torch.randn(1, 2, 64), kv_cache=(kc, kc))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_paged_decode_layout_checks_precede_dtype_routes(dtype):
    """Every pool dtype (the fp32 route included) checks the pools' contiguity, the
    tables' dtype and their width against max_context_len before anything reads them;
    on host tensors these raise before the device check."""
    from fastest_flash_attention_amd.ops.kv_cache import fastest_flash_paged_decode

    P, Hkv, D = 4, 2, 8
    kp = torch.zeros(6, Hkv, P, D, dtype=dtype)
    q = torch.zeros(2, 4, D, dtype=dtype)
    lens = torch.tensor([9, 3], dtype=torch.int32)
    narrow = torch.zeros(2, 2, dtype=torch.int32)  # 2 pages of 4 < 9 tokens
    with pytest.raises(ValueError, match="fewer columns"):
        fastest_flash_paged_decode(q, kp, kp, narrow, lens)
    wide = torch.zeros(2, 3, dtype=torch.int32)
    strided = torch.zeros(6, Hkv, P, 2 * D, dtype=dtype)[..., ::2]
    with pytest.raises(ValueError, match="contiguous"):
        fastest_flash_paged_decode(q, strided, strided, wide, lens)
    with pytest.raises(TypeError, match="int32"):
        fastest_flash_paged_decode(q, kp, kp, wide.long(), lens)
    with pytest.raises(RuntimeError, match="ROCm"):  # valid layout: the device check
        fastest_flash_paged_decode(q, kp, kp, wide, lens)
