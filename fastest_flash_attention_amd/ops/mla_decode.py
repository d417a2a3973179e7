"""MLA decode over the compressed latent cache (no counterpart in the reference).

The reference FastestFlashMLA (modules/flash_mla.py:116-172) up-projects every cached
token to per-head K_nope / V and attends with D = head_dim + rope_dim; it has no decode
path, so a decode step through it re-reads H * (2 * head_dim + rope_dim) values per
cached token. Absorbing the up-projection into the query gives the same scores and
output from the latent cache alone: with W_uk_h, W_uv_h the head-h slices of
kv_up_proj,

    q_h . k_h(t) = [W_uk_h^T q_nope_h, q_rope_h] . [c_t, r_t]
    o_h          = sum_t p_h(t) W_uv_h c_t = W_uv_h (sum_t p_h(t) c_t)

so every head attends over one shared row [c_t | r_t] per token (latent_dim + rope_dim
values), and the latent-space output is up-projected once per head afterwards. The
attention runs in ``ffa_mla_decode_fwd`` (libffa.so); the two small per-head
projections are torch batched GEMMs.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import torch

from ..kernels import _lib
from .kv_cache import check_page_ids

MLA_ROPE_DIM = 64
MLA_LATENT_DIMS = (256, 512)


def _auto_mla_tokens_per_split(batch: int, head_groups: int, max_len: int) -> int:
    """Largest split (<= 1024 tokens, >= 64) that still gives >= 256 workgroups (one per
    CU on 256 CUs); fewer splits mean fewer partials to write and merge. On MI355X at
    batch 32, context 4096 this picks 512 tokens (34.4-35.8 us per step; 256 tokens with
    two workgroups per CU: 38.6 us; 1024 tokens, 128 workgroups: about 51 us)."""
    tps = 1024
    while tps > 64 and batch * head_groups * max(1, math.ceil(max_len / tps)) < 256:
        tps //= 2
    return tps


def mla_decode_workspace_bytes(batch: int, heads_q: int, dim_v: int, max_context_len: int,
                               tokens_per_split: int) -> int:
    return int(_lib.load().ffa_mla_decode_workspace_bytes(
        batch, heads_q, dim_v, max_context_len, tokens_per_split))


@dataclass
class MlaDecodeCall:
    """A fully resolved MLA decode launch: the ABI struct plus the tensors it points to
    (kept alive with it). ``launch_mla_decode`` runs it on the current stream; a serving
    loop that refills q / context_lens in place can launch the same call every step, as
    long as every length stays within the ``max_context_len`` it was prepared with
    (longer sequences are cut to that many tokens)."""

    args: _lib.MlaDecodeArgs
    q: torch.Tensor
    out: torch.Tensor
    lse: Optional[torch.Tensor]
    keep: tuple = ()


def prepare_mla_decode(
    q: torch.Tensor,
    kv_pages: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    dim_v: int,
    scale: float,
    return_lse: bool = False,
    max_context_len: Optional[int] = None,
    tokens_per_split: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
    check_block_tables: bool = False,
    out: Optional[torch.Tensor] = None,
) -> MlaDecodeCall:
    """Check the arguments of ``fastest_flash_mla_decode``, allocate outputs (or take
    ``out``) and the workspace, build the ABI struct. Launches nothing.

    ``max_context_len`` is required here: a call prepared once may be launched again
    after ``context_lens`` has been refilled in place, and the prepared bound fixes the
    split count, the workspace size and the table width the kernels may read. Every
    later launch attends to the first ``min(context_lens[b], max_context_len)`` tokens
    of sequence b, so a serving loop whose lengths grow passes the largest length it
    will reach (and a block table that wide) or prepares the call again."""
    if max_context_len is None:
        raise ValueError("prepare_mla_decode needs an explicit max_context_len: it bounds "
                         "every context length the prepared call will be launched with")
    if q.dim() != 3 or kv_pages.dim() != 3:
        raise ValueError("q must be [B, H, dim_v + 64] and kv_pages [num_pages, page_size, dim_v + 64]")
    B, H, dqk = q.shape
    num_pages, page_size, dk = kv_pages.shape
    if dim_v not in MLA_LATENT_DIMS or dqk != dim_v + MLA_ROPE_DIM or dk != dqk:
        raise ValueError(f"MLA decode needs dim_v in {MLA_LATENT_DIMS} and rope dim "
                         f"{MLA_ROPE_DIM} (q last dim {dqk}, pages {dk}, dim_v {dim_v})")
    for name, t in (("q", q), ("kv_pages", kv_pages), ("block_tables", block_tables),
                    ("context_lens", context_lens)):
        if t.device.type != "cuda":
            raise RuntimeError(f"fastest_flash_attention_amd MLA decode runs on ROCm tensors "
                               f"only; {name} is on {t.device}")
    if q.dtype != kv_pages.dtype:
        raise TypeError("q and kv_pages must share a dtype")
    code = _lib.dtype_code(q.dtype)
    if not kv_pages.is_contiguous():
        raise ValueError("kv_pages must be contiguous")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise TypeError("block_tables and context_lens must be int32")
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if q.stride(-1) != 1 or q.data_ptr() % 16 or q.stride(0) % 8 or q.stride(1) % 8:
        q = q.contiguous() if not q.is_contiguous() else q.clone()
    max_context_len = int(max_context_len)
    if max_context_len < 0:
        raise ValueError("max_context_len must be >= 0")
    if block_tables.size(1) * page_size < max_context_len:
        raise ValueError("block_tables has fewer columns than max_context_len needs")
    if check_block_tables:
        check_page_ids(block_tables, context_lens, page_size, num_pages, max_context_len)
    if tokens_per_split is None:
        tokens_per_split = _auto_mla_tokens_per_split(B, (H + 31) // 32, max_context_len)

    lib = _lib.load()
    if out is None:
        out = torch.empty((B, H, dim_v), dtype=q.dtype, device=q.device)
    elif (tuple(out.shape) != (B, H, dim_v) or out.dtype != q.dtype or out.device != q.device
          or out.stride(-1) != 1 or out.data_ptr() % 4):
        raise ValueError(f"out must be a [B, H, dim_v] {q.dtype} tensor on {q.device} with "
                         f"unit last stride")
    lse = torch.empty((B, H), dtype=torch.float32, device=q.device) if return_lse else None
    need = int(lib.ffa_mla_decode_workspace_bytes(B, H, dim_v, max_context_len, tokens_per_split))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q.device)

    a = _lib.MlaDecodeArgs()
    a.q = q.data_ptr()
    a.kv_pages = kv_pages.data_ptr()
    a.o = out.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.block_tables = block_tables.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    a.q_stride[:] = [q.stride(0), q.stride(1)]
    a.o_stride[:] = [out.stride(0), out.stride(1)]
    if lse is not None:
        a.lse_stride[:] = [lse.stride(0), lse.stride(1)]
    a.block_table_stride = block_tables.size(1)
    a.batch = B
    a.heads_q = H
    a.dim_v = dim_v
    a.dim_rope = MLA_ROPE_DIM
    a.page_size = page_size
    a.num_pages = num_pages
    a.max_context_len = max_context_len
    a.tokens_per_split = int(tokens_per_split)
    a.scale = float(scale)
    a.dtype = code
    return MlaDecodeCall(args=a, q=q, out=out, lse=lse,
                         keep=(kv_pages, block_tables, context_lens, workspace))


def launch_mla_decode(call: MlaDecodeCall) -> None:
    lib = _lib.load()
    stream = _lib.current_stream_handle(call.q.device)
    with torch.cuda.device(call.q.device):
        rc = lib.ffa_mla_decode_fwd(ctypes.byref(call.args), ctypes.c_void_p(stream))
    _lib.check(rc)


def fastest_flash_mla_decode(
    q: torch.Tensor,
    kv_pages: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    dim_v: int,
    scale: float,
    return_lse: bool = False,
    max_context_len: Optional[int] = None,
    tokens_per_split: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
    check_block_tables: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Latent-space attention of one query token per sequence.

    Page ids outside the pool exclude the tokens they would hold, or raise IndexError
    with ``check_block_tables=True`` (as for ``fastest_flash_paged_decode``).

    q: ``[B, H, dim_v + 64]`` absorbed queries ``[W_uk^T q_nope, q_rope]``; kv_pages:
    ``[num_pages, page_size, dim_v + 64]`` rows ``[c_t | r_t]``; block_tables int32
    ``[B, max_blocks]``; context_lens int32 ``[B]``. Sequence b attends to its first
    ``context_lens[b]`` tokens. Returns ``(o_lat [B, H, dim_v], lse [B, H] or None)``.
    """
    if max_context_len is None:
        max_context_len = (int(context_lens.max().item())
                           if context_lens.numel() > 0 and q.size(0) > 0 else 0)
    call = prepare_mla_decode(q, kv_pages, block_tables, context_lens, dim_v=dim_v,
                              scale=scale, return_lse=return_lse,
                              max_context_len=max_context_len,
                              tokens_per_split=tokens_per_split, workspace=workspace,
                              check_block_tables=check_block_tables)
    launch_mla_decode(call)
    return call.out, call.lse


class MLALatentCache:
    """Paged cache of MLA latent rows ``[c_t | r_t]`` (latent_dim + rope_dim values per
    token, shared by all heads).

    Page bookkeeping follows PagedKVCache (reference ops/kv_cache.py:110-240): a free
    list popped from the front, per-sequence page tables, token t of a sequence at
    ``(page_table[t // page_size], t % page_size)``, pages returned to the tail of the
    free list. ``pages`` is ``[max_pages, page_size, latent_dim + rope_dim]``.
    """

    def __init__(self, max_pages: int = 1024, page_size: int = 64, latent_dim: int = 512,
                 rope_dim: int = MLA_ROPE_DIM, dtype: torch.dtype = torch.bfloat16,
                 device: torch.device | str = "cpu"):
        self.max_pages = max_pages
        self.page_size = page_size
        self.latent_dim = latent_dim
        self.rope_dim = rope_dim
        self.pages = torch.zeros(max_pages, page_size, latent_dim + rope_dim, dtype=dtype,
                                 device=device)
        self.free_pages = list(range(max_pages))
        self.sequences: dict = {}

    def allocate_page(self) -> int:
        if not self.free_pages:
            raise RuntimeError("MLALatentCache: out of physical pages")
        return self.free_pages.pop(0)

    def free_sequence(self, seq_id: int) -> None:
        if seq_id in self.sequences:
            self.free_pages.extend(self.sequences[seq_id]["page_table"])
            del self.sequences[seq_id]

    def seq_len(self, seq_id: int) -> int:
        return self.sequences.get(seq_id, {"len": 0})["len"]

    def append(self, seq_id: int, latent: torch.Tensor, k_rope: torch.Tensor) -> int:
        """Append ``latent [S, latent_dim]`` and rotated ``k_rope [S, rope_dim]`` rows;
        returns the new length. Out of pages: the rows that fit are written, then
        RuntimeError (PagedKVCache semantics)."""
        if latent.dim() != 2 or k_rope.dim() != 2 or latent.size(0) != k_rope.size(0):
            raise ValueError("latent must be [S, latent_dim] and k_rope [S, rope_dim]")
        if latent.size(1) != self.latent_dim or k_rope.size(1) != self.rope_dim:
            raise ValueError("latent / rope dims do not match the cache")
        seq = self.sequences.setdefault(seq_id, {"page_table": [], "len": 0})
        S_new = latent.size(0)
        if S_new == 0:
            return seq["len"]
        L0, P = seq["len"], self.page_size
        need_pages = (L0 + S_new + P - 1) // P
        out_of_pages = False
        while len(seq["page_table"]) < need_pages:
            if not self.free_pages:
                out_of_pages = True
                break
            seq["page_table"].append(self.allocate_page())
        n_fit = min(S_new, len(seq["page_table"]) * P - L0)
        if n_fit > 0:
            rows = torch.cat([latent[:n_fit], k_rope[:n_fit]], dim=-1).to(
                self.pages.device, self.pages.dtype).contiguous()
            if self.pages.device.type == "cuda":
                self._append_device(seq, L0, rows)
            else:
                t = torch.arange(L0, L0 + n_fit, dtype=torch.int64)
                table = torch.tensor(seq["page_table"], dtype=torch.int64)
                self.pages[table[t // P], t % P] = rows
            seq["len"] = L0 + n_fit
        if out_of_pages:
            raise RuntimeError("MLALatentCache: out of physical pages")
        return seq["len"]

    def _append_device(self, seq: dict, start: int, rows: torch.Tensor) -> None:
        """One K-only ``ffa_paged_append`` launch (the pool seen as one KV head)."""
        table = torch.tensor(seq["page_table"], dtype=torch.int32, device=self.pages.device)
        a = _lib.PagedAppendArgs()
        a.k_pages = self.pages.data_ptr()
        a.v_pages = None
        a.k_new = rows.data_ptr()
        a.v_new = None
        a.page_table = table.data_ptr()
        a.k_new_stride[:] = [rows.numel(), rows.stride(0)]
        a.v_new_stride[:] = [0, 0]
        a.num_pages = self.max_pages
        a.heads_kv = 1
        a.page_size = self.page_size
        a.head_dim = self.latent_dim + self.rope_dim
        a.start = start
        a.n_tokens = rows.size(0)
        a.elem_bytes = self.pages.element_size()
        if a.elem_bytes not in (2, 4):
            raise TypeError(f"MLALatentCache: pool dtype {self.pages.dtype} is not supported")
        lib = _lib.load()
        with torch.cuda.device(self.pages.device):
            stream = _lib.current_stream_handle(self.pages.device)
            _lib.check(lib.ffa_paged_append(ctypes.byref(a), ctypes.c_void_p(stream)))

    def block_tables(self, seq_ids: Sequence[int],
                     device: Optional[torch.device | str] = None
                     ) -> Tuple[torch.Tensor, torch.Tensor]:
        """int32 ``[B, max_blocks]`` block tables (rows padded with 0) and int32 ``[B]``
        lengths of ``seq_ids``."""
        device = self.pages.device if device is None else torch.device(device)
        tables = [self.sequences.get(s, {"page_table": []})["page_table"] for s in seq_ids]
        width = max([1] + [len(t) for t in tables])
        bt = torch.zeros(len(tables), width, dtype=torch.int32)
        for i, t in enumerate(tables):
            if t:
                bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        lens = torch.tensor([self.seq_len(s) for s in seq_ids], dtype=torch.int32)
        return bt.to(device), lens.to(device)

    def decode(self, q: torch.Tensor, seq_ids: Sequence[int], *, scale: float,
               return_lse: bool = False) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """``fastest_flash_mla_decode`` of absorbed queries ``[B, H, latent + rope]`` over
        the cached rows of ``seq_ids``."""
        bt, lens = self.block_tables(seq_ids)
        max_len = max([0] + [self.seq_len(s) for s in seq_ids])
        return fastest_flash_mla_decode(q, self.pages, bt, lens, dim_v=self.latent_dim,
                                        scale=scale, return_lse=return_lse,
                                        max_context_len=max_len)

    @property
    def num_free_pages(self) -> int:
        return len(self.free_pages)
