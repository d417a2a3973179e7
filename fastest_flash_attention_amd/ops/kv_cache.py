"""PagedKVCache and the batched paged-decode read path.

``PagedKVCache`` keeps the reference interface and bookkeeping exactly
(ops/kv_cache.py:110-240): pool ``[max_pages, num_heads, page_size, head_dim]``,
free list consumed from the front and refilled at the tail, per-sequence Python
page tables, index law ``token t -> (page_table[t // page_size], t % page_size)``.

What changes is the read path. ``get_kv`` (reference :208-232, a Python loop of
per-page copies) is one launch of ``ffa_paged_gather``; and decode attention no
longer needs the gather at all: ``fastest_flash_paged_decode`` /
``PagedKVCache.decode`` stream the pages in place through block tables with the
split-K HIP kernel ``ffa_paged_decode_fwd``. ``append_tokens`` (the write path) keeps
its semantics but writes all new tokens with one indexed copy instead of a
per-token loop.

Decode runs on ROCm tensors only. A pool in host memory (the constructor's
default device, as in the reference) is filled by ``append_tokens`` and read by
``get_kv`` with indexed host copies, which move data and compute nothing.

Page ids outside the pool never address memory in the kernels: decode excludes the
tokens such an id would hold (see include/ffa.h). ``check_block_tables=True``
restores the reference's IndexError (ops/kv_cache.py:226-227) at the cost of one
device reduction and a host sync.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence, Tuple

import torch

from ..kernels import _lib
from .attention_forward import launch_prefill, prepare_prefill


def _auto_tokens_per_split(batch: int, heads_kv: int, max_len: int) -> int:
    """Largest power-of-two split in [64, 2048] tokens that still gives at least one
    workgroup per CU (256 on MI355X), counting every sequence at max_len. Each workgroup
    pays a fixed start (block-table stage, first tile loads), so long splits stream
    faster. Measured on MI355X against 512-token splits: +7% on the decode benchmark
    (B=64, 8 KV heads, lengths U[512, 32768]), +4% on 16 x 8k and 2 x 32k contexts
    (the latter with only 256 workgroups), -1% on 128 contexts of at most 2k tokens."""
    tps = 2048
    while tps > 64 and batch * heads_kv * max(1, math.ceil(max_len / tps)) < 256:
        tps //= 2
    return tps


def check_page_ids(block_tables: torch.Tensor, context_lens: torch.Tensor, page_size: int,
                   num_pages: int, max_context_len: int) -> None:
    """Raise IndexError if a page id the lengths reach lies outside ``[0, num_pages)``:
    entry j of row b is used when ``j * page_size < min(context_lens[b],
    max_context_len)``. One device reduction and a host sync."""
    if block_tables.numel() == 0:
        return
    lens = torch.clamp(context_lens.to(torch.int64), min=0, max=max_context_len)
    used = (torch.arange(block_tables.size(1), device=block_tables.device)[None, :] * page_size
            < lens[:, None])
    bad = used & ((block_tables < 0) | (block_tables >= num_pages))
    if bool(bad.any()):
        b, j = (int(x) for x in bad.nonzero()[0])
        raise IndexError(f"block_tables[{b}, {j}] = {int(block_tables[b, j])} is outside the "
                         f"pool of {num_pages} pages")


def _paged_decode_fp32(q3, k_pages, v_pages, block_tables, context_lens, scale, softcap,
                       sliding_window, return_lse, max_context_len):
    """Decode over fp32 pools: per sequence, ``ffa_paged_gather`` of its pages and one
    ``ffa_prefill_fwd`` on the fp32 MFMA kernel with the query at position L - 1 (the
    reference's get_kv + forward, ops/kv_cache.py:208-232, in fp32 as it computes).
    Two launches per sequence instead of the batched split-K kernels, which take
    16-bit pools; page ids are always checked (IndexError). The caller has checked the
    pools' contiguity, the tables' dtype and their width against max_context_len."""
    B, Hq, D = q3.shape
    P_total, Hkv, page_size, _ = k_pages.shape
    lens = [min(n, int(max_context_len))
            for n in context_lens.to(torch.int64).clamp(min=0).tolist()]
    bt = block_tables  # int32, contiguous, wide enough for max_context_len (checked)
    check_page_ids(bt, context_lens, page_size, P_total, int(max_context_len))
    out = torch.zeros((B, Hq, D), dtype=torch.float32, device=q3.device)
    lse = (torch.full((B, Hq), float("-inf"), dtype=torch.float32, device=q3.device)
           if return_lse else None)
    lib = _lib.load()
    stream = _lib.current_stream_handle(q3.device)
    for b, L in enumerate(lens):
        if L == 0:
            continue
        k = torch.empty(Hkv, L, D, dtype=torch.float32, device=q3.device)
        v = torch.empty_like(k)
        g = _lib.PagedGatherArgs()
        g.k_pages = k_pages.data_ptr()
        g.v_pages = v_pages.data_ptr()
        g.k_out = k.data_ptr()
        g.v_out = v.data_ptr()
        g.page_table = bt[b].data_ptr()
        g.num_pages = P_total
        g.heads_kv = Hkv
        g.page_size = page_size
        g.head_dim = D
        g.context_len = L
        g.elem_bytes = 4
        with torch.cuda.device(q3.device):
            _lib.check(lib.ffa_paged_gather(ctypes.byref(g), ctypes.c_void_p(stream)))
        call = prepare_prefill(q3[b, :, None, :].unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0),
                               scale=scale, causal=True, softcap=softcap,
                               sliding_window=sliding_window, num_kv_heads=Hkv,
                               return_lse=return_lse)
        call.args.q_offset = L - 1  # the query is the sequence's last token
        launch_prefill(call)
        out[b] = call.out[0, :, 0, :D]
        if lse is not None:
            lse[b] = call.lse[0, :, 0, 0]
    return out, lse


def decode_workspace_bytes(batch: int, heads_q: int, head_dim: int, max_context_len: int,
                           tokens_per_split: int) -> int:
    return int(_lib.load().ffa_paged_decode_workspace_bytes(
        batch, heads_q, head_dim, max_context_len, tokens_per_split))


def fastest_flash_paged_decode(
    q: torch.Tensor,
    k_pages: torch.Tensor,
    v_pages: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    *,
    scale: Optional[float] = None,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    return_lse: bool = False,
    max_context_len: Optional[int] = None,
    tokens_per_split: Optional[int] = None,
    workspace: Optional[torch.Tensor] = None,
    check_block_tables: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """One decode step for a batch of paged sequences.

    Page ids outside ``[0, num_pages)`` in the first ``ceil(L_b / page_size)`` entries
    of a row exclude the tokens they would hold (the kernels never read through them);
    with ``check_block_tables=True`` they raise IndexError instead, as the reference's
    page indexing does (ops/kv_cache.py:226-227).

    fp32 pools (the reference test's dtype) take another route: per sequence, a gather
    of its pages and the fp32 prefill kernel, two launches and a host sync per
    sequence. On that route page ids are always checked (IndexError, whatever
    ``check_block_tables`` says), and ``tokens_per_split`` and ``workspace`` are unused.

    q: ``[B, Hq, D]`` or ``[B, Hq, 1, D]``; k_pages/v_pages: ``[P, Hkv, page_size, D]``
    (PagedKVCache layout); block_tables: int32 ``[B, max_blocks]``; context_lens: int32
    ``[B]``. Sequence b attends to its first ``context_lens[b]`` tokens with the query at
    position ``context_lens[b] - 1``: the result equals the reference
    ``fastest_flash_attn_forward(q_b, k_new, v_new, kv_cache=get_kv(b)[:L-1],
    num_kv_heads=Hkv, ...)`` for the last token (ops/attention_forward.py:82-96,
    ops/kv_cache.py:208-232). Returns ``(O, lse)`` with O shaped like q and lse fp32
    ``[B, Hq]`` (``[B, Hq, 1, 1]`` for 4D q) or None.
    """
    squeeze = q.dim() == 3
    if q.dim() == 4:
        if q.size(2) != 1:
            raise ValueError("paged decode takes one query token per sequence")
        q3 = q[:, :, 0, :]
    elif q.dim() == 3:
        q3 = q
    else:
        raise ValueError("q must be [B, Hq, D] or [B, Hq, 1, D]")
    B, Hq, D = q3.shape
    if k_pages.dim() != 4 or k_pages.shape != v_pages.shape:
        raise ValueError("k_pages / v_pages must both be [num_pages, Hkv, page_size, D]")
    P_total, Hkv, page_size, Dk = k_pages.shape
    if Dk != D:
        raise ValueError(f"head_dim mismatch: q {D}, pages {Dk}")
    if Hq % Hkv != 0:
        raise ValueError(f"heads_q {Hq} is not a multiple of heads_kv {Hkv}")
    if not (q3.dtype == k_pages.dtype == v_pages.dtype):
        raise TypeError("q and the page pools must share a dtype")
    # checks every pool dtype shares: the kernels (and the fp32 route's gather) index
    # the pools as contiguous and read ceil(L / page_size) entries of a table row
    if not (k_pages.is_contiguous() and v_pages.is_contiguous()):
        raise ValueError("page pools must be contiguous")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise TypeError("block_tables and context_lens must be int32")
    if (block_tables.dim() != 2 or block_tables.size(0) < B or context_lens.dim() != 1
            or context_lens.size(0) < B):
        raise ValueError("block_tables must be [B, max_blocks] and context_lens [B]")
    block_tables = block_tables.contiguous()
    context_lens = context_lens.contiguous()
    if max_context_len is None:
        max_context_len = int(context_lens.max().item()) if B > 0 else 0
    if block_tables.size(1) * page_size < max_context_len:
        raise ValueError("block_tables has fewer columns than max_context_len needs")
    for name, t in (("q", q3), ("k_pages", k_pages), ("v_pages", v_pages),
                    ("block_tables", block_tables), ("context_lens", context_lens)):
        if t.device.type != "cuda":
            raise RuntimeError(
                f"fastest_flash_attention_amd paged decode runs on ROCm tensors only; "
                f"{name} is on {t.device}"
            )
    if q3.dtype == torch.float32:
        out, lse = _paged_decode_fp32(q3, k_pages, v_pages, block_tables, context_lens,
                                      scale, softcap, sliding_window, return_lse,
                                      max_context_len)
        if not squeeze:
            out = out.unsqueeze(2)
            if lse is not None:
                lse = lse[:, :, None, None]
        return out, lse
    code = _lib.dtype_code(q3.dtype)
    if D % 8 != 0:
        raise ValueError(f"paged decode needs head_dim % 8 == 0 (got {D})")
    if q3.stride(-1) != 1 or q3.data_ptr() % 16 or q3.stride(0) % 8 or q3.stride(1) % 8:
        q3 = q3.contiguous() if not q3.is_contiguous() else q3.clone()
    if check_block_tables:
        check_page_ids(block_tables, context_lens, page_size, P_total, max_context_len)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    if sliding_window is not None and int(sliding_window) <= 0:
        raise ValueError("sliding_window must be positive")
    if softcap is not None and float(softcap) <= 0.0:
        raise ValueError("softcap must be positive")
    if tokens_per_split is None:
        tokens_per_split = _auto_tokens_per_split(B, Hkv, max_context_len)

    lib = _lib.load()
    out = torch.empty((B, Hq, D), dtype=q3.dtype, device=q3.device)
    lse = torch.empty((B, Hq), dtype=torch.float32, device=q3.device) if return_lse else None
    need = int(lib.ffa_paged_decode_workspace_bytes(B, Hq, D, max_context_len, tokens_per_split))
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 4), dtype=torch.uint8, device=q3.device)

    a = _lib.PagedDecodeArgs()
    a.q = q3.data_ptr()
    a.k_pages = k_pages.data_ptr()
    a.v_pages = v_pages.data_ptr()
    a.o = out.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.block_tables = block_tables.data_ptr()
    a.context_lens = context_lens.data_ptr()
    a.workspace = workspace.data_ptr()
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    a.q_stride[:] = [q3.stride(0), q3.stride(1)]
    a.o_stride[:] = [out.stride(0), out.stride(1)]
    if lse is not None:
        a.lse_stride[:] = [lse.stride(0), lse.stride(1)]
    a.block_table_stride = block_tables.size(1)
    a.batch = B
    a.heads_q = Hq
    a.heads_kv = Hkv
    a.head_dim = D
    a.page_size = page_size
    a.num_pages = P_total
    a.max_context_len = max_context_len
    a.tokens_per_split = int(tokens_per_split)
    a.window = int(sliding_window) if sliding_window is not None else 0
    a.scale = float(scale)
    a.softcap = float(softcap) if softcap is not None else 0.0
    a.dtype = code
    stream = _lib.current_stream_handle(q3.device)
    with torch.cuda.device(q3.device):
        rc = lib.ffa_paged_decode_fwd(ctypes.byref(a), ctypes.c_void_p(stream))
    _lib.check(rc)
    if not squeeze:
        out = out.unsqueeze(2)
        if lse is not None:
            lse = lse[:, :, None, None]
    return out, lse


class ContinuousKVCache:
    """Contiguous KV-cache appended in place (reference ops/kv_cache.py:18-107).

    Buffers ``k_cache`` / ``v_cache`` are ``[max_batch, num_heads, max_seq_len,
    head_dim]`` zeros; ``seq_lens`` (int64, on ``device``) holds each entry's length and
    is the source of truth, as in the reference. ``append`` writes every batch entry's
    new block with one scatter (the reference loops over the batch).
    """

    def __init__(
        self,
        max_batch: int,
        max_seq_len: int,
        num_heads: int,
        head_dim: int,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
    ):
        self.max_batch = max_batch
        self.max_seq_len = max_seq_len
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.k_cache = torch.zeros(max_batch, num_heads, max_seq_len, head_dim,
                                   dtype=dtype, device=device)
        self.v_cache = torch.zeros(max_batch, num_heads, max_seq_len, head_dim,
                                   dtype=dtype, device=device)
        self.seq_lens = torch.zeros(max_batch, dtype=torch.long, device=device)

    def reset(self, batch_indices: Optional[torch.Tensor] = None):
        """Reset all entries, or the indexed ones (reference :61-66)."""
        if batch_indices is None:
            self.seq_lens.zero_()
        else:
            self.seq_lens[batch_indices] = 0

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
        """Append ``[B, H, S_new, D]`` K/V at each entry's current length and return the
        cached ``[B, H, max_len, D]`` views (reference :68-97). On overflow the entries
        before the first overflowing one are written and advanced, then AssertionError
        is raised, as in the reference loop."""
        B, H, S_new, D = k_new.shape
        starts = self.seq_lens[:B].tolist()
        fail = next((b for b in range(B) if starts[b] + S_new > self.max_seq_len), B)
        dev = self.k_cache.device
        if S_new > 0 and fail > 0:
            pos = (torch.tensor(starts[:fail], dtype=torch.int64).unsqueeze(1)
                   + torch.arange(S_new, dtype=torch.int64).unsqueeze(0)).to(dev)
            bidx = torch.arange(fail, device=dev).unsqueeze(1).expand(fail, S_new)
            dt = self.k_cache.dtype
            self.k_cache[bidx, :, pos, :] = k_new[:fail].to(dev, dt).permute(0, 2, 1, 3)
            self.v_cache[bidx, :, pos, :] = v_new[:fail].to(dev, dt).permute(0, 2, 1, 3)
        self.seq_lens[:fail] += S_new
        if fail < B:
            end = starts[fail] + S_new
            raise AssertionError(f"KV-cache overflow: {end} > {self.max_seq_len}")
        max_len = max(starts) + S_new if B > 0 else 0
        return self.k_cache[:B, :, :max_len, :], self.v_cache[:B, :, :max_len, :]

    def get_cache(self, batch_size: int) -> Tuple[Optional[torch.Tensor], Optional[torch.Tensor]]:
        """Cached ``[batch_size, H, max_len, D]`` views, or ``(None, None)`` when empty
        (reference :99-107)."""
        max_len = int(self.seq_lens[:batch_size].max().item()) if batch_size > 0 else 0
        if max_len == 0:
            return None, None
        return self.k_cache[:batch_size, :, :max_len, :], self.v_cache[:batch_size, :, :max_len, :]


class PagedKVCache:
    """Paged KV-cache (vLLM-style page tables), reference ops/kv_cache.py:110-240.

    Args:
        max_pages: total number of physical pages.
        page_size: tokens per page.
        num_heads: number of KV heads.
        head_dim: dimension per head.
        dtype: pool dtype.
        device: pool device (a ROCm device for get_kv / decode).
    """

    def __init__(
        self,
        max_pages: int = 1024,
        page_size: int = 64,
        num_heads: int = 8,
        head_dim: int = 64,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
    ):
        self.max_pages = max_pages
        self.page_size = page_size
        self.num_heads = num_heads
        self.head_dim = head_dim
        self.k_pages = torch.zeros(max_pages, num_heads, page_size, head_dim,
                                   dtype=dtype, device=device)
        self.v_pages = torch.zeros(max_pages, num_heads, page_size, head_dim,
                                   dtype=dtype, device=device)
        self.free_pages = list(range(max_pages))
        self.sequences: dict = {}

    def allocate_page(self) -> int:
        """Take the first free physical page (reference :157-161)."""
        if not self.free_pages:
            raise RuntimeError("PagedKVCache: out of physical pages")
        return self.free_pages.pop(0)

    def free_sequence(self, seq_id: int):
        """Return a sequence's pages to the tail of the free list (reference :163-168)."""
        if seq_id in self.sequences:
            for page_id in self.sequences[seq_id]["page_table"]:
                self.free_pages.append(page_id)
            del self.sequences[seq_id]

    def append_tokens(self, seq_id: int, k_tokens: torch.Tensor, v_tokens: torch.Tensor) -> int:
        """Append ``[num_heads, S_new, head_dim]`` K/V tokens; returns the new length.

        Same pages, slots and error behaviour as the reference per-token loop
        (:186-206): pages are taken in token order; when the pool runs dry the tokens
        that fit are written, the length updated, then RuntimeError is raised.
        """
        if seq_id not in self.sequences:
            self.sequences[seq_id] = {"page_table": [], "len": 0}
        seq = self.sequences[seq_id]
        S_new = k_tokens.size(1)
        if S_new == 0:
            return seq["len"]
        L0 = seq["len"]
        P = self.page_size
        need_pages = (L0 + S_new + P - 1) // P
        out_of_pages = False
        while len(seq["page_table"]) < need_pages:
            if not self.free_pages:
                out_of_pages = True
                break
            seq["page_table"].append(self.allocate_page())
        n_fit = min(S_new, len(seq["page_table"]) * P - L0)
        if n_fit > 0:
            dev = self.k_pages.device
            dt = self.k_pages.dtype  # slice assignment in the reference casts implicitly
            kn = k_tokens[:, :n_fit, :].to(dev, dt)
            vn = v_tokens[:, :n_fit, :].to(dev, dt)
            if dev.type == "cuda":
                self._append_device(seq, L0, kn, vn)
            else:
                t = torch.arange(L0, L0 + n_fit, dtype=torch.int64)
                table = torch.tensor(seq["page_table"], dtype=torch.int64)
                phys, slot = table[t // P], t % P
                self.k_pages[phys, :, slot, :] = kn.transpose(0, 1)
                self.v_pages[phys, :, slot, :] = vn.transpose(0, 1)
            seq["len"] = L0 + n_fit
        if out_of_pages:
            raise RuntimeError("PagedKVCache: out of physical pages")
        return seq["len"]

    def _append_device(self, seq: dict, start: int, kn: torch.Tensor, vn: torch.Tensor) -> None:
        """One ``ffa_paged_append`` launch: scatter [H, n, D] new rows into the pages."""
        if kn.stride(-1) != 1:
            kn = kn.contiguous()
        if vn.stride(-1) != 1:
            vn = vn.contiguous()
        table = torch.tensor(seq["page_table"], dtype=torch.int32, device=self.k_pages.device)
        a = _lib.PagedAppendArgs()
        a.k_pages = self.k_pages.data_ptr()
        a.v_pages = self.v_pages.data_ptr()
        a.k_new = kn.data_ptr()
        a.v_new = vn.data_ptr()
        a.page_table = table.data_ptr()
        a.k_new_stride[:] = [kn.stride(0), kn.stride(1)]
        a.v_new_stride[:] = [vn.stride(0), vn.stride(1)]
        a.num_pages = self.max_pages
        a.heads_kv = self.num_heads
        a.page_size = self.page_size
        a.head_dim = self.head_dim
        a.start = start
        a.n_tokens = kn.size(1)
        a.elem_bytes = self.k_pages.element_size()
        if a.elem_bytes not in (2, 4):
            raise TypeError(f"PagedKVCache: pool dtype {self.k_pages.dtype} is not supported on the GPU")
        lib = _lib.load()
        with torch.cuda.device(self.k_pages.device):
            stream = _lib.current_stream_handle(self.k_pages.device)
            _lib.check(lib.ffa_paged_append(ctypes.byref(a), ctypes.c_void_p(stream)))

    def _page_table_tensor(self, seq_id: int) -> torch.Tensor:
        return torch.tensor(self.sequences[seq_id]["page_table"], dtype=torch.int32,
                            device=self.k_pages.device)

    def _get_kv_host(self, seq_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """``get_kv`` of a pool in host memory (the constructor's default device): one
        indexed copy by the index law, token t from (page_table[t // P], t % P). It is a
        data copy of the cache the caller keeps on the host, like the reference's
        per-page slice copies (:224-230), bit-identical to them; no attention runs."""
        seq = self.sequences[seq_id]
        L = seq["len"]
        P = self.page_size
        t = torch.arange(L, dtype=torch.int64)
        table = torch.tensor(seq["page_table"], dtype=torch.int64)
        phys, slot = table[t // P], t % P
        # advanced indices on dims 0 and 2 put the token dim first: [L, H, D] -> [H, L, D]
        k_out = self.k_pages[phys, :, slot, :].transpose(0, 1).contiguous()
        v_out = self.v_pages[phys, :, slot, :].transpose(0, 1).contiguous()
        return k_out, v_out

    def get_kv(self, seq_id: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """Contiguous ``([H, L, D], [H, L, D])`` of a sequence, or ``(None, None)``
        (reference :208-232). A ROCm pool is gathered by one ``ffa_paged_gather``
        launch; a host pool by one indexed host copy."""
        if seq_id not in self.sequences or self.sequences[seq_id]["len"] == 0:
            return None, None
        if self.k_pages.device.type != "cuda":
            return self._get_kv_host(seq_id)
        if self.k_pages.element_size() not in (2, 4):
            raise TypeError(f"unsupported pool dtype {self.k_pages.dtype}")
        L = self.sequences[seq_id]["len"]
        k_out = torch.empty(self.num_heads, L, self.head_dim, dtype=self.k_pages.dtype,
                            device=self.k_pages.device)
        v_out = torch.empty_like(k_out)
        table = self._page_table_tensor(seq_id)
        a = _lib.PagedGatherArgs()
        a.k_pages = self.k_pages.data_ptr()
        a.v_pages = self.v_pages.data_ptr()
        a.k_out = k_out.data_ptr()
        a.v_out = v_out.data_ptr()
        a.page_table = table.data_ptr()
        a.num_pages = self.max_pages
        a.heads_kv = self.num_heads
        a.page_size = self.page_size
        a.head_dim = self.head_dim
        a.context_len = L
        a.elem_bytes = self.k_pages.element_size()
        lib = _lib.load()
        stream = _lib.current_stream_handle(self.k_pages.device)
        with torch.cuda.device(self.k_pages.device):
            rc = lib.ffa_paged_gather(ctypes.byref(a), ctypes.c_void_p(stream))
        _lib.check(rc)
        return k_out, v_out

    def block_tables(
        self, seq_ids: Sequence[int], device: Optional[torch.device | str] = None
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        """int32 ``[B, max_blocks]`` block tables (rows padded with 0) and int32 ``[B]``
        context lengths of ``seq_ids``, on ``device`` (default: the pool's)."""
        device = self.k_pages.device if device is None else torch.device(device)
        tables = []
        lens = []
        for sid in seq_ids:
            seq = self.sequences.get(sid, {"page_table": [], "len": 0})
            tables.append(seq["page_table"])
            lens.append(seq["len"])
        width = max([1] + [len(t) for t in tables])
        bt = torch.zeros(len(tables), width, dtype=torch.int32)
        for i, t in enumerate(tables):
            if t:
                bt[i, : len(t)] = torch.tensor(t, dtype=torch.int32)
        return bt.to(device), torch.tensor(lens, dtype=torch.int32).to(device)

    def decode(
        self,
        q: torch.Tensor,
        seq_ids: Sequence[int],
        *,
        scale: Optional[float] = None,
        softcap: Optional[float] = None,
        sliding_window: Optional[int] = None,
        return_lse: bool = False,
    ) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
        """Decode attention of ``q`` (``[B, Hq, D]``, one token per sequence of
        ``seq_ids``) over the cached tokens, read in place from the pages."""
        bt, lens = self.block_tables(seq_ids)
        max_len = max([0] + [self.sequences[s]["len"] for s in seq_ids if s in self.sequences])
        return fastest_flash_paged_decode(
            q, self.k_pages, self.v_pages, bt, lens, scale=scale, softcap=softcap,
            sliding_window=sliding_window, return_lse=return_lse, max_context_len=max_len,
        )

    @property
    def num_free_pages(self) -> int:
        return len(self.free_pages)

    @property
    def total_capacity(self) -> int:
        return self.max_pages * self.page_size
