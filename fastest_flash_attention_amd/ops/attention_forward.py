"""fastest_flash_attn_forward — the drop-in forward entry point.

Argument handling mirrors the reference dispatcher (ops/attention_forward.py:23-167):
config precedence (:66-73), 3D -> 4D (:76), kv_cache concatenation with
``q_offset = S_kv_total - S_q`` (:82-89), GQA (:94-96), default scale (:98-99) and
block-size resolution (:102-109). The dispatch (:112-159) is replaced by a single
path: one call of ``ffa_prefill_fwd`` in libffa.so (hand-written gfx950 HIP) on the
current HIP stream. There is no Triton, no autotuner, no alternative GPU kernel and
no CPU fallback: non-ROCm tensors, unsupported dtypes or features raise.

GQA is applied by index inside the kernel (q head h reads kv head h // (Hq // Hkv)),
so ``num_kv_heads`` costs no ``repeat_kv`` copy. The block size only selects the
reference tiling that defines the LSE of rows with no visible key; the kernel's own
tiles do not change any other result.
"""

from __future__ import annotations

import ctypes
import math
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from ..config import AttentionConfig
from ..kernels import _lib
from ..utils import auto_select_block_size, maybe_unsqueeze_head


@dataclass
class ResolvedForward:
    """Arguments after the reference dispatcher's resolution (host logic only)."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    B: int
    H_q: int
    H_kv: int
    S_q: int
    S_kv: int
    D: int
    q_offset: int
    scale: float
    causal: bool
    sliding_window: Optional[int]
    softcap: Optional[float]
    two_pass: bool
    compute_dtype: Optional[torch.dtype]
    block_mask: Optional[torch.Tensor]
    block_q: int
    block_kv: int
    return_lse: bool
    squeezed: bool
    Dv: int = 0  # v's head dim (<= D; a narrower v is taken as zero-padded to D)


@dataclass
class PrefillCall:
    """A fully resolved prefill launch: the ABI struct plus the tensors it points to."""

    args: _lib.PrefillArgs
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    out: torch.Tensor
    lse: Optional[torch.Tensor]
    squeezed: bool
    d_user: int = 0
    keep: tuple = ()  # device buffers the launch reads (block-mask words, counts)


def _expand_block_mask(block_mask, r: "ResolvedForward", device) -> Tuple[torch.Tensor, int, torch.Tensor]:
    """The reference's ``[n_br, n_bc]`` tile mask (cpu_reference.py:220-222) in the form
    the kernel reads: per query tile i, bit k of the 64-bit word array = mask[i][k //
    block_kv] (keys >= S_kv clear), plus the number of tiles the reference loop visits
    per query tile (mask set, not past the causal bound, not left of the window;
    cpu_reference.py:215-231), which fixes the LSE sentinel of rows with no visible
    key. All on the device."""
    bq, bkv = r.block_q, r.block_kv
    n_br = math.ceil(r.S_q / bq)
    n_bc = math.ceil(r.S_kv / bkv) if r.S_kv > 0 else 0
    bm = torch.as_tensor(block_mask)
    if bm.dim() != 2 or bm.shape[0] < n_br or bm.shape[1] < n_bc:
        raise ValueError(f"block_mask of shape {tuple(bm.shape)} does not cover the "
                         f"[{n_br}, {n_bc}] tiles of block size ({bq}, {bkv})")
    bm = bm[:n_br, :n_bc].to(device=device, dtype=torch.bool)
    words = max(1, math.ceil(r.S_kv / 64))
    keys = torch.arange(words * 64, device=device)
    if n_bc > 0:
        bits = bm[:, torch.clamp(keys // bkv, max=n_bc - 1)] & (keys < r.S_kv)[None, :]
    else:
        bits = torch.zeros(n_br, words * 64, dtype=torch.bool, device=device)
    shifts = torch.arange(64, device=device, dtype=torch.int64)
    packed = (bits.view(n_br, words, 64).to(torch.int64) << shifts).sum(dim=-1).contiguous()
    i = torch.arange(n_br, device=device)
    j = torch.arange(n_bc, device=device)
    visit = bm.clone()
    if r.causal:
        q_last = r.q_offset + torch.clamp((i + 1) * bq, max=r.S_q) - 1
        visit &= (j * bkv)[None, :] <= q_last[:, None]
    if r.sliding_window is not None:
        q_first = r.q_offset + i * bq
        k_last = torch.clamp((j + 1) * bkv, max=r.S_kv) - 1
        visit &= k_last[None, :] >= (q_first - r.sliding_window + 1)[:, None]
    visited = visit.sum(dim=1).to(torch.int32).contiguous()
    return packed, words, visited


def _conform(t: torch.Tensor, d_pad: int) -> torch.Tensor:
    """Return ``t`` (or a copy) in the form the kernels load in 16-byte chunks: unit
    dim stride, 16-byte aligned base, batch/head/seq strides multiple of 8 elements,
    dim zero-padded to ``d_pad`` (zeros leave q.k and the stored O dims unchanged)."""
    if t.size(-1) != d_pad:
        return torch.nn.functional.pad(t, (0, d_pad - t.size(-1))).contiguous()
    ok = (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
          and all(st % 8 == 0 for st, n in zip(t.stride()[:3], t.shape[:3]) if n > 1))
    if ok:
        return t
    out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
    out.copy_(t)
    return out


def _batch_strides(t: torch.Tensor, B: int, name: str) -> list[int]:
    """[b, h, s, d] element strides; a size-1 batch broadcasts against B (torch.matmul
    broadcasting in the reference CPU path)."""
    st = list(t.stride())
    if t.size(0) != B:
        if t.size(0) != 1:
            raise ValueError(f"{name} batch {t.size(0)} does not match q batch {B}")
        st[0] = 0
    if t.size(-1) == 1:
        st[3] = 1
    return st


def resolve_forward_args(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    config: Optional[AttentionConfig] = None,
    *,
    scale: Optional[float] = None,
    causal: bool = False,
    block_size: Optional[int] = None,
    block_mask: Optional[torch.Tensor] = None,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    two_pass: bool = False,
    compute_dtype: Optional[torch.dtype] = None,
    num_kv_heads: Optional[int] = None,
    kv_cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    return_lse: bool = False,
) -> ResolvedForward:
    """Argument resolution of the reference dispatcher (ops/attention_forward.py:65-109)."""
    if config is not None:
        causal = config.causal
        softcap = config.softcap
        sliding_window = config.sliding_window
        two_pass = config.two_pass
        compute_dtype = config.compute_dtype
        num_kv_heads = config.num_kv_heads
        return_lse = config.return_lse

    q, k, v, squeezed = maybe_unsqueeze_head(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 3D [B, S, D] or 4D [B, H, S, D]")
    B, H_q, S_q, D = q.shape
    H_kv = k.size(1)

    q_offset = 0
    if kv_cache is not None:
        k_cache, v_cache = kv_cache
        if k_cache.dim() == 3:
            k_cache = k_cache.unsqueeze(1)
            v_cache = v_cache.unsqueeze(1)
        k = torch.cat([k_cache, k], dim=2)
        v = torch.cat([v_cache, v], dim=2)
        q_offset = k.size(2) - S_q
    S_kv = k.size(2)

    # v may be narrower than q / k: it is then taken as zero-padded to D (the MLA
    # module's V, which the reference pads itself, modules/flash_mla.py:151-152), and
    # the output keeps q's shape
    if v.shape[:3] != k.shape[:3] or k.size(3) != D or not 1 <= v.size(3) <= D:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    if H_q != H_kv:
        if num_kv_heads is None and H_kv != 1:
            raise ValueError(f"q has {H_q} heads and k/v have {H_kv}: pass num_kv_heads for GQA")
        if H_q % H_kv != 0:
            raise ValueError(f"num heads {H_q} is not a multiple of kv heads {H_kv}")
    if sliding_window is not None and int(sliding_window) <= 0:
        raise ValueError("sliding_window must be positive")
    if softcap is not None and float(softcap) <= 0.0:
        raise ValueError("softcap must be positive")

    if scale is None:
        scale = 1.0 / math.sqrt(D)

    if block_size is None:
        if config is not None:
            bq, bkv = config.resolve_block_sizes(S_q, S_kv, D)
        else:
            bq = bkv = auto_select_block_size(S_q, S_kv, D)
    else:
        bq = bkv = block_size

    return ResolvedForward(
        q=q, k=k, v=v, B=B, H_q=H_q, H_kv=H_kv, S_q=S_q, S_kv=S_kv, D=D,
        q_offset=q_offset, scale=float(scale), causal=bool(causal),
        sliding_window=None if sliding_window is None else int(sliding_window),
        softcap=None if softcap is None else float(softcap), two_pass=bool(two_pass),
        compute_dtype=compute_dtype, block_mask=block_mask, block_q=int(bq),
        block_kv=int(bkv), return_lse=bool(return_lse), squeezed=squeezed, Dv=int(v.size(3)),
    )


def build_prefill_args(
    r: ResolvedForward, out: torch.Tensor, lse: Optional[torch.Tensor], dtype_code: int
) -> _lib.PrefillArgs:
    """Fill ``ffa_prefill_args`` from resolved arguments (no launch, no device access)."""
    a = _lib.PrefillArgs()
    a.q = r.q.data_ptr()
    a.k = r.k.data_ptr()
    a.v = r.v.data_ptr()
    a.o = out.data_ptr()
    a.lse = lse.data_ptr() if lse is not None else None
    a.q_stride[:] = _batch_strides(r.q, r.B, "q")
    a.k_stride[:] = _batch_strides(r.k, r.B, "k")
    a.v_stride[:] = _batch_strides(r.v, r.B, "v")
    a.o_stride[:] = list(out.stride())
    if lse is not None:
        a.lse_stride[:] = list(lse.stride()[:3])
    a.batch = r.B
    a.heads_q = r.H_q
    a.heads_kv = r.H_kv
    a.seqlen_q = r.S_q
    a.seqlen_kv = r.S_kv
    a.head_dim = r.D
    a.q_offset = r.q_offset
    a.causal = 1 if r.causal else 0
    a.window = r.sliding_window if r.sliding_window is not None else 0
    a.scale = r.scale
    a.softcap = r.softcap if r.softcap is not None else 0.0
    a.ref_block_q = r.block_q
    a.ref_block_kv = r.block_kv
    a.masked_lse_mode = 1 if r.two_pass else 0
    a.dtype = dtype_code
    a.v_head_dim = r.Dv if 0 < r.Dv < r.D else 0
    return a


def prepare_prefill(*args, out: Optional[torch.Tensor] = None, **kwargs) -> PrefillCall:
    """Resolve arguments, check device/dtype/features, allocate outputs, build the ABI
    struct. Launches nothing."""
    r = resolve_forward_args(*args, **kwargs)
    for name, t in (("q", r.q), ("k", r.k), ("v", r.v)):
        if t.device.type != "cuda":
            raise RuntimeError(
                f"fastest_flash_attention_amd runs on ROCm GPU tensors only; {name} is on "
                f"{t.device} (there is no CPU path)"
            )
    if not (r.q.device == r.k.device == r.v.device):
        raise RuntimeError("q, k, v must be on the same device")
    if not (r.q.dtype == r.k.dtype == r.v.dtype):
        raise TypeError(f"q/k/v dtypes differ: {r.q.dtype}, {r.k.dtype}, {r.v.dtype}")
    code = _lib.dtype_code(r.q.dtype, allow_fp32=True)
    if r.compute_dtype is not None and r.compute_dtype != r.q.dtype:
        # The reference rounds q and k (not v) to compute_dtype before the fp32 product
        # (cpu_reference.py:260-262). fp32 is exact for 16-bit inputs; a 16-bit compute
        # dtype is applied as an exact round trip q -> compute_dtype -> q.dtype (every
        # bf16/fp16 value of the rounded tensor is representable in the input dtype).
        # fp32 inputs with a 16-bit compute dtype take the same round trip (the values
        # stay fp32, rounded as the reference rounds them).
        if r.compute_dtype in (torch.bfloat16, torch.float16):
            r.q = r.q.to(r.compute_dtype).to(r.q.dtype)
            r.k = r.k.to(r.compute_dtype).to(r.k.dtype)
        elif r.compute_dtype != torch.float32:
            raise TypeError(f"unsupported compute_dtype {r.compute_dtype}")
    if r.D > 256:
        raise ValueError(f"head_dim {r.D} > 256 is not supported")
    d_pad = (r.D + 7) // 8 * 8
    # A narrower v runs natively where the library has kernels for it (16-bit inputs,
    # head_dim 129..192, v_head_dim <= 128 and a multiple of 8); elsewhere it is
    # zero-padded here, which gives the same result.
    narrow_v = (r.Dv < d_pad and code != _lib.FFA_DTYPE_FP32 and 128 < d_pad <= 192
                and r.Dv <= 128 and r.Dv % 8 == 0)
    r.q = _conform(r.q, d_pad)
    r.k = _conform(r.k, d_pad)
    r.v = _conform(r.v, r.Dv if narrow_v else d_pad)
    d_user = r.D
    r.D = d_pad
    r.Dv = r.Dv if narrow_v else d_pad
    if out is None or d_pad != d_user:
        out = torch.empty((r.B, r.H_q, r.S_q, d_pad), dtype=r.q.dtype, device=r.q.device)
    lse = (
        torch.empty((r.B, r.H_q, r.S_q, 1), dtype=torch.float32, device=r.q.device)
        if r.return_lse
        else None
    )
    call = PrefillCall(build_prefill_args(r, out, lse, code), r.q, r.k, r.v, out, lse,
                       r.squeezed)
    call.d_user = d_user
    if r.block_mask is not None:
        packed, words, visited = _expand_block_mask(r.block_mask, r, r.q.device)
        call.args.block_key_mask = packed.data_ptr()
        call.args.block_key_mask_words = words
        call.args.block_visited = visited.data_ptr()
        call.keep = (packed, visited)
    return call


def launch_prefill(call: PrefillCall) -> None:
    lib = _lib.load()
    stream = _lib.current_stream_handle(call.q.device)
    with torch.cuda.device(call.q.device):
        rc = lib.ffa_prefill_fwd(ctypes.byref(call.args), ctypes.c_void_p(stream))
    _lib.check(rc)


def fastest_flash_attn_forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    config: Optional[AttentionConfig] = None,
    *,
    scale: Optional[float] = None,
    causal: bool = False,
    block_size: Optional[int] = None,
    block_mask: Optional[torch.Tensor] = None,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    two_pass: bool = False,
    compute_dtype: Optional[torch.dtype] = None,
    num_kv_heads: Optional[int] = None,
    kv_cache: Optional[Tuple[torch.Tensor, torch.Tensor]] = None,
    return_lse: bool = False,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Forward attention on MI355X. Same signature and results as the reference's
    ``fastest_flash_attn_forward`` (ops/attention_forward.py:23-167).

    Returns ``(output, lse_or_None)``: output has q's shape and dtype; lse is fp32
    ``[B, H, S_q, 1]`` (``[B, S_q, 1]`` for 3D input), natural log.
    """
    call = prepare_prefill(
        q, k, v, config,
        scale=scale, causal=causal, block_size=block_size, block_mask=block_mask,
        softcap=softcap, sliding_window=sliding_window, two_pass=two_pass,
        compute_dtype=compute_dtype, num_kv_heads=num_kv_heads, kv_cache=kv_cache,
        return_lse=return_lse,
    )
    launch_prefill(call)
    output, lse = call.out, call.lse
    if output.size(-1) != call.d_user:
        output = output[..., : call.d_user].contiguous()
    if call.squeezed:
        output = output.squeeze(1)
        if lse is not None:
            lse = lse.squeeze(1)
    return output, lse
