"""fastest_flash_attn_backward — the drop-in backward entry point.

Mirrors the reference dispatcher (ops/attention_backward.py:19-76): same signature,
same results as its CPU branch flash_attn_cpu_backward (kernels/cpu_reference.py:
319-427), which also covers softcap, sliding window and q_offset (the reference's
Triton branch does not). The dispatch is replaced by one call of ``ffa_attn_bwd`` in
libffa.so on the current HIP stream: a preprocess kernel, a dK/dV kernel and a dQ
kernel, with no atomics (run-to-run deterministic). There is no CPU fallback.

Beyond the reference: K/V with fewer heads than q (GQA / MQA) get dK/dV summed over
each head group inside the kernel — the gradient of the forward's head map
h -> h // (Hq // Hkv) — and a K/V batch of 1 broadcast against q's batch gets dK/dV
summed over the batch. ``block_size`` only picks the reference's tiling, which does
not change the gradients, so it is accepted and ignored.
"""

from __future__ import annotations

import ctypes
import math
from typing import Optional, Tuple

import torch

from ..kernels import _lib
from .attention_forward import _conform


def fastest_flash_attn_backward(
    grad_output: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    output: torch.Tensor,
    lse: torch.Tensor,
    *,
    scale: Optional[float] = None,
    causal: bool = False,
    block_size: int = 64,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    q_offset: int = 0,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Backward pass (reference ops/attention_backward.py:19-76).

    Args:
        grad_output: [B, H, S_q, D] (or [B, S_q, D])
        q, k, v, output: as in the forward (k, v may have fewer heads: GQA).
        lse: [B, H, S_q, 1] natural-log logsumexp from the forward.

    Returns:
        (dq, dk, dv) in the dtypes and shapes of q, k, v.
    """
    del block_size  # tiling of the reference loop only; gradients do not depend on it
    squeezed = q.dim() == 3
    if squeezed:
        grad_output, q, k, v, output = (t.unsqueeze(1) for t in (grad_output, q, k, v, output))
        if lse.dim() == 3:
            lse = lse.unsqueeze(1)
    if lse.dim() == 3:
        lse = lse.unsqueeze(-1)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be 3D [B, S, D] or 4D [B, H, S, D]")
    B, Hq, Sq, D = q.shape
    Bk, Hkv, Skv, _ = k.shape
    # v may be narrower than q / k (taken as zero-padded, as the forward takes it): dv
    # then has v's dims
    if v.shape[:3] != k.shape[:3] or k.size(3) != D or not 1 <= v.size(3) <= D:
        raise ValueError(f"k {tuple(k.shape)} / v {tuple(v.shape)} do not match q {tuple(q.shape)}")
    Dv = v.size(3)
    if grad_output.shape != q.shape or output.shape != q.shape:
        raise ValueError("grad_output and output must have q's shape")
    if tuple(lse.shape) != (B, Hq, Sq, 1):
        raise ValueError(f"lse of shape {tuple(lse.shape)}, expected {(B, Hq, Sq, 1)}")
    if Hq % Hkv != 0:
        raise ValueError(f"num heads {Hq} is not a multiple of kv heads {Hkv}")
    if Bk != B and Bk != 1:
        raise ValueError(f"k/v batch {Bk} does not match q batch {B}")
    for name, t in (("grad_output", grad_output), ("q", q), ("k", k), ("v", v),
                    ("output", output), ("lse", lse)):
        if t.device.type != "cuda":
            raise RuntimeError(
                f"fastest_flash_attention_amd runs on ROCm GPU tensors only; {name} is on "
                f"{t.device} (there is no CPU path)"
            )
    dtype = q.dtype
    if not (k.dtype == v.dtype == output.dtype == grad_output.dtype == dtype):
        raise TypeError("grad_output, q, k, v and output must share one dtype")
    code = _lib.dtype_code(dtype, allow_fp32=True)  # bf16 / fp16 / fp32 (TypeError otherwise)
    if D > 256:
        raise ValueError(f"head_dim {D} > 256 is not supported by the backward kernels")
    if sliding_window is not None and int(sliding_window) <= 0:
        raise ValueError("sliding_window must be positive")
    if softcap is not None and float(softcap) <= 0.0:
        raise ValueError("softcap must be positive")
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    dev = q.device
    d_pad = (D + 7) // 8 * 8
    # a narrower v runs natively where the library has kernels for it (16-bit inputs,
    # head_dim 129..192, v dims <= 128 and a multiple of 8), zero-padded here otherwise
    narrow_v = (Dv < d_pad and code != _lib.FFA_DTYPE_FP32 and 128 < d_pad <= 192
                and Dv <= 128 and Dv % 8 == 0)
    dv_pad = Dv if narrow_v else d_pad
    if Bk != B:
        k = k.expand(B, -1, -1, -1)
        v = v.expand(B, -1, -1, -1)
    do_c, q_c, o_c = (_conform(t, d_pad) for t in (grad_output, q, output))
    k_c, v_c = _conform(k, d_pad), _conform(v, dv_pad)
    lse_c = lse.to(torch.float32)
    dq = torch.empty((B, Hq, Sq, d_pad), dtype=dtype, device=dev)
    dk = torch.empty((B, Hkv, Skv, d_pad), dtype=dtype, device=dev)
    dv = torch.empty((B, Hkv, Skv, dv_pad), dtype=dtype, device=dev)
    if B == 0 or Sq == 0:
        dq.zero_()
        dk.zero_()
        dv.zero_()
    else:
        lib = _lib.load()
        ws_bytes = lib.ffa_attn_bwd_workspace_bytes(B, Hq, Sq)
        ws = torch.empty((max(ws_bytes, 16) + 3) // 4, dtype=torch.float32, device=dev)
        a = _lib.AttnBwdArgs()
        a.dout, a.q, a.k, a.v, a.o = (t.data_ptr() for t in (do_c, q_c, k_c, v_c, o_c))
        a.lse = lse_c.data_ptr()
        a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
        a.workspace = ws.data_ptr()
        a.workspace_bytes = ws.numel() * 4
        a.do_stride[:] = list(do_c.stride())
        a.q_stride[:] = list(q_c.stride())
        a.k_stride[:] = list(k_c.stride())
        a.v_stride[:] = list(v_c.stride())
        a.o_stride[:] = list(o_c.stride())
        a.dq_stride[:] = list(dq.stride())
        a.dk_stride[:] = list(dk.stride())
        a.dv_stride[:] = list(dv.stride())
        a.lse_stride[:] = list(lse_c.stride()[:3])
        a.batch, a.heads_q, a.heads_kv = B, Hq, Hkv
        a.seqlen_q, a.seqlen_kv, a.head_dim = Sq, Skv, d_pad
        a.q_offset = int(q_offset)
        a.causal = 1 if causal else 0
        a.window = int(sliding_window) if sliding_window is not None else 0
        a.scale = float(scale)
        a.softcap = float(softcap) if softcap is not None else 0.0
        a.dtype = code
        a.v_head_dim = Dv if narrow_v else 0
        stream = _lib.current_stream_handle(dev)
        with torch.cuda.device(dev):
            rc = lib.ffa_attn_bwd(ctypes.byref(a), ctypes.c_void_p(stream))
        _lib.check(rc)
    if d_pad != D:
        dq, dk = (t[..., :D].contiguous() for t in (dq, dk))
    if dv.size(-1) != Dv:
        dv = dv[..., :Dv].contiguous()
    if Bk != B:
        dk = dk.sum(dim=0, keepdim=True, dtype=torch.float32).to(dtype)
        dv = dv.sum(dim=0, keepdim=True, dtype=torch.float32).to(dtype)
    if squeezed:
        dq, dk, dv = dq.squeeze(1), dk.squeeze(1), dv.squeeze(1)
    return dq, dk, dv
