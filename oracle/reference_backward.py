"""CPU restatement of the reference attention backward, in numpy fp32.

TEST INFRASTRUCTURE ONLY (the checker of ffa_attn_bwd).

Restates, step by step:
  * flash_attn_cpu_backward      kernels/cpu_reference.py:319-427 (recompute backward
                                 from q, k, v, O and the stored LSE)
  * fastest_flash_attn_backward  ops/attention_backward.py:19-76 (dispatch; its CPU
                                 branch passes block_size as block_q = block_kv)
and adds the GQA reduction the HIP backward performs when the forward ran with
num_kv_heads (the reference backward only sees pre-repeated K/V: dK/dV of a KV head
are the sums over its repeated copies, the adjoint of repeat_kv, utils.py:111-130).

Pinned by tests/test_oracle_backward.py: torch.autograd in fp64 through the textbook
attention (softcap, causal / window masks) on small shapes, block-size invariance,
the GQA sum == explicit repeat, and planted mistakes (softcap derivative dropped,
D_i dropped, scale missing on dK) that must fail.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

from .reference_forward import F32, apply_softcap, causal_mask, window_mask


def flash_attn_cpu_backward(do: np.ndarray, q: np.ndarray, k: np.ndarray, v: np.ndarray,
                            o: np.ndarray, lse: np.ndarray, scale: Optional[float] = None,
                            causal: bool = False, block_q: int = 64, block_kv: int = 64,
                            softcap: Optional[float] = None,
                            sliding_window: Optional[int] = None,
                            q_offset: int = 0) -> Tuple[np.ndarray, np.ndarray, np.ndarray]:
    """do, q, o [B, H, S_q, D]; k, v [B, H, S_kv, D]; lse [B, H, S_q, 1].
    Returns fp32 (dq, dk, dv) (the reference casts to the input dtype last)."""
    B, H, S_q, D = q.shape
    S_kv = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scale = F32(scale)
    n_br = math.ceil(S_q / block_q)
    n_bc = math.ceil(S_kv / block_kv)
    dq = np.zeros(q.shape, F32)
    dk = np.zeros(k.shape, F32)
    dv = np.zeros(v.shape, F32)
    d_i = (do.astype(F32) * o.astype(F32)).sum(axis=-1, keepdims=True)          # :366
    for i in range(n_br):
        qs, qe = i * block_q, min((i + 1) * block_q, S_q)
        q_abs_s, q_abs_e = q_offset + qs, q_offset + qe
        qb = q[:, :, qs:qe].astype(F32)
        dob = do[:, :, qs:qe].astype(F32)
        lseb = lse[:, :, qs:qe].astype(F32)
        dib = d_i[:, :, qs:qe]
        for j in range(n_bc):
            ks, ke = j * block_kv, min((j + 1) * block_kv, S_kv)
            if causal and ks > q_abs_e - 1:                                       # :384
                break
            if sliding_window is not None and ke - 1 < q_abs_s - sliding_window + 1:
                continue
            kb = k[:, :, ks:ke].astype(F32)
            vb = v[:, :, ks:ke].astype(F32)
            s = np.matmul(qb, np.swapaxes(kb, -1, -2)) * scale                   # :393
            s_raw = s
            if softcap is not None:
                s = apply_softcap(s, softcap)
            if causal:
                s = np.where(causal_mask(q_abs_s, q_abs_e, ks, ke)[None, None], -np.inf, s)
            if sliding_window is not None:
                s = np.where(window_mask(q_abs_s, q_abs_e, ks, ke, sliding_window)[None, None],
                             -np.inf, s)
            with np.errstate(invalid="ignore"):
                p = np.exp(s - lseb).astype(F32)                                  # :409
            dv[:, :, ks:ke] += np.matmul(np.swapaxes(p, -1, -2), dob)             # :412
            dp = np.matmul(dob, np.swapaxes(vb, -1, -2))                          # :415
            ds = p * (dp - dib)                                                   # :418
            if softcap is not None:
                t = np.tanh(s_raw / F32(softcap))                                 # :422
                ds = ds * (F32(1.0) - t * t)
            dq[:, :, qs:qe] += np.matmul(ds, kb) * scale                          # :427
            dk[:, :, ks:ke] += np.matmul(np.swapaxes(ds, -1, -2), qb) * scale
    return dq, dk, dv


def backward(do, q, k, v, o, lse, *, scale=None, causal=False, block_size=64, softcap=None,
             sliding_window=None, q_offset=0, num_kv_heads=None):
    """The reference backward with GQA: K/V of ``num_kv_heads`` heads are repeated to
    q's heads (utils.py:127-130) and dK/dV summed back over each group."""
    Hq, Hkv = q.shape[1], k.shape[1]
    ratio = Hq // Hkv
    if ratio > 1:
        k = np.repeat(k, ratio, axis=1)
        v = np.repeat(v, ratio, axis=1)
    dq, dk, dv = flash_attn_cpu_backward(do, q, k, v, o, lse, scale=scale, causal=causal,
                                         block_q=block_size, block_kv=block_size,
                                         softcap=softcap, sliding_window=sliding_window,
                                         q_offset=q_offset)
    if ratio > 1:
        B, _, S, D = dk.shape
        dk = dk.reshape(B, Hkv, ratio, S, D).sum(axis=2)
        dv = dv.reshape(B, Hkv, ratio, S, D).sum(axis=2)
    return dq, dk, dv
