"""CPU restatement of the reference forward attention, in numpy fp32.

TEST INFRASTRUCTURE ONLY — the parity checker. Only tests/, __graft_entry__.smoke()
and bench.py's cpu_baseline leg may import this module; the product
(fastest_flash_attention_amd) never does.

Restates, step by step and in the same fp32 arithmetic order:
  * flash_attn_cpu_forward        kernels/cpu_reference.py:132-312
  * _compute_logsumexp_pass1      kernels/cpu_reference.py:63-125
  * helpers                       kernels/cpu_reference.py:28-56
  * the dispatcher's CPU branch   ops/attention_forward.py:23-167 (forward())
  * auto_select_block_size, repeat_kv, maybe_unsqueeze_head  utils.py:36-67,98-130
Inputs are numpy arrays (bf16/fp16 tensors are handed over as their exact fp32
values). Outputs: O in fp32 (the reference casts to q.dtype last, :304) and LSE
fp32 [B, H, S_q, 1].

Pinned by tests/test_oracle.py against: the reference's own test oracle (_naive_sdpa,
tests/test_fastest_flash.py:55-88) restated in fp64 (oracle/naive.py) on the
reference tests' seeded inputs, scipy.special.logsumexp / softmax, closed forms
(single key, identical keys, constant V, fully-masked-row sentinel), block-size
invariance, explicit GQA repetition, and planted-mistake mutants that must fail.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np

F32 = np.float32
NEG_INF = F32(-np.inf)


# ----------------------------------------------------------------------------------
# dtype simulation (kernels/cpu_reference.py:28-32)
# ----------------------------------------------------------------------------------

def round_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bfloat16 (nearest-even), returned as fp32."""
    x = np.ascontiguousarray(x, dtype=F32)
    u = x.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16) << 16
    out = r.astype(np.uint32).view(F32).copy()
    nan = np.isnan(x)
    out[nan] = x[nan]
    return out


def round_to_dtype(x: np.ndarray, dtype: Optional[str]) -> np.ndarray:
    """_to_compute_dtype: cast to a lower-precision dtype (simulation)."""
    if dtype is None or dtype == "float32":
        return x
    if dtype == "float16":
        return x.astype(np.float16).astype(F32)
    if dtype == "bfloat16":
        return round_to_bf16(x)
    raise ValueError(f"unknown compute dtype {dtype!r}")


def apply_softcap(scores: np.ndarray, softcap: float) -> np.ndarray:
    """_apply_softcap (:35-37): softcap * tanh(scores / softcap)."""
    c = F32(softcap)
    return (c * np.tanh(scores / c)).astype(F32)


def causal_mask(q_start: int, q_end: int, k_start: int, k_end: int) -> np.ndarray:
    """_build_causal_mask (:40-46): True where masked (row < col)."""
    rows = np.arange(q_start, q_end)[:, None]
    cols = np.arange(k_start, k_end)[None, :]
    return rows < cols


def window_mask(q_start: int, q_end: int, k_start: int, k_end: int, window: int) -> np.ndarray:
    """_build_window_mask (:49-56): True where the key is left of the window."""
    rows = np.arange(q_start, q_end)[:, None]
    cols = np.arange(k_start, k_end)[None, :]
    return cols < (rows - window + 1)


def _scores(q_blk, k_blk, scale, softcap, causal, window, q_abs_s, q_abs_e, ks, ke,
            compute_dtype=None):
    q_lp = round_to_dtype(q_blk, compute_dtype)
    k_lp = round_to_dtype(k_blk, compute_dtype)
    s = np.matmul(q_lp.astype(F32), np.swapaxes(k_lp.astype(F32), -1, -2)) * F32(scale)
    s = s.astype(F32)
    if softcap is not None:
        s = apply_softcap(s, softcap)
    if causal:
        s = np.where(causal_mask(q_abs_s, q_abs_e, ks, ke), NEG_INF, s)
    if window is not None:
        s = np.where(window_mask(q_abs_s, q_abs_e, ks, ke, window), NEG_INF, s)
    return s.astype(F32)


def _logaddexp(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    return np.logaddexp(a, b).astype(F32)


def _logsumexp_last(x: np.ndarray) -> np.ndarray:
    """torch.logsumexp over the last axis (keepdim); all -inf rows give -inf."""
    m = np.max(x, axis=-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, F32(0))
    s = np.sum(np.exp(x - m_safe), axis=-1, keepdims=True)
    with np.errstate(divide="ignore"):
        return (np.log(s) + m_safe).astype(F32)


def logsumexp_pass1(q, k, scale, causal, block_q, block_kv, block_mask, softcap,
                    sliding_window, q_offset=0):
    """_compute_logsumexp_pass1 (:63-125): exact per-row LSE, [B, H, S_q, 1]."""
    B, H, S_q, _ = q.shape
    S_k = k.shape[2]
    n_br = math.ceil(S_q / block_q)
    n_bc = math.ceil(S_k / block_kv)
    blocks = []
    for i in range(n_br):
        qs, qe = i * block_q, min(i * block_q + block_q, S_q)
        q_abs_s, q_abs_e = q_offset + qs, q_offset + qe
        blk = np.full((B, H, qe - qs, 1), NEG_INF, dtype=F32)
        for j in range(n_bc):
            ks, ke = j * block_kv, min(j * block_kv + block_kv, S_k)
            if block_mask is not None and not block_mask[i, j]:
                continue
            if causal and ks > (q_abs_e - 1):
                break
            if sliding_window is not None and ke - 1 < q_abs_s - sliding_window + 1:
                continue
            s = _scores(q[:, :, qs:qe], k[:, :, ks:ke], scale, softcap, causal,
                        sliding_window, q_abs_s, q_abs_e, ks, ke)
            blk = _logaddexp(blk, _logsumexp_last(s))
        blocks.append(blk)
    return np.concatenate(blocks, axis=2)


def flash_attn_cpu_forward(
    q: np.ndarray,
    k: np.ndarray,
    v: np.ndarray,
    scale: Optional[float] = None,
    causal: bool = False,
    block_q: int = 64,
    block_kv: int = 64,
    block_mask: Optional[np.ndarray] = None,
    softcap: Optional[float] = None,
    sliding_window: Optional[int] = None,
    two_pass: bool = False,
    compute_dtype: Optional[str] = None,
    q_offset: int = 0,
    return_lse: bool = False,
) -> Tuple[np.ndarray, Optional[np.ndarray]]:
    """flash_attn_cpu_forward (kernels/cpu_reference.py:132-312), fp32.

    q [B, H, S_q, D], k/v [B, H or 1, S_kv, D] (matmul broadcasting as in torch).
    Returns (O fp32 [B, H, S_q, D], LSE fp32 [B, H, S_q, 1] or None).
    """
    q = np.asarray(q, dtype=F32)
    k = np.asarray(k, dtype=F32)
    v = np.asarray(v, dtype=F32)
    B, H, S_q, D = q.shape
    S_kv = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    n_br = math.ceil(S_q / block_q)
    n_bc = math.ceil(S_kv / block_kv)
    out_b = max(B, k.shape[0])
    out_h = max(H, k.shape[1])

    with np.errstate(invalid="ignore", divide="ignore", over="ignore"):
        exact_lse = None
        if two_pass:
            exact_lse = logsumexp_pass1(q, k, scale, causal, block_q, block_kv, block_mask,
                                        softcap, sliding_window, q_offset)
        outs, lses = [], []
        for i in range(n_br):                                        # :195
            qs, qe = i * block_q, min(i * block_q + block_q, S_q)
            br = qe - qs
            q_blk = q[:, :, qs:qe]
            q_abs_s, q_abs_e = q_offset + qs, q_offset + qe
            o_i = np.zeros((out_b, out_h, br, D), dtype=F32)        # :205
            lse_i = np.full((out_b, out_h, br, 1), NEG_INF, dtype=F32)
            for j in range(n_bc):                                    # :215
                ks, ke = j * block_kv, min(j * block_kv + block_kv, S_kv)
                if block_mask is not None and not block_mask[i, j]:  # :220-222
                    continue
                if causal and ks > (q_abs_e - 1):                    # :225-226
                    break
                if sliding_window is not None and ke - 1 < q_abs_s - sliding_window + 1:
                    continue                                         # :229-231
                s = _scores(q_blk, k[:, :, ks:ke], scale, softcap, causal, sliding_window,
                            q_abs_s, q_abs_e, ks, ke, compute_dtype)  # :260-278
                v_blk = v[:, :, ks:ke]
                if two_pass and exact_lse is not None:               # :281-285
                    p = np.exp(s - exact_lse[:, :, qs:qe]).astype(F32)
                    o_i = (o_i + np.matmul(p, v_blk)).astype(F32)
                else:                                                # :287-302
                    m = np.max(s, axis=-1, keepdims=True)
                    m = np.where(m == NEG_INF, F32(0), m).astype(F32)
                    p = np.exp(s - m).astype(F32)
                    l_sum = np.maximum(np.sum(p, axis=-1, keepdims=True), F32(1e-30))
                    lse_ij = (m + np.log(l_sum)).astype(F32)
                    lse_new = _logaddexp(lse_i, lse_ij)
                    alpha = np.exp(lse_i - lse_new).astype(F32)
                    tile_scale = np.exp(m - lse_new).astype(F32)
                    o_i = (alpha * o_i + tile_scale * np.matmul(p, v_blk)).astype(F32)
                    lse_i = lse_new
            outs.append(o_i)
            if return_lse:
                lses.append(exact_lse[:, :, qs:qe] if (two_pass and exact_lse is not None)
                            else lse_i)
    out = np.concatenate(outs, axis=2) if outs else np.zeros((out_b, out_h, 0, D), F32)
    lse = (np.concatenate(lses, axis=2) if lses else np.zeros((out_b, out_h, 0, 1), F32)) \
        if return_lse else None
    return out, lse


# ----------------------------------------------------------------------------------
# Dispatcher CPU branch (ops/attention_forward.py:23-167) and helpers (utils.py)
# ----------------------------------------------------------------------------------

def auto_select_block_size(S_q: int, S_kv: int, D: int, max_block: int = 256,
                           min_block: int = 16) -> int:
    """utils.py:36-67."""
    bs = max(min_block, min(4096 // max(D, 1), max_block))
    while bs > min_block and math.ceil(S_kv / bs) < 4:
        bs //= 2
    if bs > 0:
        bs = 1 << (bs.bit_length() - 1)
    return max(min_block, min(bs, max_block))


def repeat_kv(kv: np.ndarray, num_q_heads: int, num_kv_heads: int) -> np.ndarray:
    """utils.py:111-130: q head h reads kv head h // (Hq // Hkv)."""
    if num_q_heads == num_kv_heads:
        return kv
    return np.repeat(kv, num_q_heads // num_kv_heads, axis=1)


def forward(q, k, v, config=None, *, scale=None, causal=False, block_size=None,
            block_mask=None, softcap=None, sliding_window=None, two_pass=False,
            compute_dtype=None, num_kv_heads=None, kv_cache=None, return_lse=False):
    """The reference dispatcher with the CPU kernel (ops/attention_forward.py:23-167).

    ``config`` is duck-typed (the attributes of AttentionConfig, config.py:58-81).
    """
    if config is not None:                                           # :66-73
        causal = config.causal
        softcap = config.softcap
        sliding_window = config.sliding_window
        two_pass = config.two_pass
        compute_dtype = config.compute_dtype
        num_kv_heads = config.num_kv_heads
        return_lse = config.return_lse
    squeezed = q.ndim == 3                                           # :76
    if squeezed:
        q, k, v = q[:, None], k[:, None], v[:, None]
    B, H_q, S_q, D = q.shape
    H_kv = k.shape[1]
    q_offset = 0
    if kv_cache is not None:                                         # :82-89
        kc, vc = kv_cache
        if kc.ndim == 3:
            kc, vc = kc[:, None], vc[:, None]
        k = np.concatenate([kc, k], axis=2)
        v = np.concatenate([vc, v], axis=2)
        q_offset = k.shape[2] - S_q
    S_kv = k.shape[2]
    if num_kv_heads is not None and H_q != H_kv:                     # :94-96
        k = repeat_kv(k, H_q, H_kv)
        v = repeat_kv(v, H_q, H_kv)
    if scale is None:                                                # :98-99
        scale = 1.0 / math.sqrt(D)
    if block_size is None:                                           # :102-109
        if config is not None:
            bq = config.block_size_q or auto_select_block_size(S_q, S_kv, D)
            bkv = config.block_size_kv or auto_select_block_size(S_q, S_kv, D)
        else:
            bq = bkv = auto_select_block_size(S_q, S_kv, D)
    else:
        bq = bkv = block_size
    if compute_dtype is not None and not isinstance(compute_dtype, str):
        compute_dtype = str(compute_dtype).replace("torch.", "")
    out, lse = flash_attn_cpu_forward(
        q, k, v, scale=scale, causal=causal, block_q=bq, block_kv=bkv,
        block_mask=block_mask, softcap=softcap, sliding_window=sliding_window,
        two_pass=two_pass, compute_dtype=compute_dtype, q_offset=q_offset,
        return_lse=return_lse,
    )
    if squeezed:                                                     # :162-165
        out = out[:, 0]
        if lse is not None:
            lse = lse[:, 0]
    return out, lse
