"""ctypes binding of libffa.so (C ABI declared in include/ffa.h).

This module is the only place Python touches the native library. It replaces the
reference's Triton availability probe and kernel imports
(reference utils.py:20-29, kernels/__init__.py:28-39): the library is loaded once,
after torch, so the process keeps a single HIP runtime.

No fallback exists: when the library is missing or a call fails, a RuntimeError
carrying ``ffa_strerror(rc)`` is raised.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

import torch  # noqa: F401  (must load torch's HIP runtime before libffa.so)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libffa.so")

FFA_ABI_VERSION = 7
FFA_DTYPE_BF16 = 0
FFA_DTYPE_FP16 = 1
FFA_DTYPE_FP32 = 2
FFA_NOALLOC_SCRATCH_BYTES = 64 << 20  # include/ffa.h

_I64x4 = ctypes.c_int64 * 4
_I64x3 = ctypes.c_int64 * 3
_I64x2 = ctypes.c_int64 * 2


class PrefillArgs(ctypes.Structure):
    """Mirror of ``ffa_prefill_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("q_stride", _I64x4),
        ("k_stride", _I64x4),
        ("v_stride", _I64x4),
        ("o_stride", _I64x4),
        ("lse_stride", _I64x3),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("q_offset", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("ref_block_q", ctypes.c_int32),
        ("ref_block_kv", ctypes.c_int32),
        ("masked_lse_mode", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("block_key_mask", ctypes.c_void_p),
        ("block_key_mask_words", ctypes.c_int32),
        ("block_visited", ctypes.c_void_p),
        ("v_head_dim", ctypes.c_int32),
    ]


class PagedGatherArgs(ctypes.Structure):
    """Mirror of ``ffa_paged_gather_args``."""

    _fields_ = [
        ("k_pages", ctypes.c_void_p),
        ("v_pages", ctypes.c_void_p),
        ("k_out", ctypes.c_void_p),
        ("v_out", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("num_pages", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("context_len", ctypes.c_int32),
        ("elem_bytes", ctypes.c_int32),
    ]


class PagedAppendArgs(ctypes.Structure):
    """Mirror of ``ffa_paged_append_args``."""

    _fields_ = [
        ("k_pages", ctypes.c_void_p),
        ("v_pages", ctypes.c_void_p),
        ("k_new", ctypes.c_void_p),
        ("v_new", ctypes.c_void_p),
        ("page_table", ctypes.c_void_p),
        ("k_new_stride", _I64x2),
        ("v_new_stride", _I64x2),
        ("num_pages", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("start", ctypes.c_int32),
        ("n_tokens", ctypes.c_int32),
        ("elem_bytes", ctypes.c_int32),
    ]


class PagedDecodeArgs(ctypes.Structure):
    """Mirror of ``ffa_paged_decode_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k_pages", ctypes.c_void_p),
        ("v_pages", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("context_lens", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("q_stride", _I64x2),
        ("o_stride", _I64x2),
        ("lse_stride", _I64x2),
        ("block_table_stride", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("max_context_len", ctypes.c_int32),
        ("tokens_per_split", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class MlaDecodeArgs(ctypes.Structure):
    """Mirror of ``ffa_mla_decode_args``."""

    _fields_ = [
        ("q", ctypes.c_void_p),
        ("kv_pages", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("block_tables", ctypes.c_void_p),
        ("context_lens", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("q_stride", _I64x2),
        ("o_stride", _I64x2),
        ("lse_stride", _I64x2),
        ("block_table_stride", ctypes.c_int32),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("dim_v", ctypes.c_int32),
        ("dim_rope", ctypes.c_int32),
        ("page_size", ctypes.c_int32),
        ("num_pages", ctypes.c_int32),
        ("max_context_len", ctypes.c_int32),
        ("tokens_per_split", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("dtype", ctypes.c_int32),
    ]


class AttnBwdArgs(ctypes.Structure):
    """Mirror of ``ffa_attn_bwd_args``."""

    _fields_ = [
        ("dout", ctypes.c_void_p),
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p),
        ("dk", ctypes.c_void_p),
        ("dv", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("do_stride", _I64x4),
        ("q_stride", _I64x4),
        ("k_stride", _I64x4),
        ("v_stride", _I64x4),
        ("o_stride", _I64x4),
        ("dq_stride", _I64x4),
        ("dk_stride", _I64x4),
        ("dv_stride", _I64x4),
        ("lse_stride", _I64x3),
        ("batch", ctypes.c_int32),
        ("heads_q", ctypes.c_int32),
        ("heads_kv", ctypes.c_int32),
        ("seqlen_q", ctypes.c_int32),
        ("seqlen_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("q_offset", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("window", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("softcap", ctypes.c_float),
        ("dtype", ctypes.c_int32),
        ("v_head_dim", ctypes.c_int32),
    ]


# Every symbol include/ffa.h declares, with its ctypes signature.
EXPORTS = {
    "ffa_prefill_fwd": (ctypes.c_int, [ctypes.POINTER(PrefillArgs), ctypes.c_void_p]),
    "ffa_paged_gather": (ctypes.c_int, [ctypes.POINTER(PagedGatherArgs), ctypes.c_void_p]),
    "ffa_paged_append": (ctypes.c_int, [ctypes.POINTER(PagedAppendArgs), ctypes.c_void_p]),
    "ffa_paged_decode_num_splits": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int32]),
    "ffa_paged_decode_workspace_bytes": (
        ctypes.c_size_t,
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32],
    ),
    "ffa_paged_decode_fwd": (ctypes.c_int, [ctypes.POINTER(PagedDecodeArgs), ctypes.c_void_p]),
    "ffa_paged_decode_fwd_noalloc": (
        ctypes.c_int, [ctypes.POINTER(PagedDecodeArgs), ctypes.c_void_p],
    ),
    "ffa_mla_decode_workspace_bytes": (
        ctypes.c_size_t,
        [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32, ctypes.c_int32],
    ),
    "ffa_mla_decode_fwd": (ctypes.c_int, [ctypes.POINTER(MlaDecodeArgs), ctypes.c_void_p]),
    "ffa_attn_bwd_workspace_bytes": (
        ctypes.c_size_t, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32],
    ),
    "ffa_attn_bwd": (ctypes.c_int, [ctypes.POINTER(AttnBwdArgs), ctypes.c_void_p]),
    "ffa_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "ffa_abi_version": (ctypes.c_int, []),
}

_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return LIB_PATH


def load() -> ctypes.CDLL:
    """Load libffa.so once; raise RuntimeError when it is missing or mismatched."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"fastest_flash_attention_amd: native library not built ({LIB_PATH}); "
                "run `python -m fastest_flash_attention_amd.kernels.hip.build`"
            )
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, argtypes) in EXPORTS.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = argtypes
        ver = lib.ffa_abi_version()
        if ver != FFA_ABI_VERSION:
            raise RuntimeError(f"libffa ABI version {ver} != expected {FFA_ABI_VERSION}")
        _lib = lib
        return lib


def is_available() -> bool:
    """True when libffa.so loads and a ROCm device is visible."""
    try:
        load()
    except (RuntimeError, OSError):
        return False
    return torch.cuda.is_available()


def check(rc: int) -> None:
    if rc != 0:
        msg = load().ffa_strerror(rc).decode()
        raise RuntimeError(f"{msg} (rc={rc})")


def strerror(rc: int) -> str:
    return load().ffa_strerror(rc).decode()


def dtype_code(dtype: torch.dtype, allow_fp32: bool = False) -> int:
    """ABI dtype code; float32 only where the entry point has an fp32 kernel (prefill)."""
    if dtype == torch.bfloat16:
        return FFA_DTYPE_BF16
    if dtype == torch.float16:
        return FFA_DTYPE_FP16
    if dtype == torch.float32 and allow_fp32:
        return FFA_DTYPE_FP32
    raise TypeError(
        f"fastest_flash_attention_amd: dtype {dtype} is not supported by this HIP kernel "
        f"(bfloat16, float16{', float32' if allow_fp32 else ''})"
    )


def current_stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
