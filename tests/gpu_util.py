"""Helpers shared by the GPU parity tests (not a test module)."""

from __future__ import annotations

import ctypes
import os
import sys

import numpy as np
import pytest
import torch

# north-star parity tolerances: fp32-accumulated 16-bit O within
# max-abs 2e-2 and mean-abs 2e-3, LSE within 1e-3
O_MAX_ABS = 2e-2
O_MEAN_ABS = 2e-3
LSE_ABS = 1e-3

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROBE_LIB = os.path.join(REPO, "tests", "hip", "libffa_probe.so")


def require_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")


def say(msg: str) -> None:
    """Name the case before a GPU step (a box that dies keeps only stdout)."""
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def seeded(shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def assert_parity(o_gpu, o_ref, lse_gpu=None, lse_ref=None, what=""):
    """Compare kernel output with the oracle at the north-star tolerances.

    Rows whose oracle LSE is finite and above the fully-masked sentinel range are
    checked by tolerance; rows with no visible key must be exactly O = 0 and carry
    the oracle's sentinel LSE (-inf or log(n * 1e-30))."""
    o = np32(o_gpu).astype(np.float64)
    r = np.asarray(o_ref, dtype=np.float64)
    assert o.shape == r.shape, (o.shape, r.shape)
    assert np.isfinite(o).all(), f"{what}: non-finite output"
    diff = np.abs(o - r)
    max_abs, mean_abs = float(diff.max(initial=0.0)), float(diff.mean()) if diff.size else 0.0
    assert max_abs <= O_MAX_ABS, f"{what}: O max-abs {max_abs:.3e}"
    assert mean_abs <= O_MEAN_ABS, f"{what}: O mean-abs {mean_abs:.3e}"
    if lse_gpu is not None:
        lg = np32(lse_gpu).astype(np.float64)
        lr = np.asarray(lse_ref, dtype=np.float64)
        assert lg.shape == lr.shape, (lg.shape, lr.shape)
        both_inf = np.isneginf(lg) & np.isneginf(lr)
        finite = ~both_inf
        assert np.isfinite(lg[finite]).all() and np.isfinite(lr[finite]).all(), \
            f"{what}: LSE -inf mismatch"
        ld = np.abs(lg[finite] - lr[finite])
        lmax = float(ld.max(initial=0.0))
        assert lmax <= LSE_ABS, f"{what}: LSE max-abs {lmax:.3e}"
    return max_abs, mean_abs


def probe_lib():
    if not os.path.exists(PROBE_LIB):
        pytest.skip("tests/hip/libffa_probe.so not built (run __graft_entry__.build())")
    lib = ctypes.CDLL(PROBE_LIB)
    for name in ("ffa_probe_mfma32", "ffa_probe_mfma16", "ffa_probe_mfma16k16",
                 "ffa_probe_mfma32f32"):
        getattr(lib, name).restype = ctypes.c_int
        getattr(lib, name).argtypes = [ctypes.c_void_p] * 3
    lib.ffa_probe_tr16.restype = ctypes.c_int
    lib.ffa_probe_tr16.argtypes = [ctypes.c_int, ctypes.c_void_p]
    lib.ffa_probe_load_lds.restype = ctypes.c_int
    lib.ffa_probe_load_lds.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    lib.ffa_probe_pair.restype = ctypes.c_int
    lib.ffa_probe_pair.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
    return lib
