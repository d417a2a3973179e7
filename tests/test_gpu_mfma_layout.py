"""Device check of the MFMA lane layouts the kernels are built on (tests/hip/mfma_probe.hip)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from tests.gpu_util import probe_lib, require_gpu, say

pytestmark = pytest.mark.gpu


def _small_ints(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(-4, 5, shape, generator=g).to(torch.bfloat16)


def test_mfma_32x32x16_layout():
    require_gpu()
    lib = probe_lib()
    A = _small_ints((32, 16), 0)
    B = _small_ints((16, 32), 1)
    C = (A.double() @ B.double()).numpy()
    out = torch.zeros(64, 16, dtype=torch.float32, device="cuda")
    say("mfma 32x32x16 layout probe")
    assert lib.ffa_probe_mfma32(A.cuda().data_ptr(), B.cuda().data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy()
    for lane in range(64):
        g = lane // 32
        for i in range(4):
            for j in range(4):
                assert got[lane, 4 * i + j] == C[8 * i + 4 * g + j, lane % 32], (lane, i, j)


def test_mfma_16x16x32_layout():
    require_gpu()
    lib = probe_lib()
    A = _small_ints((16, 32), 2)
    B = _small_ints((32, 16), 3)
    C = (A.double() @ B.double()).numpy()
    out = torch.zeros(64, 4, dtype=torch.float32, device="cuda")
    say("mfma 16x16x32 layout probe")
    assert lib.ffa_probe_mfma16(A.cuda().data_ptr(), B.cuda().data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy()
    for lane in range(64):
        for j in range(4):
            assert got[lane, j] == C[4 * (lane // 16) + j, lane % 16], (lane, j)
