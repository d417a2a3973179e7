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


def test_mfma_16x16x16_layout():
    require_gpu()
    lib = probe_lib()
    A = _small_ints((16, 16), 6)
    B = _small_ints((16, 16), 7)
    C = (A.double() @ B.double()).numpy()
    out = torch.zeros(64, 4, dtype=torch.float32, device="cuda")
    say("mfma 16x16x16 layout probe")
    assert lib.ffa_probe_mfma16k16(A.cuda().data_ptr(), B.cuda().data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy()
    for lane in range(64):
        for j in range(4):
            assert got[lane, j] == C[4 * (lane // 16) + j, lane % 16], (lane, j)


def test_mfma_32x32x2_f32_layout():
    require_gpu()
    lib = probe_lib()
    g = torch.Generator().manual_seed(8)
    A = torch.randint(-4, 5, (32, 2), generator=g).float()
    B = torch.randint(-4, 5, (2, 32), generator=g).float()
    C = (A.double() @ B.double()).numpy()
    out = torch.zeros(64, 16, dtype=torch.float32, device="cuda")
    say("mfma 32x32x2 f32 layout probe")
    assert lib.ffa_probe_mfma32f32(A.cuda().data_ptr(), B.cuda().data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy()
    for lane in range(64):
        g2 = lane // 32
        for i in range(4):
            for j in range(4):
                assert got[lane, 4 * i + j] == C[8 * i + 4 * g2 + j, lane % 32], (lane, i, j)


def test_global_load_lds_lane_placement():
    """global_load_lds_dwordx4: lane l's 16 bytes land at LDS base + 16 l."""
    require_gpu()
    lib = probe_lib()
    g = torch.arange(256, dtype=torch.int32, device="cuda")
    out = torch.zeros(256, dtype=torch.int32, device="cuda")
    say("global_load_lds probe")
    assert lib.ffa_probe_load_lds(g.data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy().reshape(64, 4)
    want = np.arange(256).reshape(64, 4)[::-1]
    assert np.array_equal(got, want)


@pytest.mark.parametrize("mode", [0, 1])
def test_ds_read_tr16_b64_layout(mode):
    """Records the element each lane receives from ds_read_b64_tr_b16 (printed) and
    checks the transpose law the V operand loader relies on: within each group of 16
    lanes, lane i receives element (i % 4) ... see the kernel comment."""
    require_gpu()
    lib = probe_lib()
    out = torch.zeros(256, dtype=torch.int16, device="cuda")
    say(f"ds_read_tr16 probe mode {mode}")
    assert lib.ffa_probe_tr16(mode, out.data_ptr()) == 0
    got = out.cpu().numpy().reshape(64, 4)
    print(f"tr16 mode {mode}:")
    for l in range(64):
        print(l, got[l].tolist())
    # every element read must come from one of the 64 lanes' own 4-element windows
    addrs = [4 * l if mode == 0 else 64 * (l % 16) + 4 * (l // 16) for l in range(64)]
    window = {a + e for a in addrs for e in range(4)}
    assert set(got.flatten().tolist()) <= window


def test_lane_pair_reductions():
    """wave_pair_max / wave_pair_sum combine lanes l and l ^ 32 (v_permlane32_swap)."""
    require_gpu()
    lib = probe_lib()
    g = torch.Generator().manual_seed(5)
    x = torch.randn(64, generator=g, dtype=torch.float32)
    out = torch.zeros(128, dtype=torch.float32, device="cuda")
    say("lane pair reduction probe")
    assert lib.ffa_probe_pair(x.cuda().data_ptr(), out.data_ptr()) == 0
    got = out.cpu().numpy()
    xn = x.numpy()
    partner = xn[np.arange(64) ^ 32]
    assert np.array_equal(got[:64], np.maximum(xn, partner))
    assert np.allclose(got[64:], xn + partner, rtol=0, atol=0)
