"""CPU check that the prefill and backward grids cover every output tile exactly once.

The workgroup -> (batch x head, tile) maps live in kernels/hip/ffa_grid.h as constexpr
integer functions that the kernels call on the device; tests/hip/grid_check.cpp
compiles the same header with g++ and sweeps grid shapes (every BASELINE
configuration, all unit counts to 96 against all tile counts to 70, some large grids)
through the map the launchers select. A planted mistake in a copy of the header must
make the checker fail, so the check is known to bite.
"""

from __future__ import annotations

import os
import shutil
import subprocess

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIP_DIR = os.path.join(REPO, "fastest_flash_attention_amd", "kernels", "hip")
SRC = os.path.join(REPO, "tests", "hip", "grid_check.cpp")


def _build_and_run(tmp_path, include_dir):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    exe = os.path.join(tmp_path, "grid_check")
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{include_dir}", SRC, "-o", exe],
                   check=True, capture_output=True, text=True)
    return subprocess.run([exe], capture_output=True, text=True, timeout=120)


def test_grid_maps_are_bijections(tmp_path):
    r = _build_and_run(str(tmp_path), HIP_DIR)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "grid_check ok" in r.stdout


@pytest.mark.parametrize("old,new", [
    # interleaved tail: tile index computed from the wrong group size
    ("jq = r / gl;", "jq = r / xcd_group;"),
    # units run in turn: unit index within the XCD dropped
    ("      unit = x * hx + u;", "      unit = x * hx;"),
])
def test_grid_check_catches_planted_mistakes(tmp_path, old, new):
    with open(os.path.join(HIP_DIR, "ffa_grid.h")) as f:
        text = f.read()
    assert old in text
    mutant_dir = tmp_path / "mutant"
    mutant_dir.mkdir()
    (mutant_dir / "ffa_grid.h").write_text(text.replace(old, new))
    r = _build_and_run(str(tmp_path), str(mutant_dir))
    assert r.returncode != 0, "the planted mistake was not detected"
