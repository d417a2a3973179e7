"""Build libffa.so (the gfx950 HIP kernels behind include/ffa.h).

Each ``*.hip`` translation unit is compiled with ``hipcc --offload-arch=gfx950`` in
parallel and linked into ``fastest_flash_attention_amd/kernels/libffa.so``. The
library's RUNPATH points at torch's bundled ``lib/`` first so that, once torch is
imported, the process holds a single HIP runtime (``libamdhip64.so.7``).

Usage: ``python -m fastest_flash_attention_amd.kernels.hip.build [--quiet]``
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
PKG_KERNELS = os.path.dirname(HERE)
REPO = os.path.dirname(os.path.dirname(PKG_KERNELS))
INCLUDE = os.path.join(REPO, "include")
OUT_LIB = os.path.join(PKG_KERNELS, "libffa.so")
SOURCES = ["ffa_api.hip", "ffa_prefill.hip", "ffa_decode.hip", "ffa_backward.hip"]
ARCH = "gfx950"

# -packed-fp32-ops: no v_pk_{add,mul,fma}_f32 are emitted (scalar fp32 VALU only).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found (expected a ROCm install under /opt/rocm)")
    return path


def torch_lib_dir() -> str:
    import torch  # noqa: WPS433  (build-time only)

    return os.path.join(os.path.dirname(torch.__file__), "lib")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}")


def compile_objects(sources: list[str], src_dir: str, obj_dir: str, includes: list[str],
                    jobs: int) -> list[str]:
    os.makedirs(obj_dir, exist_ok=True)
    cc = hipcc()
    objs = []
    cmds = []
    for src in sources:
        obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
        objs.append(obj)
        cmd = [cc, *HIPCC_FLAGS, *[f"-I{i}" for i in includes], "-c",
               os.path.join(src_dir, src), "-o", obj]
        cmds.append(cmd)
    with concurrent.futures.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    return objs


def link_shared(objs: list[str], out: str) -> None:
    tl = torch_lib_dir()
    tmp = out + ".tmp"
    _run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp,
          f"-Wl,-rpath,{tl}"])
    os.replace(tmp, out)


def build(verbose: bool = True, jobs: int | None = None) -> str:
    """Compile and link libffa.so; returns its path."""
    t0 = time.time()
    jobs = jobs or min(len(SOURCES), os.cpu_count() or 1)
    obj_dir = os.path.join(HERE, "_build")
    objs = compile_objects(SOURCES, HERE, obj_dir, [INCLUDE, HERE], jobs)
    link_shared(objs, OUT_LIB)
    if verbose:
        print(f"[ffa build] {OUT_LIB} ({time.time() - t0:.1f}s)", flush=True)
    return OUT_LIB


if __name__ == "__main__":
    build(verbose="--quiet" not in sys.argv)
