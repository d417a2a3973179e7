#!/usr/bin/env python3
"""Benchmark of the forward-attention hot path on one MI355X.

Headline workload: bf16 causal prefill, B=4, H=32, S=8192,
D=128, through the drop-in ``fastest_flash_attn_forward``. A step is one forward over
that batch with q/k/v already resident in HBM. Second workload in the same line:
paged GQA decode (BASELINE cfg4: B=64, 32 q heads / 8 kv heads, D=128, page 16,
context lengths U[512, 32768], random page permutation), a third: MLA decode over the
compressed latent cache (BASELINE cfg5 decode: batch 32 at context 4096), and a fourth:
the attention backward at the north-star shape.

Algorithmic work: prefill FLOPs = 2 * B * H * (D + Dv) * N_valid (= 4 * B * H * D * N_valid
where V has q's head dim), N_valid = exact number of unmasked (q, k) pairs; decode bytes = K/V bytes of exactly context_len tokens + q + o +
lse + block tables + context lengths (split-K workspace traffic not counted).

Timing: HIP events recorded on the stream the kernels launch on (torch's current
stream) around exactly --steps steps, after --warmup untimed steps, bracketed by
torch.cuda.synchronize(). The CPU baseline is the oracle restatement of the reference
CPU path (oracle/reference_forward.py) on a bounded row sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2516.6   # MI355X dense bf16 MFMA (256 CU x 4096 flop/clk x 2.4 GHz)
PEAK_HBM_GBS = 8000.0        # MI355X HBM3E

PREFILL = {
    "north_star": dict(B=4, Hq=32, Hkv=32, S=8192, D=128, causal=True, window=None, softcap=None),
    "cfg2": dict(B=4, Hq=32, Hkv=32, S=4096, D=128, causal=True, window=None, softcap=None),
    "cfg3": dict(B=2, Hq=32, Hkv=8, S=8192, D=128, causal=True, window=4096, softcap=50.0),
    # the MLA module's attention call: q / k of 128 + 64 rope dims, V at its 128 dims
    # (taken as zero-padded to 192, as the reference pads it; no work on the pad)
    "cfg5": dict(B=2, Hq=32, Hkv=32, S=4096, D=192, Dv=128, causal=True, window=None,
                 softcap=None),
}


def n_valid_pairs(S_q: int, S_kv: int, causal: bool, window, q_offset: int = 0) -> int:
    """Exact count of visible (q, k) pairs per (batch, head)."""
    total = 0
    for i in range(S_q):
        row = q_offset + i
        hi = min(S_kv - 1, row) if causal else S_kv - 1
        lo = max(0, row - window + 1) if window else 0
        total += max(0, hi - lo + 1)
    return total


def n_valid_pairs_fast(S: int, causal: bool, window) -> int:
    if not causal and not window:
        return S * S
    if causal and not window:
        return S * (S + 1) // 2
    return n_valid_pairs(S, S, causal, window)


def time_steps(fn, steps: int, warmup: int):
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fn()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / steps, wall * 1e3 / steps


def time_graph(fn, steps: int, warmup: int):
    """`steps` calls of fn captured into one HIP graph (torch.cuda.CUDAGraph) and timed as
    one replay: the serving-loop form of a short step, with no host launch gaps between
    steps. The calls must only launch kernels on torch's current stream."""
    import torch

    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(steps):
            fn()
    graph.replay()  # first replay uploads the graph
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    graph.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return start.elapsed_time(stop) / steps, wall * 1e3 / steps


def blas_threads() -> int:
    try:
        from threadpoolctl import threadpool_info

        n = [p["num_threads"] for p in threadpool_info() if p.get("user_api") == "blas"]
        return max(n) if n else 1
    except Exception:  # pragma: no cover - informational only
        return 1


PROFILES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles")


def profiled_traffic(summary: str, key: str = "traffic_bytes_per_launch"):
    """HBM bytes per launch of a kernel as measured by the committed rocprofv3 PMC
    summary ``profiles/<summary>`` (line ``<key>: N``: FETCH_SIZE and WRITE_SIZE per
    dispatch, each scaled by its calibration factor), or None."""
    try:
        with open(os.path.join(PROFILES, summary)) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return int(line.split(":", 1)[1].strip())
    except OSError:
        return None
    return None


def cpu_threads() -> dict:
    """Host thread counts reported beside every CPU figure."""
    import torch

    return {"os_cpu_count": os.cpu_count(), "torch_num_threads": torch.get_num_threads(),
            "blas_threads": blas_threads()}


def cpu_baseline_prefill(cfg: dict, q, k, v, budget_s: float) -> dict:
    """Oracle restatement of the reference CPU path (numpy, the reference dispatcher's
    block size) over whole (batch 0, head h) slices, h = 0, 1, ... until the time
    budget is spent; FLOPs counted exactly for the heads processed."""
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import reference_forward as rf

    S, D, ratio = cfg["S"], cfg["D"], cfg["Hq"] // cfg["Hkv"]
    Dv = cfg.get("Dv", D)
    bs = rf.auto_select_block_size(S, S, D)
    pairs = n_valid_pairs_fast(S, cfg["causal"], cfg["window"])
    secs, heads = 0.0, 0
    while heads < cfg["Hq"] and (heads == 0 or secs < budget_s):
        h = heads
        qh = q[0:1, h:h + 1].float().numpy()
        kh = k[0:1, h // ratio:h // ratio + 1].float().numpy()
        vh = v[0:1, h // ratio:h // ratio + 1].float()
        vh = torch.nn.functional.pad(vh, (0, D - Dv)).numpy()  # the reference's padded V
        t = time.perf_counter()
        rf.flash_attn_cpu_forward(qh, kh, vh, scale=1 / math.sqrt(D), causal=cfg["causal"],
                                  block_q=bs, block_kv=bs, softcap=cfg["softcap"],
                                  sliding_window=cfg["window"])
        secs += time.perf_counter() - t
        heads += 1
    flops = 2.0 * (D + Dv) * pairs * heads
    return {
        "value": flops / secs / 1e12,
        "unit": "TFLOP/s",
        "cores": blas_threads(),
        **cpu_threads(),
        "kind": "port",
        "sample": (f"oracle/reference_forward.flash_attn_cpu_forward (numpy fp32, the "
                   f"reference CPU algorithm) on batch 0, heads 0..{heads - 1} "
                   f"({heads}/{cfg['B'] * cfg['Hq']} of the batch), all {S} rows, block {bs} "
                   f"as the reference dispatcher picks; {secs:.1f} s for {flops:.3e} FLOP; "
                   f"os.cpu_count()={os.cpu_count()}"),
    }


def bench_prefill(name: str, steps: int, warmup: int, cpu_budget: float):
    import torch

    import fastest_flash_attention_amd as ffa

    cfg = PREFILL[name]
    B, Hq, Hkv, S, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["S"], cfg["D"]
    Dv = cfg.get("Dv", D)
    g = torch.Generator().manual_seed(0)
    # BASELINE recipe: fp32 randn on the host in the order q, k, v, cast to bf16 on the
    # host (identical bits on both sides), then moved to HBM.
    q = torch.randn(B, Hq, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, Dv, generator=g).to(torch.bfloat16)
    qd, kd, vd = q.cuda(), k.cuda(), v.cuda()
    kw = dict(causal=cfg["causal"], sliding_window=cfg["window"], softcap=cfg["softcap"])
    if Hq != Hkv:
        kw["num_kv_heads"] = Hkv

    def step():
        ffa.fastest_flash_attn_forward(qd, kd, vd, **kw)

    ms_event, ms_wall = time_steps(step, steps, warmup)
    pairs = n_valid_pairs_fast(S, cfg["causal"], cfg["window"])
    flops = 2.0 * B * Hq * (D + Dv) * pairs
    achieved = flops / (ms_event * 1e-3) / 1e12
    cpu = cpu_baseline_prefill(cfg, q, k, v, cpu_budget) if cpu_budget > 0 else None
    return {
        "ms_per_step": ms_wall,
        "kernel_ms": ms_event,
        "value": flops / (ms_wall * 1e-3) / 1e12,
        "flops": flops,
        "roofline": {
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_BF16_TFLOPS,
            "traffic": profiled_traffic(f"prefill_kernel_{name}.md"),
        },
        "config": {"workload": f"{name}_prefill", "batch": B, "heads_q": Hq, "heads_kv": Hkv,
                   "seq_len": S, "head_dim": D, "v_head_dim": Dv, "causal": cfg["causal"],
                   "sliding_window": cfg["window"], "softcap": cfg["softcap"],
                   "n_valid_pairs_per_head": pairs},
        "cpu_baseline": cpu,
    }


def bench_backward(steps: int, warmup: int):
    """Attention backward (fastest_flash_attn_backward: preprocess, dK/dV and dQ kernels)
    at the north-star shape, from the forward's O and LSE. Algorithmic FLOPs =
    10 * D per visible (q, k) pair (S, dP, dV, dQ, dK: five products); the kernels
    execute 14 * D (S and dP are recomputed by the dQ kernel instead of accumulating dQ
    with atomics)."""
    import torch

    import fastest_flash_attention_amd as ffa
    from fastest_flash_attention_amd.ops.attention_backward import fastest_flash_attn_backward

    cfg = PREFILL["north_star"]
    B, H, S, D = cfg["B"], cfg["Hq"], cfg["S"], cfg["D"]
    g = torch.Generator().manual_seed(0)
    q, k, v, do = (torch.randn(B, H, S, D, generator=g).to(torch.bfloat16).cuda()
                   for _ in range(4))
    o, lse = ffa.fastest_flash_attn_forward(q, k, v, causal=True, return_lse=True)

    def step():
        fastest_flash_attn_backward(do, q, k, v, o, lse, causal=True)

    ms_event, ms_wall = time_steps(step, steps, warmup)
    pairs = n_valid_pairs_fast(S, True, None)
    flops = 10.0 * B * H * D * pairs
    achieved = flops / (ms_event * 1e-3) / 1e12
    return {
        "metric": "attention backward TFLOP/s (10 * D per visible pair)",
        "value": flops / (ms_wall * 1e-3) / 1e12,
        "unit": "TFLOP/s",
        "ms_per_step": ms_wall,
        "kernel_ms": ms_event,
        "flops": flops,
        "roofline": {"bound": "mfma", "achieved": achieved, "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": achieved / PEAK_BF16_TFLOPS,
                     # the whole step: preprocess + dK/dV + dQ kernels
                     "traffic": profiled_traffic("bwd_dkdv_kernel_north_star.md",
                                                 "step_traffic_bytes")},
        "config": {"workload": "north_star_backward", "batch": B, "heads": H, "seq_len": S,
                   "head_dim": D, "causal": True},
    }


def cpu_baseline_decode(k_pages, v_pages, q, bt, lens, budget_s: float) -> dict:
    """The reference CPU decode path on sequences 0, 1, ... of the same seeded cfg4
    batch until the time budget is spent: ``get_kv`` (the per-page copy loop,
    oracle/paged.gather_sequence, moving the pool's 16-bit words as they are) and the
    one-token attention over the gathered K/V (bf16 -> fp32, repeat_kv, the reference
    CPU kernel with the query at position L - 1: oracle/reference_forward). Timed
    separately and together; GB/s on the same algorithmic bytes as the GPU leg."""
    import numpy as np
    import torch

    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from oracle import paged as opaged
    from oracle import reference_forward as rf

    B, Hq, D = q.shape
    Hkv, P = k_pages.shape[1], k_pages.shape[2]
    # the pools move to host memory once (16-bit words, as the reference's bf16 pool
    # would hold them); the copy is not timed
    kh = k_pages.view(torch.int16).cpu().numpy()
    vh = v_pages.view(torch.int16).cpu().numpy()
    qh = q.float().cpu().numpy()
    bth = bt.cpu().numpy()
    lens_h = [int(x) for x in lens.cpu()]

    def f32(words):  # exact bf16 -> fp32 widening of the gathered words
        return (words.astype(np.uint16).astype(np.uint32) << 16).view(np.float32)

    t_gather = t_attn = 0.0
    nbytes = 0
    n = 0
    bs = None
    while n < B and (n == 0 or t_gather + t_attn < budget_s):
        L = lens_h[n]
        pages = bth[n, :(L + P - 1) // P].tolist()
        t = time.perf_counter()
        kb, vb = opaged.gather_sequence(kh, vh, pages, L)
        t_gather += time.perf_counter() - t
        t = time.perf_counter()
        kf = rf.repeat_kv(f32(kb)[None], Hq, Hkv)
        vf = rf.repeat_kv(f32(vb)[None], Hq, Hkv)
        bs = rf.auto_select_block_size(1, L, D)
        rf.flash_attn_cpu_forward(qh[n][None, :, None, :], kf, vf, scale=1 / math.sqrt(D),
                                  causal=True, block_q=bs, block_kv=bs, q_offset=L - 1,
                                  return_lse=True)
        t_attn += time.perf_counter() - t
        nbytes += L * Hkv * D * 2 * 2 + 2 * Hq * D * 2 + Hq * 4 + len(pages) * 4 + 4
        n += 1
    total = t_gather + t_attn
    return {
        "value": nbytes / total / 1e9,
        "unit": "GB/s",
        "cores": 1,
        **cpu_threads(),
        "kind": "port",
        "gather_GBps": nbytes / t_gather / 1e9,
        "attention_GBps": nbytes / t_attn / 1e9,
        "gather_s": t_gather,
        "attention_s": t_attn,
        "sample": (f"sequences 0..{n - 1} of the {B}-sequence cfg4 batch ({sum(lens_h[:n])} "
                   f"of {sum(lens_h)} tokens, {nbytes:.3e} B): oracle/paged.gather_sequence "
                   f"(the reference get_kv page loop, numpy) then the one-token reference "
                   f"CPU attention (oracle/reference_forward, fp32, block {bs} as the "
                   f"reference dispatcher picks for the last sequence); gather "
                   f"{t_gather:.2f} s + attention {t_attn:.2f} s; numpy copies and "
                   f"per-tile products of one query row run on one thread"),
    }


def bench_decode(steps: int, warmup: int, cpu_budget: float = 0.0):
    import torch

    import fastest_flash_attention_amd as ffa

    B, Hq, Hkv, D, P = 64, 32, 8, 128, 16
    g = torch.Generator().manual_seed(0)
    lens = torch.randint(512, 32769, (B,), generator=g)
    pages = (lens + P - 1) // P
    total = int(pages.sum())
    perm = torch.randperm(total, generator=g).to(torch.int32)
    bt = torch.zeros(B, int(pages.max()), dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(pages[b])
        bt[b, :n] = perm[off:off + n]
        off += n
    # the 2 x 2.2 GB pools are drawn on the device (seeded) to keep host time short
    gd = torch.Generator(device="cuda").manual_seed(0)
    k_pages = torch.randn(total, Hkv, P, D, generator=gd, device="cuda").to(torch.bfloat16)
    v_pages = torch.randn(total, Hkv, P, D, generator=gd, device="cuda").to(torch.bfloat16)
    q = torch.randn(B, Hq, D, generator=gd, device="cuda").to(torch.bfloat16)
    btd, lensd = bt.cuda(), lens.to(torch.int32).cuda()
    max_len = int(lens.max())

    def step():
        ffa.fastest_flash_paged_decode(q, k_pages, v_pages, btd, lensd, return_lse=True,
                                       max_context_len=max_len)

    ms_event, ms_wall = time_steps(step, steps, warmup)
    kv_bytes = int(lens.sum()) * Hkv * D * 2 * 2
    nbytes = kv_bytes + 2 * B * Hq * D * 2 + B * Hq * 4 + int(pages.sum()) * 4 + B * 4
    achieved = nbytes / (ms_event * 1e-3) / 1e9
    return {
        "metric": "paged-decode HBM GB/s",
        "value": nbytes / (ms_wall * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": ms_wall,
        "kernel_ms": ms_event,
        "bytes": nbytes,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS,
                     "traffic": profiled_traffic("decode_split_kernel_cfg4.md")},
        "config": {"workload": "cfg4_paged_decode", "batch": B, "heads_q": Hq, "heads_kv": Hkv,
                   "head_dim": D, "page_size": P, "context_lens": "U[512, 32768] seed 0",
                   "total_tokens": int(lens.sum())},
        "cpu_baseline": (cpu_baseline_decode(k_pages, v_pages, q, btd, lensd, cpu_budget)
                         if cpu_budget > 0 else None),
    }


def bench_mla_decode(steps: int, warmup: int):
    """cfg5 decode: MLA layer (32 heads, latent 512, rope 64), batch 32 at context 4096,
    over the compressed latent cache (ffa_mla_decode_fwd). Bytes = the latent rows of
    exactly context_len tokens + absorbed q + latent o + lse + block tables."""
    import torch

    B, H, L, lat, R, P = 32, 32, 4096, 512, 64, 64
    gd = torch.Generator(device="cuda").manual_seed(0)
    n_pages = B * L // P
    pool = torch.randn(n_pages, P, lat + R, generator=gd, device="cuda").to(torch.bfloat16)
    perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(0)).to(torch.int32)
    bt = perm.view(B, L // P).contiguous().cuda()
    lens = torch.full((B,), L, dtype=torch.int32, device="cuda")
    q = torch.randn(B, H, lat + R, generator=gd, device="cuda").to(torch.bfloat16)
    scale = 1.0 / math.sqrt(128 + R)  # the module's 1/sqrt(head_dim + rope_dim)
    # a serving loop keeps its split-K workspace (caller-owned) across steps
    from fastest_flash_attention_amd.ops.mla_decode import (_auto_mla_tokens_per_split,
                                                            mla_decode_workspace_bytes)
    tps = _auto_mla_tokens_per_split(B, (H + 31) // 32, L)
    ws = torch.empty(mla_decode_workspace_bytes(B, H, lat, L, tps), dtype=torch.uint8,
                     device="cuda")

    # the call is resolved once and launched every step, as a serving loop would: the
    # ~30 us of Python argument handling per call would otherwise exceed the kernel time
    from fastest_flash_attention_amd.ops.mla_decode import launch_mla_decode, prepare_mla_decode
    call = prepare_mla_decode(q, pool, bt, lens, dim_v=lat, scale=scale, return_lse=True,
                              max_context_len=L, tokens_per_split=tps, workspace=ws)

    def step():
        launch_mla_decode(call)

    # A 36 us step is short enough for host launch gaps to show between eagerly launched
    # steps; a serving loop replays its decode step as a captured graph, and so does this
    # leg (the eager per-call figure is reported beside it).
    ms_eager, _ = time_steps(step, steps, warmup)
    ms_event, ms_wall = time_graph(step, steps, warmup)
    nbytes = B * L * (lat + R) * 2 + B * H * (lat + R) * 2 + B * H * lat * 2 + B * H * 4 + \
        n_pages * 4
    achieved = nbytes / (ms_event * 1e-3) / 1e9
    return {
        "metric": "MLA latent-cache decode HBM GB/s",
        "value": nbytes / (ms_wall * 1e-3) / 1e9,
        "unit": "GB/s",
        "ms_per_step": ms_wall,
        "kernel_ms": ms_event,
        "eager_kernel_ms": ms_eager,
        "timing": "HIP graph of the timed steps, one replay",
        "bytes": nbytes,
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": achieved / PEAK_HBM_GBS,
                     "traffic": profiled_traffic("mla_decode_split8_kernel_cfg5.md")},
        "config": {"workload": "cfg5_mla_decode", "batch": B, "heads_q": H, "latent_dim": lat,
                   "rope_dim": R, "context_len": L, "page_size": P},
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    # 50 untimed steps (~0.1 s of prefill work at the north-star shape): the MI355X clock
    # needs that long under load to settle, and a cold start reads ~5 % low.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="north_star", choices=sorted(PREFILL))
    ap.add_argument("--no-decode", action="store_true")
    ap.add_argument("--no-backward", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0,
                    help="time budget of the prefill CPU baseline sample (0 disables it)")
    ap.add_argument("--cpu-decode-seconds", type=float, default=6.0,
                    help="time budget of the decode CPU baseline sample (0 disables it)")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="run one fp32 elementwise kernel over this many MiB first (a "
                         "known-size kernel for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU; --gpus must be 1 (the hot path "
              "would shard by (batch, head) with no exchange; no multi-GPU figure is "
              "produced)", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    torch.cuda.set_device(0)
    if args.calibrate_copy_mib > 0:
        # one elementwise kernel reading and writing exactly N MiB (fp32 negate)
        src = torch.ones((args.calibrate_copy_mib << 20) // 4, dtype=torch.float32,
                         device="cuda")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        torch.neg(src, out=dst)
        torch.cuda.synchronize()
        del src, dst
    # The headline prefill leg runs last: the other legs bring the GPU out of idle first
    # (its clock ramps over ~0.1-0.3 s of load), so the headline's own W warm-up steps
    # are not also spent on the ramp.
    dec = None if args.no_decode else bench_decode(args.steps, args.warmup,
                                                   args.cpu_decode_seconds)
    mla = None if args.no_decode else bench_mla_decode(args.steps, args.warmup)
    bwd = None if args.no_backward else bench_backward(args.steps, args.warmup)
    pre = bench_prefill(args.workload, args.steps, args.warmup, args.cpu_seconds)
    line = {
        "metric": "prefill attn TFLOP/s (% bf16 MFMA peak); paged-decode HBM GB/s (% peak)",
        "value": pre["value"],
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1), no dataset)",
        "config": pre["config"],
        "roofline": pre["roofline"],
        "cpu_baseline": pre["cpu_baseline"],
        "decode": dec,
        "mla_decode": mla,
        "backward": bwd,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
