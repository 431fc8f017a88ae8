"""Benchmark of the hot path on one MI355X: prints ONE JSON line (rank 0).

Metric: "µs/layer + achieved HBM GB/s (%roofline): decode attn b8@4k, W4 GEMV M=1".
``value`` is the W4 GEMV at M=1 on configs[1] (K=4096, N=28672) in GB/s of algorithmic bytes;
the decode-attention b8@4k leg, the other M values and prefill are reported beside it.

A "step" is one launch of the kernel over one batch of synthetic input.  Inputs are resident in
HBM before the timed region and rotate over enough copies (> 2x the 256 MB Infinity Cache) that
every step reads its bytes from HBM.  Timing: HIP events recorded on the stream the kernels run
on (torch's current stream), ``--warmup`` untimed steps, then exactly ``--steps`` timed steps.
The CPU baseline is the oracle's torch-CPU fp32 dequant path on a bounded sample (rank 0, N=1).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import statistics
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "gfx1201-tuning-log_amd"))
sys.path.insert(0, REPO)

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, 8 TB/s
ROTATE_BYTES = 1 << 30         # >= 4x the 256 MB MALL


def w4_bytes(N: int, K: int, M: int) -> int:
    """Algorithmic bytes of one matvec: codes + scales + x + out."""
    return N * K // 2 + N * K // 32 + 2 * M * K + 2 * M * N


def time_launches(launch, n_sets: int, steps: int, warmup: int):
    """Run ``launch(i % n_sets)`` warmup + steps times; return (avg ms per step, per-step ms list)."""
    import torch
    for i in range(warmup):
        launch(i % n_sets)
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
    ev[0].record()
    for i in range(steps):
        launch(i % n_sets)
        ev[i + 1].record()
    torch.cuda.synchronize()
    per = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps)]
    total = ev[0].elapsed_time(ev[steps])
    return total / steps, per


def bench_w4(N: int, K: int, M: int, steps: int, warmup: int):
    import torch
    from fp8kv_amd import ops
    dev = torch.device("cuda")
    per_set = N * K // 2 + N * K // 32
    n_sets = max(4, -(-ROTATE_BYTES // per_set))
    g = torch.Generator(device=dev).manual_seed(1234 + M)
    Ws = [torch.randint(0, 256, (N, K // 2), dtype=torch.uint8, device=dev, generator=g)
          for _ in range(n_sets)]
    Ss = [torch.randint(119, 124, (N, K // 32), dtype=torch.uint8, device=dev, generator=g)
          for _ in range(n_sets)]
    X = torch.randn(M, K, device=dev, generator=g).to(torch.bfloat16)
    Y = torch.empty(M, N, dtype=torch.bfloat16, device=dev)

    def launch(i):
        ops.h4mv(X, Ws[i], Ss[i], out=Y)

    ms, per = time_launches(launch, n_sets, steps, warmup)
    b = w4_bytes(N, K, M)
    del Ws, Ss
    torch.cuda.empty_cache()
    return {"us": ms * 1e3, "us_median_event": statistics.median(per) * 1e3,
            "bytes": b, "gbs": b / (ms * 1e-3) / 1e9, "rotation_sets": n_sets}


def cpu_baseline_w4(N: int, K: int, budget_s: float = 15.0):
    """Oracle-style torch CPU fp32 dequant + GEMV at M=1 on the full cfg1 shape."""
    import torch
    from fp8kv_amd import workloads
    from oracle.formats import E2M1, E8M0
    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    case = workloads.w4_case(N=N, K=K, M=1, seed=5)
    lut = torch.tensor(E2M1, dtype=torch.float32)
    e8 = torch.tensor(E8M0, dtype=torch.float32)
    W, St, x = case["W"], case["St"], case["X"].float()

    def once():
        w = torch.empty(N, K, dtype=torch.float32)
        w[:, 0::2] = lut[(W & 15).long()]
        w[:, 1::2] = lut[(W >> 4).long()]
        w = (w.view(N, K // 32, 32) * e8[St.long()][:, :, None]).view(N, K)
        return x @ w.t()

    for _ in range(3):
        once()
    times = []
    t_start = time.perf_counter()
    while len(times) < 10 or (time.perf_counter() - t_start < budget_s and len(times) < 50):
        t0 = time.perf_counter()
        once()
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    med = statistics.median(times)
    return {"value": w4_bytes(N, K, 1) / med / 1e9, "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"full cfg1 (N={N}, K={K}, M=1) torch-CPU fp32 dequant+GEMV, median of "
                      f"{len(times)} after 3 warm-ups ({med * 1e3:.1f} ms/call)",
            "cpu_model": platform.processor() or platform.machine()}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU: every box here has one GPU; "
                                   "run with --gpus 1 (multi-GPU sharding is described in "
                                   "DESIGN.md, not benchmarked)"}))
        sys.exit(2)

    import torch
    assert torch.cuda.is_available(), "bench.py needs a GPU"
    N, K = 28672, 4096
    m1 = bench_w4(N, K, 1, args.steps, args.warmup)
    m4 = bench_w4(N, K, 4, args.steps, args.warmup)
    m8 = bench_w4(N, K, 8, args.steps, args.warmup)
    cpu = None if args.no_cpu_baseline else cpu_baseline_w4(N, K)
    line = {
        "metric": "µs/layer + achieved HBM GB/s (%roofline): decode attn b8@4k, W4 GEMV M=1",
        "value": round(m1["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(m1["us"] / 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "e2m1xbf16->f32",
        "data": "synthetic (seeded random codes/scales/activations, rotated over >1 GB)",
        "config": {"workload": "configs[1] MXFP4 W4A16 matvec K=4096 N=28672 M=1",
                   "rotation_sets": m1["rotation_sets"]},
        "roofline": {"bound": "hbm", "achieved": round(m1["gbs"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(m1["gbs"] / HBM_PEAK_GBS, 4),
                     "traffic": None},
        "cpu_baseline": cpu,
        "legs": {
            "w4_gemv_M1": {"us": round(m1["us"], 2), "us_median": round(m1["us_median_event"], 2),
                           "GBps": round(m1["gbs"], 1), "frac": round(m1["gbs"] / HBM_PEAK_GBS, 4)},
            "w4_gemv_M4": {"us": round(m4["us"], 2), "GBps": round(m4["gbs"], 1),
                           "frac": round(m4["gbs"] / HBM_PEAK_GBS, 4)},
            "w4_gemv_M8": {"us": round(m8["us"], 2), "GBps": round(m8["gbs"], 1),
                           "frac": round(m8["gbs"] / HBM_PEAK_GBS, 4)},
        },
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
