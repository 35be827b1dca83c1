"""Benchmark of the pufferlean training-step hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu-baseline]

Prints ONE JSON line. Workloads (synthetic, seeded, inputs resident in HBM before timing):
  gemm    policy GEMMs M=16384 (256 segments x 64 steps), K=N=512: forward X.W^T, dgrad dY.W,
          wgrad dY^T.X, bf16 MFMA with fp32 accumulate (fp32 storage in, fp32 out)
  vtrace  V-trace reverse scan, fp32 time-major, 4096 segments x horizon 64, replicated 64x in
          one launch so the working set (403 MB) exceeds the 256 MB Infinity Cache
A "step" is one pass of the workload's hot path over one batch. Timed with HIP events on the
stream the kernels run on.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
F32_PEAK_TFLOPS = 157.3
METRIC = "PPO update samples/sec @ hidden 512 (1 GPU); GEMM/NS MFMA util %; V-trace GB/s"


def _events():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_loop(fn, steps, warmup):
    """Average ms per call of fn() over `steps` calls after `warmup`, bracketed by syncs."""
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    s, e = _events()
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


# ------------------------------------------------------------------------------------------------
def bench_gemm(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    M, K, N = 16384, 512, 512
    X = torch.from_numpy(rng.normal(rng.seed_for(2, 0), M * K).astype(np.float32)).cuda().view(M, K)
    W = torch.from_numpy((rng.normal(rng.seed_for(2, 1), N * K) / np.sqrt(512)).astype(np.float32)).cuda().view(N, K)
    dY = torch.from_numpy(rng.normal(rng.seed_for(2, 2), M * N).astype(np.float32)).cuda().view(M, N)
    Xb, Wb, dYb = X.bfloat16(), W.bfloat16(), dY.bfloat16()
    Y = torch.empty(M, N, device="cuda")
    Yb = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    dX = torch.empty(M, K, device="cuda")
    dW = torch.empty(N, K, device="cuda")
    flops = 2.0 * M * N * K
    out = {}
    forms = {
        "nn_fwd_f32io": lambda: D.gemm(X, W, trans_b=True, out=Y),
        "nt_dgrad_f32io": lambda: D.gemm(dY, W, out=dX),
        "tn_wgrad_f32io": lambda: D.gemm(dY, X, trans_a=True, out=dW),
        "nn_fwd_bf16io": lambda: D.gemm(Xb, Wb, trans_b=True, out=Yb),
        "nt_dgrad_bf16in": lambda: D.gemm(dYb, Wb, out=dX),
        "tn_wgrad_bf16in": lambda: D.gemm(dYb, Xb, trans_a=True, out=dW),
        "nn_fwd_f32math": lambda: D.gemm(X, W, trans_b=True, out=Y, math="f32"),
    }
    for name, fn in forms.items():
        ms = time_loop(fn, steps, warmup)
        peak = F32_PEAK_TFLOPS if name.endswith("f32math") else BF16_PEAK_TFLOPS
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac": round(tf / peak, 4)}
    return out


def bench_vtrace(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    B, T, R = 4096, 64, 64
    n = B * T
    cols = []
    for i in range(4):
        base = [rng.normal(rng.seed_for(4, 1), n), rng.normal(rng.seed_for(4, 2), n),
                rng.bernoulli(rng.seed_for(4, 3), n, 0.01),
                rng.normal(rng.seed_for(4, 4), n, 0.0, 0.1)][i]
        t = torch.from_numpy(base.astype(np.float32)).cuda().view(T, B)
        cols.append(t.repeat(1, R).contiguous())
    val, rew, done, logr = cols
    boot = torch.from_numpy(rng.normal(rng.seed_for(4, 5), B).astype(np.float32)).cuda().repeat(R).contiguous()
    adv = torch.empty_like(val)
    tgt = torch.empty_like(val)
    fn = lambda: D.vtrace(rew, val, done, logr, boot, variant=1, time_major=True, rho_is_log=True,
                          out_adv=adv, out_tgt=tgt)
    ms = time_loop(fn, steps, warmup)
    bytes_ = 24.0 * n * R + 4.0 * B * R
    gbs = bytes_ / (ms * 1e-3) / 1e9
    # single (non-replicated) call latency
    v1, r1, d1, l1 = (c[:, :B].contiguous() for c in cols)
    b1 = boot[:B].contiguous()
    ms1 = time_loop(lambda: D.vtrace(r1, v1, d1, l1, b1, variant=1, time_major=True,
                                     rho_is_log=True), steps, warmup)
    return {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": bytes_, "single_call_us": round(ms1 * 1e3, 2)}


# ------------------------------------------------------------------------------------------------
def cpu_baseline_gemm():
    """The oracle's OpenMP f64 GEMM (forward form) on a 2048-row sample of the 16384x512x512 forward."""
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    from pufferlean_amd import rng
    cores = os.cpu_count() or 1
    cores = min(cores, 16)
    rows, K, N = 2048, 512, 512
    X = rng.normal(1, rows * K).reshape(rows, K)
    W = rng.normal(2, N * K).reshape(N, K)
    t0 = time.perf_counter()
    reps = 0
    while True:
        O.gemm(0, 1, X, W, rows, N, K, threads=cores)
        reps += 1
        if time.perf_counter() - t0 > 10.0:
            break
    dt = (time.perf_counter() - t0) / reps
    return {"value": round(2.0 * rows * N * K / dt / 1e9, 2), "unit": "GFLOP/s (f64)", "cores": cores,
            "kind": "port", "sample": f"forward GEMM {rows}x{K}x{N} (of 16384 rows), {reps} reps"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the path would shard segments/rows across GPUs; see DESIGN.md)", file=sys.stderr)
        return 2
    import torch
    from pufferlean_amd import _lib
    _lib.lib()
    assert torch.cuda.is_available(), "bench needs a GPU"
    res = {}
    if args.workload in ("all", "gemm"):
        res["gemm"] = bench_gemm(args.steps, args.warmup)
    if args.workload in ("all", "vtrace"):
        res["vtrace"] = bench_vtrace(args.steps, args.warmup)
    g = res.get("gemm", {})
    head = g.get("nn_fwd_bf16io")
    line = {
        "metric": METRIC,
        "value": head["tflops"] if head else None,
        "unit": "TFLOP/s (policy GEMM forward, bf16 MFMA)",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(head["us"] / 1e3, 4) if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded splitmix64)",
        "config": {"workload": "policy GEMM 16384x512x512 (configs: gemm, vtrace)"},
        "roofline": ({"bound": "mfma", "achieved": head["tflops"], "peak": BF16_PEAK_TFLOPS,
                      "unit": "TFLOP/s", "frac": head["frac"], "traffic": None} if head else None),
        "components": res,
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline_gemm()
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
