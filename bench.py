"""Benchmark of the pufferlean training-step hot path on one MI355X.

python bench.py [--gpus 1] [--steps K] [--warmup W] [--only NAME] [--no-cpu-baseline] [--eager]

Prints ONE JSON line. The headline workload (value) is the full PPO+Muon minibatch step of a
2-layer MinGRU policy at hidden 512: obs 128 -> encoder 512 -> 2 MinGRU layers of 512 -> 16-way
categorical head + value head, 4096 segments x horizon 64 (262,144 rows), V-trace -> advantage
normalisation -> forward -> clipped PPO loss (clip 0.2, vf 0.5, ent 0.01) -> backward -> grad-norm
clip -> Muon (5 constant-coefficient Newton-Schulz steps) on every matrix, bias steps on biases.
fp32 master weights, bf16 activations and bf16 MFMA GEMMs. A "step" is one such minibatch update,
captured once into a HIP graph and replayed (--eager: launched directly).

Components, each on its own synthetic seeded inputs already resident in HBM:
  gemm    policy GEMMs M=16384, K=N=512 in the three forms (forward X.W^T, dgrad dY.W, wgrad dY^T.X)
  ns      Newton-Schulz batch: 4 x (512x512) + 2 x (512x1024), 5 steps, constant coefficients
  vtrace  V-trace, fp32 time-major, 4096 segments x 64, replicated 64x in one launch (403 MB)
  rollout one rollout timestep of the headline policy over 4096 envs (MinGRU step + categorical
          draw), bf16 and fp32 MFMA products
  replay  prioritised replay between V-trace and the BPTT on 4096 segments x 64 with 4096 draws:
          segment |adv| sums, sampler, minibatch gather (+ normalisation), value/ratio iterate, in
          the fp32 time-major layout and in the reference's f64 segment-major layout
  cartpole the CartPole-sized PPO+Muon update: 1024 envs x 64 steps, MLP 4 -> 128 -> 128 -> (2 + 1),
          V-trace -> normalisation -> gradient -> Muon, fp32 and bf16 MFMA products
  heads   multi-discrete (heads 9 and 5, 262,144 rows) and Gaussian (4 dims, 131,072 rows) loss
          gradients with their dashboard losses, the two samplers over one step of 4096 / 2048
          agents, and the whole wide update (4 epochs, hidden 128) through its host-buffer entry
          (wall time, PCIe upload of the f64 columns included)
Component times are HIP-event times of a HIP graph holding `steps` launches (device time per launch,
no host launch path; "us_eager" is the same loop launched from Python). Events are recorded on the
stream the kernels run on.

CPU baselines (the oracle, on up to 16 host cores of the same box, in the same run): cpu_baseline is the
headline's (the MinGRU gradient over a sample of segments plus Muon); cpu_baselines holds one per config
(CartPole update, policy GEMMs, Newton-Schulz batch, V-trace), each the median of repeated runs.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
F32_PEAK_TFLOPS = 157.3
METRIC = "PPO update samples/sec @ hidden 512 (1 GPU); GEMM/NS MFMA util %; V-trace GB/s"

# the headline workload
B5, T5, D5, H5, L5, A5 = 4096, 64, 128, 512, 2, 16


def _ev():
    import torch
    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


# The GPU's clocks ramp up over the first tens of milliseconds of sustained work (a 0.5 ms GEMM runs
# about 20 % slower in its first ~60 launches of a process); warm-up therefore runs for at least this
# long, whatever the warm-up count, so the timed region measures steady state.
WARM_S = 0.25


def warm(fn, warmup, min_s=WARM_S):
    """Run fn() `warmup` times, then keep running it until `min_s` seconds of device work have passed."""
    import time
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < min_s:
        for _ in range(4):
            fn()
        torch.cuda.synchronize()


def time_loop(fn, steps, warmup):
    """Average ms per call of fn() over `steps` calls after the warm-up, bracketed by syncs."""
    import torch
    warm(fn, warmup)
    s, e = _ev()
    s.record()
    for _ in range(steps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / steps


def _t(x, dtype=None):
    import numpy as np
    import torch
    return torch.from_numpy(np.ascontiguousarray(x, dtype or np.float32)).cuda()


# ------------------------------------------------------------------------------------------------
def mingru_inputs(B, T, D, H, L, A, seed_base=5):
    """Seeded synthetic minibatch of the headline workload (time-major columns)."""
    import numpy as np
    from pufferlean_amd import rng
    s = lambda k: rng.seed_for(seed_base, k)
    n = B * T
    parts = [rng.normal(s(0), H * D) / np.sqrt(D), np.zeros(H)]
    for l in range(L):
        parts.append(rng.normal(s(1 + l), 3 * H * H) / np.sqrt(H))
    parts += [rng.normal(s(8), A * H) / np.sqrt(H), np.zeros(A), rng.normal(s(9), H) / np.sqrt(H),
              np.zeros(1)]
    params = np.concatenate(parts)
    cols = dict(
        obs=rng.normal(s(10), n * D),
        act=rng.randint(s(11), n, A).astype(np.int32),
        rew=rng.normal(s(12), n),
        done=rng.bernoulli(s(13), n, 0.01),
        logrho=rng.normal(s(14), n, 0.0, 0.1),
        val=rng.normal(s(15), n),
        boot=rng.normal(s(16), B),
        # behaviour log-probs of the (near-uniform) initial policy, perturbed
        old=np.log(1.0 / A) + rng.normal(s(17), n, 0.0, 0.05),
    )
    return params, cols


def bench_ppo_step(steps, warmup, eager=False):
    import numpy as np
    import torch
    from pufferlean_amd import device as D

    cfg = D.MinGRUConfig(B5, T5, D5, H5, L5, A5, lr=0.015, mu=0.95, max_grad_norm=0.5,
                         gscale=1.0 / (B5 * T5), vf_clip=0.0)
    params, cols = mingru_inputs(B5, T5, D5, H5, L5, A5)
    p = _t(params)
    mom = torch.zeros_like(p)
    g = torch.zeros_like(p)
    obs = _t(cols["obs"]).view(T5, B5, D5)
    act = _t(cols["act"], np.int32).view(T5, B5)
    old, val, rew, done, logrho = (_t(cols[k]).view(T5, B5) for k in ("old", "val", "rew", "done", "logrho"))
    boot = _t(cols["boot"])
    losses = torch.zeros(7, device="cuda", dtype=torch.float64)

    def step():
        D.mingru_step(cfg, p, mom, obs, act, old, val, rew, done, logrho, boot, G=g, losses=losses)

    for _ in range(max(warmup, 1)):
        step()
    torch.cuda.synchronize()
    graph = None
    if not eager:
        graph = torch.cuda.CUDAGraph()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        run = graph.replay
    else:
        run = step
    warm(run, 2)
    e0, e1 = _ev()
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    finite = bool(torch.isfinite(p).all().item())
    ns_valid = ns_ok()
    rows = B5 * T5
    out = {"ms": round(ms, 4), "samples_per_s": round(rows / (ms * 1e-3), 1), "rows": rows,
           "params": cfg.P, "graph": graph is not None, "finite": finite, "ns_ok": ns_valid,
           "losses": [round(float(x), 5) for x in losses.cpu().tolist()]}
    out["dominant_kernel"] = dominant_kernel()
    return out


DGRAD_SETS = 3  # operand sets the dominant-kernel loop rotates through (2.4 GB of dy: not cache-resident)


def dgrad_operands(sets=DGRAD_SETS):
    """The step's data-gradient product of one layer as the step runs it: dh_in = dy W_l + skip, with dy
    [262144 x 1536] bf16, the transposed weight copy W_l^T [512 x 1536] bf16 (an NT product over k = 1536)
    and the gate-skip term the top layer's backward scan writes, added by the AXPBY epilogue into dh_in
    [262144 x 512] bf16. `sets` independent operand sets, so a loop over them reads dy from HBM."""
    import torch
    rows = B5 * T5
    ops = []
    for _ in range(sets):
        dy = (torch.randn(rows, 3 * H5, device="cuda") * 0.1).bfloat16()
        wt = (torch.randn(H5, 3 * H5, device="cuda") / 39.2).bfloat16()
        skip = (torch.randn(rows, H5, device="cuda") * 0.1).bfloat16()
        out = torch.empty(rows, H5, device="cuda", dtype=torch.bfloat16)
        ops.append((dy, wt, skip, out))
    return ops


def dgrad_launch(op):
    from pufferlean_amd import _lib as L
    from pufferlean_amd import device as D
    dy, wt, skip, out = op
    D.gemm(dy, wt, trans_b=True, out=out, epilogue=L.PH_EPI_AXPBY, aux=skip, alpha=1.0, beta=1.0)


def dominant_kernel():
    """The data-gradient GEMM (the step's largest kernel family: two launches per step), timed with HIP
    events on the stream it runs on over 30 launches that rotate through three operand sets, after 0.25 s
    of warm-up launches."""
    import torch
    rows = B5 * T5
    ops = dgrad_operands()
    it = [0]

    def fn():
        dgrad_launch(ops[it[0] % len(ops)])
        it[0] += 1
    gms = time_loop(fn, 30, 6)
    flops = 2.0 * rows * H5 * 3 * H5
    tf = flops / (gms * 1e-3) / 1e12
    del ops
    torch.cuda.empty_cache()
    return {"name": "k_gemm_nt_dma (data gradient 262144x512x1536, bf16, AXPBY epilogue)", "us": round(gms * 1e3, 1),
            "tflops": round(tf, 1), "flops": flops,
            "hbm_bytes": 2.0 * (rows * 3 * H5 + H5 * 3 * H5 + 2 * rows * H5)}


def ns_ok():
    """False if a fused Newton-Schulz launch since the last check gave up a bounded wait or left a work
    queue without blocks on its XCD: its matrices, and every update that used them, are invalid. The
    library keeps that record on the device; reading it synchronises and clears it."""
    from pufferlean_amd import device as D
    try:
        D.ns_status()
        return True
    except Exception as e:  # noqa: BLE001 - the library's error text is the report
        print(f"# newton-schulz status: {e}", file=sys.stderr, flush=True)
        return False


def time_graph(fn, steps, warmup):
    """Average ms per call of fn() with `steps` calls captured in one HIP graph and replayed, so the
    figure is device time per call without the host launch path (kernel-scale components are shorter
    than a Python-level launch). fn must not allocate; the warm-up calls size the library's buffers."""
    import torch
    for _ in range(max(warmup, 1)):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(steps):
                fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    warm(g.replay, 1)
    a, b = _ev()
    a.record()
    g.replay()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / steps


def bench_gemm(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    M, K, N = 16384, 512, 512
    X = _t(rng.normal(rng.seed_for(2, 0), M * K)).view(M, K)
    W = _t(rng.normal(rng.seed_for(2, 1), N * K) / np.sqrt(512)).view(N, K)
    dY = _t(rng.normal(rng.seed_for(2, 2), M * N)).view(M, N)
    Xb, Wb, dYb = X.bfloat16(), W.bfloat16(), dY.bfloat16()
    Y = torch.empty(M, N, device="cuda")
    Yb = torch.empty(M, N, device="cuda", dtype=torch.bfloat16)
    dX = torch.empty(M, K, device="cuda")
    dXb = torch.empty(M, K, device="cuda", dtype=torch.bfloat16)
    dW = torch.empty(N, K, device="cuda")
    flops = 2.0 * M * N * K
    forms = {
        "fwd_bf16": (lambda: D.gemm(Xb, Wb, trans_b=True, out=Yb), BF16_PEAK_TFLOPS),
        "dgrad_bf16": (lambda: D.gemm(dYb, Wb, out=dXb), BF16_PEAK_TFLOPS),
        "wgrad_bf16": (lambda: D.gemm(dYb, Xb, trans_a=True, out=dW), BF16_PEAK_TFLOPS),
        "fwd_f32io_bf16math": (lambda: D.gemm(X, W, trans_b=True, out=Y), BF16_PEAK_TFLOPS),
        "dgrad_f32io_bf16math": (lambda: D.gemm(dY, W, out=dX), BF16_PEAK_TFLOPS),
        "wgrad_f32io_bf16math": (lambda: D.gemm(dY, X, trans_a=True, out=dW), BF16_PEAK_TFLOPS),
        "fwd_f32math": (lambda: D.gemm(X, W, trans_b=True, out=Y, math="f32"), F32_PEAK_TFLOPS),
    }
    out = {}
    for name, (fn, peak) in forms.items():
        ms = time_graph(fn, steps, warmup)
        ms_eager = time_loop(fn, steps, warmup)
        tf = flops / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 2), "tflops": round(tf, 1), "frac": round(tf / peak, 4),
                     "us_eager": round(ms_eager * 1e3, 2)}
    return out


def bench_ns(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    shapes = [(512, 512)] * 4 + [(512, 1024)] * 2
    mats = [_t(rng.normal(rng.seed_for(3, i), r * c, 0.0, 0.02)).view(r, c) for i, (r, c) in enumerate(shapes)]
    work = [m.clone() for m in mats]

    # the six matrices in one fused launch (ph_newton_schulz_batch)
    run = lambda: D.newton_schulz_batch(work, coeffs=D.CONST_COEFFS, math="bf16")
    ms = time_graph(run, max(steps // 5, 3), warmup)
    ms_eager = time_loop(run, max(steps // 5, 3), warmup)
    flops = sum(5 * (4 * min(r, c) ** 2 * max(r, c) + 2 * min(r, c) ** 3) for r, c in shapes)
    tf = flops / (ms * 1e-3) / 1e12
    return {"us": round(ms * 1e3, 1), "tflops": round(tf, 2), "frac": round(tf / BF16_PEAK_TFLOPS, 4),
            "flops": flops, "matrices": len(shapes), "us_eager": round(ms_eager * 1e3, 1), "ns_ok": ns_ok()}


def bench_vtrace(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    B, T, R = 4096, 64, 64
    n = B * T
    base = [rng.normal(rng.seed_for(4, 1), n), rng.normal(rng.seed_for(4, 2), n),
            rng.bernoulli(rng.seed_for(4, 3), n, 0.01), rng.normal(rng.seed_for(4, 4), n, 0.0, 0.1)]
    cols = [_t(x).view(T, B).repeat(1, R).contiguous() for x in base]
    val, rew, done, logr = cols
    boot = _t(rng.normal(rng.seed_for(4, 5), B)).repeat(R).contiguous()
    adv = torch.empty_like(val)
    tgt = torch.empty_like(val)
    fn = lambda: D.vtrace(rew, val, done, logr, boot, variant=1, time_major=True, rho_is_log=True,
                          out_adv=adv, out_tgt=tgt)
    ms = time_graph(fn, steps, warmup)
    bytes_ = 24.0 * n * R + 4.0 * B * R
    gbs = bytes_ / (ms * 1e-3) / 1e9
    v1, r1, d1, l1 = (c[:, :B].contiguous() for c in cols)
    b1 = boot[:B].contiguous()
    a1, t1 = torch.empty_like(v1), torch.empty_like(v1)
    ms1 = time_graph(lambda: D.vtrace(r1, v1, d1, l1, b1, variant=1, time_major=True, rho_is_log=True,
                                      out_adv=a1, out_tgt=t1), steps, warmup)
    return {"us": round(ms * 1e3, 2), "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
            "bytes": bytes_, "single_call_us": round(ms1 * 1e3, 2)}


# CartPole-sized update: 1024 envs x 64 steps, obs 4 -> 128 -> 128 -> (2 + 1)
CP_B, CP_T, CP_D, CP_H, CP_L, CP_A = 1024, 64, 4, 128, 2, 2


def cartpole_inputs(seed_base=1):
    """Seeded CartPole workload: weights N(0, 1/fan_in), zero biases, obs U[-1,1], actions uniform over 2,
    rewards 1, dones Bernoulli(0.02); the behaviour log-probs are filled in from the forward."""
    import numpy as np
    from pufferlean_amd import rng
    s = lambda k: rng.seed_for(seed_base, k)
    N = CP_B * CP_T
    parts = []
    for l in range(CP_L):
        fan = CP_D if l == 0 else CP_H
        parts += [rng.normal(s(l), CP_H * fan) / np.sqrt(fan), np.zeros(CP_H)]
    parts += [rng.normal(s(8), (CP_A + 1) * CP_H) / np.sqrt(CP_H), np.zeros(CP_A + 1)]
    return np.concatenate(parts), dict(obs=rng.randf(s(10), N * CP_D, -1.0, 1.0), act=rng.randint(s(11), N, CP_A),
                                       rew=np.ones(N), done=rng.bernoulli(s(12), N, 0.02),
                                       noise=rng.normal(s(13), N, 0.0, 0.05))


def bench_cartpole(steps, warmup):
    """The whole CartPole PPO update (forward, V-trace, advantage normalisation, PPO gradient, Muon on
    every matrix) through ph_mlp_update, graph-captured; samples/s = 65,536 rows / update time."""
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    params, c = cartpole_inputs()
    N = CP_B * CP_T
    out = {"rows": N, "envs": CP_B, "horizon": CP_T, "net": f"{CP_D}->{CP_H}x{CP_L}->{CP_A}+1"}
    flops_fwd = 2.0 * N * (CP_D * CP_H + (CP_L - 1) * CP_H * CP_H + CP_H * (CP_A + 1))
    # fp32 tier: fp32 products and fp32-MFMA Newton-Schulz; bf16 tier: bf16 products, and the three
    # matrices' Newton-Schulz in one fused bf16 launch ("bf16_ns_f32": the bf16 products with the fp32
    # Newton-Schulz)
    for name, math_, mm in (("f32", "f32", "f32"), ("bf16", "bf16", "bf16"), ("bf16_ns_f32", "bf16", "f32")):
        cfg = D.MLPConfig(N, CP_D, CP_H, CP_L, CP_A, math=math_, muon_math=mm)
        p0 = _t(params)
        obs = _t(c["obs"]).view(N, CP_D)
        act = _t(c["act"], np.int32)
        lg = D.mlp_forward(cfg, p0, obs)
        lp = torch.log_softmax(lg[:, :CP_A].double(), 1).gather(1, act.long().view(-1, 1)).view(-1)
        behav = (lp + _t(c["noise"], np.float64)).float()
        rew, done = _t(c["rew"]), _t(c["done"])
        p = p0.clone()
        mom = torch.zeros_like(p)
        G = torch.empty_like(p)
        ms = time_graph(lambda: D.mlp_update(cfg, CP_T, p, mom, obs, act, behav, rew, done, G=G), steps, warmup)
        tf = 3.0 * flops_fwd / (ms * 1e-3) / 1e12
        out[name] = {"us": round(ms * 1e3, 1), "samples_per_s": round(N / (ms * 1e-3), 1),
                     "gemm_tflops": round(tf, 2), "finite": bool(torch.isfinite(p).all().item()),
                     "ns_ok": ns_ok()}
    out["gemm_flops"] = 3.0 * flops_fwd
    return out


def bench_replay(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    N, T, Bd = B5, T5, B5
    n = N * T
    out = {}
    for name, dt, tm in (("f32_time_major", torch.float32, True), ("f64_segment_major", torch.float64, False)):
        esz = 4 if dt == torch.float32 else 8
        mk = lambda k, f=rng.normal: _t(f(rng.seed_for(6, k), n), np.float64).to(dt)
        adv, val, logp = mk(0), mk(1), mk(2)
        act = _t(rng.randint(rng.seed_for(6, 3), n, A5), np.float64).to(dt)
        term = _t(rng.bernoulli(rng.seed_for(6, 4), n, 0.01), np.float64).to(dt)
        ratio = torch.ones_like(val)
        cols = D.ReplayColumns(N, T, adv=adv, value=val, ratio=ratio, act=act, logp=logp, term=term,
                               time_major=tm)
        L1 = torch.empty(N, device="cuda", dtype=torch.float64)
        seg = torch.empty(Bd, device="cuda", dtype=torch.int32)
        mp = torch.empty(Bd, device="cuda", dtype=torch.float64)
        mb = torch.empty(6 * Bd * T, device="cuda", dtype=dt)
        newlp = _t(rng.normal(rng.seed_for(6, 5), Bd * T) - 2.0)
        newval = _t(rng.normal(rng.seed_for(6, 6), Bd * T))
        f_l1 = lambda: D.seg_l1(cols, out=L1)
        f_ps = lambda: D.prio_sample(L1, Bd, alpha=0.8, beta=0.2, rng_state=0x5EED, seg=seg, mbprio=mp)
        f_ga = lambda: D.mb_gather(cols, seg, mp, out=mb)
        f_it = lambda: D.mb_iterate(cols, seg, newlp, newval)

        def chain():
            f_l1(); f_ps(); f_ga(); f_it()
        f_l1(); f_ps()
        torch.cuda.synchronize()
        uniq = int(torch.unique(seg).numel())
        r = {}
        for k, fn in (("seg_l1", f_l1), ("prio_sample", f_ps), ("gather", f_ga), ("iterate", f_it),
                      ("chain", chain)):
            r[k + "_us"] = round(time_graph(fn, steps, warmup) * 1e3, 2)
        # algorithmic HBM bytes: gather reads 5 columns through the draws and writes 6, then the
        # normalisation reads and writes adv; the iterate reads new_logp/new_value of every draw and
        # logp of each distinct segment, and writes value/ratio of each distinct segment
        g_bytes = n * (11 * esz + 2 * esz) + Bd * (4 + 8)
        it_bytes = Bd * T * 8 + uniq * T * 3 * esz + Bd * 4
        r["gather_gbs"] = round(g_bytes / (r["gather_us"] * 1e-6) / 1e9, 1)
        r["gather_frac"] = round(r["gather_gbs"] / HBM_PEAK_GBS, 4)
        r["gather_bytes"] = g_bytes
        r["iterate_gbs"] = round(it_bytes / (r["iterate_us"] * 1e-6) / 1e9, 1)
        r["distinct_segments"] = uniq
        out[name] = r
    out["shape"] = {"segments": N, "horizon": T, "draws": Bd}
    return out


def bench_rollout(steps, warmup):
    import numpy as np
    import torch
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    N = B5
    params, _ = mingru_inputs(B5, 1, D5, H5, L5, A5)
    p = _t(params)
    obs = _t(rng.normal(rng.seed_for(7, 0), N * D5)).view(N, D5)
    state = torch.zeros(N, L5, H5, device="cuda")
    out = torch.empty(N, A5 + 1, device="cuda")
    act = torch.empty(N, device="cuda", dtype=torch.int32)
    lp = torch.empty(N, device="cuda")
    val = torch.empty(N, device="cuda")
    flops = 2.0 * N * (D5 * H5 + L5 * 3 * H5 * H5 + (A5 + 1) * H5)
    r = {"envs": N, "flops": flops}
    for name, prec, peak in (("bf16", 0, BF16_PEAK_TFLOPS), ("f32", 1, F32_PEAK_TFLOPS)):
        def fn():
            D.mingru_rollout_step(p, obs, state, out, D=D5, H=H5, L_layers=L5, A=A5, precision=prec)
            D.sample_actions(out, A5, rng_state=0x5EED, act=act, logp=lp, value=val)
        ms = time_graph(fn, steps, warmup)
        tf = flops / (ms * 1e-3) / 1e12
        r[name] = {"us": round(ms * 1e3, 2), "env_steps_per_s": round(N / (ms * 1e-3), 1),
                   "tflops": round(tf, 1), "frac": round(tf / peak, 4)}
    return r


# multi-discrete heads: the reference's `target` env (config/target.ini, ocean/target/adapter.c: 4096
# agents, obs 28, heads {9, 5}, minibatch 32768); Gaussian: its `drone` env (config/drone.ini,
# ocean/drone: 2048 agents, obs 21, 4 dims, minibatch 16384); default horizon 64, hidden 128, 4 epochs
MD_AGENTS, MD_OBS, MD_HEADS, MD_MB = 4096, 28, (9, 5), 32768
CT_AGENTS, CT_OBS, CT_DIM, CT_MB = 2048, 21, 4, 16384
HD_T, HD_H, HD_EPOCHS = 64, 128, 4


def bench_heads(steps, warmup):
    import ctypes as C
    import numpy as np
    import torch
    from pufferlean_amd import _lib as L
    from pufferlean_amd import device as D
    from pufferlean_amd import rng

    out = {}
    K = len(MD_HEADS)
    # loss gradients over a whole rollout of rows, dashboard losses folded in the same launch
    for name, N, O, Wd in (("md_grad", MD_AGENTS * HD_T, sum(MD_HEADS) + 1, K),
                           ("cont_grad", CT_AGENTS * HD_T, 2 * CT_DIM + 1, CT_DIM)):
        y = _t(rng.normal(rng.seed_for(8, 0), N * O)).view(N, O)
        if name == "md_grad":
            act = torch.stack([_t(rng.randint(rng.seed_for(8, 1 + h), N, s), np.int32) for h, s in enumerate(MD_HEADS)],
                              1).contiguous()
        else:
            act = _t(rng.normal(rng.seed_for(8, 1), N * Wd)).view(N, Wd)
        adv, ret = _t(rng.normal(rng.seed_for(8, 8), N)), _t(rng.normal(rng.seed_for(8, 9), N))
        old, ov = _t(rng.normal(rng.seed_for(8, 10), N) - 3.0), _t(rng.normal(rng.seed_for(8, 11), N))
        dout = torch.empty_like(y)
        losses = torch.zeros(7, device="cuda", dtype=torch.float64)
        if name == "md_grad":
            fn = lambda: D.ppo_grad_md(y, act, adv, ret, old, ov, head_sizes=MD_HEADS, vf_clip=0.2, dout=dout,
                                       losses=losses)
        else:
            fn = lambda: D.ppo_grad_cont(y, act, adv, ret, old, ov, dim=CT_DIM, vf_clip=0.2, dout=dout, losses=losses)
        us = time_graph(fn, steps, warmup) * 1e3
        if name == "md_grad":
            fn0 = lambda: D.ppo_grad_md(y, act, adv, ret, old, ov, head_sizes=MD_HEADS, vf_clip=0.2, dout=dout)
        else:
            fn0 = lambda: D.ppo_grad_cont(y, act, adv, ret, old, ov, dim=CT_DIM, vf_clip=0.2, dout=dout)
        us0 = time_graph(fn0, steps, warmup) * 1e3
        # per row: the O head outputs read and their O gradients written, Wd actions, adv/ret/old/ov
        nbytes = N * (2 * O * 4 + Wd * 4 + 4 * 4)
        gbs = nbytes / (us * 1e-6) / 1e9
        out[name] = {"rows": N, "us": round(us, 2), "us_no_losses": round(us0, 2), "bytes": nbytes,
                     "gbs": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    # samplers over one rollout step of the env's agents
    Ym = _t(rng.normal(rng.seed_for(8, 20), MD_AGENTS * (sum(MD_HEADS) + 1))).view(MD_AGENTS, -1)
    om = torch.empty((K + 2) * MD_AGENTS, device="cuda", dtype=torch.float64)
    out["md_sample_us"] = round(time_graph(lambda: D.sample_actions_md(Ym, MD_HEADS, rng_state=0x5EED, out=om),
                                           steps, warmup) * 1e3, 2)
    Yc = _t(rng.normal(rng.seed_for(8, 21), CT_AGENTS * (2 * CT_DIM + 1))).view(CT_AGENTS, -1)
    oc = torch.empty((CT_DIM + 2) * CT_AGENTS, device="cuda", dtype=torch.float64)
    out["cont_sample_us"] = round(time_graph(lambda: D.sample_actions_cont(Yc, CT_DIM, rng_state=0x5EED, out=oc),
                                             steps, warmup) * 1e3, 2)
    # the whole wide update through its host-buffer entry: f64 columns uploaded once, 4 epochs of
    # minibatches on the device, exact f64 Muon; wall time per call, PCIe upload included
    dp = lambda a: np.ascontiguousarray(a, np.float64).ctypes.data_as(L.dptr)
    for name, mode, agents, Dm, O, Wd, mb in (("md_update", 1, MD_AGENTS, MD_OBS, sum(MD_HEADS) + 1, K, MD_MB),
                                              ("cont_update", 2, CT_AGENTS, CT_OBS, 2 * CT_DIM + 1, CT_DIM, CT_MB)):
        NT = agents * HD_T
        P = HD_H * Dm + HD_H + O * HD_H + O
        pm = np.concatenate([rng.normal(rng.seed_for(8, 30), P) * 0.1, np.zeros(P)])
        obs = rng.normal(rng.seed_for(8, 31), NT * Dm)
        if mode == 1:
            acts = np.stack([rng.randint(rng.seed_for(8, 32 + h), NT, s) for h, s in enumerate(MD_HEADS)],
                            1).astype(np.float64)
        else:
            acts = rng.normal(rng.seed_for(8, 32), NT * Wd)
        adv, ret = rng.normal(rng.seed_for(8, 40), NT), rng.normal(rng.seed_for(8, 41), NT)
        olp, ov = rng.normal(rng.seed_for(8, 42), NT) - 3.0, rng.normal(rng.seed_for(8, 43), NT)
        perm = np.concatenate([np.random.default_rng(e).permutation(NT) for e in range(HD_EPOCHS)]).astype(np.float64)
        hs = np.array(MD_HEADS, np.float64)
        h = C.c_size_t(0)
        L.call("ph_cuda_policy_load", dp(pm), P, C.byref(h))
        peek = np.zeros(1)
        args = [dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), dp(ov), NT, dp(perm), dp(hs), len(hs), NT, Dm, HD_H, O,
                Wd, mode, HD_EPOCHS, NT // mb, 0.015, 0.0, 0.95, 1e-12, 2.0, 0.001, 0.2, 0.2, 1.5, 1, dp(peek)]
        try:
            n_calls = max(2, min(steps, 5))
            L.call("ph_cuda_train_update_wide_resident", h.value, *args)
            t0 = time.perf_counter()
            for _ in range(n_calls):
                L.call("ph_cuda_train_update_wide_resident", h.value, *args)
            ms = (time.perf_counter() - t0) / n_calls * 1e3
        finally:
            L.call("ph_cuda_policy_free", h.value)
        out[name] = {"rows": NT, "obs": Dm, "hidden": HD_H, "out": O, "epochs": HD_EPOCHS, "minibatch": mb,
                     "ms": round(ms, 2), "rows_per_s": round(NT / (ms * 1e-3), 1),
                     "upload_bytes": 8 * (NT * (Dm + Wd + 4) + HD_EPOCHS * NT)}
    out["heads"] = list(MD_HEADS)
    out["cont_dims"] = CT_DIM
    return out


def traffic_kernels():
    """Launches for the two HBM-traffic counter runs (rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE):
    the dominant kernel (the data-gradient GEMM, one operand set per launch) 3 times, then a plain
    512 MiB device copy 3 times, whose known byte count scales the counters."""
    import torch
    ops = dgrad_operands()
    for op in ops:
        dgrad_launch(op)
    torch.cuda.synchronize()
    a = torch.ones(1 << 28, device="cuda", dtype=torch.bfloat16)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    return {"gemm": [B5 * T5, H5, 3 * H5], "copy_bytes": 2 * a.numel()}


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_dgrad_262144x512x1536_traffic.json")


def measured_traffic():
    """HBM bytes per launch of the dominant kernel from the committed counter summary (null if the
    summary is absent or was taken on another tile configuration)."""
    try:
        with open(TRAFFIC_FILE) as f:
            t = json.load(f)
        return t.get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


# ------------------------------------------------------------------------------------------------
# CPU baselines: the oracle (the reference CPU path's algorithm, f64 unless noted) on the host cores of
# the GPU box, in the same run. Each figure is the median of repeated runs (after one warm-up) within a
# time budget; the sample each one covers is stated.

def cpu_threads():
    return max(1, min(16, os.cpu_count() or 1))


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


WARMUPS, REPS = 3, 10  # CPU baselines: median of REPS timed runs after WARMUPS untimed ones


def _median_time(fn, budget_s, reps=REPS, warmups=WARMUPS, min_reps=3):
    """Median wall time of fn() over `reps` runs after `warmups` untimed ones. A leg whose runs are too
    long for `budget_s` stops after at least `min_reps` and says so: returns (median, timing record)."""
    import statistics
    for _ in range(warmups):
        fn()
    ts = []
    t_start = time.perf_counter()
    while len(ts) < reps and (len(ts) < min_reps or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    rec = {"reps": len(ts), "warmups": warmups}
    if len(ts) < reps:
        rec["budget_limited"] = f"{len(ts)} of {reps} reps within the {budget_s:.0f} s budget of this leg"
    return statistics.median(ts), rec


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as O
    return O


def cpu_baseline_gemm(nt, budget_s=15.0):
    """Config 2 on the oracle's blocked f64 GEMM over nt threads (the reference's CPU GEMMs are OpenBLAS
    dgemm): GFLOP/s per form."""
    import numpy as np
    from pufferlean_amd import rng
    O = _oracle()
    M, K, N = 16384, 512, 512
    X = rng.normal(rng.seed_for(2, 0), M * K).reshape(M, K)
    W = rng.normal(rng.seed_for(2, 1), N * K).reshape(N, K) / np.sqrt(512)
    dY = rng.normal(rng.seed_for(2, 2), M * N).reshape(M, N)
    C1 = np.zeros((M, N)); C2 = np.zeros((M, K)); C3 = np.zeros((N, K))
    forms = {"fwd": lambda: O.lib().orc_gemm_blocked(0, 1, M, N, K, O.P(X), K, O.P(W), K, O.P(C1), N, nt),
             "dgrad": lambda: O.lib().orc_gemm_blocked(0, 0, M, K, N, O.P(dY), N, O.P(W), K, O.P(C2), K, nt),
             "wgrad": lambda: O.lib().orc_gemm_blocked(1, 0, N, K, M, O.P(dY), N, O.P(X), K, O.P(C3), K, nt)}
    out = {}
    for name, fn in forms.items():
        t, rec = _median_time(fn, budget_s / 3)
        out[name] = dict({"value": round(2.0 * M * N * K / t / 1e9, 2), "unit": "GFLOP/s", "ms": round(t * 1e3, 1)},
                         **rec)
    return {"forms": out, "cores": nt, "kind": "port",
            "sample": "the whole 16384x512x512 product per form, f64, blocked and packed, OpenMP"}


def cpu_baseline_ns(nt, budget_s=25.0):
    """Config 3: the oracle's Newton-Schulz (the reference's naive f64 products) on the six matrices over
    nt threads, and on one thread for one step of one 512x512 matrix, scaled to the batch by flops."""
    import numpy as np
    from pufferlean_amd import rng
    O = _oracle()
    shapes = [(512, 512)] * 4 + [(512, 1024)] * 2
    mats = [rng.normal(rng.seed_for(3, i), r * c, 0.0, 0.02).reshape(r, c) for i, (r, c) in enumerate(shapes)]
    flops = sum(5 * (4 * min(r, c) ** 2 * max(r, c) + 2 * min(r, c) ** 3) for r, c in shapes)
    old = O.lib().orc_set_threads(nt)
    try:
        t_mt, rec = _median_time(lambda: [O.newton_schulz(m, O.BASELINE_COEFFS, 1e-7, form=1) for m in mats],
                                 budget_s * 0.6)
    finally:
        O.lib().orc_set_threads(old)
    one = mats[0]
    t_1, rec1 = _median_time(lambda: O.newton_schulz(one, O.BASELINE_COEFFS[:1], 1e-7, form=1), budget_s * 0.4)
    f1 = 4 * 512 ** 3 + 2 * 512 ** 3
    return dict({"value": round(flops / t_mt / 1e9, 2), "unit": "GFLOP/s", "us": round(t_mt * 1e6, 1),
                 "cores": nt, "single_thread": dict({"value": round(f1 / t_1 / 1e9, 3), "unit": "GFLOP/s",
                                                     "batch_us_scaled": round(t_1 * flops / f1 * 1e6, 1)}, **rec1),
                 "kind": "port", "sample": "all six matrices x 5 steps on nt threads; one step of one 512x512 "
                                           "matrix on one thread, scaled to the batch's flops"}, **rec)


def cpu_baseline_vtrace(nt, budget_s=3.0):
    """Config 4: the oracle's fp32 V-trace scan (puffercuda.cu:120-132 restated) on 4096 x 64,
    time-major, one thread and nt threads over segments."""
    import numpy as np
    from pufferlean_amd import rng
    O = _oracle()
    B, T = 4096, 64
    n = B * T
    val, rew = O.f32(rng.normal(rng.seed_for(4, 1), n)), O.f32(rng.normal(rng.seed_for(4, 2), n))
    done = O.f32(rng.bernoulli(rng.seed_for(4, 3), n, 0.01))
    lr = O.f32(rng.normal(rng.seed_for(4, 4), n, 0.0, 0.1))
    boot = O.f32(rng.normal(rng.seed_for(4, 5), B))
    adv = np.zeros(n, np.float32); tgt = np.zeros(n, np.float32)
    args = lambda: (O.P(rew), O.P(val), O.P(done), O.P(lr), O.P(boot), B, T, 1, 1, 1, 1, 0.99, 0.95, 1.0, 1.0,
                    O.P(adv), O.P(tgt))
    t1, r1 = _median_time(lambda: O.lib().orc_vtrace_f32(*args()), budget_s / 2, reps=21)
    tm, rm = _median_time(lambda: O.lib().orc_vtrace_f32_mt(*args(), nt), budget_s / 2, reps=21)
    by = 24.0 * n + 4.0 * B
    return dict({"value": round(by / tm / 1e9, 2), "unit": "GB/s", "us": round(tm * 1e6, 1), "cores": nt,
                 "single_thread": dict({"value": round(by / t1 / 1e9, 2), "unit": "GB/s", "us": round(t1 * 1e6, 1)},
                                       **r1),
                 "kind": "port", "sample": "the whole 4096 x 64 fp32 scan (bootstrapped variant, log-ratio input)"},
                **rm)


def cpu_baseline_cartpole(nt, budget_s=20.0):
    """Config 1: the whole CartPole update on the oracle (f64): forward, V-trace, normalisation, the
    gradient of the 4->128->128->3 MLP, Muon on the three matrices; GEMMs and NS products on nt threads."""
    import numpy as np
    O = _oracle()
    params, c = cartpole_inputs()
    N = CP_B * CP_T
    act = c["act"].astype(float)
    z = np.zeros(N)
    _, lp, _ = O.mlp_deep_ppo_grad(params, c["obs"], act, z, z, z, None, N, CP_D, CP_H, CP_L, CP_A, threads=nt)
    behav = lp + c["noise"]
    cf = O.coeffs_array(O.BASELINE_COEFFS)

    def update():
        _, lpn, val = O.mlp_deep_ppo_grad(params, c["obs"], act, z, z, z, None, N, CP_D, CP_H, CP_L, CP_A,
                                          threads=nt)
        adv, tgt = O.vtrace(c["rew"], val, c["done"], lpn - behav, None, CP_B, CP_T, variant=0, time_major=True,
                            rho_is_log=True)
        advn = np.zeros(N)
        O.lib().orc_adv_normalize(O.P(adv), N, O.P(advn))
        g, _, _ = O.mlp_deep_ppo_grad(params, c["obs"], act, advn, tgt, behav, None, N, CP_D, CP_H, CP_L, CP_A,
                                      threads=nt)
        off = 0
        for l in range(CP_L + 1):
            rows, cols = (CP_A + 1 if l == CP_L else CP_H), (CP_D if l == 0 else CP_H)
            k = rows * cols
            a = np.zeros(k); b = np.zeros(k)
            O.lib().orc_muon_mat(rows, cols, O.P(params[off:off + k].copy()), O.P(g[off:off + k] / N),
                                 O.P(np.zeros(k)), O.P(a), O.P(b), 1.0, 0.015, 0.0, 0.95, 1e-7, O.P(cf), 5, 1)
            off += k + rows

    old = O.lib().orc_set_threads(nt)
    try:
        t, rec = _median_time(update, budget_s)
    finally:
        O.lib().orc_set_threads(old)
    return dict({"value": round(N / t, 1), "unit": "samples/s", "ms": round(t * 1e3, 1), "cores": nt,
                 "kind": "port", "sample": "the whole 65,536-row update (two forwards: V-trace inputs, then the "
                                           "gradient's), f64"}, **rec)


def cpu_baseline_ppo(nt, budget_s=40.0):
    """Config 5 (the headline) on the oracle, in the trainer's order: V-trace (bootstrapped, time-major, log
    ratios) and the advantage normalisation over all 262,144 rows, then the single-sequence MinGRU PPO
    gradient (f64, the reference CPU path's algorithm) over a sample of segments spread on nt threads and
    scaled to the 4096 segments, the grad-norm clip, and Muon (f64 Newton-Schulz, nt threads) on the five
    matrices. samples/s = 262,144 / (V-trace + normalisation + scaled gradient + clip + Muon)."""
    import numpy as np
    O = _oracle()
    params, cols = mingru_inputs(B5, T5, D5, H5, L5, A5)
    P = params.size
    n = B5 * T5
    rew, val, done, logrho = (O.f64(cols[k]) for k in ("rew", "val", "done", "logrho"))
    boot = O.f64(cols["boot"])
    adv = np.zeros(n)

    def vtrace_norm():
        a, tg = O.vtrace(rew, val, done, logrho, boot, B5, T5, variant=1, time_major=True, rho_is_log=True)
        O.lib().orc_adv_normalize(O.P(a), n, O.P(adv))
        return tg

    t_v, rec_v = _median_time(vtrace_norm, budget_s * 0.1)
    tgt = vtrace_norm().reshape(T5, B5)
    S = min(B5, 4 * nt)
    obs = O.f64(cols["obs"].reshape(T5, B5, D5)[:, :S, :])
    pick = lambda x: O.f64(x.reshape(T5, B5)[:, :S])
    act, old_, vals, term, advs, tgts = (pick(x) for x in (cols["act"], cols["old"], val, done, adv, tgt))
    out = np.zeros(P + 2 * T5 * S)
    grad = lambda: O.lib().orc_mingru_ppo_grad_batch(
        O.P(params), O.P(obs), O.P(act), O.P(advs), O.P(tgts), O.P(old_), O.P(term), O.P(vals), S, T5, H5,
        D5, L5, A5, 0.5, 0.01, 0.2, 0.0, O.P(out), nt)
    t_g, rec_g = _median_time(grad, budget_s * 0.4)
    cf = O.coeffs_array(O.BASELINE_COEFFS)
    szE, szL = H5 * D5, 3 * H5 * H5
    mats = [(0, H5, D5)] + [(szE + H5 + l * szL, 3 * H5, H5) for l in range(L5)]
    offDec = szE + H5 + L5 * szL
    mats += [(offDec, A5, H5), (offDec + A5 * H5 + A5, 1, H5)]
    g = out[:P].copy()

    def clip_muon():
        gc = g.copy()
        O.lib().orc_gclip(O.P(gc), P, 1.0 / n, 0.5)
        for off, r, c in mats:
            k = r * c
            a = np.zeros(k); b = np.zeros(k)
            O.lib().orc_muon_mat(r, c, O.P(params[off:off + k].copy()), O.P(gc[off:off + k].copy()),
                                 O.P(np.zeros(k)), O.P(a), O.P(b), 1.0, 0.015, 0.0, 0.95, 1e-7, O.P(cf), 5, 1)

    old = O.lib().orc_set_threads(nt)
    try:
        t_m, rec_m = _median_time(clip_muon, budget_s * 0.5)
    finally:
        O.lib().orc_set_threads(old)
    t_step = t_v + t_g * B5 / S + t_m
    return {"value": round(n / t_step, 1), "unit": "samples/s", "cores": nt, "kind": "port",
            "sample": f"V-trace + normalisation over all 4096 segments; gradient over {S} of 4096 segments "
                      f"({100.0 * S / B5:.1f} %) x 64 steps on {nt} threads, scaled to 4096; clip + Muon on "
                      f"the 5 matrices ({nt} threads); step {t_step:.1f} s",
            "sampled_fraction": round(S / B5, 5),
            "vtrace_norm_s": round(t_v, 4), "vtrace_norm_timing": rec_v,
            "gradient_s_per_segment": round(t_g / S, 4), "gradient_timing": rec_g,
            "muon_s": round(t_m, 3), "muon_timing": rec_m}


def cpu_baselines(only):
    nt = cpu_threads()
    out = {"threads": nt, "cpu_model": cpu_model(), "nproc": os.cpu_count()}
    for name, fn in (("cartpole", cpu_baseline_cartpole), ("gemm", cpu_baseline_gemm), ("ns", cpu_baseline_ns),
                     ("vtrace", cpu_baseline_vtrace)):
        if only in ("all", name):
            out[name] = fn(nt)
            print(f"# cpu baseline {name} done", file=sys.stderr, flush=True)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--only", default="all")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--eager", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported in this build "
              "(the step would shard segments across GPUs with one gradient all-reduce per minibatch)",
              file=sys.stderr)
        return 2
    import torch
    from pufferlean_amd import _lib
    _lib.lib()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.only == "traffic":
        print(json.dumps(traffic_kernels()))
        return 0
    comps = {}
    head = None
    if args.only in ("all", "ppo"):
        head = bench_ppo_step(args.steps, args.warmup, eager=args.eager)
        print(f"# ppo step {head['ms']} ms", file=sys.stderr, flush=True)
    if args.only in ("all", "gemm"):
        comps["gemm"] = bench_gemm(args.steps, args.warmup)
        print("# gemm done", file=sys.stderr, flush=True)
    if args.only in ("all", "ns"):
        comps["ns"] = bench_ns(args.steps, args.warmup)
        print("# ns done", file=sys.stderr, flush=True)
    if args.only in ("all", "vtrace"):
        comps["vtrace"] = bench_vtrace(args.steps, args.warmup)
        print("# vtrace done", file=sys.stderr, flush=True)
    if args.only in ("all", "rollout"):
        comps["rollout"] = bench_rollout(args.steps, args.warmup)
        print("# rollout done", file=sys.stderr, flush=True)
    if args.only in ("all", "replay"):
        comps["replay"] = bench_replay(args.steps, args.warmup)
        print("# replay done", file=sys.stderr, flush=True)
    if args.only in ("all", "heads"):
        comps["heads"] = bench_heads(args.steps, args.warmup)
        print("# heads done", file=sys.stderr, flush=True)
    if args.only in ("all", "cartpole"):
        comps["cartpole"] = bench_cartpole(args.steps, args.warmup)
        print("# cartpole done", file=sys.stderr, flush=True)
    # a step whose Newton-Schulz gave up has no valid figure: no value is printed for it
    valid = head is not None and head["finite"] and head["ns_ok"]
    line = {
        "metric": METRIC,
        "value": head["samples_per_s"] if valid else None,
        "unit": "samples/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": head["ms"] if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (seeded splitmix64; random-init weights)",
        "config": {"workload": "MinGRU PPO+Muon minibatch step: obs 128 -> enc 512 -> 2x MinGRU 512 "
                               "(sequential scan over the 64 steps, as the reference trains) -> 16-way + value; "
                               "4096 segments x 64 steps",
                   "segments": B5, "horizon": T5, "hidden": H5, "layers": L5, "actions": A5,
                   "obs": D5, "scan": "sequential"},
    }
    if head:
        dk = head["dominant_kernel"]
        line["roofline"] = {"bound": "mfma", "achieved": dk["tflops"], "peak": BF16_PEAK_TFLOPS,
                            "unit": "TFLOP/s", "frac": round(dk["tflops"] / BF16_PEAK_TFLOPS, 4),
                            "traffic": measured_traffic(), "kernel": dk["name"], "kernel_us": dk["us"],
                            "algorithmic_bytes": dk["hbm_bytes"]}
        line["step"] = {k: v for k, v in head.items() if k != "dominant_kernel"}
    line["components"] = comps
    if head is not None and not valid:
        line["error"] = "the timed step produced invalid weights (non-finite, or a Newton-Schulz launch gave up)"
    if "ns" in comps and not comps["ns"]["ns_ok"]:
        comps["ns"]["us"] = comps["ns"]["tflops"] = comps["ns"]["frac"] = None
    if not args.no_cpu_baseline:
        nt = cpu_threads()
        if head:
            line["cpu_baseline"] = dict(cpu_baseline_ppo(nt), cpu_model=cpu_model())
            print("# cpu baseline ppo done", file=sys.stderr, flush=True)
        line["cpu_baselines"] = cpu_baselines(args.only)
    print(json.dumps(line))
    return 0 if (head is None or valid) else 1


if __name__ == "__main__":
    sys.exit(main())
