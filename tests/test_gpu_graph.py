"""The MinGRU PPO+Muon step captured in a HIP graph (as the benchmark runs it) replays exactly.

The step forks its per-matrix Muon updates onto library stream lanes and joins them back, and its
reductions reset their own arrival counters; a captured step must therefore reproduce the eager
step bit for bit on every replay. Eager torch work and device synchronisations sit between the
replays.
"""
import numpy as np
import pytest
import torch

from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def _t(x, dt=np.float32):
    return torch.from_numpy(np.ascontiguousarray(x, dt)).cuda()


@pytest.mark.parametrize("precision", ["bf16", "f32"])
def test_graph_replays_match_eager(gpu, precision):
    B, T, Dm, H, L, A = 64, 16, 8, 32, 2, 5
    cfg = D.MinGRUConfig(B, T, Dm, H, L, A, lr=0.015, mu=0.95, max_grad_norm=0.5,
                         gscale=1.0 / (B * T), precision=precision, math=precision)
    n = B * T
    p0 = rng.normal(0x900, cfg.P) * 0.1
    obs = _t(rng.normal(0x901, n * Dm)).view(T, B, Dm)
    act = _t(rng.randint(0x902, n, A), np.int32).view(T, B)
    old = _t(np.log(1.0 / A) + rng.normal(0x903, n, 0.0, 0.05)).view(T, B)
    val = _t(rng.normal(0x904, n)).view(T, B)
    rew = _t(rng.normal(0x905, n)).view(T, B)
    done = _t(rng.bernoulli(0x906, n, 0.05)).view(T, B)
    logrho = _t(rng.normal(0x907, n, 0.0, 0.1)).view(T, B)
    boot = _t(rng.normal(0x908, B))

    def run_eager(p, m, g, k):
        outs = []
        for _ in range(k):
            D.mingru_step(cfg, p, m, obs, act, old, val, rew, done, logrho, boot, G=g)
            torch.cuda.synchronize()
            outs.append((p.clone(), m.clone()))
        return outs

    # eager reference chain of 3 steps
    ref = run_eager(_t(p0), torch.zeros(cfg.P, device="cuda"), torch.zeros(cfg.P, device="cuda"), 3)

    # warm up (library buffers, lane streams) on throw-away copies, then capture one step
    run_eager(_t(p0), torch.zeros(cfg.P, device="cuda"), torch.zeros(cfg.P, device="cuda"), 1)
    p = _t(p0)
    m = torch.zeros(cfg.P, device="cuda")
    g = torch.zeros(cfg.P, device="cuda")
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            D.mingru_step(cfg, p, m, obs, act, old, val, rew, done, logrho, boot, G=g)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    # capture records work without running it: the parameters are still the initial ones
    assert torch.equal(p, _t(p0))
    for k in range(3):
        graph.replay()
        torch.cuda.synchronize()
        _ = (torch.ones(1000, device="cuda") * 2).sum().item()  # eager work between replays
        assert torch.equal(p, ref[k][0]), f"replay {k}: parameters differ from the eager step"
        assert torch.equal(m, ref[k][1]), f"replay {k}: momentum differs from the eager step"


def test_captured_gemm_survives_scratch_growth(gpu):
    """A graph captured around a GEMM that stages zero-padded operand copies (a 28-wide reduction)
    keeps valid staging memory when a later, larger call grows the same scratch slots: the old
    buffers are retired, not freed, until ph_release_scratch."""
    M, N, K = 4096, 128, 28
    a = _t(rng.normal(0x910, M * K)).view(M, K)
    b = _t(rng.normal(0x911, N * K) / np.sqrt(K)).view(N, K)
    ref = D.gemm(a, b, trans_b=True, math="bf16")
    c = torch.empty_like(ref)
    D.gemm(a, b, trans_b=True, math="bf16", out=c)  # warm-up sizes the slots for this shape
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(graph, stream=s):
            D.gemm(a, b, trans_b=True, math="bf16", out=c)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    n0, _ = D.scratch_retired()
    # a larger unaligned call than any before it grows the padding slots
    M2 = 1 << 20
    a2 = _t(rng.normal(0x912, M2 * K)).view(M2, K)
    big = D.gemm(a2, b, trans_b=True, math="bf16")
    torch.cuda.synchronize()
    n1, b1 = D.scratch_retired()
    assert n1 > n0 and b1 > 0
    for k in range(3):
        c.zero_()
        graph.replay()
        torch.cuda.synchronize()
        _ = (torch.ones(1000, device="cuda") * 2).sum().item()
        assert torch.equal(c, ref), f"replay {k} after the slot grew"
    assert big.shape == (M2, N)
    del graph
    D.release_scratch()
    assert D.scratch_retired() == (0, 0)


def test_step_error_after_fork_joins_lane(gpu):
    """An argument error found after the step forked its lane 0 (V-trace and the normalisation already
    queued there; the gradient then rejects 40 logits, more than the padded head holds) still joins the
    lane: a capture around the failing call ends cleanly and the library's error is what surfaces, and
    the stream's later work is unaffected."""
    from pufferlean_amd._lib import PufferHipError
    B, T, Dm, H, L = 16, 8, 8, 32, 1
    n = B * T
    obs = _t(rng.normal(0x940, n * Dm)).view(T, B, Dm)
    old = _t(rng.normal(0x941, n, -2.0, 0.1)).view(T, B)
    val = _t(rng.normal(0x942, n)).view(T, B)
    rew = _t(rng.normal(0x943, n)).view(T, B)
    done = _t(rng.bernoulli(0x944, n, 0.05)).view(T, B)
    logrho = _t(rng.normal(0x945, n, 0.0, 0.1)).view(T, B)
    boot = _t(rng.normal(0x946, B))

    cfgs = {A: D.MinGRUConfig(B, T, Dm, H, L, A, gscale=1.0 / n, precision="bf16", math="bf16") for A in (5, 40)}
    acts = {A: _t(rng.randint(0x947, n, A), np.int32).view(T, B) for A in (5, 40)}
    gs = {A: torch.zeros(cfgs[A].P, device="cuda") for A in (5, 40)}

    def step(A, p, m):  # no allocation or host copy: it also runs under capture
        D.mingru_step(cfgs[A], p, m, obs, acts[A], old, val, rew, done, logrho, boot, G=gs[A])

    good, bad_P = cfgs[5], cfgs[40].P
    p0 = rng.normal(0x948, good.P) * 0.1
    ref_p, ref_m = _t(p0), torch.zeros(good.P, device="cuda")
    step(5, ref_p, ref_m)
    torch.cuda.synchronize()
    with pytest.raises(PufferHipError, match="at most"):  # eager: sizes the buffers, fails after the fork
        step(40, _t(np.zeros(bad_P)), torch.zeros(bad_P, device="cuda"))
    torch.cuda.synchronize()
    pb, mb = _t(np.zeros(bad_P)), torch.zeros(bad_P, device="cuda")
    graph = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with pytest.raises(PufferHipError, match="at most"):
        with torch.cuda.stream(s):
            with torch.cuda.graph(graph, stream=s):
                step(40, pb, mb)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    p, m = _t(p0), torch.zeros(good.P, device="cuda")
    step(5, p, m)
    torch.cuda.synchronize()
    assert torch.equal(p, ref_p) and torch.equal(m, ref_m)
