"""Rollout policy forward and categorical sampler on the GPU vs the CPU oracle (the twins
pufferffi.c:896-918 and the f64 restatement of lean_cuda_mingru_step).

Bars: value column exact; actions exact except a draw whose uniform lies within rounding of a
cumulative softmax boundary (1e-12 for f64 logits, 1e-5 for f32, where the running sum is f32 as in
the reference's f32 sampler); logp 1e-13 (f64) / 1e-5 (f32) relative; the fp32 step 1e-5 relative,
the bf16 step 2e-2 relative Frobenius (bf16 operands).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def cu(x, dt=torch.float64):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dt)


def dp(a):
    return np.ascontiguousarray(a, np.float64).ctypes.data_as(C.POINTER(C.c_double))


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def _sample(Y, ldy, N, A, has_value, state, dtype):
    t = torch.float64 if dtype == L.PH_F64 else torch.float32
    gY = cu(Y, t)
    act = torch.empty(N, device="cuda", dtype=torch.int32)
    lp = torch.empty(N, device="cuda", dtype=t)
    val = torch.empty(N, device="cuda", dtype=t)
    L.call("ph_sample_actions", dtype, C.c_void_p(gY.data_ptr()), ldy, N, A, has_value, state,
           C.c_void_p(act.data_ptr()), C.c_void_p(lp.data_ptr()), C.c_void_p(val.data_ptr()),
           C.c_void_p(torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return act.cpu().numpy(), lp.cpu().numpy().astype(np.float64), val.cpu().numpy().astype(np.float64)


def _check_actions(act, ref_act, Y, A, state, band):
    N = len(act)
    lg = Y[:, :A]
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    cum = np.cumsum(p, axis=1)
    u = rng.uniform01(rng.words(state, N))
    bad = np.nonzero(act != ref_act)[0]
    for n in bad:  # only draws within rounding of a cumulative boundary may differ
        k = int(min(act[n], ref_act[n]))
        assert abs(act[n] - ref_act[n]) == 1 and abs(cum[n, k] - u[n]) < band, (n, act[n], ref_act[n])
    assert len(bad) <= max(1, N // 500)


@pytest.mark.parametrize("N,A", [(1, 1), (5, 2), (4096, 16), (10000, 7)])
def test_sample_f64_matches_cpu_twin(gpu, N, A):
    print(f"sample f64 N={N} A={A}", flush=True)
    Y = rng.normal(0x701 + N, N * (A + 1)).reshape(N, A + 1) * 3.0
    state = 0x1234567 + A
    act, lp, val = _sample(Y, A + 1, N, A, 1, state, L.PH_F64)
    ra, rl, rv = O.sample_actions(Y, A, state)
    _check_actions(act, ra, Y, A, state, 1e-12)
    ok = act == ra
    assert np.allclose(lp[ok], rl[ok], rtol=1e-13, atol=1e-15)
    assert np.array_equal(val, rv)


def test_sample_f32_rows_strided_no_value(gpu):
    N, A, ldy = 4096, 12, 32
    Y = (rng.normal(0x702, N * ldy).reshape(N, ldy) * 2.0).astype(np.float32)
    state = 0xABCDEF
    act, lp, val = _sample(Y, ldy, N, A, 0, state, L.PH_F32)
    Y64 = Y.astype(np.float64)
    ra, rl, _ = O.sample_actions(np.ascontiguousarray(Y64[:, :A + 1]), A, state)
    _check_actions(act, ra, Y64, A, state, 1e-5)
    ok = act == ra
    assert np.allclose(lp[ok], rl[ok], rtol=1e-5, atol=1e-6)
    assert np.all(val == 0.0)


def test_cuda_sample_actions_host_entry(gpu):
    N, A, Ocols = 2048, 9, 10
    Y = rng.normal(0x703, N * Ocols).reshape(N, Ocols)
    out = np.zeros(3 * N)
    L.call("ph_cuda_sample_actions", dp(Y), N, A, Ocols, 0x5151, dp(out))
    ra, rl, rv = O.sample_actions(Y, A, 0x5151)
    _check_actions(out[:N], ra, Y, A, 0x5151, 1e-12)
    assert np.array_equal(out[2 * N:], rv)
    ok = out[:N] == ra
    assert np.allclose(out[N:2 * N][ok], rl[ok], rtol=1e-13, atol=1e-15)


# ---- MinGRU rollout step ------------------------------------------------------------------------
def _mg_params(seed, D, H, Lr, A, scale=0.3):
    P = H * D + H + Lr * 3 * H * H + A * H + A + H + 1
    return rng.normal(seed, P) * scale / np.sqrt(max(D, H) / 8)


@pytest.mark.parametrize("prec,tol", [(1, 1e-5), (0, 2e-2)])
def test_rollout_step_matches_oracle_over_three_steps(gpu, prec, tol):
    N, Dm, H, Lr, A = 300, 16, 64, 2, 7
    params = _mg_params(0x711, Dm, H, Lr, A)
    dims = L.MinGRUDims(N, 1, Dm, H, Lr, A, prec)
    gp = cu(params, torch.float32)
    state = torch.zeros(N * Lr * H, device="cuda", dtype=torch.float32)
    out = torch.empty(N * (A + 1), device="cuda", dtype=torch.float32)
    ref_state = np.zeros((N, Lr, H))
    for t in range(3):
        obs = rng.normal(0x712 + t, N * Dm).reshape(N, Dm)
        gobs = cu(obs, torch.float32)  # held until after the synchronize: the kernel reads it
        L.call("ph_mingru_rollout_step", C.byref(dims), C.c_void_p(gp.data_ptr()),
               C.c_void_p(gobs.data_ptr()), C.c_void_p(state.data_ptr()),
               C.c_void_p(out.data_ptr()), C.c_void_p(torch.cuda.current_stream().cuda_stream))
        torch.cuda.synchronize()
        ref_out, ref_state = O.mingru_step(params.astype(np.float32).astype(np.float64),
                                           obs.astype(np.float32).astype(np.float64), ref_state, N, Dm, H, Lr, A)
        assert rel(out.cpu().numpy().reshape(N, A + 1), ref_out) < tol, t
        assert rel(state.cpu().numpy().reshape(N, Lr, H), ref_state) < tol, t
        ref_state = state.cpu().numpy().astype(np.float64).reshape(N, Lr, H)  # continue from the device state


@pytest.mark.parametrize("bf16,tol", [(0, 1e-5), (1, 2e-2)])
def test_cuda_mingru_step_host_entry_headline_shape(gpu, bf16, tol):
    N, Dm, H, Lr, A = 256, 128, 512, 2, 16
    params = _mg_params(0x721, Dm, H, Lr, A)
    obs = rng.normal(0x722, N * Dm)
    st = rng.normal(0x723, N * Lr * H) * 0.5
    out = np.zeros(N * (A + 1) + N * Lr * H)
    L.call("ph_cuda_mingru_step", dp(params), dp(obs), dp(st), N, Dm, H, Lr, A, bf16, dp(out))
    ro, rs = O.mingru_step(params, obs, st, N, Dm, H, Lr, A)
    assert rel(out[:N * (A + 1)], ro.ravel()) < tol
    assert rel(out[N * (A + 1):], rs.ravel()) < tol


@pytest.mark.parametrize("bf16,tol", [(0, 1e-5), (1, 1e-2)])
def test_cuda_mlp_forward(gpu, bf16, tol):
    N, Dm, H, Oc = 1000, 24, 128, 5
    P = H * Dm + H + Oc * H + Oc
    p = rng.normal(0x731, P) / np.sqrt(Dm)
    X = rng.normal(0x732, N * Dm)
    out = np.zeros(N * Oc)
    L.call("ph_cuda_mlp_forward", dp(p), dp(X), N, Dm, H, Oc, bf16, dp(out))
    ref = np.zeros(N * Oc)
    O.lib().orc_mlp_forward(O.P(p), O.P(X), N, Dm, H, Oc, O.P(ref))
    assert rel(out, ref) < tol


def test_rollout_step_then_sample_in_one_graph(gpu):
    """A horizon of rollout steps + draws captured once in a HIP graph and replayed equals the same
    launches made directly."""
    N, Dm, H, Lr, A, T = 512, 32, 64, 2, 6, 4
    params = cu(_mg_params(0x741, Dm, H, Lr, A), torch.float32)
    obs = cu(rng.normal(0x742, T * N * Dm).reshape(T, N, Dm), torch.float32)
    dims = L.MinGRUDims(N, 1, Dm, H, Lr, A, 0)

    def run(state, out, act, lp):
        s = C.c_void_p(torch.cuda.current_stream().cuda_stream)
        for t in range(T):
            L.call("ph_mingru_rollout_step", C.byref(dims), C.c_void_p(params.data_ptr()),
                   C.c_void_p(obs[t].data_ptr()), C.c_void_p(state.data_ptr()), C.c_void_p(out[t].data_ptr()), s)
            L.call("ph_sample_actions", L.PH_F32, C.c_void_p(out[t].data_ptr()), A + 1, N, A, 1, 0x99 + t * N,
                   C.c_void_p(act[t].data_ptr()), C.c_void_p(lp[t].data_ptr()), None, s)

    mk = lambda: (torch.zeros(N * Lr * H, device="cuda"), torch.empty(T, N * (A + 1), device="cuda"),
                  torch.empty(T, N, device="cuda", dtype=torch.int32), torch.empty(T, N, device="cuda"))
    ref = mk()
    run(*ref)
    torch.cuda.synchronize()
    bufs = mk()
    run(*bufs)  # sizes the library's buffers before capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        bufs[0].zero_()
        with torch.cuda.graph(g, stream=s):
            run(*bufs)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    for _ in range(3):
        bufs[0].zero_()
        g.replay()
        torch.cuda.synchronize()
        for a, b in zip(ref, bufs):
            assert torch.equal(a, b)
