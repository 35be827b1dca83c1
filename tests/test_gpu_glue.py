"""The Lean glue on the GPU: reference symbols called through their Lean ABI (owned FloatArrays,
unboxed scalars, IO results; the stand-in lean.h of tests/lean_stub) against the oracle.

* lean_cuda_selftest: 2i + 1.
* lean_cuda_vtrace on the verify-vtrace-gpu inputs: bit-exact with orc_vtrace_vec.
* lean_cuda_train_step on the verify-train-step shapes: the oracle's step (fp32 products 1e-5).
* lean_cuda_mingru_ppo_grad, host mode: the oracle's summed sequence gradient (1e-5); and the
  trainer's resident chain (mg_prep -> mg_vtrace_prio -> gradient with empty scal/params -> resident
  Muon with empty gClip), whose empty results and final weights match the same chain through the
  host-buffer entries bit for bit.
* lean_ffi_mlp_policy_load / _forward / _update / _free: the oracle's f64 MLP forward within the bf16
  bar; the bench entries return positive GF/s.
Every call releases its owned arguments: the stand-in's live-object count returns to where it was.
"""
import ctypes as C
import os

import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import rng
from test_gpu_host_abi import init_mlp, mlp_batch, oracle_train_step, vt_inputs

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GLUE = os.path.join(ROOT, "tests", "lean_stub", "libglue_stub.so")
vp, sz, dbl, u8, u64 = C.c_void_p, C.c_size_t, C.c_double, C.c_uint8, C.c_uint64


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def G(gpu):
    L.lib()  # the glue links libpufferhip.so; loading it first keeps one copy in the process
    h = C.CDLL(GLUE)
    h.stub_array.restype = vp
    h.stub_array.argtypes = [C.POINTER(C.c_double), sz]
    h.stub_array_size.restype = sz
    h.stub_array_size.argtypes = [vp]
    h.stub_array_data.restype = C.POINTER(C.c_double)
    h.stub_array_data.argtypes = [vp]
    h.stub_io_ok.argtypes = [vp]
    h.stub_io_value.restype = vp
    h.stub_io_value.argtypes = [vp]
    h.stub_io_error.restype = C.c_char_p
    h.stub_io_error.argtypes = [vp]
    h.stub_unbox.restype = sz
    h.stub_unbox.argtypes = [vp]
    h.stub_live.restype = C.c_long
    h.stub_release.argtypes = [vp]
    return h


def arr(G, x):
    x = np.ascontiguousarray(np.asarray(x, np.float64).ravel())
    return G.stub_array(x.ctypes.data_as(C.POINTER(C.c_double)), x.size)


def take(G, a):
    """numpy copy of a Lean FloatArray, then released"""
    n = G.stub_array_size(a)
    out = np.ctypeslib.as_array(G.stub_array_data(a), (max(n, 1),))[:n].copy()
    G.stub_release(a)
    return out


def io(G, r):
    """value of an IO result (raises with the library's message on an IO error); releases the result"""
    if not G.stub_io_ok(r):
        msg = G.stub_io_error(r).decode()
        G.stub_release(r)
        raise RuntimeError(msg)
    v = G.stub_io_value(r)
    return r, v


def fn(G, name, res, args):
    f = getattr(G, name)
    f.restype = res
    f.argtypes = args
    return f


def test_selftest_and_vtrace(G):
    live = G.stub_live()
    out = take(G, fn(G, "lean_cuda_selftest", vp, [sz])(1000))
    assert np.array_equal(out, 2.0 * np.arange(1000) + 1.0)
    B, T, gam, lam, rc, cc = 8, 12, 0.99, 0.95, 2.1, 1.08  # verify-vtrace-gpu (Exe/Puffer.lean:1075-1084)
    rew, val, term, imp = vt_inputs(0x5C1A, B, T)
    f = fn(G, "lean_cuda_vtrace", vp, [vp, vp, vp, vp, sz, sz, dbl, dbl, dbl, dbl])
    adv = take(G, f(arr(G, rew), arr(G, val), arr(G, term), arr(G, imp), B, T, gam, lam, rc, cc))
    ref = np.zeros(B * T)
    O.lib().orc_vtrace_vec(O.P(rew), O.P(val), O.P(term), O.P(imp), B, T, gam, lam, rc, cc, O.P(ref))
    assert np.array_equal(adv, ref)
    assert G.stub_live() == live


def test_train_step(G):
    live = G.stub_live()
    N, D, H, A = 96, 12, 16, 5
    params, s = init_mlp(D, H, A + 1, 0x77E5)
    obs, acts, adv, ret, olp = mlp_batch(s, N, D, A, -2.0, 2.0)
    Pn = params.size
    mom = s.randf(-0.1, 0.1, Pn)
    pm = np.concatenate([params, mom])
    ref = oracle_train_step(pm, obs, acts, adv, ret, olp, N, H, D, A, 0.1, 0.0, 0.95, 1e-7)
    f = fn(G, "lean_cuda_train_step", vp, [vp] * 6 + [sz] * 4 + [dbl] * 7 + [u8])
    out = take(G, f(arr(G, pm), arr(G, obs), arr(G, acts), arr(G, adv), arr(G, ret), arr(G, olp), N, H, D, A, 0.1,
                    0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0))
    assert out.size == 2 * Pn
    assert rel(out[:Pn] - params, ref[:Pn] - params) < 1e-5
    assert rel(out[Pn:], ref[Pn:]) < 1e-5
    assert G.stub_live() == live


GRAD_ARGS = [vp, vp, vp] + [sz] * 7 + [vp] + [dbl] * 4 + [vp, vp, vp]


def test_mingru_grad_host_mode(G, monkeypatch):
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    live = G.stub_live()
    B, T, D, H, Ln, A = 6, 9, 8, 16, 2, 5
    Pn = H * D + H + Ln * 3 * H * H + A * H + A + H + 1
    n = B * T
    p = rng.normal(0x1C1, Pn) * 0.3
    obs = rng.normal(0x1C2, n * D).reshape(T, B, D)
    act = rng.randint(0x1C3, n, A).reshape(T, B).astype(np.float64)
    adv, ret = rng.normal(0x1C4, n).reshape(T, B), rng.normal(0x1C5, n).reshape(T, B)
    old = rng.randf(0x1C6, n, -2.5, -1.0).reshape(T, B)
    term = rng.bernoulli(0x1C7, n, 0.05).reshape(T, B)
    ov = rng.normal(0x1C8, n).reshape(T, B)
    scal = np.concatenate([a.ravel() for a in (act, adv, ret, old, term, ov)])
    f = fn(G, "lean_cuda_mingru_ppo_grad", vp, GRAD_ARGS)
    r, v = io(G, f(arr(G, p), arr(G, obs), arr(G, scal), B, T, H, D, Ln, A, 1, arr(G, []), 0.5, 0.01, 0.2, 0.2,
                   arr(G, []), arr(G, []), None))
    got = np.ctypeslib.as_array(G.stub_array_data(v), (G.stub_array_size(v),)).copy()
    G.stub_release(r)
    assert got.size == Pn + 2 * n  # host form
    g = np.zeros(Pn)
    for b in range(B):
        o = np.zeros(Pn + 2 * T)
        O.lib().orc_mingru_ppo_grad_seq(O.P(p), O.P(O.f64(obs[:, b, :])), O.P(O.f64(act[:, b])),
                                        O.P(O.f64(adv[:, b])), O.P(O.f64(ret[:, b])), O.P(O.f64(old[:, b])),
                                        O.P(O.f64(term[:, b])), O.P(O.f64(ov[:, b])), T, H, D, Ln, A, 0.5, 0.01, 0.2,
                                        0.2, O.P(o))
        g += o[:Pn]
    assert rel(got[:Pn], g) < 1e-5
    assert G.stub_live() == live


def test_mingru_resident_chain(G, monkeypatch):
    """The trainer's minibatch loop through the Lean ABI (MinGRUTrain.lean:814-849) and through the
    host-buffer entries, from the same columns, weights and sampler state: identical weights."""
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    monkeypatch.delenv("PUFFER_MUON_EXACT", raising=False)
    monkeypatch.delenv("PUFFER_MG_DEVPRIO", raising=False)
    live = G.stub_live()
    N, T, Dm, H, Ln, A, mb, numMB = 16, 8, 8, 16, 2, 5, 6, 3
    P = H * Dm + H + Ln * 3 * H * H + A * H + A + H + 1
    n = N * T
    params = rng.normal(0x1D1, P) * 0.3
    cols = [rng.normal(0x1D2, n), rng.bernoulli(0x1D3, n, 0.05), rng.randint(0x1D4, n, A).astype(np.float64),
            rng.randf(0x1D5, n, -2.5, -1.0), rng.normal(0x1D6, n), rng.normal(0x1D7, N)]  # rew term act logp val boot
    traj = rng.normal(0x1D8, n * Dm)
    lr, wd, mu, eps, maxgn = 0.02, 0.0, 0.95, 1e-7, 0.5
    sc = 1.0 / (mb * T)
    f_prep = fn(G, "lean_cuda_mg_prep", vp, [vp] * 6 + [sz] * 3)
    f_load = fn(G, "lean_cuda_policy_load", vp, [vp, sz, vp])
    f_down = fn(G, "lean_cuda_policy_download", vp, [sz, sz, vp])
    f_free = fn(G, "lean_cuda_policy_free", vp, [sz, vp])
    f_prio = fn(G, "lean_cuda_mg_vtrace_prio", vp, [sz, sz] + [dbl] * 4 + [sz, dbl, dbl, u64, vp])
    f_grad = fn(G, "lean_cuda_mingru_ppo_grad", vp, GRAD_ARGS)
    f_muon = fn(G, "lean_cuda_mingru_muon_resident", vp, [sz, vp] + [sz] * 4 + [dbl] * 6 + [vp])

    def lean_chain():
        r, _ = io(G, f_prep(*[arr(G, c) for c in cols], N, T, 1))
        G.stub_release(r)
        L.call("ph_cuda_mg_obs_traj", traj.ctypes.data_as(L.dptr), N, T, Dm)
        r, v = io(G, f_load(arr(G, np.concatenate([params, np.zeros(P)])), P, None))
        h = G.stub_unbox(v)
        G.stub_release(r)
        state, w = 0x4321, params.copy()
        for _ in range(numMB):
            r, v = io(G, f_prio(N, T, 0.99, 0.95, 1.0, 1.0, mb, 0.8, 0.3, state, None))
            assert G.stub_unbox(v) == 1  # the draws stay on the device
            G.stub_release(r)
            r, v = io(G, f_grad(arr(G, w), arr(G, []), arr(G, []), mb, T, H, Dm, Ln, A, 1, arr(G, []), 0.5, 0.01,
                                0.2, 0.2, arr(G, []), arr(G, []), None))
            assert G.stub_array_size(v) == 0  # resident gradient
            G.stub_release(r)
            r, v = io(G, f_muon(h, arr(G, []), H, Dm, Ln, A, lr, wd, mu, eps, maxgn, sc, None))
            w = np.ctypeslib.as_array(G.stub_array_data(v), (max(G.stub_array_size(v), 1),))[:G.stub_array_size(v)].copy()
            assert w.size == 0  # the weights stay in the handle
            G.stub_release(r)
            state = (state + mb * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        r, v = io(G, f_down(h, P, None))
        full = np.ctypeslib.as_array(G.stub_array_data(v), (2 * P,)).copy()
        G.stub_release(r)
        r, _ = io(G, f_free(h, None))
        G.stub_release(r)
        return full

    def abi_chain():
        dp = lambda a: np.ascontiguousarray(a, np.float64).ctypes.data_as(L.dptr)
        L.call("ph_cuda_mg_prep", *[dp(c) for c in cols], N, T, 1)
        L.call("ph_cuda_mg_obs_traj", dp(traj), N, T, Dm)
        h = C.c_size_t(0)
        L.call("ph_cuda_policy_load", dp(np.concatenate([params, np.zeros(P)])), P, C.byref(h))
        state, ln, used = 0x4321, C.c_size_t(0), C.c_uint8(0)
        out = np.zeros(P + 2 * T * mb)
        for i in range(numMB):
            L.call("ph_cuda_mg_vtrace_prio", N, T, 0.99, 0.95, 1.0, 1.0, mb, 0.8, 0.3, state, C.byref(used))
            L.call("ph_cuda_mingru_ppo_grad", dp(params) if i == 0 else None, P if i == 0 else 0, None, 0, None, 0,
                   mb, T, H, Dm, Ln, A, 1, None, 0, 0.5, 0.01, 0.2, 0.2, None, 0, None, 0, dp(out), C.byref(ln))
            L.call("ph_cuda_mingru_muon_resident", h.value, None, 0, H, Dm, Ln, A, lr, wd, mu, eps, maxgn, sc, None,
                   C.byref(ln))
            state = (state + mb * 0x9E3779B97F4A7C15) & 0xFFFFFFFFFFFFFFFF
        full = np.zeros(2 * P)
        L.call("ph_cuda_policy_download", h.value, P, dp(full))
        L.call("ph_cuda_policy_free", h.value)
        return full

    a = lean_chain()
    b = abi_chain()
    assert np.all(np.isfinite(a)) and rel(a[:P] - params, np.zeros(P)) > 0
    assert np.array_equal(a, b)
    assert G.stub_live() == live


def test_mlp_policy_handle_and_benches(G):
    live = G.stub_live()
    N, D, H, O_ = 512, 12, 64, 6
    params, _ = init_mlp(D, H, O_, 0x5EA1)
    X = rng.randf(0x5EA2, N * D, -1.0, 1.0)
    ref = np.zeros(N * O_)
    O.lib().orc_mlp_forward(O.P(params), O.P(X), N, D, H, O_, O.P(ref))
    load = fn(G, "lean_ffi_mlp_policy_load", sz, [vp, sz, sz, sz])
    fwd = fn(G, "lean_ffi_mlp_policy_forward", vp, [sz, vp, sz])
    upd = fn(G, "lean_ffi_mlp_policy_update", u8, [sz, vp])
    free = fn(G, "lean_ffi_mlp_policy_free", u8, [sz])
    h = load(arr(G, params), D, H, O_)
    assert h != 0
    y = take(G, fwd(h, arr(G, X), N))
    assert y.size == N * O_ and rel(y, ref) < 1e-2
    # weights re-uploaded in place: the forward follows the new weights
    p2 = params * 0.5
    O.lib().orc_mlp_forward(O.P(p2), O.P(X), N, D, H, O_, O.P(ref))
    assert upd(h, arr(G, p2)) == 1
    y2 = take(G, fwd(h, arr(G, X), N))
    assert rel(y2, ref) < 1e-2
    y3 = take(G, fwd(h, arr(G, X[: 7 * D]), 7))  # fewer rows reuse the grown buffers
    assert np.array_equal(y3, y2[: 7 * O_])
    assert free(h) == 1
    for name, args in (("lean_ffi_bench_mlp2_bf16_resident", (4096, 32, 128, 9, 20)),
                       ("lean_ffi_bench_mlp2_bf16_wres", (4096, 32, 128, 9, 20)),
                       ("lean_ffi_bench_cublaslt_bf16_resident", (8192, 256, 512, 20))):
        gf = fn(G, name, dbl, [sz] * len(args))(*args)
        assert gf > 0.0, name
    assert fn(G, "lean_ffi_cuda_available", u8, [vp])(G.stub_array(None, 0)) == 1
    assert G.stub_live() == live
