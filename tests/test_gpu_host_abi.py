"""Host-buffer entry points (the Lean @[extern] mirror) on the GPU, driven by the reference's own
verify-* inputs (Exe/Puffer.lean: same seeds, shapes and interleaved draw order) and checked against
the oracle with the tolerances of the path: bit-exact for the f64 scans and the exact-tier Muon,
1e-5 relative for fp32 GEMM work, 1e-2 relative for bf16 MFMA work.
"""
import ctypes as C
import math
import os

import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def dp(a):
    return np.ascontiguousarray(a, np.float64).ctypes.data_as(C.POINTER(C.c_double))


class Stream:
    """Sequential splitmix64 draws as the reference's `randF lo hi rng` chain consumes them."""

    def __init__(self, seed):
        self.seed, self.i = seed, 0

    def u(self, n=1):
        w = rng.words(self.seed, n, self.i)
        self.i += n
        return rng.uniform01(w)

    def randf(self, lo, hi, n=1):
        return lo + (hi - lo) * self.u(n)


def init_mlp(din, H, dout, seed):
    """initMLP (Puffer/RL/NNTrain.lean:418-422): W1 ~ U[-s1, s1) with s1 = sqrt(2)/sqrt(din), W2 ~
    U[-s2, s2) with s2 = 1/sqrt(H), row-major draws; zero biases. Returns (flat params, stream)."""
    s = Stream(seed)
    s1 = math.sqrt(2.0) * (1.0 / math.sqrt(din))
    s2 = 1.0 / math.sqrt(H)
    W1 = s.u(H * din) * (2.0 * s1) - s1
    W2 = s.u(dout * H) * (2.0 * s2) - s2
    return np.concatenate([W1, np.zeros(H), W2, np.zeros(dout)]), s


def mlp_batch(s, N, D, A, adv_lo=-1.0, adv_hi=1.0):
    obs, acts, adv, ret, olp = [], [], [], [], []
    for _ in range(N):
        obs.append(s.randf(-1.0, 1.0, D))
        acts.append(math.floor(s.randf(0.0, float(A))[0]))
        adv.append(s.randf(adv_lo, adv_hi)[0])
        ret.append(s.randf(-1.0, 1.0)[0])
        olp.append(s.randf(-1.5, 0.0)[0])
    return (np.concatenate(obs), np.array(acts, np.float64), np.array(adv), np.array(ret), np.array(olp))


def vt_inputs(seed, B, T, boot=False):
    s = Stream(seed)
    rew, val, term, imp = [], [], [], []
    for _ in range(B * T):
        rew.append(s.randf(-1.5, 1.5)[0])
        val.append(s.randf(-2.0, 2.0)[0])
        term.append(1.0 if s.randf(0.0, 1.0)[0] < 0.12 else 0.0)
        imp.append(s.randf(0.1, 2.0)[0])
    out = [np.array(v) for v in (rew, val, term, imp)]
    if boot:
        out.append(s.randf(-2.0, 2.0, B))
    return out


REF = O.coeffs_array(O.REF_COEFFS)


# ---- V-trace / advantage normalisation -------------------------------------------------------------
def test_vtrace_verify_inputs_bit_exact(gpu):
    B, T = 8, 12
    rew, val, term, imp = vt_inputs(0x5C1A, B, T)
    got = np.zeros(B * T)
    L.call("ph_cuda_vtrace", dp(rew), dp(val), dp(term), dp(imp), B, T, 0.99, 0.95, 2.1, 1.08, dp(got))
    ref = np.zeros(B * T)
    O.lib().orc_vtrace_vec(O.P(rew), O.P(val), O.P(term), O.P(imp), B, T, 0.99, 0.95, 2.1, 1.08, O.P(ref))
    assert np.array_equal(got, ref)


def test_vtrace_mingru_verify_inputs_bit_exact(gpu):
    B, T = 8, 12
    rew, val, term, imp, boot = vt_inputs(0x5C1B, B, T, boot=True)
    got = np.zeros(B * T)
    L.call("ph_cuda_vtrace_mingru", dp(rew), dp(val), dp(term), dp(imp), dp(boot), B, T, 0.99, 0.95, 2.1,
           1.08, dp(got))
    ref = np.zeros(B * T)
    O.lib().orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(imp), O.P(boot), B, T, 0.99, 0.95, 2.1, 1.08,
                              O.P(ref))
    assert np.array_equal(got, ref)


@pytest.mark.parametrize("n", [257, 1, 100003])
def test_adv_normalize(gpu, n):
    adv = Stream(0xAD7).randf(-3.0, 3.0, n)
    got = np.zeros(n)
    L.call("ph_cuda_adv_normalize", dp(adv), n, dp(got))
    ref = np.zeros(n)
    O.lib().orc_adv_normalize(O.P(adv), n, O.P(ref))
    # a parallel fold vs the sequential one: a normalisation, equal to roundoff
    np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)


# ---- MLP PPO gradient and whole steps ------------------------------------------------------------------
def test_mlp_ppo_grad_verify_inputs(gpu):
    N, D, H, A = 64, 12, 16, 5
    Ocnt = A + 1
    params, s = init_mlp(D, H, Ocnt, 0x9A73)
    obs, acts, adv, ret, olp = mlp_batch(s, N, D, A)
    Pn = params.size
    ref = np.zeros(Pn)
    O.lib().orc_mlp_ppo_grad(O.P(params), O.P(obs), O.P(acts), O.P(adv), O.P(ret), O.P(olp), N, H, D, A, 0.5,
                             0.01, 0.2, O.P(ref), 1)
    for bf, tol in ((0, 1e-5), (1, 1e-2)):
        g = np.zeros(Pn)
        L.call("ph_cuda_mlp_ppo_grad", dp(params), dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), N, H, D, A, 0.5,
               0.01, 0.2, bf, dp(g))
        assert rel(g, ref) < tol, (bf, rel(g, ref))


def oracle_train_step(pm, obs, acts, adv, ret, olp, N, H, D, A, lr, wd, mu, eps):
    """normalizeAdv -> mlpPPOGradBatchBlas -> (mean) -> applyMuon (the reference's shadow oracle of
    verify-train-step-gpu, Exe/Puffer.lean:1210-1226)."""
    Pn = H * D + H + (A + 1) * H + A + 1
    advn = np.zeros(N)
    O.lib().orc_adv_normalize(O.P(adv), N, O.P(advn))
    g = np.zeros(Pn)
    O.lib().orc_mlp_ppo_grad(O.P(pm[:Pn]), O.P(obs), O.P(acts), O.P(advn), O.P(ret), O.P(olp), N, H, D, A, 0.5,
                             0.01, 0.2, O.P(g), 1)
    out = np.zeros(2 * Pn)
    O.lib().orc_muon_step_mlp(O.P(pm), O.P(g), H, D, A + 1, 1.0 / N, lr, wd, mu, eps, O.P(out))
    return out


def test_train_step_verify_inputs(gpu):
    N, D, H, A = 96, 12, 16, 5
    params, s = init_mlp(D, H, A + 1, 0x77E5)
    obs, acts, adv, ret, olp = mlp_batch(s, N, D, A, -2.0, 2.0)
    Pn = params.size
    mom = s.randf(-0.1, 0.1, Pn)
    pm = np.concatenate([params, mom])
    ref = oracle_train_step(pm, obs, acts, adv, ret, olp, N, H, D, A, 0.1, 0.0, 0.95, 1e-7)
    for bf, tol in ((0, 1e-5), (1, 2e-2)):
        out = np.zeros(2 * Pn)
        L.call("ph_cuda_train_step", dp(pm), dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), N, H, D, A, 0.1, 0.0,
               0.95, 1e-7, 0.5, 0.01, 0.2, bf, dp(out))
        assert rel(out[:Pn] - params, ref[:Pn] - params) < tol, (bf, rel(out[:Pn] - params, ref[:Pn] - params))
        assert rel(out[Pn:], ref[Pn:]) < tol, (bf, rel(out[Pn:], ref[Pn:]))


def update_inputs(NT=48, D=12, H=16, A=5, epochs=3):
    """verify-train-update-resident shapes (Exe/Puffer.lean:1228-1262); the permutations are seeded
    numpy shuffles (the property checked does not depend on which permutation)."""
    Pn = H * D + H + (A + 1) * H + A + 1
    s = Stream(0x9A7C33)
    pm0 = s.randf(-0.3, 0.3, 2 * Pn)
    obs = s.randf(-1.0, 1.0, NT * D)
    acts, adv, ret, olp = [], [], [], []
    for _ in range(NT):
        acts.append(math.floor(s.randf(0.0, float(A))[0]))
        adv.append(s.randf(-2.0, 2.0)[0])
        ret.append(s.randf(-1.0, 1.0)[0])
        olp.append(s.randf(-1.5, 0.0)[0])
    r = np.random.default_rng(0x1234)
    perms = [r.permutation(NT) for _ in range(epochs)]
    return Pn, pm0, obs, np.array(acts, np.float64), np.array(adv), np.array(ret), np.array(olp), perms


def test_train_update_equals_minibatch_loop(gpu):
    """Whole update on device == looping the single-step entry over the same minibatches (the
    reference's verify-train-update-resident check): bit-exact in the fp32 tier."""
    NT, D, H, A, epochs, numMB = 48, 12, 16, 5, 3, 4
    Pn, pm0, obs, acts, adv, ret, olp, perms = update_inputs(NT, D, H, A, epochs)
    permflat = np.concatenate(perms).astype(np.float64)
    got = np.zeros(2 * Pn)
    L.call("ph_cuda_train_update", dp(pm0), dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), dp(permflat), NT, D, H,
           A, epochs, numMB, 0.05, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0, dp(got))
    pm = pm0.copy()
    mb = NT // numMB
    for e in range(epochs):
        for m in range(numMB):
            lo, hi = m * mb, (NT if m + 1 == numMB else (m + 1) * mb)
            idx = perms[e][lo:hi]
            ob = obs.reshape(NT, D)[idx].ravel()
            out = np.zeros(2 * Pn)
            L.call("ph_cuda_train_step", dp(pm), dp(ob), dp(acts[idx]), dp(adv[idx]), dp(ret[idx]), dp(olp[idx]),
                   len(idx), H, D, A, 0.05, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0, dp(out))
            pm = out
    assert np.array_equal(got, pm)


def test_train_update_resident_matches_host_update(gpu):
    NT, D, H, A, epochs, numMB = 48, 12, 16, 5, 3, 4
    Pn, pm0, obs, acts, adv, ret, olp, perms = update_inputs(NT, D, H, A, epochs)
    permflat = np.concatenate(perms).astype(np.float64)
    host = np.zeros(2 * Pn)
    L.call("ph_cuda_train_update", dp(pm0), dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), dp(permflat), NT, D, H,
           A, epochs, numMB, 0.05, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0, dp(host))
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm0), Pn, C.byref(h))
    try:
        peek = np.zeros(1)
        L.call("ph_cuda_train_update_resident", h.value, dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), None, 0,
               dp(permflat), NT, D, H, A, epochs, numMB, 0.05, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, 0.0, 0.0, 0,
               dp(peek))
        res = np.zeros(2 * Pn)
        L.call("ph_cuda_policy_download", h.value, Pn, dp(res))
    finally:
        L.call("ph_cuda_policy_free", h.value)
    assert np.array_equal(res, host)
    assert peek[0] == host[0]


def test_train_update_resident_value_clip_and_grad_clip(gpu):
    """One minibatch, one epoch, with the value-loss clip and the global grad-norm clip, against an
    f64 chain: forward (orc_mlp_forward), per-row PPO gradient with the clip (orc_ppo_grad), f64
    backward, orc_gclip, exact Muon (orc_muon_step_mlp with gscale 1 on the clipped gradient)."""
    NT, D, H, A = 48, 12, 16, 5
    Pn, pm0, obs, acts, adv, ret, olp, _ = update_inputs(NT, D, H, A, 1)
    ov = Stream(0x0F0F).randf(-1.0, 1.0, NT)
    ident = np.arange(NT, dtype=np.float64)
    vfclip, mgn = 0.1, 0.05
    # oracle
    Oc = A + 1
    W1, b1 = pm0[:H * D].reshape(H, D), pm0[H * D:H * D + H]
    W2 = pm0[H * D + H:H * D + H + Oc * H].reshape(Oc, H)
    X = obs.reshape(NT, D)
    H1 = np.maximum(X @ W1.T + b1, 0.0)
    out = np.zeros(NT * Oc)
    O.lib().orc_mlp_forward(O.P(pm0[:Pn]), O.P(obs), NT, D, H, Oc, O.P(out))
    out = out.reshape(NT, Oc)
    advn = np.zeros(NT)
    O.lib().orc_adv_normalize(O.P(adv), NT, O.P(advn))
    dl, dv, _, _ = O.ppo_grad(out[:, :A], out[:, A], acts, advn, ret, olp, ov, vf=0.5, ent=0.01, clip=0.2,
                              vfclip=vfclip, max_shift=False)
    dOut = np.concatenate([dl, dv.reshape(NT, 1)], axis=1)
    dZ = (dOut @ W2) * (H1 > 0)
    g = np.concatenate([(dZ.T @ X).ravel(), dZ.sum(0), (dOut.T @ H1).ravel(), dOut.sum(0)])
    O.lib().orc_gclip(O.P(g), Pn, 1.0 / NT, mgn)
    ref = np.zeros(2 * Pn)
    O.lib().orc_muon_step_mlp(O.P(pm0), O.P(g), H, D, Oc, 1.0, 0.05, 0.0, 0.95, 1e-7, O.P(ref))
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm0), Pn, C.byref(h))
    try:
        peek = np.zeros(1)
        L.call("ph_cuda_train_update_resident", h.value, dp(obs), dp(acts), dp(adv), dp(ret), dp(olp), dp(ov), NT,
               dp(ident), NT, D, H, A, 1, 1, 0.05, 0.0, 0.95, 1e-7, 0.5, 0.01, 0.2, vfclip, mgn, 0, dp(peek))
        res = np.zeros(2 * Pn)
        L.call("ph_cuda_policy_download", h.value, Pn, dp(res))
    finally:
        L.call("ph_cuda_policy_free", h.value)
    assert rel(res[:Pn] - pm0[:Pn], ref[:Pn] - pm0[:Pn]) < 1e-5
    assert rel(res[Pn:], ref[Pn:]) < 1e-5


# ---- Muon ------------------------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(16, 24), (24, 16), (20, 20)])
def test_muon_stepmat_verify_inputs_bit_exact(gpu, shape):
    rows, cols = shape
    n = rows * cols
    s = Stream(0x3E7A)
    # the reference draws the three shapes from one continuing stream; each shape here restarts at
    # the offset the earlier shapes consumed
    for r0, c0 in [(16, 24), (24, 16), (20, 20)]:
        if (r0, c0) == shape:
            break
        s.u(3 * r0 * c0)
    W, G, M = np.zeros(n), np.zeros(n), np.zeros(n)
    for i in range(n):
        W[i] = s.randf(-0.5, 0.5)[0]
        G[i] = s.randf(-0.3, 0.3)[0]
        M[i] = s.randf(-0.2, 0.2)[0]
    got = np.zeros(2 * n)
    L.call("ph_cuda_muon_stepmat", dp(W), dp(G), dp(M), rows, cols, 0.1, 0.0, 0.95, 1e-7, dp(got))
    nW, nM = np.zeros(n), np.zeros(n)
    O.lib().orc_muon_mat(rows, cols, O.P(W), O.P(G), O.P(M), O.P(nW), O.P(nM), 1.0, 0.1, 0.0, 0.95, 1e-7, O.P(REF), 5,
                         0)
    assert np.array_equal(got[:n], nW)
    assert np.array_equal(got[n:], nM)


def test_muon_step_mlp_resident_verify_inputs_bit_exact(gpu):
    H, D, Oc = 24, 16, 6
    Pn = H * D + H + Oc * H + Oc
    s = Stream(0x51A7)
    par, grad, mom = np.zeros(Pn), np.zeros(Pn), np.zeros(Pn)
    for i in range(Pn):
        par[i] = s.randf(-0.5, 0.5)[0]
        grad[i] = s.randf(-2.0, 2.0)[0]
        mom[i] = s.randf(-0.1, 0.1)[0]
    pm = np.concatenate([par, mom])
    ref = np.zeros(2 * Pn)
    O.lib().orc_muon_step_mlp(O.P(pm), O.P(grad), H, D, Oc, 1.0 / 64.0, 0.1, 0.0, 0.95, 1e-7, O.P(ref))
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm), Pn, C.byref(h))
    try:
        newp = np.zeros(Pn)
        L.call("ph_cuda_muon_step_mlp_resident", h.value, dp(grad), H, D, Oc, 1.0 / 64.0, 0.1, 0.0, 0.95, 1e-7,
               dp(newp))
        full = np.zeros(2 * Pn)
        L.call("ph_cuda_policy_download", h.value, Pn, dp(full))
    finally:
        L.call("ph_cuda_policy_free", h.value)
    assert np.array_equal(newp, ref[:Pn])
    assert np.array_equal(full, ref)


def test_policy_handle_roundtrip(gpu):
    Pn = 1001
    pm = Stream(0x77).randf(-1, 1, 2 * Pn)
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm), Pn, C.byref(h))
    assert h.value != 0
    back = np.zeros(2 * Pn)
    L.call("ph_cuda_policy_download", h.value, Pn, dp(back))
    L.call("ph_cuda_policy_free", h.value)
    assert np.array_equal(back, pm)


# ---- dense forward ----------------------------------------------------------------------------------
def test_dense_forward_f64_bit_exact_and_bf16(gpu):
    N, D, H = 300, 37, 65
    s = Stream(0xDE45)
    X, W, b = s.randf(-1, 1, N * D), s.randf(-0.5, 0.5, H * D), s.randf(-0.2, 0.2, H)
    ref = np.zeros(N * H)
    O.lib().orc_dense_forward(O.P(X), O.P(W), O.P(b), N, D, H, O.P(ref))
    got = np.zeros(N * H)
    L.call("ph_ffi_dense_forward_gpu", dp(X), dp(W), dp(b), N, D, H, dp(got))
    assert np.array_equal(got, ref)
    L.call("ph_ffi_dense_forward_bf16", dp(X), dp(W), dp(b), N, D, H, dp(got))
    assert rel(got, ref) < 1e-2


def test_mlp_forward_batch_bf16(gpu):
    N, D, H, Oc = 512, 16, 128, 3
    params, s = init_mlp(D, H, Oc, 0xF0F0)
    X = s.randf(-1, 1, N * D)
    ref = np.zeros(N * Oc)
    O.lib().orc_mlp_forward(O.P(params), O.P(X), N, D, H, Oc, O.P(ref))
    got = np.zeros(N * Oc)
    L.call("ph_ffi_mlp_forward_batch_bf16", dp(params), dp(X), N, D, H, Oc, dp(got))
    assert rel(got, ref) < 1e-2


def test_availability_and_bench(gpu):
    assert L.lib().ph_ffi_cuda_available() == 1
    gf = L.lib().ph_ffi_bench_bf16_resident(4096, 256, 256, 5)
    assert gf > 0


# ---- MinGRU host mode -------------------------------------------------------------------------------
def test_mingru_grad_host_mode_matches_oracle(gpu, monkeypatch):
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    B, T, D, H, Ln, A = 8, 16, 8, 16, 2, 5
    n = B * T
    Pn = H * D + H + Ln * 3 * H * H + A * H + A + H + 1
    p = rng.normal(0x1A1, Pn) * 0.3
    obs = rng.normal(0x1A2, n * D).reshape(T, B, D)
    act = rng.randint(0x1A3, n, A).reshape(T, B).astype(np.float64)
    adv = rng.normal(0x1A4, n).reshape(T, B)
    ret = rng.normal(0x1A5, n).reshape(T, B)
    old = rng.randf(0x1A6, n, -2.5, -1.0).reshape(T, B)
    term = rng.bernoulli(0x1A7, n, 0.05).reshape(T, B)
    ov = rng.normal(0x1A8, n).reshape(T, B)
    scal = np.concatenate([a.ravel() for a in (act, adv, ret, old, term, ov)])
    out = np.zeros(Pn + 2 * n)
    ln = C.c_size_t(0)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), n * D, dp(scal), 6 * n, B, T, H, D, Ln, A, 1, None, 0,
           0.5, 0.01, 0.2, 0.2, None, 0, None, 0, dp(out), C.byref(ln))
    assert ln.value == out.size
    g = np.zeros(Pn)
    nlp = np.zeros((T, B))
    for b in range(B):
        o = np.zeros(Pn + 2 * T)
        O.lib().orc_mingru_ppo_grad_seq(O.P(p), O.P(O.f64(obs[:, b, :])), O.P(O.f64(act[:, b])), O.P(O.f64(adv[:, b])),
                                        O.P(O.f64(ret[:, b])), O.P(O.f64(old[:, b])), O.P(O.f64(term[:, b])),
                                        O.P(O.f64(ov[:, b])), T, H, D, Ln, A, 0.5, 0.01, 0.2, 0.2, O.P(o))
        g += o[:Pn]
        nlp[:, b] = o[Pn:Pn + T]
    assert rel(out[:Pn], g) < 1e-5
    assert rel(out[Pn:Pn + n], nlp.ravel()) < 1e-5


def test_mingru_muon_resident_host_gradient(gpu, monkeypatch):
    H, D, Ln, A = 16, 8, 2, 5
    Pn = H * D + H + Ln * 3 * H * H + A * H + A + H + 1
    s = Stream(0x2B2B)
    W, G, M = s.randf(-0.5, 0.5, Pn), s.randf(-0.3, 0.3, Pn), s.randf(-0.1, 0.1, Pn)
    # oracle: exact Muon per flattenMG matrix (reference op order), stepvec per bias
    ref_w, ref_m = W.copy(), M.copy()
    szE, szL = H * D, 3 * H * H
    offW = szE + H
    offDec = offW + Ln * szL
    mats = [(0, H, D)] + [(offW + l * szL, 3 * H, H) for l in range(Ln)] + [(offDec, A, H), (offDec + A * H + A, 1, H)]
    vecs = [(szE, H), (offDec + A * H, A), (offDec + A * H + A + H, 1)]
    for off, r, c in mats:
        k = r * c
        a, bb = np.zeros(k), np.zeros(k)
        O.lib().orc_muon_mat(r, c, O.P(W[off:off + k].copy()), O.P(G[off:off + k].copy()), O.P(M[off:off + k].copy()),
                             O.P(a), O.P(bb), 1.0, 0.02, 0.0, 0.95, 1e-7, O.P(REF), 5, 0)
        ref_w[off:off + k], ref_m[off:off + k] = a, bb
    for off, k in vecs:
        a, bb = np.zeros(k), np.zeros(k)
        O.lib().orc_stepvec(k, O.P(W[off:off + k].copy()), O.P(G[off:off + k].copy()), O.P(M[off:off + k].copy()),
                            O.P(a), O.P(bb), 1.0, 0.02, 0.0, 0.95)
        ref_w[off:off + k], ref_m[off:off + k] = a, bb
    for exact, tol in (("1", 0.0), ("0", 1e-4)):
        monkeypatch.setenv("PUFFER_MUON_EXACT", exact)
        h = C.c_size_t(0)
        L.call("ph_cuda_policy_load", dp(np.concatenate([W, M])), Pn, C.byref(h))
        try:
            wout = np.zeros(Pn)
            wl = C.c_size_t(0)
            L.call("ph_cuda_mingru_muon_resident", h.value, dp(G), Pn, H, D, Ln, A, 0.02, 0.0, 0.95, 1e-7, 0.5, 1.0,
                   dp(wout), C.byref(wl))
            assert wl.value == Pn
            full = np.zeros(2 * Pn)
            L.call("ph_cuda_policy_download", h.value, Pn, dp(full))
        finally:
            L.call("ph_cuda_policy_free", h.value)
        assert np.array_equal(wout, full[:Pn])
        if tol == 0.0:
            assert np.array_equal(full[:Pn], ref_w) and np.array_equal(full[Pn:], ref_m)
        else:
            assert rel(full[:Pn] - W, ref_w - W) < tol
            assert rel(full[Pn:], ref_m) < 1e-12  # momentum is f64 in both tiers
