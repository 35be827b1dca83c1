"""A whole MinGRU update through the host-buffer entries, in the call order of the reference's
trainer (MinGRUTrain.lean:786-849): resident columns and obs trajectory, then per minibatch the
device V-trace + prioritised draws, the device-column gradient (gather, BPTT, value/ratio iterate),
the trainer's gradient clip (MinGRUTrain.lean:640-649) and the resident Muon step; against the same
chain composed from the oracle's functions.

Bars: per-minibatch segment sums within 1e-6 relative and identical draws; the final weights'
change within 1e-3 relative of the oracle chain's (fp32 BPTT against f64, exact-tier Muon).
"""
import ctypes as C

import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu

GOLD = 0x9E3779B97F4A7C15
REF = O.coeffs_array(O.REF_COEFFS)


def dp(a):
    return np.ascontiguousarray(a, np.float64).ctypes.data_as(C.POINTER(C.c_double))


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def grad_clip(g, max_norm, sc):
    """The trainer's clip (MinGRUTrain.lean:640-649): g * sc * min(1, maxNorm / |g * sc|)."""
    gnorm = np.sqrt(np.sum((g * sc) ** 2))
    cc = (max_norm / gnorm if (max_norm > 0 and gnorm > max_norm) else 1.0) * sc
    return g * cc


def oracle_muon(w, m, g, H, Dm, Lr, A, lr, wd, mu, eps):
    w, m = w.copy(), m.copy()
    szE, szL = H * Dm, 3 * H * H
    offW = szE + H
    offDec = offW + Lr * szL
    mats = [(0, H, Dm)] + [(offW + l * szL, 3 * H, H) for l in range(Lr)] + [(offDec, A, H),
                                                                            (offDec + A * H + A, 1, H)]
    vecs = [(szE, H), (offDec + A * H, A), (offDec + A * H + A + H, 1)]
    for off, r, c in mats:
        k = r * c
        a, b = np.zeros(k), np.zeros(k)
        O.lib().orc_muon_mat(r, c, O.P(w[off:off + k].copy()), O.P(g[off:off + k].copy()),
                             O.P(m[off:off + k].copy()), O.P(a), O.P(b), 1.0, lr, wd, mu, eps, O.P(REF), 5, 0)
        w[off:off + k], m[off:off + k] = a, b
    for off, k in vecs:
        a, b = np.zeros(k), np.zeros(k)
        O.lib().orc_stepvec(k, O.P(w[off:off + k].copy()), O.P(g[off:off + k].copy()), O.P(m[off:off + k].copy()),
                            O.P(a), O.P(b), 1.0, lr, wd, mu)
        w[off:off + k], m[off:off + k] = a, b
    return w, m


def test_mingru_update_chain_matches_oracle(gpu, monkeypatch):
    monkeypatch.setenv("PUFFER_MUON_EXACT", "1")
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    monkeypatch.delenv("PUFFER_MG_DEVPRIO", raising=False)
    N, T, Dm, H, Lr, A = 16, 8, 8, 16, 2, 5
    mbSegs, numMB = 6, 3
    gam, lam, rc, cc = 0.99, 0.95, 1.0, 1.0
    alpha, beta = 0.8, 0.3
    lr, wd, mu, eps, maxgn = 0.02, 0.0, 0.95, 1e-7, 0.5
    vf, ent, clip, vfclip = 0.5, 0.01, 0.2, 0.2
    P = H * Dm + H + Lr * 3 * H * H + A * H + A + H + 1
    n = N * T
    params = rng.normal(0x801, P) * 0.3
    mom = np.zeros(P)
    rew = rng.normal(0x802, n)
    term = rng.bernoulli(0x803, n, 0.05)
    act = rng.randint(0x804, n, A).astype(np.float64)
    logp = rng.randf(0x805, n, -2.5, -1.0)
    val = rng.normal(0x806, n)
    boot = rng.normal(0x807, N)
    traj = rng.normal(0x808, n * Dm)  # row e*T + t

    # ---- device chain, as the trainer calls it
    L.call("ph_cuda_mg_prep", dp(rew), dp(term), dp(act), dp(logp), dp(val), dp(boot), N, T, 1)
    L.call("ph_cuda_mg_obs_traj", dp(traj), N, T, Dm)
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(np.concatenate([params, mom])), P, C.byref(h))
    dev_draws, dev_l1 = [], []
    try:
        wflat, state = params.copy(), 0x1234
        for _ in range(numMB):
            l1 = np.zeros(N)
            L.call("ph_cuda_mg_vtrace", N, T, gam, lam, rc, cc, dp(l1))  # the sums the draws below use
            idx, mp = np.zeros(mbSegs), np.zeros(mbSegs)
            L.call("ph_ffi_prio_sample", dp(l1), N, T, mbSegs, alpha, beta, state, dp(idx), dp(mp))
            dev_l1.append(l1)
            dev_draws.append(idx)
            used = C.c_uint8(0)
            L.call("ph_cuda_mg_vtrace_prio", N, T, gam, lam, rc, cc, mbSegs, alpha, beta, state, C.byref(used))
            assert used.value == 1
            out = np.zeros(P + 2 * T * mbSegs)
            L.call("ph_cuda_mingru_ppo_grad", dp(wflat), None, 0, None, 0, mbSegs, T, H, Dm, Lr, A, 1, None, 0, vf,
                   ent, clip, vfclip, None, 0, None, 0, dp(out))
            sc = 1.0 / (mbSegs * T)
            gclip = grad_clip(out[:P], maxgn, sc)
            wout = np.zeros(P)
            L.call("ph_cuda_mingru_muon_resident", h.value, dp(gclip), P, H, Dm, Lr, A, lr, wd, mu, eps, maxgn, sc,
                   dp(wout))
            wflat = wout
            state = (state + mbSegs * GOLD) & 0xFFFFFFFFFFFFFFFF
    finally:
        L.call("ph_cuda_policy_free", h.value)

    # ---- the same chain from the oracle's functions
    value, ratio = val.copy(), np.ones(n)
    w, m, state = params.copy(), mom.copy(), 0x1234
    obs3 = traj.reshape(N, T, Dm)
    for mb in range(numMB):
        adv = np.zeros(n)
        O.lib().orc_vtrace_mingru(O.P(rew), O.P(value), O.P(term), O.P(ratio), O.P(boot), N, T, gam, lam, rc, cc,
                                  O.P(adv))
        l1 = O.seg_l1(adv, N, T)
        assert rel(dev_l1[mb], l1) < 1e-6, mb
        idx, mp, _, _ = O.prio_sample(l1, mbSegs, alpha, beta, state)
        assert np.array_equal(idx, dev_draws[mb]), mb
        scal, _ = O.gather_seq_minibatch(act, logp, term, adv, value, idx, mp, T)
        nb = T * mbSegs
        cols = [scal[k * nb:(k + 1) * nb].reshape(T, mbSegs) for k in range(6)]  # act adv ret old term ov
        g = np.zeros(P)
        nlp, nv = np.zeros((T, mbSegs)), np.zeros((T, mbSegs))
        for bi in range(mbSegs):
            o = np.zeros(P + 2 * T)
            seq = [O.f64(c[:, bi]) for c in cols]
            O.lib().orc_mingru_ppo_grad_seq(O.P(w), O.P(O.f64(obs3[int(idx[bi])])), O.P(seq[0]),
                                            O.P(seq[1]), O.P(seq[2]), O.P(seq[3]), O.P(seq[4]), O.P(seq[5]), T, H, Dm,
                                            Lr, A, vf, ent, clip, vfclip, O.P(o))
            g += o[:P]
            nlp[:, bi], nv[:, bi] = o[P:P + T], o[P + T:]
        w, m = oracle_muon(w, m, grad_clip(g, maxgn, 1.0 / nb), H, Dm, Lr, A, lr, wd, mu, eps)
        value, ratio = O.mb_iterate(value, ratio, logp, nlp.ravel().astype(np.float32),
                                    nv.ravel().astype(np.float32), idx, T)
        state = (state + mbSegs * GOLD) & 0xFFFFFFFFFFFFFFFF
    assert rel(wflat - params, w - params) < 1e-3
