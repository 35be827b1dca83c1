"""A whole MinGRU update through the host-buffer entries, in the call order of the reference's
trainer (MinGRUTrain.lean:786-849): resident columns and obs trajectory, then per minibatch the
device V-trace + prioritised draws, the device-column gradient (gather, BPTT, value/ratio iterate)
left resident on the device, and the resident Muon step that clips and consumes it and leaves the
weights for the next gradient (empty gClip / empty params, puffercuda.cu:5237-5248, 5727-5768);
against the same chain composed from the oracle's functions. The resident hand-off is also checked
bit for bit against the host-gradient form of the same minibatch.

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
            # the gradient decides the mode by its result length (MinGRUTrain.lean:832-849): zero = resident
            out = np.zeros(P + 2 * T * mbSegs)
            ln = C.c_size_t(0)
            L.call("ph_cuda_mingru_ppo_grad", dp(wflat) if wflat.size else None, wflat.size, None, 0, None, 0,
                   mbSegs, T, H, Dm, Lr, A, 1, None, 0, vf, ent, clip, vfclip, None, 0, None, 0, dp(out),
                   C.byref(ln))
            assert ln.value == 0  # device-column mode keeps the gradient on the device
            sc = 1.0 / (mbSegs * T)
            wout = np.zeros(P)
            wl = C.c_size_t(0)
            L.call("ph_cuda_mingru_muon_resident", h.value, None, 0, H, Dm, Lr, A, lr, wd, mu, eps, maxgn, sc,
                   dp(wout), C.byref(wl))
            assert wl.value == 0  # ... and the Muon leaves the weights there for the next gradient
            wflat = wout[:wl.value]
            state = (state + mbSegs * GOLD) & 0xFFFFFFFFFFFFFFFF
        full = np.zeros(2 * P)
        L.call("ph_cuda_policy_download", h.value, P, dp(full))
        wflat = full[:P]
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


@pytest.mark.parametrize("maxgn", [0.0, 0.05])
def test_resident_handoff_equals_host_mode(gpu, monkeypatch, maxgn):
    """One minibatch both ways from the same draws and weights: (host) the gradient returned to the host,
    clipped there, uploaded to the Muon; (resident) the gradient left on the device and clipped and
    consumed by the Muon. Without an active clip the new weights and momentum are identical bit for
    bit; with one, the clip's norm is summed in another order (device tree vs host loop), so they agree
    to 1e-13. The next gradient from the resident weights (empty params) equals the host-weights one."""
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    monkeypatch.delenv("PUFFER_MUON_EXACT", raising=False)
    N, T, Dm, H, Lr, A, B = 24, 8, 8, 16, 2, 5, 8
    P = H * Dm + H + Lr * 3 * H * H + A * H + A + H + 1
    n = N * T
    params = rng.normal(0x851, P) * 0.3
    mom = rng.normal(0x852, P) * 0.01
    rew, term = rng.normal(0x853, n), rng.bernoulli(0x854, n, 0.05)
    act = rng.randint(0x855, n, A).astype(np.float64)
    logp, val, boot = rng.randf(0x856, n, -2.5, -1.0), rng.normal(0x857, n), rng.normal(0x858, N)
    traj = rng.normal(0x859, n * Dm)
    L.call("ph_cuda_mg_prep", dp(rew), dp(term), dp(act), dp(logp), dp(val), dp(boot), N, T, 1)
    L.call("ph_cuda_mg_obs_traj", dp(traj), N, T, Dm)
    l1 = np.zeros(N)
    L.call("ph_cuda_mg_vtrace", N, T, 0.99, 0.95, 1.0, 1.0, dp(l1))
    idx, mp = np.zeros(B), np.zeros(B)
    L.call("ph_ffi_prio_sample", dp(l1), N, T, B, 0.8, 0.3, 0x77, dp(idx), dp(mp))
    adv = np.zeros(n)
    O.lib().orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(np.ones(n)), O.P(boot), N, T, 0.99, 0.95, 1.0,
                              1.0, O.P(adv))
    scal = np.zeros(6 * T * B)
    L.call("ph_ffi_gather_seq_minibatch", None, dp(act), dp(logp), dp(term), dp(adv), dp(val), dp(idx), dp(mp),
           T, B, Dm, N, dp(scal))
    obs = np.ascontiguousarray(traj.reshape(N, T, Dm)[idx.astype(np.int64)].transpose(1, 0, 2))
    args = (B, T, H, Dm, Lr, A, 1, None, 0, 0.5, 0.01, 0.2, 0.2)
    sc = 1.0 / (B * T)
    hh, hr = C.c_size_t(0), C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(np.concatenate([params, mom])), P, C.byref(hh))
    L.call("ph_cuda_policy_load", dp(np.concatenate([params, mom])), P, C.byref(hr))
    try:
        ln, wl = C.c_size_t(0), C.c_size_t(0)
        out = np.zeros(P + 2 * T * B)
        # host form
        L.call("ph_cuda_mingru_ppo_grad", dp(params), P, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0,
               None, 0, dp(out), C.byref(ln))
        assert ln.value == out.size
        gclip = grad_clip(out[:P], maxgn, sc)
        w_host = np.zeros(P)
        L.call("ph_cuda_mingru_muon_resident", hh.value, dp(gclip), P, H, Dm, Lr, A, 0.02, 0.0, 0.95, 1e-7, maxgn,
               sc, dp(w_host), C.byref(wl))
        assert wl.value == P
        # resident form, same draws (device gather of the same columns)
        L.call("ph_cuda_mingru_ppo_grad", dp(params), P, None, 0, None, 0, *args, dp(idx), B, dp(mp), B, dp(out),
               C.byref(ln))
        assert ln.value == 0
        g_res = np.zeros(P)
        L.call("ph_cuda_mg_resident_grad", P, dp(g_res))
        L.call("ph_cuda_mingru_muon_resident", hr.value, None, 0, H, Dm, Lr, A, 0.02, 0.0, 0.95, 1e-7, maxgn, sc,
               None, C.byref(wl))
        assert wl.value == 0
        with pytest.raises(L.PufferHipError, match="no resident gradient"):  # the stamp was consumed
            L.call("ph_cuda_mingru_muon_resident", hr.value, None, 0, H, Dm, Lr, A, 0.02, 0.0, 0.95, 1e-7, maxgn,
                   sc, None, C.byref(wl))
        fh, fr = np.zeros(2 * P), np.zeros(2 * P)
        L.call("ph_cuda_policy_download", hh.value, P, dp(fh))
        L.call("ph_cuda_policy_download", hr.value, P, dp(fr))
        assert np.array_equal(fh[:P], w_host)
        if maxgn == 0.0:
            assert np.array_equal(fr, fh)
        else:
            assert rel(fr[:P] - params, fh[:P] - params) < 1e-13 and rel(fr[P:], fh[P:]) < 1e-13
        # the next gradient: empty params take the resident handle's weights (the last Muon's handle)
        o1, o2 = np.zeros(P + 2 * T * B), np.zeros(P + 2 * T * B)
        L.call("ph_cuda_mingru_ppo_grad", None, 0, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0, None, 0,
               dp(o1), C.byref(ln))
        L.call("ph_cuda_mingru_ppo_grad", dp(fr[:P]), P, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0,
               None, 0, dp(o2), C.byref(ln))
        assert np.array_equal(o1, o2)
    finally:
        L.call("ph_cuda_policy_free", hh.value)
        L.call("ph_cuda_policy_free", hr.value)
    with pytest.raises(L.PufferHipError, match="no resident weights"):  # freed with its handle
        L.call("ph_cuda_mingru_ppo_grad", None, 0, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0, None, 0,
               dp(o1), C.byref(ln))

