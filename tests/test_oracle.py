"""Pins the CPU oracle: known answers, closed forms, invariants, brute force and finite differences.

None of these checks retypes the oracle's formula: each uses a different formulation (a textbook
identity, an explicit sum, a finite difference, a library routine) so a dropped term, a wrong sign
or index, or a transposed operand fails at least one of them.
"""
import ctypes as C
import math

import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import rng

L = O.lib()


# ---------------------------------------------------------------------------------------------
# generator

def test_splitmix64_known_answer():
    # Published splitmix64 outputs for seed 0 (Vigna's reference implementation).
    expect = [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F, 0xF88BB8A8724C81EC]
    s = C.c_uint64(0)
    got = [L.orc_rng_next(C.byref(s)) for _ in range(4)]
    assert got == expect
    assert [int(w) for w in rng.words(0, 4)] == expect


def test_python_and_c_generators_agree():
    s = C.c_uint64(0x5C1A)
    out = np.zeros(1000)
    L.orc_randf(O.P(out), 1000, -1.5, 1.5, C.byref(s))
    assert np.array_equal(out, rng.randf(0x5C1A, 1000, -1.5, 1.5))
    assert s.value == rng.state_after(0x5C1A, 1000)


# ---------------------------------------------------------------------------------------------
# V-trace / GAE

def _vt_inputs(seed, B, T, p_done=0.12):
    """The reference's verify-vtrace-gpu draw order (Exe/Puffer.lean:1075-1084)."""
    w = rng.uniform01(rng.words(seed, 4 * B * T)).reshape(B * T, 4)
    rew = -1.5 + (1.5 - -1.5) * w[:, 0]
    val = -2.0 + (2.0 - -2.0) * w[:, 1]
    term = (w[:, 2] < p_done).astype(np.float64)
    imp = 0.1 + (2.0 - 0.1) * w[:, 3]
    return rew, val, term, imp


def _vec(rew, val, term, imp, B, T, g, lam, rb, cb):
    adv = np.zeros(B * T)
    L.orc_vtrace_vec(O.P(rew), O.P(val), O.P(term), O.P(imp), B, T, g, lam, rb, cb, O.P(adv))
    return adv


def _brute_vec(rew, val, term, imp, T, g, lam, rb, cb):
    """adv_t = sum_{s=t}^{T-2} (g*lam)^{s-t} (prod_{u=t}^{s-1} c_u nnt_u) delta_s  (one segment)."""
    r = np.clip(rew, -1, 1)
    nnt = (term == 0).astype(float)
    rho = np.minimum(imp, rb)
    c = np.minimum(imp, cb)
    delta = [rho[t] * (r[t] + g * val[t + 1] * nnt[t] - val[t]) for t in range(T - 1)]
    out = np.zeros(T)
    for t in range(T - 1):
        tot, w = 0.0, 1.0
        for s in range(t, T - 1):
            tot += w * delta[s]
            w *= g * lam * c[s] * nnt[s]
        out[t] = tot
    return out


def test_vtrace_vec_brute_force():
    B, T = 5, 9
    rew, val, term, imp = _vt_inputs(0x5C1A, B, T)
    adv = _vec(rew, val, term, imp, B, T, 0.99, 0.95, 2.1, 1.08).reshape(B, T)
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        ref = _brute_vec(rew[sl], val[sl], term[sl], imp[sl], T, 0.99, 0.95, 2.1, 1.08)
        np.testing.assert_allclose(adv[b], ref, rtol=1e-12, atol=1e-12)


def test_vtrace_vec_is_gae_at_unit_ratio():
    B, T = 16, 33
    rew, val, term, _ = _vt_inputs(0x1111, B, T)
    imp = np.ones(B * T)
    adv = _vec(rew, val, term, imp, B, T, 0.99, 0.95, 1.0, 1.0)
    out = np.zeros(2 * B * T)
    L.orc_gae_soa(O.P(val), O.P(rew), O.P(term), B, T, 0.99, 0.95, O.P(out))
    assert np.array_equal(adv, out[: B * T])  # bit-exact
    np.testing.assert_array_equal(out[B * T:], out[: B * T] + val)


def test_vtrace_vec_closed_forms():
    B, T = 4, 10
    rew, val, _, imp = _vt_inputs(0x2222, B, T)
    ones = np.ones(B * T)
    adv = _vec(rew, val, ones, imp, B, T, 0.99, 0.95, 2.1, 1.08).reshape(B, T)
    rho = np.minimum(imp, 2.1).reshape(B, T)
    r = np.clip(rew, -1, 1).reshape(B, T)
    v = val.reshape(B, T)
    np.testing.assert_allclose(adv[:, :-1], (rho * (r - v))[:, :-1], rtol=1e-14)
    assert np.all(adv[:, -1] == 0.0)
    _, _, term, _ = _vt_inputs(0x3333, B, T)
    adv0 = _vec(rew, val, term, imp, B, T, 0.0, 0.95, 2.1, 1.08).reshape(B, T)
    np.testing.assert_allclose(adv0[:, :-1], (rho * (r - v))[:, :-1], rtol=1e-14)


def test_vtrace_mingru_brute_force_and_gae_boot():
    B, T = 6, 11
    rew, val, term, imp = _vt_inputs(0x5C1B, B, T)
    boot = rng.randf(0x77, B, -2.0, 2.0)
    adv = np.zeros(B * T)
    L.orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(imp), O.P(boot), B, T, 0.99, 0.95,
                        2.1, 1.08, O.P(adv))
    # explicit sum
    for b in range(B):
        sl = slice(b * T, (b + 1) * T)
        r = np.clip(rew[sl], -1, 1); v = val[sl]; nnt = (term[sl] <= 0.5).astype(float)
        rho = np.minimum(imp[sl], 2.1); c = np.minimum(imp[sl], 1.08)
        vnext = np.append(v[1:], boot[b])
        delta = rho * r + 0.99 * vnext * nnt - v
        for t in range(T):
            tot, w = 0.0, 1.0
            for s in range(t, T):
                tot += w * delta[s]
                w *= 0.99 * 0.95 * c[s] * nnt[s]
            assert abs(adv[b * T + t] - tot) < 1e-12
    # rho = c = 1 without the clamp is GAE with bootstrap: the targets match gae_boot_norm's
    # returns bit for bit (time-major).
    tm = lambda x: np.ascontiguousarray(x.reshape(B, T).T).ravel()
    _, tgt = O.vtrace(tm(rew), tm(val), tm(term), np.ones(B * T), boot, B, T, variant=1,
                      time_major=True, clamp=False)
    out = np.zeros(2 * B * T)
    L.orc_gae_boot_norm(O.P(tm(val)), O.P(tm(rew)), O.P(tm(term)), O.P(boot), B, T, 0.99, 0.95,
                        O.P(out))
    assert np.array_equal(tgt, out[B * T:])


@pytest.mark.parametrize("variant", [0, 1])
def test_vtrace_general_matches_reference_forms(variant):
    B, T = 13, 17
    rew, val, term, imp = _vt_inputs(0x4444 + variant, B, T)
    boot = rng.randf(0x78, B, -2.0, 2.0)
    adv, tgt = O.vtrace(rew, val, term, imp, boot, B, T, variant=variant, time_major=False,
                        rho_clip=2.1, c_clip=1.08)
    if variant == 0:
        ref = _vec(rew, val, term, imp, B, T, 0.99, 0.95, 2.1, 1.08)
    else:
        ref = np.zeros(B * T)
        L.orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(imp), O.P(boot), B, T, 0.99, 0.95,
                            2.1, 1.08, O.P(ref))
    assert np.array_equal(adv, ref)
    np.testing.assert_array_equal(tgt, ref + val)
    # time-major layout is the transpose
    tm = lambda x: np.ascontiguousarray(x.reshape(B, T).T).ravel()
    adv_t, _ = O.vtrace(tm(rew), tm(val), tm(term), tm(imp), boot, B, T, variant=variant,
                        time_major=True, rho_clip=2.1, c_clip=1.08)
    assert np.array_equal(adv_t, tm(adv))
    # log-ratio input
    adv_l, _ = O.vtrace(rew, val, term, np.log(imp), boot, B, T, variant=variant,
                        time_major=False, rho_is_log=True, rho_clip=2.1, c_clip=1.08)
    np.testing.assert_allclose(adv_l, adv, rtol=1e-12, atol=1e-12)
    # f32 twin within 1e-5 relative Frobenius
    a32, _ = O.vtrace(rew, val, term, imp, boot, B, T, variant=variant, time_major=False,
                      rho_clip=2.1, c_clip=1.08, dtype=np.float32)
    assert np.linalg.norm(a32 - adv) / np.linalg.norm(adv) < 1e-5


def test_adv_normalize_closed_form():
    x = rng.randf(0xAD7, 257, -3.0, 3.0)
    out = np.zeros_like(x)
    L.orc_adv_normalize(O.P(x), 257, O.P(out))
    assert abs(out.mean()) < 1e-14
    np.testing.assert_allclose(out.std(), 1.0, rtol=1e-7)
    np.testing.assert_allclose(out, (x - x.mean()) / (x.std() + 1e-8), rtol=1e-13)


# ---------------------------------------------------------------------------------------------
# PPO loss gradient: finite differences of an independently written objective

def _objective(lg, v, a, adv, ret, old, ov, vf, ent, clip, vfclip):
    lse = np.log(np.sum(np.exp(lg - lg.max()))) + lg.max()
    p = np.exp(lg - lse)
    ratio = math.exp(lg[a] - lse - old)
    surr = min(adv * ratio, adv * min(max(ratio, 1 - clip), 1 + clip))
    H = -np.sum(p * (lg - lse))
    vl = (v - ret) ** 2
    if vfclip > 0 and ov is not None:
        vc = ov + min(max(v - ov, -vfclip), vfclip)
        vl = max(vl, (vc - ret) ** 2)
    return surr + ent * H - vf * 0.5 * vl


@pytest.mark.parametrize("vfclip", [0.0, 0.3])
def test_ppo_grad_finite_differences(vfclip):
    N, A = 40, 5
    lg = rng.normal(1, N * A).reshape(N, A)
    v = rng.normal(2, N)
    act = rng.randint(3, N, A).astype(float)
    adv = rng.normal(4, N)
    ret = rng.normal(5, N)
    old = np.array([lg[n, int(act[n])] - np.log(np.exp(lg[n]).sum()) for n in range(N)])
    old += rng.normal(6, N, 0.0, 0.3)  # ratios away from 1, some clipped
    ov = v + rng.normal(7, N, 0.0, 0.5)
    dl, dv, nlp, nv = O.ppo_grad(lg, v, act, adv, ret, old, ov, vfclip=vfclip)
    h = 1e-6
    checked = 0
    for n in range(N):
        a = int(act[n])
        f = lambda L_, V_: _objective(L_, V_, a, adv[n], ret[n], old[n], ov[n], 0.5, 0.01, 0.2, vfclip)
        ratio = math.exp(nlp[n] - old[n])
        if abs(ratio - 0.8) < 1e-3 or abs(ratio - 1.2) < 1e-3:
            continue  # kink of the clip
        if vfclip > 0 and abs(abs(v[n] - ov[n]) - vfclip) < 1e-3:
            continue
        for k in range(A):
            e = np.zeros(A); e[k] = h
            fd = (f(lg[n] + e, v[n]) - f(lg[n] - e, v[n])) / (2 * h)
            assert abs(fd - dl[n, k]) < 1e-6 * max(1.0, abs(fd)), (n, k, fd, dl[n, k])
        fdv = (f(lg[n], v[n] + h) - f(lg[n], v[n] - h)) / (2 * h)
        assert abs(fdv - dv[n]) < 1e-6 * max(1.0, abs(fdv))
        checked += 1
    assert checked > N // 2
    # max-shifted log-sum-exp is the same function
    dl2, dv2, _, _ = O.ppo_grad(lg, v, act, adv, ret, old, ov, vfclip=vfclip, max_shift=True)
    np.testing.assert_allclose(dl2, dl, rtol=1e-10, atol=1e-13)


def test_ppo_grad_uniform_logits():
    # equal logits: p = 1/A, entropy gradient 0, ratio = exp(-log A - old)
    N, A = 8, 4
    lg = np.zeros((N, A))
    act = np.arange(N) % A
    old = np.full(N, -math.log(A))  # ratio exactly 1: unclipped branch
    adv = np.linspace(-1, 1, N)
    dl, dv, _, _ = O.ppo_grad(lg, np.zeros(N), act, adv, np.ones(N), old)
    for n in range(N):
        expect = adv[n] * (np.eye(A)[act[n]] - 1.0 / A)
        np.testing.assert_allclose(dl[n], expect, atol=1e-15)
    np.testing.assert_allclose(dv, 0.5 * np.ones(N))  # -vf*(0-1)


def test_ppo_losses_hand_computed():
    lg = np.array([[0.0, 0.0], [math.log(3.0), 0.0]])
    act = np.array([0.0, 1.0])
    old = np.array([math.log(0.5), math.log(0.25)])  # ratios 1.0 and 1.0
    adv = np.array([2.0, -1.0])
    ret = np.array([1.0, 0.0])
    v = np.array([0.0, 2.0])
    L7 = O.ppo_losses(lg, v, act, adv, ret, old)
    pg = ((-2.0) + (1.0)) / 2
    vl = (0.5 * 1.0 + 0.5 * 4.0) / 2
    H0 = math.log(2.0)
    H1 = -(0.75 * math.log(0.75) + 0.25 * math.log(0.25))
    ent = (H0 + H1) / 2
    np.testing.assert_allclose(L7, [pg, vl, ent, pg + 0.5 * vl - 0.01 * ent, 0.0, 0.0, 0.0],
                               atol=1e-14)


# ---------------------------------------------------------------------------------------------
# GEMM and the MLP chain

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_vs_numpy(ta, tb):
    M, N, K = 37, 23, 19
    A = rng.normal(10, M * K).reshape((K, M) if ta else (M, K))
    B = rng.normal(11, K * N).reshape((N, K) if tb else (K, N))
    ref = (A.T if ta else A) @ (B.T if tb else B)
    got = O.gemm(ta, tb, A, B, M, N, K, threads=2)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-12)


def _mlp_objective(p, obs, act, adv, ret, old, N, H, D, A):
    O_ = A + 1
    W1 = p[: H * D].reshape(H, D); b1 = p[H * D: H * D + H]
    W2 = p[H * D + H: H * D + H + O_ * H].reshape(O_, H); b2 = p[H * D + H + O_ * H:]
    h = np.maximum(obs.reshape(N, D) @ W1.T + b1, 0)
    out = h @ W2.T + b2
    return sum(_objective(out[n, :A], out[n, A], int(act[n]), adv[n], ret[n], old[n], None,
                          0.5, 0.01, 0.2, 0.0) for n in range(N))


def test_mlp_ppo_grad_finite_differences():
    N, D, H, A = 12, 5, 7, 3
    O_ = A + 1
    P_ = H * D + H + O_ * H + O_
    p = rng.normal(20, P_) * 0.5
    obs = rng.randf(21, N * D, -1, 1)
    act = rng.randint(22, N, A).astype(float)
    adv = rng.normal(23, N)
    ret = rng.normal(24, N)
    old = rng.randf(25, N, -1.5, -0.5)
    g = np.zeros(P_)
    L.orc_mlp_ppo_grad(O.P(p), O.P(obs), O.P(act), O.P(adv), O.P(ret), O.P(old), N, H, D, A, 0.5,
                       0.01, 0.2, O.P(g), 1)
    h = 1e-6
    fd = np.zeros(P_)
    for i in range(P_):
        e = np.zeros(P_); e[i] = h
        fd[i] = (_mlp_objective(p + e, obs, act, adv, ret, old, N, H, D, A)
                 - _mlp_objective(p - e, obs, act, adv, ret, old, N, H, D, A)) / (2 * h)
    np.testing.assert_allclose(g, fd, rtol=1e-5, atol=1e-6)


def _deep_objective(p, obs, act, adv, ret, old, ov, N, D, H, L, A, vfclip):
    O_ = A + 1
    x = obs.reshape(N, D)
    off = 0
    for l in range(L):
        fan = D if l == 0 else H
        W = p[off: off + H * fan].reshape(H, fan); off += H * fan
        b = p[off: off + H]; off += H
        x = np.maximum(x @ W.T + b, 0)
    Wo = p[off: off + O_ * H].reshape(O_, H); off += O_ * H
    out = x @ Wo.T + p[off: off + O_]
    return sum(_objective(out[n, :A], out[n, A], int(act[n]), adv[n], ret[n], old[n],
                          None if ov is None else ov[n], 0.5, 0.01, 0.2, vfclip) for n in range(N))


def test_mlp_deep_one_layer_is_reference_mlp():
    N, D, H, A = 33, 6, 9, 4
    O_ = A + 1
    P_ = H * D + H + O_ * H + O_
    p = rng.normal(40, P_) * 0.5
    obs = rng.randf(41, N * D, -1, 1)
    act = rng.randint(42, N, A).astype(float)
    adv, ret = rng.normal(43, N), rng.normal(44, N)
    old = rng.randf(45, N, -1.8, -0.8)
    g = np.zeros(P_)
    L.orc_mlp_ppo_grad(O.P(p), O.P(obs), O.P(act), O.P(adv), O.P(ret), O.P(old), N, H, D, A, 0.5,
                       0.01, 0.2, O.P(g), 1)
    gd, _, _ = O.mlp_deep_ppo_grad(p, obs, act, adv, ret, old, None, N, D, H, 1, A, threads=1)
    assert np.array_equal(gd, g)


@pytest.mark.parametrize("L_,vfclip", [(2, 0.0), (3, 0.0), (2, 0.25)])
def test_mlp_deep_finite_differences(L_, vfclip):
    N, D, H, A = 10, 4, 6, 2
    P_ = O.mlp_deep_param_count(D, H, L_, A)
    p = rng.normal(50 + L_, P_) * 0.6
    obs = rng.randf(51, N * D, -1, 1)
    act = rng.randint(52, N, A).astype(float)
    adv, ret = rng.normal(53, N), rng.normal(54, N)
    old = rng.randf(55, N, -1.2, -0.4)
    ov = rng.normal(56, N)
    g, nlp, nv = O.mlp_deep_ppo_grad(p, obs, act, adv, ret, old, ov, N, D, H, L_, A, vfclip=vfclip,
                                     threads=1)
    h = 1e-6
    fd = np.zeros(P_)
    for i in range(P_):
        e = np.zeros(P_); e[i] = h
        fd[i] = (_deep_objective(p + e, obs, act, adv, ret, old, ov, N, D, H, L_, A, vfclip)
                 - _deep_objective(p - e, obs, act, adv, ret, old, ov, N, D, H, L_, A, vfclip)) / (2 * h)
    np.testing.assert_allclose(g, fd, rtol=1e-5, atol=1e-6)
    assert np.all(np.isfinite(nlp)) and np.all(nlp < 0) and nv.shape == (N,)


def test_mlp_forward_matches_numpy():
    N, D, H, O_ = 9, 4, 6, 3
    p = rng.normal(30, H * D + H + O_ * H + O_)
    X = rng.normal(31, N * D)
    Y = np.zeros(N * O_)
    L.orc_mlp_forward(O.P(p), O.P(X), N, D, H, O_, O.P(Y))
    W1 = p[: H * D].reshape(H, D); b1 = p[H * D: H * D + H]
    W2 = p[H * D + H: H * D + H + O_ * H].reshape(O_, H); b2 = p[H * D + H + O_ * H:]
    ref = np.maximum(X.reshape(N, D) @ W1.T + b1, 0) @ W2.T + b2
    np.testing.assert_allclose(Y.reshape(N, O_), ref, rtol=1e-12)


# ---------------------------------------------------------------------------------------------
# Newton-Schulz / Muon

def _scalar_quintic(s, coeffs):
    for a, b, c in coeffs:
        s = a * s + b * s ** 3 + c * s ** 5
    return s


@pytest.mark.parametrize("form", [0, 1])
@pytest.mark.parametrize("shape", [(6, 10), (10, 6), (8, 8)])
def test_ns_scaled_orthogonal_closed_form(form, shape):
    m, n = shape
    q, _ = np.linalg.qr(rng.normal(40, max(m, n) ** 2).reshape(max(m, n), max(m, n)))
    Q = q[:m, :n] if m <= n else q[:m, :n]
    sigma = 0.37
    X0 = sigma * Q
    eps = 1e-7
    s0 = sigma / (sigma * math.sqrt(min(m, n)) + eps)
    for coeffs in (O.REF_COEFFS, O.BASELINE_COEFFS):
        out = O.newton_schulz(X0, coeffs, eps, form)
        np.testing.assert_allclose(out, _scalar_quintic(s0, coeffs) * Q, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("form", [0, 1])
def test_ns_diagonal_closed_form(form):
    d = np.array([0.3, -1.2, 2.0, 0.05, 0.9])
    eps = 1e-7
    out = O.newton_schulz(np.diag(d), O.REF_COEFFS, eps, form)
    s = d / (np.linalg.norm(d) + eps)
    np.testing.assert_allclose(out, np.diag(_scalar_quintic(s, O.REF_COEFFS)), rtol=1e-11, atol=1e-14)


def test_ns_forms_agree_and_transpose_symmetry():
    X = rng.normal(41, 12 * 20).reshape(12, 20) * 0.02
    for coeffs in (O.REF_COEFFS, O.BASELINE_COEFFS):
        a = O.newton_schulz(X, coeffs, 1e-7, 0)
        b = O.newton_schulz(X, coeffs, 1e-7, 1)
        np.testing.assert_allclose(a, b, rtol=1e-11, atol=1e-13)
        at = O.newton_schulz(np.ascontiguousarray(X.T), coeffs, 1e-7, 0)
        np.testing.assert_allclose(at, a.T, rtol=1e-11, atol=1e-13)


def test_muon_mat_diagonal_and_mlp_wrapper():
    # W, G, M diagonal: the step stays diagonal and reduces to the scalar recurrences
    n = 6
    w = rng.normal(50, n); g = rng.normal(51, n); m = rng.normal(52, n)
    lr, wd, mu, eps, gs = 0.1, 0.01, 0.95, 1e-7, 0.25
    nW = np.zeros((n, n)); nM = np.zeros((n, n))
    c = O.coeffs_array(O.REF_COEFFS)
    L.orc_muon_mat(n, n, O.P(np.diag(w)), O.P(np.diag(g)), O.P(np.diag(m)), O.P(nW), O.P(nM), gs,
                   lr, wd, mu, eps, O.P(c), 5, 0)
    mm = mu * m + g * gs
    u = g * gs + mu * mm
    s = _scalar_quintic(u / (np.linalg.norm(u) + eps), O.REF_COEFFS)
    np.testing.assert_allclose(np.diag(nM), mm, rtol=1e-15)
    np.testing.assert_allclose(nW, np.diag((1 - lr * wd) * w + lr * s), rtol=1e-10, atol=1e-14)
    # whole-MLP wrapper equals the per-tensor calls
    H, D, O_ = 5, 3, 4
    P_ = H * D + H + O_ * H + O_
    pm = rng.normal(53, 2 * P_); gg = rng.normal(54, P_)
    out = np.zeros(2 * P_)
    L.orc_muon_step_mlp(O.P(pm), O.P(gg), H, D, O_, gs, lr, wd, mu, eps, O.P(out))
    offs = [(0, H, D), (H * D, H, None), (H * D + H, O_, H), (H * D + H + O_ * H, O_, None)]
    for off, r, cdim in offs:
        if cdim is None:
            nb = np.zeros(r); nm = np.zeros(r)
            L.orc_stepvec(r, O.P(pm[off:off + r].copy()), O.P(gg[off:off + r].copy()),
                          O.P(pm[P_ + off:P_ + off + r].copy()), O.P(nb), O.P(nm), gs, lr, wd, mu)
            np.testing.assert_array_equal(out[off:off + r], nb)
            np.testing.assert_array_equal(out[P_ + off:P_ + off + r], nm)
            np.testing.assert_allclose(nm, mu * pm[P_ + off:P_ + off + r] + gs * gg[off:off + r])
        else:
            k = r * cdim
            a = np.zeros(k); b = np.zeros(k)
            L.orc_muon_mat(r, cdim, O.P(pm[off:off + k].copy()), O.P(gg[off:off + k].copy()),
                           O.P(pm[P_ + off:P_ + off + k].copy()), O.P(a), O.P(b), gs, lr, wd, mu,
                           eps, O.P(c), 5, 0)
            np.testing.assert_array_equal(out[off:off + k], a)
            np.testing.assert_array_equal(out[P_ + off:P_ + off + k], b)


def test_gclip_closed_form():
    g = rng.normal(60, 100)
    g1 = g.copy()
    gn = L.orc_gclip(O.P(g1), 100, 0.5, 1.0)
    np.testing.assert_allclose(gn, np.linalg.norm(0.5 * g), rtol=1e-14)
    np.testing.assert_allclose(g1, g * 0.5 * (1.0 / gn), rtol=1e-14)
    g2 = g.copy()
    L.orc_gclip(O.P(g2), 100, 0.5, 1e9)
    np.testing.assert_allclose(g2, 0.5 * g, rtol=1e-15)


# ---------------------------------------------------------------------------------------------
# MinGRU

def _mg_unpack(p, H, D, Lr, A):
    o = 0
    def take(n):
        nonlocal o
        v = p[o:o + n]; o += n
        return v
    wE = take(H * D).reshape(H, D); bE = take(H)
    Ws = [take(3 * H * H).reshape(3 * H, H) for _ in range(Lr)]
    wD = take(A * H).reshape(A, H); bD = take(A); wV = take(H); bV = take(1)
    return wE, bE, Ws, wD, bD, wV, bV


def _mg_objective(p, obs, act, adv, ret, old, term, ov, T, H, D, Lr, A, vfclip):
    sig = lambda x: 1 / (1 + np.exp(-x))
    wE, bE, Ws, wD, bD, wV, bV = _mg_unpack(p, H, D, Lr, A)
    st = np.zeros((Lr, H))
    tot = 0.0
    for t in range(T):
        h = wE @ obs[t * D:(t + 1) * D] + bE
        for l in range(Lr):
            y = Ws[l] @ h
            hid, gate, proj = y[:H], y[H:2 * H], y[2 * H:]
            z = sig(gate)
            g = np.where(hid >= 0, hid + 0.5, sig(hid))
            o = (1 - z) * st[l] + z * g
            hg = sig(proj)
            h = hg * o + (1 - hg) * h
            st[l] = o
        lg = wD @ h + bD
        v = wV @ h + bV[0]
        tot += _objective(lg, v, int(act[t]), adv[t], ret[t], old[t], ov[t], 0.5, 0.01, 0.2, vfclip)
        if term[t] != 0:
            st[:] = 0
    return tot


def test_mingru_seq_grad_finite_differences():
    T, H, D, Lr, A = 6, 4, 3, 2, 3
    P_ = H * D + H + Lr * 3 * H * H + A * H + A + H + 1
    p = rng.normal(70, P_) * 0.6
    obs = rng.normal(71, T * D)
    act = rng.randint(72, T, A).astype(float)
    adv = rng.normal(73, T); ret = rng.normal(74, T)
    old = rng.randf(75, T, -1.6, -0.6)
    term = np.array([0, 0, 1, 0, 0, 0], dtype=float)
    ov = rng.normal(76, T)
    out = np.zeros(P_ + 2 * T)
    L.orc_mingru_ppo_grad_seq(O.P(p), O.P(obs), O.P(act), O.P(adv), O.P(ret), O.P(old), O.P(term),
                              O.P(ov), T, H, D, Lr, A, 0.5, 0.01, 0.2, 0.0, O.P(out))
    h = 1e-6
    fd = np.zeros(P_)
    for i in range(P_):
        e = np.zeros(P_); e[i] = h
        fd[i] = (_mg_objective(p + e, obs, act, adv, ret, old, term, ov, T, H, D, Lr, A, 0.0)
                 - _mg_objective(p - e, obs, act, adv, ret, old, term, ov, T, H, D, Lr, A, 0.0)) / (2 * h)
    np.testing.assert_allclose(out[:P_], fd, rtol=1e-5, atol=1e-6)


def test_heinsen_equals_sequential_recurrence():
    T, H = 64, 7
    gate = rng.normal(80, T * H).reshape(T, H) * 2
    hid = rng.normal(81, T * H).reshape(T, H) * 2
    o = np.zeros((T, H))
    L.orc_mingru_heinsen(O.P(gate), O.P(hid), T, H, O.P(o))
    sig = lambda x: 1 / (1 + np.exp(-x))
    prev = np.zeros(H)
    for t in range(T):
        z = sig(gate[t]); g = np.where(hid[t] >= 0, hid[t] + 0.5, sig(hid[t]))
        prev = (1 - z) * prev + z * g
        np.testing.assert_allclose(o[t], prev, rtol=1e-11, atol=1e-13)
