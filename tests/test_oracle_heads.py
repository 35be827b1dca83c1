"""Pins the oracle's multi-discrete and continuous heads.

Gradients: central finite differences of objectives written here independently in numpy (joint
clipped surrogate, clipped value loss, entropy), and the K = 1 multi-discrete case against the
separately pinned single-head gradient. Samplers: numpy inverse-CDF and Box-Muller on the pinned
splitmix64 words, and Gaussian draw moments.
"""
import math

import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import rng

GOLD, GOLD2, MASK = 0x9E3779B97F4A7C15, 0xD1B54A32D192ED03, 0xFFFFFFFFFFFFFFFF
HALF_LOG_2PI = 0.5 * math.log(2 * math.pi)


def word_unit(x):
    """uniform01 of the splitmix64 finaliser of x (words(s, 1) mixes s + GOLD)."""
    return float(rng.uniform01(rng.words((x - GOLD) & MASK, 1))[0])


def vloss(v, ret, ov, vfclip):
    vl = (v - ret) ** 2
    if vfclip > 0 and ov is not None:
        vc = ov + min(max(v - ov, -vfclip), vfclip)
        vl = max(vl, (vc - ret) ** 2)
    return 0.5 * vl


def obj_md(row, acts, sizes, adv, ret, old, ov, vf, ent, clip, vfclip):
    joint, H, off = 0.0, 0.0, 0
    for h, sz in enumerate(sizes):
        lg = row[off:off + sz]
        lse = lg.max() + np.log(np.exp(lg - lg.max()).sum())
        p = np.exp(lg - lse)
        joint += lg[int(acts[h])] - lse
        H += -np.sum(p * (lg - lse))
        off += sz
    r = math.exp(joint - old)
    surr = min(adv * r, adv * min(max(r, 1 - clip), 1 + clip))
    return surr + ent * H - vf * vloss(row[off], ret, ov, vfclip)


def obj_cont(row, acts, d, adv, ret, old, ov, vf, ent, clip, vfclip, lslo, lshi):
    logp, H = 0.0, 0.0
    for i in range(d):
        ls = min(max(row[d + i], lslo), lshi)
        z = (acts[i] - row[i]) * math.exp(-ls)
        logp += -0.5 * z * z - ls - HALF_LOG_2PI
        H += ls + 0.5 * (1 + math.log(2 * math.pi))
    r = math.exp(logp - old)
    surr = min(adv * r, adv * min(max(r, 1 - clip), 1 + clip))
    return surr + ent * H - vf * vloss(row[2 * d], ret, ov, vfclip)


def _fd_check(f, row, grad, skip=()):
    h = 1e-6
    for k in range(len(row)):
        if k in skip:
            continue
        e = np.zeros(len(row))
        e[k] = h
        fd = (f(row + e) - f(row - e)) / (2 * h)
        assert abs(fd - grad[k]) < 2e-6 * max(1.0, abs(fd)), (k, fd, grad[k])


@pytest.mark.parametrize("vfclip", [0.0, 0.3])
def test_md_gradient_finite_differences(vfclip):
    sizes = [3, 5, 2]
    N, W = 30, sum(sizes)
    out = rng.normal(0x901, N * (W + 1)).reshape(N, W + 1)
    acts = np.stack([rng.randint(0x902 + h, N, s) for h, s in enumerate(sizes)], axis=1).astype(np.float64)
    adv, ret = rng.normal(0x905, N), rng.normal(0x906, N)
    ov = out[:, W] + rng.normal(0x907, N, 0.0, 0.5)
    d0, nlp0, _ = O.ppo_grad_md(out, acts, adv, ret, np.zeros(N), ov, sizes)
    old = nlp0 + rng.normal(0x908, N, 0.0, 0.3)
    d, nlp, nv = O.ppo_grad_md(out, acts, adv, ret, old, ov, sizes, vfclip=vfclip)
    assert np.array_equal(nv, out[:, W])
    checked = 0
    for n in range(N):
        r = math.exp(nlp[n] - old[n])
        if abs(r - 0.8) < 1e-3 or abs(r - 1.2) < 1e-3:
            continue
        if vfclip > 0 and abs(abs(out[n, W] - ov[n]) - vfclip) < 1e-3:
            continue
        f = lambda row: obj_md(row, acts[n], sizes, adv[n], ret[n], old[n], ov[n], 0.5, 0.01, 0.2, vfclip)
        _fd_check(f, out[n], d[n])
        checked += 1
    assert checked > N // 2


def test_md_single_head_equals_categorical_gradient():
    N, A = 50, 6
    out = rng.normal(0x911, N * (A + 1)).reshape(N, A + 1)
    act = rng.randint(0x912, N, A).astype(np.float64)
    adv, ret, old = rng.normal(0x913, N), rng.normal(0x914, N), rng.normal(0x915, N, -1.8, 0.4)
    d, nlp, nv = O.ppo_grad_md(out, act[:, None], adv, ret, old, None, [A])
    dl, dv, nlp1, nv1 = O.ppo_grad(out[:, :A], out[:, A], act, adv, ret, old)
    np.testing.assert_allclose(d[:, :A], dl, rtol=1e-11, atol=1e-14)
    np.testing.assert_allclose(d[:, A], dv, rtol=1e-12, atol=1e-15)
    np.testing.assert_allclose(nlp, nlp1, rtol=1e-12)


@pytest.mark.parametrize("vfclip,lslo", [(0.0, -20.0), (0.3, -5.0)])
def test_cont_gradient_finite_differences(vfclip, lslo):
    dim, N = 3, 40
    lshi = 2.0
    out = rng.normal(0x921, N * (2 * dim + 1)).reshape(N, 2 * dim + 1)
    out[:, dim:2 * dim] *= 0.5
    acts = out[:, :dim] + rng.normal(0x922, N * dim).reshape(N, dim) * 0.8
    adv, ret = rng.normal(0x923, N), rng.normal(0x924, N)
    ov = out[:, 2 * dim] + rng.normal(0x925, N, 0.0, 0.5)
    _, nlp0, _ = O.ppo_grad_cont(out, acts, adv, ret, np.zeros(N), ov, dim, lslo=lslo, lshi=lshi)
    old = nlp0 + rng.normal(0x926, N, 0.0, 0.3)
    d, nlp, nv = O.ppo_grad_cont(out, acts, adv, ret, old, ov, dim, vfclip=vfclip, lslo=lslo, lshi=lshi)
    checked = 0
    for n in range(N):
        r = math.exp(nlp[n] - old[n])
        if abs(r - 0.8) < 1e-3 or abs(r - 1.2) < 1e-3:
            continue
        if vfclip > 0 and abs(abs(out[n, 2 * dim] - ov[n]) - vfclip) < 1e-3:
            continue
        f = lambda row: obj_cont(row, acts[n], dim, adv[n], ret[n], old[n], ov[n], 0.5, 0.01, 0.2, vfclip, lslo,
                                 lshi)
        _fd_check(f, out[n], d[n])
        checked += 1
    assert checked > N // 2


def test_cont_saturated_log_std_has_zero_gradient():
    dim, N = 2, 4
    out = rng.normal(0x931, N * 5).reshape(N, 5)
    out[:, 2] = -30.0  # dim 0: raw log-std below the clamp
    out[:, 3] = 0.0    # dim 1: inside it
    acts = out[:, :2].copy()
    acts[:, 1] += 0.3
    _, nlp, _ = O.ppo_grad_cont(out, acts, np.ones(N), np.zeros(N), np.zeros(N), None, dim)
    d, _, _ = O.ppo_grad_cont(out, acts, np.ones(N), np.zeros(N), nlp, None, dim)  # ratio 1
    assert np.all(d[:, 2] == 0.0)          # saturated: masked
    assert np.all(d[:, 3] != 0.0) and np.all(d[:, 1] != 0.0)
    out[:, 2] = 5.0                        # above the clamp: masked too
    _, nlp, _ = O.ppo_grad_cont(out, acts, np.ones(N), np.zeros(N), np.zeros(N), None, dim)
    d, _, _ = O.ppo_grad_cont(out, acts, np.ones(N), np.zeros(N), nlp, None, dim)
    assert np.all(d[:, 2] == 0.0)


def test_sample_md_equals_numpy_inverse_cdf():
    sizes = [4, 2, 7]
    N, W = 300, sum(sizes)
    Y = rng.normal(0x941, N * (W + 1)).reshape(N, W + 1) * 1.5
    state = 0xFACE
    out = O.sample_md(Y, sizes, state)
    K = len(sizes)
    for n in range(N):
        joint, off = 0.0, 0
        for h, sz in enumerate(sizes):
            lg = Y[n, off:off + sz]
            p = np.exp(lg - lg.max())
            p /= p.sum()
            u = word_unit(state + (n + 1) * GOLD + (h + 1) * GOLD2)
            cum = np.cumsum(p)
            a = next((k for k in range(sz) if u < cum[k]), sz - 1)
            assert out[h * N + n] == a, (n, h)
            joint += math.log(p[a])
            off += sz
        assert abs(out[K * N + n] - joint) < 1e-12
        assert out[(K + 1) * N + n] == Y[n, W]


def test_sample_cont_equals_numpy_box_muller_and_moments():
    dim, N = 2, 200
    Y = rng.normal(0x951, N * (2 * dim + 1)).reshape(N, 2 * dim + 1)
    state = 0xBEEF
    out = O.sample_cont(Y, dim, state)
    for n in range(0, N, 7):
        logp = 0.0
        for i in range(dim):
            base = state + (n + 1) * GOLD
            u1 = max(word_unit(base + (2 * i + 1) * GOLD2), 1e-7)
            u2 = word_unit(base + (2 * i + 2) * GOLD2)
            z = math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2)
            ls = min(max(Y[n, dim + i], -20.0), 2.0)
            assert abs(out[i * N + n] - (Y[n, i] + math.exp(ls) * z)) < 1e-12 * max(1, abs(out[i * N + n]))
            logp += -0.5 * z * z - ls - HALF_LOG_2PI
        assert abs(out[dim * N + n] - logp) < 1e-11 * max(1, abs(logp))
    # zero means and log-stds: the actions are standard normal draws
    M = 100000
    Z = O.sample_cont(np.zeros((M, 3)), 1, 0x1234)[:M]
    assert abs(Z.mean()) < 5 / math.sqrt(M) and abs(Z.var() - 1) < 5 * math.sqrt(2 / M)


def test_md_out_of_range_action_gives_nan_row():
    sizes = [3, 4]
    N, W = 4, 7
    out = rng.normal(0x961, N * (W + 1)).reshape(N, W + 1)
    acts = np.array([[0, 3], [3, 0], [-1, 2], [2, 3]], np.float64)  # rows 1 and 2 hold a bad action
    d, nlp, nv = O.ppo_grad_md(out, acts, np.ones(N), np.zeros(N), np.full(N, -2.0), None, sizes)
    for n in (1, 2):
        assert np.all(np.isnan(d[n, :W])) and np.isnan(nlp[n])
        assert np.isfinite(d[n, W]) and nv[n] == out[n, W]
    assert np.all(np.isfinite(d[[0, 3]])) and np.all(np.isfinite(nlp[[0, 3]]))


# ---- dashboard losses of the wide heads ---------------------------------------------------------
def _loss_inputs(seed, N):
    adv, ret = rng.normal(seed, N), rng.normal(seed + 1, N)
    ov = rng.normal(seed + 2, N, 0.0, 0.7)
    return adv, ret, ov


@pytest.mark.parametrize("vfclip", [0.0, 0.3])
def test_md_losses_single_head_equal_categorical_losses(vfclip):
    N, A = 300, 6
    out = rng.normal(0x971, N * (A + 1)).reshape(N, A + 1) * 1.5
    act = rng.randint(0x972, N, A).astype(np.float64)
    adv, ret, ov = _loss_inputs(0x973, N)
    old = rng.normal(0x976, N, -1.8, 0.5)
    got = O.wide_losses(1, out, act[:, None], adv, ret, old, ov, sizes=[A], vfclip=vfclip)
    ref = O.ppo_losses(out[:, :A].copy(), out[:, A].copy(), act, adv, ret, old, ov, vfclip=vfclip)
    np.testing.assert_allclose(got, ref, rtol=1e-13, atol=1e-15)


def test_md_losses_two_heads_equal_one_head_over_the_product():
    """Independent heads: the joint distribution is the product (logits l1_i + l2_j), whose log-prob and
    entropy are the sums of the heads'."""
    N, s1, s2 = 200, 3, 4
    out = rng.normal(0x981, N * (s1 + s2 + 1)).reshape(N, s1 + s2 + 1)
    a1, a2 = rng.randint(0x982, N, s1), rng.randint(0x983, N, s2)
    adv, ret, ov = _loss_inputs(0x984, N)
    old = rng.normal(0x987, N, -2.5, 0.5)
    got = O.wide_losses(1, out, np.stack([a1, a2], 1).astype(np.float64), adv, ret, old, ov, sizes=[s1, s2],
                        vfclip=0.2)
    prod = (out[:, :s1, None] + out[:, None, s1:s1 + s2]).reshape(N, s1 * s2)
    ref = O.ppo_losses(np.ascontiguousarray(prod), out[:, -1].copy(), (a1 * s2 + a2).astype(np.float64), adv, ret,
                       old, ov, vfclip=0.2)
    np.testing.assert_allclose(got, ref, rtol=1e-12, atol=1e-14)


def test_cont_losses_against_scipy_normal():
    from scipy.stats import norm
    dim, N = 3, 250
    out = rng.normal(0x991, N * (2 * dim + 1)).reshape(N, 2 * dim + 1)
    out[::17, dim] = -30.0   # below the clamp
    out[::23, dim + 1] = 4.0  # above it
    acts = out[:, :dim] + rng.normal(0x992, N * dim).reshape(N, dim) * 0.6
    acts[::17, 0] = out[::17, 0]  # z = 0 on the dim clamped at -20 keeps logp (and the log-ratio) moderate
    adv, ret, ov = _loss_inputs(0x993, N)
    ls = np.clip(out[:, dim:2 * dim], -20.0, 2.0)
    logp = norm.logpdf(acts, loc=out[:, :dim], scale=np.exp(ls)).sum(axis=1)
    old = logp + rng.normal(0x996, N, 0.0, 0.3)
    got = O.wide_losses(2, out, acts, adv, ret, old, ov, dim=dim, vfclip=0.25)
    # entropy: scipy's differential entropy of each dim
    np.testing.assert_allclose(got[2], norm.entropy(scale=np.exp(ls)).sum(axis=1).mean(), rtol=1e-13)
    # ratio and value terms: a 2-action categorical row [x, 0] with action 0 has log-prob -log(1 + e^-x);
    # shifting logp and old by the same c keeps every log-ratio, so x is chosen to give logp - c
    c = logp.max() + 1.0
    x = -np.log(np.expm1(-(logp - c)))
    cat = np.stack([x, np.zeros(N), out[:, 2 * dim]], axis=1)
    ref = O.ppo_losses(cat[:, :2].copy(), cat[:, 2].copy(), np.zeros(N), adv, ret, old - c, ov, vfclip=0.25)
    for k in (0, 1, 4, 5, 6):
        np.testing.assert_allclose(got[k], ref[k], rtol=1e-9, atol=1e-12, err_msg=str(k))
    np.testing.assert_allclose(got[3], got[0] + 0.5 * got[1] - 0.01 * got[2], rtol=1e-14)


# ---- MinGRU sequence gradient with multi-discrete heads ------------------------------------------
def _mg_layout(H, D, L, A):
    szE, szL = H * D, 3 * H * H
    offDec = szE + H + L * szL
    return offDec, offDec + A * H, offDec + A * H + A  # wDec, bDec, wVal offsets


def _mg_seq(p, obs, acts, advs, rets, olds, terms, ovs, T, H, D, L, A, sizes=None, vfclip=0.2):
    P = p.size
    out = np.zeros(P + 2 * T)
    f = lambda a: np.ascontiguousarray(a, np.float64)
    if sizes is None:
        O.lib().orc_mingru_ppo_grad_seq(O.P(f(p)), O.P(f(obs)), O.P(f(acts)), O.P(f(advs)), O.P(f(rets)),
                                        O.P(f(olds)), O.P(f(terms)), O.P(f(ovs)), T, H, D, L, A, 0.5, 0.01, 0.2,
                                        vfclip, O.P(out))
    else:
        O.lib().orc_mingru_ppo_grad_seq_md(O.P(f(p)), O.P(f(obs)), O.P(f(acts)), O.P(f(advs)), O.P(f(rets)),
                                           O.P(f(olds)), O.P(f(terms)), O.P(f(ovs)), T, H, D, L, A,
                                           O.P(np.ascontiguousarray(sizes, np.int32)), len(sizes), 0.5, 0.01, 0.2,
                                           vfclip, O.P(out))
    return out[:P], out[P:P + T], out[P + T:]


def test_mingru_md_two_heads_equal_product_head():
    """Heads of sizes 3 and 4 are one categorical head over the 12 pairs with decoder rows
    W1[i] + W2[j] (and biases b1[i] + b2[j]): the same joint log-probs, the same gradients of every
    shared layer, and each head's decoder gradient the product's summed over the other head."""
    H, D, L, T, s1, s2 = 16, 8, 2, 12, 3, 4
    W, A2 = s1 + s2, s1 * s2
    P_md = H * D + H + L * 3 * H * H + W * H + W + H + 1
    p = rng.normal(0x9A1, P_md) * 0.3
    dec, bdec, val = _mg_layout(H, D, L, W)
    W1, W2 = p[dec:dec + s1 * H].reshape(s1, H), p[dec + s1 * H:bdec].reshape(s2, H)
    b1, b2 = p[bdec:bdec + s1], p[bdec + s1:val]
    Wp = (W1[:, None, :] + W2[None, :, :]).reshape(A2, H)
    bp = (b1[:, None] + b2[None, :]).reshape(A2)
    pp = np.concatenate([p[:dec], Wp.ravel(), bp, p[val:]])
    obs = rng.normal(0x9A2, T * D)
    a1, a2 = rng.randint(0x9A3, T, s1), rng.randint(0x9A4, T, s2)
    advs, rets, ovs = rng.normal(0x9A5, T), rng.normal(0x9A6, T), rng.normal(0x9A7, T, 0.0, 0.5)
    olds = rng.normal(0x9A8, T, -2.3, 0.4)
    terms = np.zeros(T)
    terms[5] = 1.0
    g, nlp, nv = _mg_seq(p, obs, np.stack([a1, a2], 1).astype(np.float64), advs, rets, olds, terms, ovs, T, H, D, L,
                         W, sizes=[s1, s2])
    gp, nlpp, nvp = _mg_seq(pp, obs, (a1 * s2 + a2).astype(np.float64), advs, rets, olds, terms, ovs, T, H, D, L,
                            A2)
    np.testing.assert_allclose(nlp, nlpp, rtol=1e-12, atol=1e-14)
    np.testing.assert_array_equal(nv, nvp)
    dec2, bdec2, val2 = _mg_layout(H, D, L, A2)
    np.testing.assert_allclose(g[:dec], gp[:dec2], rtol=1e-9, atol=1e-12)          # encoder and layers
    np.testing.assert_allclose(g[val:], gp[val2:], rtol=1e-9, atol=1e-12)          # value head
    gW = gp[dec2:bdec2].reshape(s1, s2, H)
    gb = gp[bdec2:val2].reshape(s1, s2)
    np.testing.assert_allclose(g[dec:dec + s1 * H].reshape(s1, H), gW.sum(1), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(g[dec + s1 * H:bdec].reshape(s2, H), gW.sum(0), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(g[bdec:bdec + s1], gb.sum(1), rtol=1e-9, atol=1e-12)
    np.testing.assert_allclose(g[bdec + s1:val], gb.sum(0), rtol=1e-9, atol=1e-12)


def test_mingru_md_single_head_equals_categorical():
    H, D, L, T, A = 16, 8, 1, 9, 5
    P = H * D + H + L * 3 * H * H + A * H + A + H + 1
    p = rng.normal(0x9B1, P) * 0.3
    obs = rng.normal(0x9B2, T * D)
    acts = rng.randint(0x9B3, T, A).astype(np.float64)
    advs, rets, ovs = rng.normal(0x9B4, T), rng.normal(0x9B5, T), rng.normal(0x9B6, T)
    olds, terms = rng.normal(0x9B7, T, -1.5, 0.3), np.zeros(T)
    g, nlp, _ = _mg_seq(p, obs, acts[:, None], advs, rets, olds, terms, ovs, T, H, D, L, A, sizes=[A])
    gc, nlpc, _ = _mg_seq(p, obs, acts, advs, rets, olds, terms, ovs, T, H, D, L, A)
    np.testing.assert_allclose(g, gc, rtol=1e-10, atol=1e-13)
    np.testing.assert_allclose(nlp, nlpc, rtol=1e-12)
