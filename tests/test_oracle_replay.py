"""Pins the oracle's prioritised-replay functions (the MinGRU minibatch chain).

Each check uses a formulation other than the oracle's loops: numpy's searchsorted and power forms
(the Python reference's tools/puffer_ref.py:151-159), the first-hit linear scan of
weightedSampleReplace (Puffer/RL/VecTrain.lean:147-165), closed forms on uniform or dyadic inputs,
draw frequencies against the probabilities, numpy fancy indexing for the gather, and a dictionary
of last assignments for the iterate.
"""
import numpy as np

import oracle_lib as O
from pufferlean_amd import rng


def rel(a, b):
    return float(np.max(np.abs(a - b) / np.maximum(np.abs(b), 1e-300)))


# ---- per-segment |adv| sums ---------------------------------------------------------------------
def test_seg_l1_exact_on_dyadic_inputs():
    N, T = 37, 19
    adv = (rng.randint(0x51, N * T, 257) - 128) / 8.0  # dyadic: every summation order is exact
    got = O.seg_l1(adv, N, T)
    assert np.array_equal(got, np.abs(adv.reshape(N, T)).sum(axis=1))


def test_seg_l1_random_within_roundoff():
    N, T = 300, 64
    adv = rng.normal(0x52, N * T)
    got = O.seg_l1(adv, N, T)
    assert rel(got, np.abs(adv.reshape(N, T)).sum(axis=1)) < 1e-13


# ---- prioritised sampler ------------------------------------------------------------------------
def _draw_units(state, mb):
    # draw i uses the word of state + (i+1)*GOLD: the splitmix64 stream started at `state`
    return rng.uniform01(rng.words(state, mb))


def test_prio_draws_equal_searchsorted_and_linear_scan():
    N, mb, state = 300, 700, 0x5EED1234
    L1 = np.abs(rng.normal(0x53, N)) * 10.0
    L1[::17] = 0.0  # zero-advantage segments keep a floor probability
    idx, mp, probs, cum = O.prio_sample(L1, mb, 0.8, 0.4, state)
    u = _draw_units(state, mb) * cum[-1]
    ss = np.minimum(np.searchsorted(cum, u, side="left"), N - 1)
    assert np.array_equal(idx, ss.astype(np.float64))
    for i in range(0, mb, 7):  # weightedSampleReplace's first-hit scan
        hit = next((e for e in range(N) if cum[e] >= u[i]), N - 1)
        assert idx[i] == hit


def test_prio_probabilities_and_weights_match_power_forms():
    N, mb, state = 513, 1000, 0xABCDEF
    L1 = np.abs(rng.normal(0x54, N)) * 3.0
    alpha, beta = 0.8, 0.35
    idx, mp, probs, cum = O.prio_sample(L1, mb, alpha, beta, state)
    w = (L1 + 1e-12) ** alpha
    p = (w + 1e-6) / (w.sum() + 1e-6)
    assert rel(probs, p) < 1e-13
    assert rel(cum, np.cumsum(p)) < 1e-13
    # the floor 1e-6 is added per segment but once to the normaliser
    assert abs(cum[-1] - (w.sum() + N * 1e-6) / (w.sum() + 1e-6)) < 1e-12
    k = idx.astype(np.int64)
    assert rel(mp, (N * p[k] + 1e-12) ** (-beta)) < 1e-13


def test_prio_uniform_closed_form():
    N, mb, state = 1000, 4000, 0x77
    idx, mp, probs, cum = O.prio_sample(np.full(N, 2.5), mb, 0.8, 0.2, state)
    u = _draw_units(state, mb)
    expect = np.floor(u * N)
    near = np.abs(u * N - np.round(u * N)) < 1e-9  # within rounding of a boundary
    assert np.array_equal(idx[~near], expect[~near])
    assert np.allclose(mp, 1.0, atol=1e-9)


def test_prio_draw_frequencies_follow_probabilities():
    L1 = np.array([0.0, 1.0, 2.0, 4.0, 8.0, 0.5, 3.0, 16.0])
    N, mb = L1.size, 200000
    idx, _, probs, _ = O.prio_sample(L1, mb, 0.8, 0.2, 0x1F2E3D)
    freq = np.bincount(idx.astype(np.int64), minlength=N) / mb
    sigma = np.sqrt(probs * (1 - probs) / mb)
    assert np.all(np.abs(freq - probs) < 5 * sigma + 1e-12)


def test_prio_single_segment():
    idx, mp, probs, cum = O.prio_sample(np.array([3.0]), 10, 0.8, 0.5, 0x99)
    assert np.all(idx == 0.0)
    assert probs[0] == 1.0
    assert np.allclose(mp, 1.0, atol=1e-11)


# ---- minibatch gather ---------------------------------------------------------------------------
def _cols(seed, N, T, dyadic=False):
    if dyadic:
        adv = (rng.randint(seed, N * T, 129) - 64) / 16.0
        val = (rng.randint(seed + 1, N * T, 65) - 32) / 4.0
    else:
        adv = rng.normal(seed, N * T)
        val = rng.normal(seed + 1, N * T)
    act = rng.randint(seed + 2, N * T, 6).astype(np.float64)
    logp = rng.randf(seed + 3, N * T, -3.0, -0.1)
    term = rng.randf(seed + 4, N * T, 0.0, 1.0)
    return act, logp, term, adv, val


def test_gather_equals_fancy_index_construction():
    N, T, Bmb = 40, 12, 25
    act, logp, term, adv, val = _cols(0x61, N, T)
    seg = rng.randint(0x66, Bmb, N).astype(np.float64)
    seg[3] = seg[7] = seg[11]  # repeated draws
    mp = rng.randf(0x67, Bmb, 0.5, 2.0)
    out, st = O.gather_seq_minibatch(act, logp, term, adv, val, seg, mp, T)
    s = seg.astype(np.int64)
    tm = lambda col: col.reshape(N, T)[s].T.ravel()  # [T][Bmb], row t*Bmb + bi
    n = T * Bmb
    a = tm(adv)
    assert np.array_equal(out[:n], np.trunc(tm(act)))
    assert np.array_equal(out[2 * n:3 * n], a + tm(val))
    assert np.array_equal(out[3 * n:4 * n], tm(logp))
    assert np.array_equal(out[4 * n:5 * n], (tm(term) > 0.5).astype(np.float64))
    assert np.array_equal(out[5 * n:], tm(val))
    mean, std = a.mean(), a.std()
    assert rel(st, np.array([mean, std])) < 1e-13
    w = np.tile(mp, T)
    assert rel(out[n:2 * n], w * (a - mean) / (std + 1e-8)) < 1e-12


def test_gather_mean_std_exact_on_dyadic_inputs():
    N, T, Bmb = 16, 8, 32  # T*Bmb = 256: mean of dyadic values is exact
    act, logp, term, adv, val = _cols(0x71, N, T, dyadic=True)
    seg = rng.randint(0x76, Bmb, N).astype(np.float64)
    out, st = O.gather_seq_minibatch(act, logp, term, adv, val, seg, np.ones(Bmb), T)
    a = adv.reshape(N, T)[seg.astype(np.int64)].ravel()
    mean = a.sum() / a.size
    assert st[0] == mean
    assert st[1] == np.sqrt(((a - mean) ** 2).sum() / a.size)


# ---- value / ratio iterate ----------------------------------------------------------------------
def test_iterate_last_assignment_wins():
    N, T, Bmb = 20, 6, 30
    value = rng.normal(0x81, N * T)
    ratio = np.ones(N * T)
    logp = rng.randf(0x82, N * T, -3.0, -0.1)
    seg = rng.randint(0x83, Bmb, N).astype(np.float64)
    newlp = rng.randf(0x84, T * Bmb, -3.0, -0.1).astype(np.float32)
    newval = rng.normal(0x85, T * Bmb).astype(np.float32)
    v2, r2 = O.mb_iterate(value, ratio, logp, newlp, newval, seg, T)
    last = {}
    for bi, e in enumerate(seg.astype(np.int64)):
        last[e] = bi
    ev, er = value.copy(), ratio.copy()
    for e, bi in last.items():
        for t in range(T):
            ev[e * T + t] = float(newval[t * Bmb + bi])
            er[e * T + t] = np.exp(float(newlp[t * Bmb + bi]) - logp[e * T + t])
    assert np.array_equal(v2, ev)
    assert rel(r2, er) < 1e-15
    untouched = np.setdiff1d(np.arange(N), seg.astype(np.int64))
    for e in untouched:
        assert np.array_equal(v2[e * T:(e + 1) * T], value[e * T:(e + 1) * T])
        assert np.all(r2[e * T:(e + 1) * T] == 1.0)
