"""Pins the oracle's rollout functions: the categorical sampler and the single-step MinGRU forward.

The sampler is checked against numpy's softmax and cumulative sum on the pinned splitmix64 words, a
closed form for uniform logits, and draw frequencies; the step forward against the separately pinned
sequence forward of orc_mingru_ppo_grad_seq (its new values and new log-probs).
"""
import numpy as np

import oracle_lib as O
from pufferlean_amd import rng


def test_sample_actions_equal_numpy_inverse_cdf():
    N, A = 500, 7
    Y = rng.normal(0x601, N * (A + 1)).reshape(N, A + 1) * 2.0
    state = 0xDEC0DE
    act, logp, val = O.sample_actions(Y, A, state)
    u = rng.uniform01(rng.words(state, N))
    lg = Y[:, :A]
    p = np.exp(lg - lg.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    cum = np.cumsum(p, axis=1)
    expect = np.array([next((k for k in range(A) if u[n] < cum[n, k]), A - 1) for n in range(N)])
    assert np.array_equal(act, expect)
    a = act.astype(np.int64)
    assert np.allclose(logp, np.log(p[np.arange(N), a]), rtol=1e-13, atol=1e-15)
    assert np.array_equal(val, Y[:, A])


def test_sample_actions_uniform_logits_closed_form():
    N, A = 4000, 6
    Y = np.zeros((N, A + 1))
    act, logp, _ = O.sample_actions(Y, A, 0x42)
    u = rng.uniform01(rng.words(0x42, N))
    near = np.abs(u * A - np.round(u * A)) < 1e-9
    assert np.array_equal(act[~near], np.floor(u * A)[~near])
    assert np.allclose(logp, -np.log(A), rtol=1e-14)


def test_sample_actions_frequencies():
    N, A = 200000, 5
    logits = np.array([0.0, 1.0, -1.0, 2.0, 0.5])
    Y = np.tile(np.append(logits, 3.0), (N, 1))
    act, _, _ = O.sample_actions(Y, A, 0x77)
    p = np.exp(logits - logits.max())
    p /= p.sum()
    freq = np.bincount(act.astype(np.int64), minlength=A) / N
    assert np.all(np.abs(freq - p) < 5 * np.sqrt(p * (1 - p) / N))


def test_mingru_step_chain_equals_sequence_forward():
    T, D, H, L, A = 6, 5, 7, 2, 4
    P = H * D + H + L * 3 * H * H + A * H + A + H + 1
    params = rng.normal(0x611, P) * 0.4
    obs = rng.normal(0x612, T * D).reshape(T, D)
    acts = rng.randint(0x613, T, A).astype(np.float64)
    z = np.zeros(T)
    seq = np.zeros(P + 2 * T)
    O.lib().orc_mingru_ppo_grad_seq(O.P(params), O.P(O.f64(obs)), O.P(acts), O.P(z), O.P(z), O.P(z), O.P(z),
                                    O.P(z), T, H, D, L, A, 0.5, 0.01, 0.2, 0.0, O.P(seq))
    newlp, newval = seq[P:P + T], seq[P + T:]
    state = np.zeros((1, L, H))
    for t in range(T):
        out, state = O.mingru_step(params, obs[t], state, 1, D, H, L, A)
        lg = out[0, :A]
        lsm = lg - lg.max() - np.log(np.exp(lg - lg.max()).sum())
        assert abs(out[0, A] - newval[t]) <= 1e-12 * max(1.0, abs(newval[t]))
        assert abs(lsm[int(acts[t])] - newlp[t]) <= 1e-12 * max(1.0, abs(newlp[t]))


def test_mingru_step_envs_are_independent():
    N, D, H, L, A = 5, 4, 6, 3, 3
    P = H * D + H + L * 3 * H * H + A * H + A + H + 1
    params = rng.normal(0x621, P) * 0.3
    obs = rng.normal(0x622, N * D).reshape(N, D)
    state = rng.normal(0x623, N * L * H).reshape(N, L, H)
    out, ns = O.mingru_step(params, obs, state, N, D, H, L, A)
    for n in range(N):
        o1, s1 = O.mingru_step(params, obs[n], state[n:n + 1], 1, D, H, L, A)
        assert np.array_equal(o1[0], out[n]) and np.array_equal(s1[0], ns[n])
