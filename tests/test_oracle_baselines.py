"""The oracle's threaded CPU-baseline functions (timed by bench.py) compute what the pinned serial
functions compute."""
import numpy as np
import pytest

import oracle_lib as O
from pufferlean_amd import rng


@pytest.mark.parametrize("time_major", [0, 1])
@pytest.mark.parametrize("variant", [0, 1])
def test_vtrace_mt_equals_serial(time_major, variant):
    B, T = 37, 19
    n = B * T
    cols = [O.f32(rng.normal(900 + k, n)) for k in range(2)]
    term = O.f32(rng.bernoulli(902, n, 0.1))
    lr = O.f32(rng.normal(903, n, 0.0, 0.2))
    boot = O.f32(rng.normal(904, B))
    outs = []
    for fn, extra in ((O.lib().orc_vtrace_f32, ()), (O.lib().orc_vtrace_f32_mt, (5,))):
        adv = np.zeros(n, np.float32); tgt = np.zeros(n, np.float32)
        fn(O.P(cols[0]), O.P(cols[1]), O.P(term), O.P(lr), O.P(boot), B, T, variant, time_major, 1, 1,
           0.99, 0.95, 1.0, 1.0, O.P(adv), O.P(tgt), *extra)
        outs.append((adv, tgt))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_gemm_blocked_vs_numpy(ta, tb):
    M, N, K = 133, 75, 300
    A = rng.normal(910, M * K).reshape((K, M) if ta else (M, K))
    B = rng.normal(911, K * N).reshape((N, K) if tb else (K, N))
    C = np.zeros((M, N))
    O.lib().orc_gemm_blocked(ta, tb, M, N, K, O.P(A), A.shape[1], O.P(B), B.shape[1], O.P(C), N, 4)
    np.testing.assert_allclose(C, (A.T if ta else A) @ (B.T if tb else B), rtol=1e-12, atol=1e-11)


def test_mingru_batch_equals_sum_of_sequences():
    B, T, D, H, L, A = 5, 7, 4, 8, 2, 3
    P = H * D + H + L * 3 * H * H + A * H + A + H + 1
    p = rng.normal(920, P) * 0.3
    obs = rng.normal(921, T * B * D).reshape(T, B, D)
    act = rng.randint(922, T * B, A).astype(float).reshape(T, B)
    adv, ret = rng.normal(923, T * B).reshape(T, B), rng.normal(924, T * B).reshape(T, B)
    old = rng.randf(925, T * B, -1.5, -0.5).reshape(T, B)
    term = rng.bernoulli(926, T * B, 0.2).reshape(T, B)
    ov = rng.normal(927, T * B).reshape(T, B)
    g = np.zeros(P); lp = np.zeros((T, B)); nv = np.zeros((T, B))
    for b in range(B):
        out = np.zeros(P + 2 * T)
        O.lib().orc_mingru_ppo_grad_seq(O.P(p), O.P(O.f64(obs[:, b, :])), O.P(O.f64(act[:, b])),
                                        O.P(O.f64(adv[:, b])), O.P(O.f64(ret[:, b])), O.P(O.f64(old[:, b])),
                                        O.P(O.f64(term[:, b])), O.P(O.f64(ov[:, b])), T, H, D, L, A, 0.5, 0.01,
                                        0.2, 0.2, O.P(out))
        g += out[:P]; lp[:, b] = out[P:P + T]; nv[:, b] = out[P + T:]
    for threads in (1, 3):
        out = np.zeros(P + 2 * T * B)
        O.lib().orc_mingru_ppo_grad_batch(O.P(p), O.P(O.f64(obs)), O.P(O.f64(act)), O.P(O.f64(adv)),
                                          O.P(O.f64(ret)), O.P(O.f64(old)), O.P(O.f64(term)), O.P(O.f64(ov)),
                                          B, T, H, D, L, A, 0.5, 0.01, 0.2, 0.2, O.P(out), threads)
        if threads == 1:
            assert np.array_equal(out[:P], g)
        np.testing.assert_allclose(out[:P], g, rtol=1e-12, atol=1e-14)
        assert np.array_equal(out[P:P + T * B].reshape(T, B), lp)
        assert np.array_equal(out[P + T * B:].reshape(T, B), nv)


def test_threaded_newton_schulz_equals_serial():
    X = rng.normal(930, 48 * 80, 0.0, 0.02).reshape(48, 80)
    ref = O.newton_schulz(X, O.BASELINE_COEFFS, form=1)
    old = O.lib().orc_set_threads(4)
    try:
        got = O.newton_schulz(X, O.BASELINE_COEFFS, form=1)
        got0 = O.newton_schulz(X.T.copy(), O.REF_COEFFS, form=0)
    finally:
        O.lib().orc_set_threads(old)
    assert np.array_equal(got, ref)
    assert np.array_equal(got0, O.newton_schulz(X.T.copy(), O.REF_COEFFS, form=0))
