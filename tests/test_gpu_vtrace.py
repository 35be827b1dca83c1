"""V-trace / GAE on the GPU vs the CPU oracle (bit-exact where the op order allows)."""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def _verify_inputs(seed, B, T):
    # draw order of the reference's verify-vtrace-gpu / verify-vtrace-mingru-gpu
    # (Exe/Puffer.lean:1075-1084, 1104-1116)
    w = rng.uniform01(rng.words(seed, 4 * B * T)).reshape(B * T, 4)
    rew = -1.5 + (1.5 - -1.5) * w[:, 0]
    val = -2.0 + (2.0 - -2.0) * w[:, 1]
    term = (w[:, 2] < 0.12).astype(np.float64)
    imp = 0.1 + (2.0 - 0.1) * w[:, 3]
    boot = -2.0 + 4.0 * rng.uniform01(rng.words(seed, B, start=4 * B * T))
    return rew, val, term, imp, boot


def _cuda(x, dtype=torch.float64):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dtype)


@pytest.mark.parametrize("variant,seed", [(0, 0x5C1A), (1, 0x5C1B)])
def test_reference_verify_cases_bit_exact(gpu, variant, seed):
    B, T = 8, 12
    rew, val, term, imp, boot = _verify_inputs(seed, B, T)
    if variant == 0:
        ref = np.zeros(B * T)
        O.lib().orc_vtrace_vec(O.P(rew), O.P(val), O.P(term), O.P(imp), B, T, 0.99, 0.95, 2.1,
                               1.08, O.P(ref))
    else:
        ref = np.zeros(B * T)
        O.lib().orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(imp), O.P(boot), B, T, 0.99,
                                  0.95, 2.1, 1.08, O.P(ref))
    t = lambda x: _cuda(x).reshape(B, T)
    adv, tgt = D.vtrace(t(rew), t(val), t(term), t(imp), _cuda(boot), variant=variant,
                        time_major=False, rho_clip=2.1, c_clip=1.08)
    got = adv.cpu().numpy().ravel()
    assert np.array_equal(got, ref), f"max|d| = {np.abs(got - ref).max()}"
    assert np.array_equal(tgt.cpu().numpy().ravel(), ref + val)


def _bench_inputs(B, T, seed=0x4000):
    # time-major [T][B]: V, r ~ N(0,1), done ~ Bernoulli(0.01), log ratio ~ N(0, 0.1)
    n = B * T
    val = rng.normal(seed + 1, n)
    rew = rng.normal(seed + 2, n)
    done = rng.bernoulli(seed + 3, n, 0.01)
    logr = rng.normal(seed + 4, n, 0.0, 0.1)
    boot = rng.normal(seed + 5, B)
    return rew, val, done, logr, boot


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("time_major", [True, False])
@pytest.mark.parametrize("B,T", [(4096, 64), (1000, 37), (1, 1), (3, 2), (257, 64)])
def test_fp32_bit_exact_vs_f32_twin(gpu, variant, time_major, B, T):
    rew, val, done, logr, boot = _bench_inputs(B, T)
    ratio = np.exp(logr.astype(np.float32))  # ratio formed on the host: no device exp involved
    a32, t32 = O.vtrace(rew, val, done, ratio, boot, B, T, variant=variant, time_major=time_major,
                        dtype=np.float32)
    shape = (T, B) if time_major else (B, T)
    c = lambda x: _cuda(x, torch.float32).reshape(shape)
    adv, tgt = D.vtrace(c(rew), c(val), c(done), c(ratio), _cuda(boot, torch.float32),
                        variant=variant, time_major=time_major)
    assert np.array_equal(adv.cpu().numpy().ravel(), a32)
    assert np.array_equal(tgt.cpu().numpy().ravel(), t32)
    # and within 1e-5 relative Frobenius of the f64 oracle on the same fp32 inputs
    a64, _ = O.vtrace(rew.astype(np.float32), val.astype(np.float32), done.astype(np.float32),
                      ratio.astype(np.float64), boot.astype(np.float32), B, T, variant=variant,
                      time_major=time_major)
    den = max(np.linalg.norm(a64), 1e-30)
    assert np.linalg.norm(adv.cpu().numpy().ravel().astype(np.float64) - a64) / den < 1e-5


@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("with_rho,want_targets", [(True, True), (False, False)])
def test_fp32_streaming_path_bit_exact(gpu, variant, with_rho, want_targets):
    """Large time-major fp32 batches take the two-segments-per-lane, nontemporal kernel; it is still
    bit-identical to the f32 twin (with ratios, and as plain GAE without targets)."""
    B, T = 131072, 16
    rew, val, done, logr, boot = _bench_inputs(B, T, seed=0x4400)
    ratio = np.exp(logr.astype(np.float32)) if with_rho else np.ones(B * T, np.float32)
    a32, t32 = O.vtrace(rew, val, done, ratio, boot, B, T, variant=variant, time_major=True,
                        dtype=np.float32)
    c = lambda x: _cuda(x, torch.float32).reshape(T, B)
    adv, tgt = D.vtrace(c(rew), c(val), c(done), c(ratio) if with_rho else None,
                        _cuda(boot, torch.float32), variant=variant, time_major=True,
                        want_targets=want_targets)
    assert np.array_equal(adv.cpu().numpy().ravel(), a32)
    if want_targets:
        assert np.array_equal(tgt.cpu().numpy().ravel(), t32)
    else:
        assert tgt is None


@pytest.mark.parametrize("variant", [0, 1])
def test_log_ratio_input_within_tolerance(gpu, variant):
    B, T = 4096, 64
    rew, val, done, logr, boot = _bench_inputs(B, T, seed=0x4100)
    a64, t64 = O.vtrace(rew.astype(np.float32), val.astype(np.float32), done, logr.astype(np.float32),
                        boot.astype(np.float32), B, T, variant=variant, time_major=True,
                        rho_is_log=True)
    c = lambda x: _cuda(x, torch.float32).reshape(T, B)
    adv, tgt = D.vtrace(c(rew), c(val), c(done), c(logr), _cuda(boot, torch.float32),
                        variant=variant, time_major=True, rho_is_log=True)
    g = adv.cpu().numpy().ravel().astype(np.float64)
    assert np.linalg.norm(g - a64) / np.linalg.norm(a64) < 1e-5
    gt = tgt.cpu().numpy().ravel().astype(np.float64)
    assert np.linalg.norm(gt - t64) / np.linalg.norm(t64) < 1e-5


def test_gae_is_unit_ratio_and_matches_gae_soa(gpu):
    B, T = 300, 50
    rew, val, done, _, _ = _bench_inputs(B, T, seed=0x4200)
    out = np.zeros(2 * B * T)
    O.lib().orc_gae_soa(O.P(val), O.P(rew), O.P(done), B, T, 0.99, 0.95, O.P(out))
    c = lambda x: _cuda(x).reshape(B, T)
    adv, tgt = D.vtrace(c(rew), c(val), c(done), None, None, variant=0, time_major=False)
    assert np.array_equal(adv.cpu().numpy().ravel(), out[:B * T])
    assert np.array_equal(tgt.cpu().numpy().ravel(), out[B * T:])


def test_edge_cases(gpu):
    # all done: every step stands alone; no done: one long discounted sum; B = 0 is a no-op
    B, T = 130, 20
    rew, val, _, logr, boot = _bench_inputs(B, T, seed=0x4300)
    for done in (np.ones(B * T), np.zeros(B * T)):
        for variant in (0, 1):
            ref, _ = O.vtrace(rew, val, done, np.exp(logr), boot, B, T, variant=variant,
                              time_major=True)
            c = lambda x: _cuda(x).reshape(T, B)
            adv, _ = D.vtrace(c(rew), c(val), c(done), c(np.exp(logr)), _cuda(boot),
                              variant=variant, time_major=True)
            assert np.array_equal(adv.cpu().numpy().ravel(), ref)
    e = torch.empty((0, 5), device="cuda", dtype=torch.float32)
    D.vtrace(e, e, e, e, torch.empty(5, device="cuda"), variant=1, time_major=True)


def test_full_size_replicated_properties(gpu):
    """64 replicas of the 4096x64 workload in one launch: each replica equals the single run,
    and the targets-minus-values identity holds everywhere."""
    B, T, R = 4096, 64, 64
    rew, val, done, logr, boot = _bench_inputs(B, T, seed=0x4400)
    c = lambda x: _cuda(x, torch.float32).reshape(T, B)
    one, _ = D.vtrace(c(rew), c(val), c(done), c(logr), _cuda(boot, torch.float32), variant=1,
                      time_major=True, rho_is_log=True)
    rep = lambda x: c(x).repeat(1, R).contiguous()
    adv, tgt = D.vtrace(rep(rew), rep(val), rep(done), rep(logr),
                        _cuda(boot, torch.float32).repeat(R).contiguous(), variant=1,
                        time_major=True, rho_is_log=True)
    for r in (0, 17, 63):
        assert torch.equal(adv[:, r * B:(r + 1) * B], one)
    assert torch.equal(tgt, adv + rep(val))
