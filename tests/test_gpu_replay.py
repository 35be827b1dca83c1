"""Prioritised replay on the GPU vs the CPU oracle (the twins pufferffi.c:1094-1200 and the iterate
loop of puffercuda.cu:500-511).

Bars: segment sums, gathered act/ret/old/term/ov columns, segment choice of the iterate and the
value column bit-exact; draws bit-exact except a draw whose uniform lies within rounding of a
cumulative boundary (the sampler's sums use a fixed tree order, the twin's are sequential);
normalised advantages, mean/std and importance weights within 1e-12 relative; ratio = exp(.)
within 1e-15 relative (device exp vs the host's, both within an ulp).
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def cu(x, dt=torch.float64):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dt)


def dp(a):
    return np.ascontiguousarray(a, np.float64).ctypes.data_as(C.POINTER(C.c_double))


def relmax(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-300))


# ---- per-segment |adv| sums ---------------------------------------------------------------------
@pytest.mark.parametrize("N,T", [(1, 1), (7, 5), (1000, 129), (4096, 64)])
def test_seg_l1_segment_major_f64_bit_exact(gpu, N, T):
    print(f"seg_l1 f64 N={N} T={T}", flush=True)
    adv = rng.normal(0x101 + N, N * T)
    got = D.seg_l1(D.ReplayColumns(N, T, adv=cu(adv))).cpu().numpy()
    assert np.array_equal(got, O.seg_l1(adv, N, T))


def test_seg_l1_time_major_f32_bit_exact(gpu):
    N, T = 4096, 64
    adv = rng.normal(0x102, N * T).astype(np.float32).reshape(T, N)
    got = D.seg_l1(D.ReplayColumns(N, T, adv=cu(adv, torch.float32), time_major=True)).cpu().numpy()
    # f32 -> f64 is exact, and both sum t ascending in f64
    assert np.array_equal(got, O.seg_l1(adv.T.astype(np.float64), N, T))


# ---- prioritised sampler ------------------------------------------------------------------------
def _check_draws(seg, mp, L1, mb, alpha, beta, state):
    idx, mpr, probs, cum = O.prio_sample(L1, mb, alpha, beta, state)
    seg = seg.astype(np.float64)
    bad = np.nonzero(seg != idx)[0]
    u = rng.uniform01(rng.words(state, mb)) * cum[-1]
    for i in bad:  # only boundary draws may differ, and only to the neighbouring segment
        k = int(min(seg[i], idx[i]))
        assert abs(seg[i] - idx[i]) == 1 and abs(cum[k] - u[i]) <= 1e-12 * cum[-1], (i, seg[i], idx[i])
    assert len(bad) <= max(1, mb // 1000)
    ok = seg == idx
    assert relmax(mp[ok], mpr[ok]) < 1e-12
    return idx


@pytest.mark.parametrize("N,mb", [(1, 16), (7, 1), (1000, 777), (4096, 4096), (6144, 3000), (6145, 3000),
                                  (50000, 8192)])
def test_prio_sample_matches_cpu_twin(gpu, N, mb):
    print(f"prio_sample N={N} draws={mb}", flush=True)
    L1 = np.abs(rng.normal(0x201 + N, N)) * 20.0
    L1[::13] = 0.0
    alpha, beta, state = 0.8, 0.35, 0x0123456789ABCDEF + N
    seg, mp = D.prio_sample(cu(L1), mb, alpha=alpha, beta=beta, rng_state=state)
    torch.cuda.synchronize()
    _check_draws(seg.cpu().numpy(), mp.cpu().numpy(), L1, mb, alpha, beta, state)


def test_prio_sample_zero_and_constant_priorities(gpu):
    for L1 in (np.zeros(300), np.full(300, 4.0)):
        seg, mp = D.prio_sample(cu(L1), 2000, alpha=0.8, beta=0.2, rng_state=0x55)
        _check_draws(seg.cpu().numpy(), mp.cpu().numpy(), L1, 2000, 0.8, 0.2, 0x55)


def test_prio_sample_reproducible(gpu):
    L1 = cu(np.abs(rng.normal(0x202, 20000)))
    a = [D.prio_sample(L1, 5000, alpha=0.6, beta=0.4, rng_state=0xFEED) for _ in range(2)]
    assert torch.equal(a[0][0], a[1][0]) and torch.equal(a[0][1], a[1][1])


def test_ffi_prio_sample_matches_cpu_twin(gpu):
    N, mb, state = 2048, 512, 0xC0FFEE
    L1 = np.abs(rng.normal(0x203, N)) * 5.0
    idx, mp = np.zeros(mb), np.zeros(mb)
    L.call("ph_ffi_prio_sample", dp(L1), N, 64, mb, 0.8, 0.2, state, dp(idx), dp(mp))
    _check_draws(idx, mp, L1, mb, 0.8, 0.2, state)


# ---- minibatch gather ---------------------------------------------------------------------------
def _cols(seed, N, T, K=1):
    adv = rng.normal(seed, N * T)
    val = rng.normal(seed + 1, N * T)
    act = rng.randint(seed + 2, N * T * K, 16).astype(np.float64)
    logp = rng.randf(seed + 3, N * T, -3.0, -0.1)
    term = rng.randf(seed + 4, N * T, 0.0, 1.0)
    return act, logp, term, adv, val


def _segs(seed, B, N):
    s = rng.randint(seed, B, N)
    if B > 8:
        s[5] = s[2] = s[B - 1]  # repeated draws
    return s


@pytest.mark.parametrize("N,T,B,time_major", [(300, 16, 200, False), (300, 16, 200, True), (1, 3, 4, False),
                                              (4096, 64, 4096, False), (4096, 64, 4096, True)])
def test_gather_f64_matches_cpu_twin(gpu, N, T, B, time_major):
    print(f"mb_gather f64 N={N} T={T} B={B} time_major={time_major}", flush=True)
    act, logp, term, adv, val = _cols(0x301, N, T)
    seg = _segs(0x306, B, N)
    mp = rng.randf(0x307, B, 0.3, 3.0)
    ref, rst = O.gather_seq_minibatch(act, logp, term, adv, val, seg.astype(np.float64), mp, T)
    lay = (lambda x: x.reshape(N, T).T) if time_major else (lambda x: x)
    cols = D.ReplayColumns(N, T, adv=cu(lay(adv)), value=cu(lay(val)), act=cu(lay(act)), logp=cu(lay(logp)),
                           term=cu(lay(term)), time_major=time_major)
    st = torch.zeros(2, device="cuda", dtype=torch.float64)
    out = D.mb_gather(cols, cu(seg, torch.int32), cu(mp), stats=st).cpu().numpy()
    n = T * B
    for k in (0, 2, 3, 4, 5):
        assert np.array_equal(out[k * n:(k + 1) * n], ref[k * n:(k + 1) * n]), k
    assert relmax(out[n:2 * n], ref[n:2 * n]) < 1e-12
    assert relmax(st.cpu().numpy(), rst) < 1e-12


def test_gather_multi_component_actions(gpu):
    N, T, B, K = 50, 10, 40, 3
    act, logp, term, adv, val = _cols(0x311, N, T, K)
    seg = _segs(0x316, B, N)
    cols = D.ReplayColumns(N, T, adv=cu(adv), value=cu(val), act=cu(act), logp=cu(logp), term=cu(term), K=K)
    out = D.mb_gather(cols, cu(seg, torch.int32)).cpu().numpy()
    n = T * B
    expect = act.reshape(N, T, K)[seg].transpose(1, 0, 2).ravel()  # [T][B][K]
    assert np.array_equal(out[:K * n], expect)
    ref, _ = O.gather_seq_minibatch(act.reshape(N, T, K)[:, :, 0].ravel(), logp, term, adv, val,
                                    seg.astype(np.float64), np.ones(B), T)
    assert np.array_equal(out[(K + 1) * n:], ref[2 * n:])
    assert relmax(out[K * n:(K + 1) * n], ref[n:2 * n]) < 1e-12


def test_gather_f32_time_major(gpu):
    N, T, B = 4096, 64, 1024
    act, logp, term, adv, val = (x.astype(np.float32).astype(np.float64) for x in _cols(0x321, N, T))
    seg = _segs(0x326, B, N)
    mp = rng.randf(0x327, B, 0.3, 3.0)
    ref, rst = O.gather_seq_minibatch(act, logp, term, adv, val, seg.astype(np.float64), mp, T)
    tm = lambda x: cu(x.reshape(N, T).T, torch.float32)
    cols = D.ReplayColumns(N, T, adv=tm(adv), value=tm(val), act=tm(act), logp=tm(logp), term=tm(term),
                           time_major=True)
    out = D.mb_gather(cols, cu(seg, torch.int32), cu(mp)).cpu().numpy().astype(np.float64)
    n = T * B
    for k in (0, 3, 4, 5):
        assert np.array_equal(out[k * n:(k + 1) * n], ref[k * n:(k + 1) * n]), k
    assert relmax(out[2 * n:3 * n], ref[2 * n:3 * n]) < 1e-6  # a + v rounded to f32
    assert relmax(out[n:2 * n], ref[n:2 * n]) < 1e-6


def test_gather_out_of_range_index_gives_nan_rows(gpu):
    N, T, B = 20, 4, 6
    act, logp, term, adv, val = _cols(0x331, N, T)
    seg = np.array([0, 3, -1, 7, N, 19])
    cols = D.ReplayColumns(N, T, adv=cu(adv), value=cu(val), act=cu(act), logp=cu(logp), term=cu(term))
    out = D.mb_gather(cols, cu(seg, torch.int32)).cpu().numpy().reshape(6, T, B)
    assert np.all(np.isnan(out[:, :, [2, 4]]))
    assert np.all(np.isfinite(out[[0, 2, 3, 4, 5]][:, :, [0, 1, 3, 5]]))


def test_ffi_gather_seq_minibatch_matches_cpu_twin(gpu):
    N, T, B, Dm = 64, 16, 48, 5
    act, logp, term, adv, val = _cols(0x341, N, T)
    seg = _segs(0x346, B, N).astype(np.float64)
    mp = rng.randf(0x347, B, 0.3, 3.0)
    out = np.zeros(6 * T * B)
    L.call("ph_ffi_gather_seq_minibatch", None, dp(act), dp(logp), dp(term), dp(adv), dp(val), dp(seg), dp(mp),
           T, B, Dm, N, dp(out))
    ref, _ = O.gather_seq_minibatch(act, logp, term, adv, val, seg, mp, T)
    n = T * B
    assert np.array_equal(np.delete(out, np.s_[n:2 * n]), np.delete(ref, np.s_[n:2 * n]))
    assert relmax(out[n:2 * n], ref[n:2 * n]) < 1e-12
    bad = seg.copy()
    bad[3] = N
    with pytest.raises(L.PufferHipError, match="segIdx"):
        L.call("ph_ffi_gather_seq_minibatch", None, dp(act), dp(logp), dp(term), dp(adv), dp(val), dp(bad),
               dp(mp), T, B, Dm, N, dp(out))


# ---- value / ratio iterate ----------------------------------------------------------------------
def _iter_expect(value, ratio, logp, newlp, newval, seg, N, T):
    """Last assignment per segment over the valid draws, t ascending (segment-major columns)."""
    value, ratio = value.copy(), ratio.copy()
    B = len(seg)
    for bi, e in enumerate(seg):
        if 0 <= e < N:
            for t in range(T):
                value[e * T + t] = float(newval[t * B + bi])
                ratio[e * T + t] = np.exp(float(newlp[t * B + bi]) - logp[e * T + t])
    return value, ratio


@pytest.mark.parametrize("time_major", [False, True])
def test_iterate_f64_matches_in_order_loop(gpu, time_major):
    N, T = 500, 70  # T > 64: each wavefront loops over its steps
    value0 = rng.normal(0x401, N * T)
    logp = rng.randf(0x402, N * T, -3.0, -0.1)
    lay = (lambda x: x.reshape(N, T).T) if time_major else (lambda x: x)
    unlay = (lambda x: x.reshape(T, N).T.ravel()) if time_major else (lambda x: x)
    dv, dr = cu(lay(value0)), cu(lay(np.ones(N * T)))
    cols = D.ReplayColumns(N, T, value=dv, ratio=dr, logp=cu(lay(logp)), time_major=time_major)
    value, ratio = value0.copy(), np.ones(N * T)
    for call, B in enumerate((300, 120, 300)):  # the last-writer table must be clear between calls
        seg = _segs(0x410 + call, B, N)
        newlp = rng.randf(0x420 + call, T * B, -3.0, -0.1).astype(np.float32)
        newval = rng.normal(0x430 + call, T * B).astype(np.float32)
        D.mb_iterate(cols, cu(seg, torch.int32), cu(newlp, torch.float32), cu(newval, torch.float32))
        ov, orr = O.mb_iterate(value, ratio, logp, newlp, newval, seg.astype(np.float64), T)
        value, ratio = ov, orr
        gv, gr = unlay(dv.cpu().numpy()), unlay(dr.cpu().numpy())
        assert np.array_equal(gv, value), call
        assert relmax(gr, ratio) < 1e-15, call
        value, ratio = gv, gr  # continue from the device state


def test_iterate_f32_and_invalid_indices(gpu):
    N, T, B = 64, 33, 40
    value0 = rng.normal(0x441, N * T).astype(np.float32)
    logp = rng.randf(0x442, N * T, -3.0, -0.1).astype(np.float32)
    seg = _segs(0x443, B, N)
    seg[[1, 9]] = [-1, N]
    newlp = rng.randf(0x444, T * B, -3.0, -0.1).astype(np.float32)
    newval = rng.normal(0x445, T * B).astype(np.float32)
    dv, dr = cu(value0, torch.float32), cu(np.ones(N * T), torch.float32)
    cols = D.ReplayColumns(N, T, value=dv, ratio=dr, logp=cu(logp, torch.float32))
    D.mb_iterate(cols, cu(seg, torch.int32), cu(newlp, torch.float32), cu(newval, torch.float32))
    ev, er = _iter_expect(value0.astype(np.float64), np.ones(N * T), logp.astype(np.float64), newlp, newval,
                          seg, N, T)
    assert np.array_equal(dv.cpu().numpy().astype(np.float64), ev.astype(np.float32).astype(np.float64))
    assert np.array_equal(dr.cpu().numpy(), er.astype(np.float32))
    # the skipped draws left the table clear: a second call behaves like a fresh one
    seg2 = _segs(0x446, B, N)
    D.mb_iterate(cols, cu(seg2, torch.int32), cu(newlp, torch.float32), cu(newval, torch.float32))
    ev2, _ = _iter_expect(ev.astype(np.float32).astype(np.float64), er, logp.astype(np.float64), newlp, newval,
                          seg2, N, T)
    assert np.array_equal(dv.cpu().numpy().astype(np.float64), ev2.astype(np.float32).astype(np.float64))


# ---- the host-buffer chain of the MinGRU trainer ------------------------------------------------
def test_mg_chain_device_columns_match_host_path(gpu, monkeypatch):
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    monkeypatch.delenv("PUFFER_MG_DEVPRIO", raising=False)
    N, T, B, Dm, H, Ln, A = 24, 8, 10, 8, 16, 2, 5
    gam, lam, rc, cc, alpha, beta = 0.99, 0.95, 1.0, 1.0, 0.8, 0.3
    n = N * T
    Pn = H * Dm + H + Ln * 3 * H * H + A * H + A + H + 1
    p = rng.normal(0x501, Pn) * 0.3
    rew = rng.normal(0x502, n)
    term = rng.bernoulli(0x503, n, 0.05)
    act = rng.randint(0x504, n, A).astype(np.float64)
    logp = rng.randf(0x505, n, -2.5, -1.0)
    val = rng.normal(0x506, n)
    boot = rng.normal(0x507, N)
    obs_roll = rng.normal(0x508, n * Dm).reshape(N, T, Dm)
    L.call("ph_cuda_mg_prep", dp(rew), dp(term), dp(act), dp(logp), dp(val), dp(boot), N, T, 1)
    ready = C.c_uint8(9)
    L.call("ph_cuda_mg_cols_ready", N, T, C.byref(ready))
    assert ready.value == 0

    # V-trace + segment sums on the resident columns: bit-exact vs the oracle
    L1 = np.zeros(N)
    L.call("ph_cuda_mg_vtrace", N, T, gam, lam, rc, cc, dp(L1))
    adv = np.zeros(n)
    O.lib().orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(np.ones(n)), O.P(boot), N, T, gam, lam, rc, cc,
                              O.P(adv))
    assert np.array_equal(L1, O.seg_l1(adv, N, T))

    # host path: device twin of the sampler and gather, host-mode gradient
    idx, mp = np.zeros(B), np.zeros(B)
    L.call("ph_ffi_prio_sample", dp(L1), N, T, B, alpha, beta, 0x77, dp(idx), dp(mp))
    _check_draws(idx, mp, L1, B, alpha, beta, 0x77)
    scal = np.zeros(6 * T * B)
    L.call("ph_ffi_gather_seq_minibatch", None, dp(act), dp(logp), dp(term), dp(adv), dp(val), dp(idx), dp(mp),
           T, B, Dm, N, dp(scal))
    obs = np.ascontiguousarray(obs_roll[idx.astype(np.int64)].transpose(1, 0, 2))  # [T][B][D]
    args = (B, T, H, Dm, Ln, A, 1, None, 0, 0.5, 0.01, 0.2, 0.2)
    out_host = np.zeros(Pn + 2 * T * B)
    ln = C.c_size_t(0)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0, None, 0,
           dp(out_host), C.byref(ln))
    assert ln.value == out_host.size

    # device-column mode with the same draws: the same gather on the same resident data; the gradient
    # stays on the device (resident mode: zero-length result)
    out_dev = np.zeros_like(out_host)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, None, 0, *args, dp(idx), B, dp(mp), B,
           dp(out_dev), C.byref(ln))
    assert ln.value == 0
    g_dev = np.zeros(Pn)
    L.call("ph_cuda_mg_resident_grad", Pn, dp(g_dev))
    assert np.array_equal(g_dev, out_host[:Pn])

    # ... and it iterated value/ratio of the drawn segments: V-trace again sees the new columns
    nlp = out_host[Pn:Pn + T * B].astype(np.float32)
    nv = out_host[Pn + T * B:].astype(np.float32)
    val2, ratio2 = O.mb_iterate(val, np.ones(n), logp, nlp, nv, idx, T)
    adv2 = np.zeros(n)
    O.lib().orc_vtrace_mingru(O.P(rew), O.P(val2), O.P(term), O.P(ratio2), O.P(boot), N, T, gam, lam, rc, cc,
                              O.P(adv2))
    L1b = np.zeros(N)
    L.call("ph_cuda_mg_vtrace", N, T, gam, lam, rc, cc, dp(L1b))
    assert relmax(L1b, O.seg_l1(adv2, N, T)) < 1e-12

    # resident draws: V-trace + sampler on the device, consumed by the next gradient call
    used = C.c_uint8(0)
    L.call("ph_cuda_mg_vtrace_prio", N, T, gam, lam, rc, cc, B, alpha, beta, 0x99, C.byref(used))
    assert used.value == 1
    idx3, mp3 = np.zeros(B), np.zeros(B)
    L.call("ph_ffi_prio_sample", dp(L1b), N, T, B, alpha, beta, 0x99, dp(idx3), dp(mp3))
    obs3 = np.ascontiguousarray(obs_roll[idx3.astype(np.int64)].transpose(1, 0, 2))
    out_res = np.zeros_like(out_host)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs3), obs3.size, None, 0, *args, None, 0, None, 0, dp(out_res),
           C.byref(ln))
    assert ln.value == 0
    g_res = np.zeros(Pn)
    L.call("ph_cuda_mg_resident_grad", Pn, dp(g_res))
    scal3, _ = O.gather_seq_minibatch(act, logp, term, adv2, val2, idx3, mp3, T)
    out_chk = np.zeros_like(out_host)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs3), obs3.size, dp(scal3), scal3.size, *args, None, 0, None,
           0, dp(out_chk), C.byref(ln))
    assert relmax(g_res, out_chk[:Pn]) < 1e-5
    # the stamp was consumed: without scal or draws there is no scalar source
    with pytest.raises(L.PufferHipError, match="no scalar source"):
        L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, None, 0, *args, None, 0, None, 0,
               dp(out_res), C.byref(ln))
    monkeypatch.setenv("PUFFER_MG_DEVPRIO", "0")
    L.call("ph_cuda_mg_vtrace_prio", N, T, gam, lam, rc, cc, B, alpha, beta, 0x99, C.byref(used))
    assert used.value == 0
    with pytest.raises(L.PufferHipError, match="ph_cuda_mg_prep"):
        L.call("ph_cuda_mg_vtrace", N + 1, T, gam, lam, rc, cc, dp(L1b))
