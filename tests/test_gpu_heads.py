"""Multi-discrete and continuous heads on the GPU vs the CPU oracle (k_ppo_dout_md / k_ppo_dout_cont /
k_sample_md / k_sample_cont, puffercuda.cu:702-727, 1538-1551, 1652-1668, 1767-1790).

Bars: loss gradients and new log-probs within 1e-5 relative (fp32 against f64); values exact;
multi-discrete draws exact except within rounding of a cumulative boundary (1e-12 for f64 rows, 1e-5
for f32); Gaussian draws within 1e-12 relative (f64 rows); the MLP gradients within 1e-5 (fp32
products) and 1e-2 (bf16 products) of the f64 composition.
"""
import ctypes as C

import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu
GOLD, GOLD2, MASK = 0x9E3779B97F4A7C15, 0xD1B54A32D192ED03, 0xFFFFFFFFFFFFFFFF


def cu(x, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda", dt)


def vp(t):
    """Raw device address of t. The caller keeps t referenced while a kernel may use it: the address of
    a dropped temporary is handed to the next allocation."""
    return C.c_void_p(t.data_ptr()) if t is not None else None


def dp(a):
    return np.ascontiguousarray(a, np.float64).ctypes.data_as(C.POINTER(C.c_double))


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def st():
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def word_unit(x):
    return float(rng.uniform01(rng.words((x - GOLD) & MASK, 1))[0])


# ---- loss gradients -----------------------------------------------------------------------------
# heads 3+9+2+5 (+ value) fit the 32-wide LDS tile; 20+17+3 run the row-per-lane kernel
@pytest.mark.parametrize("sizes", [[3, 9, 2, 5], [20, 17, 3]])
@pytest.mark.parametrize("vfclip", [0.0, 0.25])
def test_ppo_grad_md_matches_oracle(gpu, vfclip, sizes):
    N, K, W = 5000, len(sizes), sum(sizes)
    print(f"md grad sizes={sizes} vfclip={vfclip}", flush=True)
    out = (rng.normal(0xA01, N * (W + 1)).reshape(N, W + 1) * 2.0).astype(np.float32).astype(np.float64)
    acts = np.stack([rng.randint(0xA02 + h, N, s) for h, s in enumerate(sizes)], axis=1)
    adv, ret = rng.normal(0xA06, N), rng.normal(0xA07, N)
    ov = out[:, W] + rng.normal(0xA08, N, 0.0, 0.5)
    _, nlp0, _ = O.ppo_grad_md(out, acts, adv, ret, np.zeros(N), ov, sizes)
    old = nlp0 + rng.normal(0xA09, N, 0.0, 0.3)
    f32 = lambda x: x.astype(np.float32).astype(np.float64)
    ref, rlp, rv = O.ppo_grad_md(out, acts, f32(adv), f32(ret), f32(old), f32(ov), sizes, vfclip=vfclip)
    g = torch.empty(N, W + 1, device="cuda")
    nlp, nv = torch.empty(N, device="cuda"), torch.empty(N, device="cuda")
    hs = (C.c_int * K)(*sizes)
    # every device input stays referenced until after the synchronize: the kernel reads them
    dout_, dact, dadv, dret, dold, dov = cu(out), cu(acts, torch.int32), cu(adv), cu(ret), cu(old), cu(ov)
    assert int(dact.min()) >= 0 and all(int(dact[:, h].max()) < s for h, s in enumerate(sizes))
    losses = torch.zeros(7, device="cuda", dtype=torch.float64)
    L.call("ph_ppo_grad_md", vp(dout_), W + 1, vp(dact), vp(dadv), vp(dret), vp(dold), vp(dov), N, hs, K, 0.5, 0.01,
           0.2, vfclip, vp(g), W + 1, vp(nlp), vp(nv), vp(losses), st())
    torch.cuda.synchronize()
    assert rel(g.cpu().numpy(), ref) < 1e-5
    assert rel(nlp.cpu().numpy(), rlp) < 1e-5
    assert np.array_equal(nv.cpu().numpy().astype(np.float64), rv)
    rL = O.wide_losses(1, out, acts, f32(adv), f32(ret), f32(old), f32(ov), sizes=sizes, vfclip=vfclip)
    np.testing.assert_allclose(losses.cpu().numpy(), rL, rtol=1e-5, atol=max(1e-6, 2.0 / N))


@pytest.mark.parametrize("sizes", [[3, 4], [20, 17]])
def test_ppo_grad_md_out_of_range_action_gives_nan_row(gpu, sizes):
    """The kernels' range check (tiled and row-per-lane forms): a bad action makes its row's logit
    gradients and log-prob NaN, as in the oracle, and reads nothing outside the row."""
    N, K, W = 4, 2, sum(sizes)
    out = rng.normal(0xA0A, N * (W + 1)).reshape(N, W + 1).astype(np.float32).astype(np.float64)
    acts = np.array([[0, sizes[1] - 1], [sizes[0], 0], [-1, 2], [2, sizes[1] - 1]], np.int32)
    ref, rlp, _ = O.ppo_grad_md(out, acts.astype(np.float64), np.ones(N), np.zeros(N), np.full(N, -2.0), None,
                                sizes)
    dout_, dact = cu(out), cu(acts, torch.int32)
    dadv, dret, dold = cu(np.ones(N)), cu(np.zeros(N)), cu(np.full(N, -2.0))
    g = torch.empty(N, W + 1, device="cuda")
    nlp = torch.empty(N, device="cuda")
    hs = (C.c_int * K)(*sizes)
    L.call("ph_ppo_grad_md", vp(dout_), W + 1, vp(dact), vp(dadv), vp(dret), vp(dold), None, N, hs, K, 0.5, 0.01, 0.2,
           0.0, vp(g), W + 1, vp(nlp), None, None, st())
    torch.cuda.synchronize()
    gg, ll = g.cpu().numpy().astype(np.float64), nlp.cpu().numpy().astype(np.float64)
    assert np.array_equal(np.isnan(gg), np.isnan(ref)) and np.array_equal(np.isnan(ll), np.isnan(rlp))
    ok = [0, 3]
    assert rel(gg[ok], ref[ok]) < 1e-5 and rel(gg[[1, 2], W], ref[[1, 2], W]) < 1e-5


# 4 dims fit the 32-wide LDS tile; 17 dims (35 columns) run the row-per-lane kernel
@pytest.mark.parametrize("dim", [4, 17])
@pytest.mark.parametrize("vfclip,lslo", [(0.0, -20.0), (0.25, -5.0)])
def test_ppo_grad_cont_matches_oracle(gpu, vfclip, lslo, dim):
    N = 5000
    print(f"cont grad dim={dim} vfclip={vfclip}", flush=True)
    O_ = 2 * dim + 1
    out = rng.normal(0xA11, N * O_).reshape(N, O_)
    out[:, dim:2 * dim] *= 0.7
    out[::50, dim] = -40.0  # saturated log-stds
    out = out.astype(np.float32).astype(np.float64)
    acts = (out[:, :dim] + rng.normal(0xA12, N * dim).reshape(N, dim) * 0.5).astype(np.float32).astype(np.float64)
    acts[::50, 0] = out[::50, 0]  # z = 0 on the saturated dim keeps logp representable in f32
    adv, ret = rng.normal(0xA13, N), rng.normal(0xA14, N)
    ov = out[:, 2 * dim] + rng.normal(0xA15, N, 0.0, 0.5)
    _, nlp0, _ = O.ppo_grad_cont(out, acts, adv, ret, np.zeros(N), ov, dim, lslo=lslo)
    old = nlp0 + rng.normal(0xA16, N, 0.0, 0.3)
    f32 = lambda x: x.astype(np.float32).astype(np.float64)
    ref, rlp, _ = O.ppo_grad_cont(out, acts, f32(adv), f32(ret), f32(old), f32(ov), dim, vfclip=vfclip, lslo=lslo)
    g = torch.empty(N, O_, device="cuda")
    nlp = torch.empty(N, device="cuda")
    dout_, dact, dadv, dret, dold, dov = cu(out), cu(acts), cu(adv), cu(ret), cu(old), cu(ov)
    losses = torch.zeros(7, device="cuda", dtype=torch.float64)
    L.call("ph_ppo_grad_cont", vp(dout_), O_, vp(dact), vp(dadv), vp(dret), vp(dold), vp(dov), N, dim, 0.5, 0.01, 0.2,
           vfclip, lslo, 2.0, vp(g), O_, vp(nlp), None, vp(losses), st())
    torch.cuda.synchronize()
    gg = g.cpu().numpy()
    assert rel(gg, ref) < 1e-5
    assert np.all(gg[::50, dim] == 0.0)
    assert rel(nlp.cpu().numpy(), rlp) < 1e-5
    rL = O.wide_losses(2, out, acts, f32(adv), f32(ret), f32(old), f32(ov), dim=dim, vfclip=vfclip, lslo=lslo)
    np.testing.assert_allclose(losses.cpu().numpy(), rL, rtol=1e-5, atol=max(1e-6, 2.0 / N))


# ---- samplers -----------------------------------------------------------------------------------
@pytest.mark.parametrize("dtype", [L.PH_F64, L.PH_F32])
def test_sample_md_matches_oracle(gpu, dtype):
    sizes = [4, 2, 7]
    N, K, W = 6000, 3, 13
    Y = rng.normal(0xA21, N * (W + 1)).reshape(N, W + 1) * 1.5
    if dtype == L.PH_F32:
        Y = Y.astype(np.float32).astype(np.float64)
    state = 0xABCD1234
    ref = O.sample_md(Y, sizes, state)
    out = torch.empty((K + 2) * N, device="cuda", dtype=torch.float64)
    hs = (C.c_int * K)(*sizes)
    dY = cu(Y, torch.float64 if dtype == L.PH_F64 else torch.float32)
    L.call("ph_sample_actions_md", dtype, vp(dY), W + 1, N, hs, K, state, vp(out), st())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    band = 1e-12 if dtype == L.PH_F64 else 1e-5
    bad = 0
    for h in range(K):
        diff = np.nonzero(got[h * N:(h + 1) * N] != ref[h * N:(h + 1) * N])[0]
        off = sum(sizes[:h])
        for n in diff:  # only draws within rounding of a cumulative boundary may differ
            lg = Y[n, off:off + sizes[h]]
            p = np.exp(lg - lg.max())
            cum = np.cumsum(p / p.sum())
            u = word_unit(state + (n + 1) * GOLD + (h + 1) * GOLD2)
            k = int(min(got[h * N + n], ref[h * N + n]))
            assert abs(cum[k] - u) < band, (h, n)
        bad += len(diff)
    assert bad <= max(1, N // 500)
    ok = np.all(np.stack([got[h * N:(h + 1) * N] == ref[h * N:(h + 1) * N] for h in range(K)]), axis=0)
    tol = 1e-12 if dtype == L.PH_F64 else 1e-5
    assert np.allclose(got[K * N:(K + 1) * N][ok], ref[K * N:(K + 1) * N][ok], rtol=tol, atol=tol)
    assert np.array_equal(got[(K + 1) * N:], ref[(K + 1) * N:])


def test_sample_cont_matches_oracle(gpu):
    dim, N = 3, 6000
    Y = rng.normal(0xA31, N * (2 * dim + 1)).reshape(N, 2 * dim + 1)
    Y[::40, dim + 1] = -35.0
    state = 0x77777
    ref = O.sample_cont(Y, dim, state)
    out = torch.empty((dim + 2) * N, device="cuda", dtype=torch.float64)
    dY = cu(Y, torch.float64)
    L.call("ph_sample_actions_cont", L.PH_F64, vp(dY), 2 * dim + 1, N, dim, state, -20.0, 2.0, vp(out), st())
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    np.testing.assert_allclose(got[:(dim + 1) * N], ref[:(dim + 1) * N], rtol=1e-12, atol=1e-12)
    assert np.array_equal(got[(dim + 1) * N:], ref[(dim + 1) * N:])


def test_host_sampler_entries(gpu):
    sizes = [5, 3]
    N, W = 1000, 8
    Y = rng.normal(0xA41, N * (W + 1)).reshape(N, W + 1)
    out = np.zeros(4 * N)
    L.call("ph_cuda_sample_actions_md", dp(Y), dp(np.array(sizes, np.float64)), N, 2, W + 1, 0x55, dp(out))
    ref = O.sample_md(Y, sizes, 0x55)
    assert np.sum(out[:2 * N] != ref[:2 * N]) <= 2 and np.array_equal(out[3 * N:], ref[3 * N:])
    dim = 2
    Yc = rng.normal(0xA42, N * (2 * dim + 1)).reshape(N, 2 * dim + 1)
    outc = np.zeros((dim + 2) * N)
    L.call("ph_cuda_sample_actions_cont", dp(Yc), N, dim, 2 * dim + 1, 0x66, dp(outc))
    np.testing.assert_allclose(outc, O.sample_cont(Yc, dim, 0x66), rtol=1e-12, atol=1e-12)


# ---- MLP gradients with the new heads -----------------------------------------------------------
def mlp_backprop(params, X, dout, H, D, O_):
    """Summed gradient of the flattenMLP net (relu hidden) given d(objective)/d(out) per row."""
    W1 = params[:H * D].reshape(H, D)
    b1 = params[H * D:H * D + H]
    W2 = params[H * D + H:H * D + H + O_ * H].reshape(O_, H)
    z1 = X @ W1.T + b1
    h1 = np.maximum(z1, 0)
    gW2 = dout.T @ h1
    gb2 = dout.sum(axis=0)
    dz = (dout @ W2) * (z1 > 0)
    return np.concatenate([(dz.T @ X).ravel(), dz.sum(axis=0), gW2.ravel(), gb2])


def test_backprop_composition_reproduces_categorical_mlp_gradient(gpu):
    N, D, H, A = 64, 6, 16, 4
    O_ = A + 1
    P = H * D + H + O_ * H + O_
    p = rng.normal(0xA51, P) * 0.5
    X = rng.normal(0xA52, N * D).reshape(N, D)
    act = rng.randint(0xA53, N, A).astype(np.float64)
    adv, ret, old = rng.normal(0xA54, N), rng.normal(0xA55, N), rng.normal(0xA56, N, -1.5, 0.3)
    out = np.zeros(N * O_)
    O.lib().orc_mlp_forward(O.P(p), O.P(X), N, D, H, O_, O.P(out))
    out = out.reshape(N, O_)
    dl, dv, _, _ = O.ppo_grad(out[:, :A], out[:, A], act, adv, ret, old)
    g = mlp_backprop(p, X, np.concatenate([dl, dv[:, None]], axis=1), H, D, O_)
    ref = np.zeros(P)
    O.lib().orc_mlp_ppo_grad(O.P(p), O.P(X), O.P(act), O.P(adv), O.P(ret), O.P(old), N, H, D, A, 0.5, 0.01, 0.2,
                             O.P(ref), 1)
    assert rel(g, ref) < 1e-12


@pytest.mark.parametrize("bf16,tol", [(0, 1e-5), (1, 1e-2)])
def test_cuda_mlp_ppo_grad_md(gpu, bf16, tol):
    sizes = [3, 4]
    N, D, H, K, W = 512, 10, 32, 2, 7
    O_ = W + 1
    P = H * D + H + O_ * H + O_
    p = rng.normal(0xA61, P) * 0.4
    X = rng.normal(0xA62, N * D).reshape(N, D)
    acts = np.stack([rng.randint(0xA63 + h, N, s) for h, s in enumerate(sizes)], axis=1).astype(np.float64)
    adv, ret = rng.normal(0xA66, N), rng.normal(0xA67, N)
    old = rng.normal(0xA68, N, -2.5, 0.3)
    g = np.zeros(P)
    L.call("ph_cuda_mlp_ppo_grad_md", dp(p), dp(X), dp(acts), dp(adv), dp(ret), dp(old),
           dp(np.array(sizes, np.float64)), N, H, D, K, 0.5, 0.01, 0.2, bf16, dp(g))
    out = np.zeros(N * O_)
    O.lib().orc_mlp_forward(O.P(p), O.P(X), N, D, H, O_, O.P(out))
    dout, _, _ = O.ppo_grad_md(out.reshape(N, O_), acts, adv, ret, old, None, sizes)
    assert rel(g, mlp_backprop(p, X, dout, H, D, O_)) < tol


@pytest.mark.parametrize("bf16,tol", [(0, 1e-5), (1, 1e-2)])
def test_cuda_mlp_ppo_grad_cont(gpu, bf16, tol):
    dim, N, D, H = 2, 512, 10, 32
    O_ = 2 * dim + 1
    P = H * D + H + O_ * H + O_
    p = rng.normal(0xA71, P) * 0.4
    # log-std rows of the output layer scaled so log-stds sit near [-1, 1]: with raw log-stds of several
    # units, d logp / d mu = z exp(-ls) runs into the thousands and the fp32 forward's rounding, not the
    # gradient, would set the error
    w2, b2 = H * D + H, H * D + H + O_ * H
    p[w2 + dim * H:w2 + 2 * dim * H] *= 0.1
    p[b2 + dim:b2 + 2 * dim] *= 0.1
    X = rng.normal(0xA72, N * D).reshape(N, D)
    out = np.zeros(N * O_)
    O.lib().orc_mlp_forward(O.P(p), O.P(X), N, D, H, O_, O.P(out))
    out = out.reshape(N, O_)
    acts = out[:, :dim] + rng.normal(0xA73, N * dim).reshape(N, dim) * 0.3
    adv, ret = rng.normal(0xA74, N), rng.normal(0xA75, N)
    _, nlp, _ = O.ppo_grad_cont(out, acts, adv, ret, np.zeros(N), None, dim)
    old = nlp + rng.normal(0xA76, N, 0.0, 0.1)
    g = np.zeros(P)
    L.call("ph_cuda_mlp_ppo_grad_cont", dp(p), dp(X), dp(acts), dp(adv), dp(ret), dp(old), N, H, D, dim, 0.5, 0.01,
           0.2, bf16, dp(g))
    dout, _, _ = O.ppo_grad_cont(out, acts, adv, ret, old, None, dim)
    assert rel(g, mlp_backprop(p, X, dout, H, D, O_)) < tol


# ---- whole wide update --------------------------------------------------------------------------
def wide_chain(pm0, obs, acts, adv, ret, olp, ov, perms, NT, D, H, O_, mode, sizes, dim, numMB, lr, wd, mu, eps,
               vfclip, mgn):
    """The wide update composed from the oracle's functions: per minibatch gather by the shuffle,
    orc_adv_normalize, orc_mlp_forward, the head gradient, the backward composition, orc_gclip and the
    exact Muon orc_muon_step_mlp. Returns [params; mom] and the last minibatch's dashboard losses."""
    Pn = H * D + H + O_ * H + O_
    pm = pm0.copy()
    X, Acol = obs.reshape(NT, D), acts.reshape(NT, -1)
    mb = NT // numMB
    last = None
    for perm in perms:
        for m in range(numMB):
            idx = perm[m * mb:(NT if m + 1 == numMB else (m + 1) * mb)]
            n = len(idx)
            Xm = np.ascontiguousarray(X[idx])
            advn = np.zeros(n)
            O.lib().orc_adv_normalize(O.P(np.ascontiguousarray(adv[idx])), n, O.P(advn))
            out = np.zeros(n * O_)
            O.lib().orc_mlp_forward(O.P(np.ascontiguousarray(pm[:Pn])), O.P(Xm), n, D, H, O_, O.P(out))
            out = out.reshape(n, O_)
            ovm = ov[idx] if ov is not None else None
            if mode == 1:
                dout, _, _ = O.ppo_grad_md(out, Acol[idx], advn, ret[idx], olp[idx], ovm, sizes, vfclip=vfclip)
                last = O.wide_losses(1, out, Acol[idx], advn, ret[idx], olp[idx], ovm, sizes=sizes, vfclip=vfclip)
            else:
                dout, _, _ = O.ppo_grad_cont(out, Acol[idx], advn, ret[idx], olp[idx], ovm, dim, vfclip=vfclip)
                last = O.wide_losses(2, out, Acol[idx], advn, ret[idx], olp[idx], ovm, dim=dim, vfclip=vfclip)
            g = mlp_backprop(pm[:Pn], Xm, dout, H, D, O_)
            gs = 1.0 / n
            if mgn > 0:
                O.lib().orc_gclip(O.P(g), Pn, gs, mgn)
                gs = 1.0
            nxt = np.zeros(2 * Pn)
            O.lib().orc_muon_step_mlp(O.P(pm), O.P(g), H, D, O_, gs, lr, wd, mu, eps, O.P(nxt))
            pm = nxt
    return pm, last


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("vfclip,mgn", [(0.0, 0.0), (0.2, 0.5)])
def test_train_update_wide_resident_matches_oracle_chain(gpu, mode, vfclip, mgn):
    NT, D, H, epochs, numMB = 96, 12, 16, 2, 3
    sizes, dim = [3, 4, 2], 3
    Wd = len(sizes) if mode == 1 else dim
    O_ = sum(sizes) + 1 if mode == 1 else 2 * dim + 1
    Pn = H * D + H + O_ * H + O_
    print(f"wide update mode={mode} vfclip={vfclip} mgn={mgn}", flush=True)
    pm0 = np.concatenate([rng.normal(0xB01, Pn) * 0.3, rng.normal(0xB02, Pn) * 0.01])
    if mode == 2:  # log-std rows of the output layer near [-1, 1] (the conditioning of the Gaussian head)
        w2, b2 = H * D + H, H * D + H + O_ * H
        pm0[w2 + dim * H:w2 + 2 * dim * H] *= 0.1
        pm0[b2 + dim:b2 + 2 * dim] *= 0.1
    obs = rng.normal(0xB03, NT * D)
    if mode == 1:
        acts = np.stack([rng.randint(0xB04 + h, NT, s) for h, s in enumerate(sizes)], 1).astype(np.float64)
    else:
        acts = rng.normal(0xB04, NT * dim).reshape(NT, dim) * 0.5
    adv, ret = rng.normal(0xB08, NT), rng.normal(0xB09, NT)
    olp = rng.normal(0xB0A, NT, -3.0 if mode == 1 else -2.5, 0.3)
    ov = rng.normal(0xB0B, NT, 0.0, 0.5) if vfclip > 0 else None
    r = np.random.default_rng(0xB0C)
    perms = [r.permutation(NT) for _ in range(epochs)]
    lr, wd, mu, eps = 0.02, 0.01, 0.95, 1e-7
    ref, refL = wide_chain(pm0, obs, acts, adv, ret, olp, ov, perms, NT, D, H, O_, mode, sizes, dim, numMB, lr, wd,
                           mu, eps, vfclip, mgn)
    h = C.c_size_t(0)
    L.call("ph_cuda_policy_load", dp(pm0), Pn, C.byref(h))
    L.call("ph_cuda_mg_loss_enable", 1)
    try:
        peek = np.zeros(1)
        L.call("ph_cuda_train_update_wide_resident", h.value, dp(obs), dp(acts), dp(adv), dp(ret), dp(olp),
               dp(ov) if ov is not None else None, NT if ov is not None else 0,
               dp(np.concatenate(perms).astype(np.float64)), dp(np.array(sizes, np.float64)), len(sizes), NT, D, H,
               O_, Wd, mode, epochs, numMB, lr, wd, mu, eps, 0.5, 0.01, 0.2, vfclip, mgn, 0, dp(peek))
        res = np.zeros(2 * Pn)
        L.call("ph_cuda_policy_download", h.value, Pn, dp(res))
        losses = np.zeros(7)
        L.call("ph_cuda_mg_read_losses", dp(losses))
    finally:
        L.call("ph_cuda_mg_loss_enable", 0)
        L.call("ph_cuda_policy_free", h.value)
    assert peek[0] == res[0]
    # fp32 gradients against the f64 chain over six minibatches of exact Muon
    assert rel(res[:Pn] - pm0[:Pn], ref[:Pn] - pm0[:Pn]) < 1e-4
    assert rel(res[Pn:], ref[Pn:]) < 1e-4
    np.testing.assert_allclose(losses, refL, rtol=1e-4, atol=2.0 / (NT // numMB))


# ---- MinGRU gradient with multi-discrete heads -----------------------------------------------------
def _mg_md_oracle(p, obs, act, adv, ret, old, term, ov, T, B, H, D, Ln, W, sizes):
    """Sum over the B sequences of the oracle's K-head sequence gradient; act [T][B][K]."""
    Pn = p.size
    g, nlp = np.zeros(Pn), np.zeros((T, B))
    for b in range(B):
        o = np.zeros(Pn + 2 * T)
        O.lib().orc_mingru_ppo_grad_seq_md(O.P(p), O.P(O.f64(obs[:, b, :])), O.P(O.f64(act[:, b, :])),
                                           O.P(O.f64(adv[:, b])), O.P(O.f64(ret[:, b])), O.P(O.f64(old[:, b])),
                                           O.P(O.f64(term[:, b])), O.P(O.f64(ov[:, b])), T, H, D, Ln, W,
                                           O.P(np.ascontiguousarray(sizes, np.int32)), len(sizes), 0.5, 0.01, 0.2,
                                           0.2, O.P(o))
        g += o[:Pn]
        nlp[:, b] = o[Pn:Pn + T]
    return g, nlp


# fp32 products: the parity bar. bf16 products: 5e-2, wider than the single-head 2e-2 because the joint
# log-prob sums the K heads' bf16 logit errors before the ratio is formed (the reference records the
# same for its bf16 multi-discrete tier, puffercuda.cu:4946-4951); 4.1 % measured on this case.
@pytest.mark.parametrize("prec,tol", [("f32", 1e-5), ("bf16", 5e-2)])
def test_mingru_md_host_mode_matches_oracle(gpu, monkeypatch, prec, tol):
    if prec == "bf16":
        monkeypatch.setenv("PUFFER_MG_PREC", "bf16")
    else:
        monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    sizes = [3, 4, 2]
    B, T, D, H, Ln, K = 8, 16, 8, 32, 2, 3
    W = sum(sizes)
    n = B * T
    Pn = H * D + H + Ln * 3 * H * H + W * H + W + H + 1
    p = rng.normal(0xB31, Pn) * 0.3
    obs = rng.normal(0xB32, n * D).reshape(T, B, D)
    act = np.stack([rng.randint(0xB33 + h, n, s) for h, s in enumerate(sizes)], 1).reshape(T, B, K).astype(np.float64)
    adv, ret = rng.normal(0xB37, n).reshape(T, B), rng.normal(0xB38, n).reshape(T, B)
    old = rng.randf(0xB39, n, -4.0, -2.5).reshape(T, B)
    term = rng.bernoulli(0xB3A, n, 0.05).reshape(T, B)
    ov = rng.normal(0xB3B, n).reshape(T, B)
    scal = np.concatenate([act.ravel()] + [a.ravel() for a in (adv, ret, old, term, ov)])
    out = np.zeros(Pn + 2 * n)
    ln = C.c_size_t(0)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), n * D, dp(scal), scal.size, B, T, H, D, Ln, W, K,
           dp(np.array(sizes, np.float64)), K, 0.5, 0.01, 0.2, 0.2, None, 0, None, 0, dp(out), C.byref(ln))
    assert ln.value == out.size
    g, nlp = _mg_md_oracle(p, obs, act, adv, ret, old, term, ov, T, B, H, D, Ln, W, sizes)
    assert rel(out[:Pn], g) < tol
    assert rel(out[Pn:Pn + n], nlp.ravel()) < tol


def test_mingru_md_device_column_mode(gpu, monkeypatch):
    """K-wide resident columns: the device gather of the drawn segments feeds the same gradient as the
    host form built from the oracle's gather (actions indexed by the draws)."""
    monkeypatch.delenv("PUFFER_MG_PREC", raising=False)
    sizes = [3, 4]
    N, T, B, D, H, Ln, K = 32, 8, 12, 8, 16, 2, 2
    W = sum(sizes)
    n = N * T
    Pn = H * D + H + Ln * 3 * H * H + W * H + W + H + 1
    p = rng.normal(0xB41, Pn) * 0.3
    rew, term = rng.normal(0xB42, n), rng.bernoulli(0xB43, n, 0.05)
    act = np.stack([rng.randint(0xB44 + h, n, s) for h, s in enumerate(sizes)], 1).astype(np.float64)  # [N*T][K]
    logp, val, boot = rng.randf(0xB46, n, -3.5, -2.0), rng.normal(0xB47, n), rng.normal(0xB48, N)
    obs_roll = rng.normal(0xB49, n * D).reshape(N, T, D)
    L.call("ph_cuda_mg_prep", dp(rew), dp(term), dp(act), dp(logp), dp(val), dp(boot), N, T, K)
    L1 = np.zeros(N)
    L.call("ph_cuda_mg_vtrace", N, T, 0.99, 0.95, 1.0, 1.0, dp(L1))
    adv = np.zeros(n)
    O.lib().orc_vtrace_mingru(O.P(rew), O.P(val), O.P(term), O.P(np.ones(n)), O.P(boot), N, T, 0.99, 0.95, 1.0, 1.0,
                              O.P(adv))
    idx, mp = np.zeros(B), np.zeros(B)
    L.call("ph_ffi_prio_sample", dp(L1), N, T, B, 0.8, 0.3, 0x5151, dp(idx), dp(mp))
    scal1, _ = O.gather_seq_minibatch(np.zeros(n), logp, term, adv, val, idx, mp, T)  # [act | adv | ret | old | term | ov]
    e = idx.astype(np.int64)
    act_mb = act.reshape(N, T, K)[e].transpose(1, 0, 2)  # [T][B][K]
    scal = np.concatenate([act_mb.ravel(), scal1[T * B:]])
    obs = np.ascontiguousarray(obs_roll[e].transpose(1, 0, 2))
    hs = np.array(sizes, np.float64)
    args = (B, T, H, D, Ln, W, K, dp(hs), K, 0.5, 0.01, 0.2, 0.2)
    out_host = np.zeros(Pn + 2 * T * B)
    ln = C.c_size_t(0)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, dp(scal), scal.size, *args, None, 0, None, 0,
           dp(out_host), C.byref(ln))
    assert ln.value == out_host.size
    # device-column mode: the gradient stays on the device (resident mode, zero-length result)
    out_dev = np.zeros_like(out_host)
    L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, None, 0, *args, dp(idx), B, dp(mp), B,
           dp(out_dev), C.byref(ln))
    assert ln.value == 0
    g_dev = np.zeros(Pn)
    L.call("ph_cuda_mg_resident_grad", Pn, dp(g_dev))
    assert rel(g_dev, out_host[:Pn]) < 1e-5
    # a K-wide call does not gather from columns of another width
    L.call("ph_cuda_mg_prep", dp(rew), dp(term), dp(act[:, 0].copy()), dp(logp), dp(val), dp(boot), N, T, 1)
    L.call("ph_cuda_mg_vtrace", N, T, 0.99, 0.95, 1.0, 1.0, dp(L1))
    with pytest.raises(L.PufferHipError, match="no scalar source"):
        L.call("ph_cuda_mingru_ppo_grad", dp(p), Pn, dp(obs), obs.size, None, 0, *args, dp(idx), B, dp(mp), B,
               dp(out_dev), C.byref(ln))


def test_mingru_rollout_step_then_multi_discrete_draw(gpu):
    """The MinGRU rollout step with W = sum of head sizes logits (its rows are [logits | value]) feeds the
    multi-discrete sampler directly: draws and joint log-probs against the oracle's step and sampler."""
    sizes = [3, 4, 2]
    N, Dm, H, Lr = 512, 16, 64, 2
    W = sum(sizes)
    P = H * Dm + H + Lr * 3 * H * H + W * H + W + H + 1
    params = rng.normal(0xB51, P) * 0.3 / np.sqrt(max(Dm, H) / 8)
    obs = rng.normal(0xB52, N * Dm).reshape(N, Dm)
    dims = L.MinGRUDims(N, 1, Dm, H, Lr, W, 1)  # fp32 products
    gp, gobs = cu(params), cu(obs)
    state = torch.zeros(N * Lr * H, device="cuda")
    out = torch.empty(N, W + 1, device="cuda")
    draws = torch.empty((len(sizes) + 2) * N, device="cuda", dtype=torch.float64)
    hs = (C.c_int * len(sizes))(*sizes)
    L.call("ph_mingru_rollout_step", C.byref(dims), vp(gp), vp(gobs), vp(state), vp(out), st())
    L.call("ph_sample_actions_md", L.PH_F32, vp(out), W + 1, N, hs, len(sizes), 0x4242, vp(draws), st())
    torch.cuda.synchronize()
    ref_out, _ = O.mingru_step(params.astype(np.float32).astype(np.float64),
                               obs.astype(np.float32).astype(np.float64), np.zeros((N, Lr, H)), N, Dm, H, Lr, W)
    y = out.cpu().numpy().astype(np.float64)
    assert rel(y, ref_out) < 1e-5
    got, ref = draws.cpu().numpy(), O.sample_md(y, sizes, 0x4242)  # the sampler on the device's own rows
    K = len(sizes)
    bad = sum(int(np.sum(got[h * N:(h + 1) * N] != ref[h * N:(h + 1) * N])) for h in range(K))
    assert bad <= max(1, N // 500)
    ok = np.all(np.stack([got[h * N:(h + 1) * N] == ref[h * N:(h + 1) * N] for h in range(K)]), axis=0)
    assert np.allclose(got[K * N:(K + 1) * N][ok], ref[K * N:(K + 1) * N][ok], rtol=1e-5, atol=1e-5)
    assert np.array_equal(got[(K + 1) * N:], ref[(K + 1) * N:])
