"""MinGRU PPO+Muon minibatch step on the GPU vs the CPU oracle.

The batched gradient (all T*B rows at once) is checked against the sum over segments of the
reference's single-sequence BPTT (lean_ffi_mingru_ppo_grad_seq, restated as
orc_mingru_ppo_grad_seq) in two precision tiers:
  fp32 tier (fp32 activations, fp32 MFMA):  1e-5 relative Frobenius on the whole gradient;
  bf16 tier (bf16 activations and weight copies, bf16 MFMA, fp32 accumulation and master weights):
    2e-2 relative Frobenius on the whole gradient. The bf16 rounding of the weights and activations
    alone accounts for 0.3-1.6% on these small shapes (a CPU emulation with exact arithmetic
    elsewhere reproduces the GPU error to three digits).
The whole step (V-trace -> normalisation -> gradient -> clip -> Muon) is checked against the
oracle chain on the momentum and the parameter update.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def init_params(D_, H, L, A, seed):
    """N(0, 1/fan_in) weights, zero biases, in the flattenMG order."""
    parts = []
    parts.append(rng.normal(seed, H * D_) / np.sqrt(D_)); parts.append(np.zeros(H))
    for l in range(L):
        parts.append(rng.normal(seed + 1 + l, 3 * H * H) / np.sqrt(H))
    parts.append(rng.normal(seed + 10, A * H) / np.sqrt(H)); parts.append(np.zeros(A))
    parts.append(rng.normal(seed + 11, H) / np.sqrt(H)); parts.append(np.zeros(1))
    return np.concatenate(parts)


def make_batch(B, T, D_, A, seed, p_done=0.05):
    n = B * T
    obs = rng.normal(seed, n * D_).reshape(T, B, D_)
    act = rng.randint(seed + 1, n, A).reshape(T, B)
    adv = rng.normal(seed + 2, n).reshape(T, B)
    ret = rng.normal(seed + 3, n).reshape(T, B)
    old = rng.randf(seed + 4, n, -3.5, -1.5).reshape(T, B)
    ov = rng.normal(seed + 5, n).reshape(T, B)
    done = rng.bernoulli(seed + 6, n, p_done).reshape(T, B)
    return obs, act, adv, ret, old, ov, done


def oracle_grad(p, obs, act, adv, ret, old, ov, done, T, B, H, D_, L, A, vfclip):
    P = p.size
    g = np.zeros(P)
    nlp = np.zeros((T, B)); nv = np.zeros((T, B))
    for b in range(B):
        out = np.zeros(P + 2 * T)
        O.lib().orc_mingru_ppo_grad_seq(
            O.P(p), O.P(O.f64(obs[:, b, :])), O.P(O.f64(act[:, b])), O.P(O.f64(adv[:, b])),
            O.P(O.f64(ret[:, b])), O.P(O.f64(old[:, b])), O.P(O.f64(done[:, b])), O.P(O.f64(ov[:, b])),
            T, H, D_, L, A, 0.5, 0.01, 0.2, vfclip, O.P(out))
        g += out[:P]
        nlp[:, b] = out[P:P + T]; nv[:, b] = out[P + T:]
    return g, nlp, nv


def cuda32(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


TOL = {"f32": 1e-5, "bf16": 2e-2}


@pytest.mark.parametrize("precision", ["f32", "bf16"])
@pytest.mark.parametrize("vfclip", [0.0, 0.2])
@pytest.mark.parametrize("dims", [(8, 16, 8, 16, 2, 5), (16, 12, 16, 32, 1, 3), (4, 9, 8, 24, 3, 16)])
def test_grad_vs_sequential_oracle(gpu, dims, vfclip, precision):
    B, T, D_, H, L, A = dims
    p = init_params(D_, H, L, A, 0x500 + H)
    obs, act, adv, ret, old, ov, done = make_batch(B, T, D_, A, 0x600 + B)
    ref, rnlp, rnv = oracle_grad(p, obs, act, adv, ret, old, ov, done, T, B, H, D_, L, A, vfclip)
    # the oracle sees the same bf16-free inputs; the GPU path rounds weights/activations to bf16
    cfg = D.MinGRUConfig(B, T, D_, H, L, A, vf_clip=vfclip, precision=precision)
    assert cfg.P == p.size
    G, nlp, nv = D.mingru_ppo_grad(cfg, cuda32(p), cuda32(obs), torch.from_numpy(act.astype(np.int32)).cuda(),
                                   cuda32(adv), cuda32(ret), cuda32(old), cuda32(ov), cuda32(done))
    g = G.cpu().numpy()
    tol = TOL[precision]
    assert rel(g, ref) < tol, rel(g, ref)
    assert rel(nlp.cpu().numpy().reshape(T, B), rnlp) < min(tol, 1e-2)
    assert rel(nv.cpu().numpy().reshape(T, B), rnv) < min(tol, 1e-2)


@pytest.mark.parametrize("A", [5, 17])
def test_grad_top_scan_forms_head_gradient(gpu, A):
    """bf16 tier with H a multiple of 256: the top layer's backward scan forms the head's data gradient
    dl.Wh itself (8 loss-gradient words a step for up to 16 head rows, 9 for 17-18) and writes the
    gate-skip term that the top data gradient adds. Against the sequential oracle at the bf16-tier
    tolerance; B = 3 leaves a whole idle wavefront in the last workgroup."""
    B, T, D_, H, L = 3, 12, 8, 256, 2
    p = init_params(D_, H, L, A, 0x700 + A)
    obs, act, adv, ret, old, ov, done = make_batch(B, T, D_, A, 0x710 + A)
    ref, rnlp, rnv = oracle_grad(p, obs, act, adv, ret, old, ov, done, T, B, H, D_, L, A, 0.2)
    cfg = D.MinGRUConfig(B, T, D_, H, L, A, vf_clip=0.2, precision="bf16")
    G, nlp, nv = D.mingru_ppo_grad(cfg, cuda32(p), cuda32(obs), torch.from_numpy(act.astype(np.int32)).cuda(),
                                   cuda32(adv), cuda32(ret), cuda32(old), cuda32(ov), cuda32(done))
    g = G.cpu().numpy()
    assert np.isfinite(g).all()
    assert rel(g, ref) < TOL["bf16"], rel(g, ref)
    assert rel(nlp.cpu().numpy().reshape(T, B), rnlp) < 1e-2
    assert rel(nv.cpu().numpy().reshape(T, B), rnv) < 1e-2


def test_grad_blocks_match_per_tensor(gpu):
    # every parameter block (encoder, each layer, heads, biases) within tolerance on its own (fp32 tier)
    B, T, D_, H, L, A = 8, 16, 8, 16, 2, 5
    p = init_params(D_, H, L, A, 0x700)
    obs, act, adv, ret, old, ov, done = make_batch(B, T, D_, A, 0x710)
    ref, _, _ = oracle_grad(p, obs, act, adv, ret, old, ov, done, T, B, H, D_, L, A, 0.0)
    cfg = D.MinGRUConfig(B, T, D_, H, L, A, precision="f32")
    G, _, _ = D.mingru_ppo_grad(cfg, cuda32(p), cuda32(obs), torch.from_numpy(act.astype(np.int32)).cuda(),
                                cuda32(adv), cuda32(ret), cuda32(old), cuda32(ov), cuda32(done))
    g = G.cpu().numpy()
    sizes = [H * D_, H] + [3 * H * H] * L + [A * H, A, H, 1]
    off = 0
    for k, s in enumerate(sizes):
        assert rel(g[off:off + s], ref[off:off + s]) < 1e-5, (k, rel(g[off:off + s], ref[off:off + s]))
        off += s


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_whole_step_vs_oracle_chain(gpu, precision):
    B, T, D_, H, L, A = 16, 16, 8, 16, 2, 5
    p = init_params(D_, H, L, A, 0x800)
    mom = rng.normal(0x801, p.size) * 0.01
    obs, act, _, _, old, val, done = make_batch(B, T, D_, A, 0x810, p_done=0.03)
    rew = rng.normal(0x820, B * T).reshape(T, B)
    logrho = rng.normal(0x821, B * T, 0.0, 0.1).reshape(T, B)
    boot = rng.normal(0x822, B)
    lr, mu, mgn = 0.015, 0.95, 0.5
    # oracle chain
    adv, tgt = O.vtrace(rew.ravel(), val.ravel(), done.ravel(), logrho.ravel(), boot, B, T, variant=1,
                        time_major=True, rho_is_log=True)
    advn = np.zeros_like(adv)
    O.lib().orc_adv_normalize(O.P(adv), adv.size, O.P(advn))
    g, _, _ = oracle_grad(p, obs, act, advn.reshape(T, B), tgt.reshape(T, B), old, val, done, T, B, H,
                          D_, L, A, 0.0)
    O.lib().orc_gclip(O.P(g), g.size, 1.0 / (B * T), mgn)
    newp = p.copy(); newm = mom.copy()
    c = O.coeffs_array(O.BASELINE_COEFFS)
    szE, szL = H * D_, 3 * H * H
    mats = [(0, H, D_)] + [(szE + H + l * szL, 3 * H, H) for l in range(L)]
    offDec = szE + H + L * szL
    mats += [(offDec, A, H), (offDec + A * H + A, 1, H)]
    vecs = [(szE, H), (offDec + A * H, A), (offDec + A * H + A + H, 1)]
    for off, r, cc in mats:
        k = r * cc
        a = np.zeros(k); bb = np.zeros(k)
        O.lib().orc_muon_mat(r, cc, O.P(p[off:off + k].copy()), O.P(g[off:off + k].copy()),
                             O.P(mom[off:off + k].copy()), O.P(a), O.P(bb), 1.0, lr, 0.0, mu, 1e-7,
                             O.P(c), 5, 1)
        newp[off:off + k] = a; newm[off:off + k] = bb
    for off, k in vecs:
        a = np.zeros(k); bb = np.zeros(k)
        O.lib().orc_stepvec(k, O.P(p[off:off + k].copy()), O.P(g[off:off + k].copy()),
                            O.P(mom[off:off + k].copy()), O.P(a), O.P(bb), 1.0, lr, 0.0, mu)
        newp[off:off + k] = a; newm[off:off + k] = bb
    # GPU step
    cfg = D.MinGRUConfig(B, T, D_, H, L, A, lr=lr, mu=mu, max_grad_norm=mgn, gscale=1.0 / (B * T),
                         precision=precision, math=precision)
    gp, gm = cuda32(p), cuda32(mom)
    D.mingru_step(cfg, gp, gm, cuda32(obs), torch.from_numpy(act.astype(np.int32)).cuda(), cuda32(old),
                  cuda32(val), cuda32(rew), cuda32(done), cuda32(logrho), cuda32(boot))
    tol = {"f32": 1e-4, "bf16": 2e-2}[precision]
    assert rel(gm.cpu().numpy(), newm) < tol
    assert rel(gp.cpu().numpy() - p, newp - p) < tol
