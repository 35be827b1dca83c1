"""The whole MinGRU PPO+Muon minibatch step at the headline policy's own dimensions against the oracle
chain: obs 128 -> encoder 512 -> 2 MinGRU layers of 512 -> 16-way categorical head + value head,
sequence 64, on 32 segments (the step's every kernel family at its real per-matrix shapes: the five
matrices of the Newton-Schulz batch are 512x128, 2 x 1536x512, 16x512 and 1x512 whatever the number of
segments). Behaviour log-probs are the policy's own log-probs at these weights plus N(0, 0.05), as in a
trainer's first epoch.

The oracle chain follows the trainer's call order (MinGRUTrain.lean:814-849, puffercuda.cu:5727-5976):
  orc_vtrace_mingru (bootstrapped, time-major, log ratios)  ->  orc_adv_normalize over the minibatch
  ->  the summed single-sequence gradient (orc_mingru_ppo_grad_batch, each segment
      lean_ffi_mingru_ppo_grad_seq, pufferffi.c:763-876)
  ->  orc_gclip (scale 1/(T*B), max norm 0.5)  ->  orc_muon_mat (form 1, the constant triple x 5) on
      every matrix, orc_stepvec on every bias.
The GPU runs ph_mingru_step once. Per matrix and per bias, relative Frobenius errors of the new momentum
and of the weight change (new - old):
  fp32 tier (fp32 activations, fp32 MFMA, fp32 Newton-Schulz): both within 1e-4 of the oracle chain.
  bf16 tier (bf16 activations, bf16 MFMA, fused bf16 Newton-Schulz):
    * momentum within 3e-2 of the oracle chain: the momentum is the clipped gradient plus mu times the
      previous momentum, and the gradient's bar in this tier is 3e-2 per block (bf16 storage of the
      activations and their gradients; the error grows with a block's depth from the loss);
    * weight change within 1e-2 of the oracle's Muon step applied to the GPU's own momentum (the
      gradient recovered as new momentum - mu * old momentum): the fused bf16 Newton-Schulz and the
      weight update alone, at the single-product bar;
    * weight change within 1e-1 of the oracle chain: Newton-Schulz amplifies an error of its input by up
      to a^5 = 3.4445^5 ~ 480 along small singular directions; the fp32 tier shows the same 5-30x
      ratio of update error to momentum error.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import device as D
from pufferlean_amd import rng
from test_gpu_mingru import init_params

pytestmark = pytest.mark.gpu

Dm, H, L, A, T = 128, 512, 2, 16, 64
LR, MU, MGN = 0.015, 0.95, 0.5


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def layout():
    """(name, offset, rows, cols) of every matrix and (name, offset, n) of every bias, flattenMG order."""
    szE, szL = H * Dm, 3 * H * H
    offW = szE + H
    offDec = offW + L * szL
    mats = [("enc.W", 0, H, Dm)] + [(f"layer{l}.W", offW + l * szL, 3 * H, H) for l in range(L)]
    mats += [("dec.W", offDec, A, H), ("val.W", offDec + A * H + A, 1, H)]
    vecs = [("enc.b", szE, H), ("dec.b", offDec + A * H, A), ("val.b", offDec + A * H + A + H, 1)]
    return mats, vecs


def minibatch(B, seed):
    n = T * B
    obs = rng.normal(seed, n * Dm).reshape(T, B, Dm)
    act = rng.randint(seed + 1, n, A).reshape(T, B)
    old = (np.log(1.0 / A) + rng.normal(seed + 2, n, 0.0, 0.3)).reshape(T, B)
    val = rng.normal(seed + 3, n).reshape(T, B)
    done = rng.bernoulli(seed + 4, n, 0.01).reshape(T, B)
    rew = rng.normal(seed + 5, n).reshape(T, B)
    logrho = rng.normal(seed + 6, n, 0.0, 0.1).reshape(T, B)
    boot = rng.normal(seed + 7, B)
    return obs, act, old, val, done, rew, logrho, boot


def oracle_logp(p, cols, B, threads=8):
    """The oracle's log-probs of the taken actions at weights p ([T][B])."""
    obs, act, old, val, done = cols[:5]
    P = p.size
    out = np.zeros(P + 2 * T * B)
    z = np.zeros(T * B)
    O.lib().orc_mingru_ppo_grad_batch(O.P(p), O.P(O.f64(obs)), O.P(O.f64(act)), O.P(z), O.P(z),
                                      O.P(O.f64(old)), O.P(O.f64(done)), O.P(O.f64(val)), B, T, H, Dm, L, A,
                                      0.5, 0.01, 0.2, 0.0, O.P(out), threads)
    return out[P:P + T * B].reshape(T, B)


def muon_mats(p, g, mom, threads=8):
    """orc_muon_mat on every matrix of p (gradient g, previous momentum mom): (new p, new momentum)."""
    newp, newm = p.copy(), mom.copy()
    c = O.coeffs_array(O.BASELINE_COEFFS)
    mats, _ = layout()
    prev = O.lib().orc_set_threads(threads)
    try:
        for _, off, r, cc in mats:
            k = r * cc
            a = np.zeros(k); b = np.zeros(k)
            O.lib().orc_muon_mat(r, cc, O.P(p[off:off + k].copy()), O.P(g[off:off + k].copy()),
                                 O.P(mom[off:off + k].copy()), O.P(a), O.P(b), 1.0, LR, 0.0, MU, 1e-7,
                                 O.P(c), 5, 1)
            newp[off:off + k] = a; newm[off:off + k] = b
    finally:
        O.lib().orc_set_threads(prev)
    return newp, newm


def oracle_step(p, mom, cols, B, threads=8):
    obs, act, old, val, done, rew, logrho, boot = cols
    adv, tgt = O.vtrace(rew.ravel(), val.ravel(), done.ravel(), logrho.ravel(), boot, B, T, variant=1,
                        time_major=True, rho_is_log=True)
    advn = np.zeros_like(adv)
    O.lib().orc_adv_normalize(O.P(adv), adv.size, O.P(advn))
    P = p.size
    out = np.zeros(P + 2 * T * B)
    O.lib().orc_mingru_ppo_grad_batch(O.P(p), O.P(O.f64(obs)), O.P(O.f64(act)), O.P(advn), O.P(tgt),
                                      O.P(O.f64(old)), O.P(O.f64(done)), O.P(O.f64(val)), B, T, H, Dm, L, A,
                                      0.5, 0.01, 0.2, 0.0, O.P(out), threads)
    g = out[:P].copy()
    O.lib().orc_gclip(O.P(g), P, 1.0 / (B * T), MGN)
    newp, newm = muon_mats(p, g, mom, threads)
    _, vecs = layout()
    for _, off, k in vecs:
        a = np.zeros(k); b = np.zeros(k)
        O.lib().orc_stepvec(k, O.P(p[off:off + k].copy()), O.P(g[off:off + k].copy()),
                            O.P(mom[off:off + k].copy()), O.P(a), O.P(b), 1.0, LR, 0.0, MU)
        newp[off:off + k] = a; newm[off:off + k] = b
    return newp, newm


def cuda32(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()


@pytest.mark.parametrize("precision", ["f32", "bf16"])
def test_h512_whole_step_vs_oracle_chain(gpu, precision):
    B = 32
    print(f"mingru h512 whole step B={B} T={T} {precision}", flush=True)
    p = init_params(Dm, H, L, A, 0xD500)
    # previous momentum at about half the clipped gradient's scale on the layers (the clipped gradient's
    # entries are ~3e-5 RMS there), so both terms of the momentum update are exercised
    mom = rng.normal(0xD501, p.size) * 2e-5
    cols = list(minibatch(B, 0xD600))
    cols[2] = oracle_logp(p, cols, B) + rng.normal(0xD6FF, T * B, 0.0, 0.05).reshape(T, B)
    ref_p, ref_m = oracle_step(p, mom, cols, B)
    obs, act, old, val, done, rew, logrho, boot = cols
    cfg = D.MinGRUConfig(B, T, Dm, H, L, A, lr=LR, mu=MU, max_grad_norm=MGN, gscale=1.0 / (B * T),
                         precision=precision, math=precision)
    assert cfg.P == p.size
    gp, gm = cuda32(p), cuda32(mom)
    D.mingru_step(cfg, gp, gm, cuda32(obs), torch.from_numpy(np.ascontiguousarray(act, np.int32)).cuda(),
                  cuda32(old), cuda32(val), cuda32(rew), cuda32(done), cuda32(logrho), cuda32(boot))
    D.ns_status()
    newp = gp.cpu().numpy().astype(np.float64)
    newm = gm.cpu().numpy().astype(np.float64)
    mats, vecs = layout()
    # the oracle's Muon step on the GPU's own momentum: isolates Newton-Schulz and the weight update
    own_p, _ = muon_mats(p, newm - MU * mom, mom)
    errs = {}
    for name, off, r, cc in mats:
        s = slice(off, off + r * cc)
        errs[name] = (rel(newm[s], ref_m[s]), rel(newp[s] - p[s], ref_p[s] - p[s]),
                      rel(newp[s] - p[s], own_p[s] - p[s]))
    for name, off, k in vecs:
        s = slice(off, off + k)
        errs[name] = (rel(newm[s], ref_m[s]), rel(newp[s] - p[s], ref_p[s] - p[s]), 0.0)
    print("momentum / update vs chain / update vs Muon of own momentum:",
          {k: tuple(f"{v:.2e}" for v in e) for k, e in errs.items()}, flush=True)
    tol_m, tol_u, tol_own = {"f32": (1e-4, 1e-4, 1e-4), "bf16": (3e-2, 1e-1, 1e-2)}[precision]
    for name, (em, eu, eo) in errs.items():
        assert em < tol_m, (name, "momentum", em)
        assert eu < tol_u, (name, "update", eu)
        assert eo < tol_own, (name, "update vs Muon of the GPU momentum", eo)
