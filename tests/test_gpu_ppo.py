"""Fused PPO loss gradient and advantage normalisation on the GPU vs the CPU oracle."""
import math

import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def _rows(N, A, seed):
    lg = rng.normal(seed, N * A).reshape(N, A).astype(np.float32)
    v = rng.normal(seed + 1, N).astype(np.float32)
    act = rng.randint(seed + 2, N, A).astype(np.int32)
    adv = rng.normal(seed + 3, N).astype(np.float32)
    ret = rng.normal(seed + 4, N).astype(np.float32)
    lse = np.log(np.exp(lg.astype(np.float64)).sum(1))
    lp = lg[np.arange(N), act] - lse
    old = (lp + rng.normal(seed + 5, N, 0.0, 0.2)).astype(np.float32)
    # No ratio within 1e-4 of a clip edge (0.8, 1.2): far beyond fp32 rounding of the log-prob, so the
    # clipped-surrogate branch of every row is decided the same way in fp32 and f64, and a disagreement
    # is a mask error, not rounding.
    for _ in range(4):
        r = np.exp(lp - old.astype(np.float64))
        near = (np.abs(r - 0.8) < 1e-4) | (np.abs(r - 1.2) < 1e-4)
        if not near.any():
            break
        old[near] = (old[near].astype(np.float64) + 3e-4).astype(np.float32)
    ov = (v + rng.normal(seed + 6, N, 0.0, 0.5)).astype(np.float32)
    return lg, v, act, adv, ret, old, ov


def clip_branch(ratio, adv, eps=0.2):
    """Rows whose clipped surrogate takes the clipped term: min(r A, clip(r) A) with the clip active."""
    r = np.asarray(ratio, np.float64)
    a = np.asarray(adv, np.float64)
    return ((a >= 0) & (r > 1 + eps)) | ((a < 0) & (r < 1 - eps))


@pytest.mark.parametrize("A", [2, 5, 16, 64])
@pytest.mark.parametrize("vfclip", [0.0, 0.2])
@pytest.mark.parametrize("max_shift", [True, False])
def test_ppo_grad_vs_oracle(gpu, A, vfclip, max_shift):
    N = 262144 if A == 16 else 5000
    lg, v, act, adv, ret, old, ov = _rows(N, A, 300 + A)
    c = lambda x: torch.from_numpy(x).cuda()
    newlp = torch.empty(N, device="cuda"); newval = torch.empty(N, device="cuda")
    losses = torch.zeros(7, device="cuda", dtype=torch.float64)
    dl, dv = D.ppo_grad(c(lg), c(v), c(act), c(adv), c(ret), c(old), c(ov) if vfclip > 0 else None,
                        vf_clip=vfclip, max_shift=max_shift, newlp=newlp, newval=newval,
                        losses=losses)
    rdl, rdv, rnlp, rnv = O.ppo_grad(lg, v, act, adv, ret, old, ov if vfclip > 0 else None,
                                     vfclip=vfclip, max_shift=max_shift)
    # The clip mask: the branch each row takes from the device's own log-prob must be the oracle's
    # branch for every row (no edge rows exist in these inputs).
    gl = newlp.cpu().numpy().astype(np.float64)
    mask_dev = clip_branch(np.exp(gl - old.astype(np.float64)), adv)
    mask_ref = clip_branch(np.exp(rnlp - old.astype(np.float64)), adv)
    assert int((mask_dev != mask_ref).sum()) == 0
    assert 0 < mask_ref.sum() < N  # both branches occur
    # row by row, against the RMS row norm: a row on the wrong branch would differ by its whole
    # policy-gradient part (of the order of the RMS norm); fp32 rounding is about 1e-7 of it
    gd = dl.cpu().numpy().astype(np.float64)
    rms = np.sqrt(np.mean(np.sum(rdl * rdl, axis=1)))
    assert (np.linalg.norm(gd - rdl, axis=1) / rms).max() < 1e-4
    assert rel(gd, rdl) < 1e-5
    assert rel(dv.cpu().numpy(), rdv) < 1e-5
    assert rel(newlp.cpu().numpy(), rnlp) < 1e-5
    assert np.array_equal(newval.cpu().numpy(), v)
    rL = O.ppo_losses(lg, v, act, adv, ret, old, ov if vfclip > 0 else None, vfclip=vfclip)
    gL = losses.cpu().numpy()
    np.testing.assert_allclose(gL, rL, rtol=1e-5, atol=max(1e-6, 2.0 / N))


def test_ppo_grad_strided_combined_head(gpu):
    """The MLP layout: logits and value share rows of width A+1 (value in column A)."""
    N, A = 4096, 5
    out = rng.normal(400, N * (A + 1)).reshape(N, A + 1).astype(np.float32)
    _, _, act, adv, ret, old, _ = _rows(N, A, 401)
    g = torch.from_numpy(out).cuda()
    dout = torch.zeros_like(g)
    c = lambda x: torch.from_numpy(x).cuda()
    D.ppo_grad(g[:, :A], g[:, A], c(act), c(adv), c(ret), c(old), max_shift=False,
               dlogits=dout[:, :A], dvalues=dout[:, A])
    rdl, rdv, _, _ = O.ppo_grad(out[:, :A].copy(), out[:, A].copy(), act, adv, ret, old)
    d = dout.cpu().numpy()
    assert rel(d[:, :A], rdl) < 1e-5
    assert rel(d[:, A], rdv) < 1e-5


def test_ppo_grad_padded_rows_partial_chunk(gpu):
    """Head rows padded to 16 columns (A = 10 logits, value in column 10), the layout of the
    MinGRU head: the rows move as float4s, the last chunk of each row partially; padding columns of
    the gradient rows are left untouched."""
    N, A, W = 4096, 10, 16
    out = rng.normal(410, N * W).reshape(N, W).astype(np.float32)
    _, _, act, adv, ret, old, _ = _rows(N, A, 411)
    g = torch.from_numpy(out).cuda()
    dout = torch.full_like(g, 7.0)
    c = lambda x: torch.from_numpy(x).cuda()
    D.ppo_grad(g[:, :A], g[:, A], c(act), c(adv), c(ret), c(old), max_shift=True,
               dlogits=dout[:, :A], dvalues=dout[:, A])
    rdl, rdv, _, _ = O.ppo_grad(out[:, :A].copy(), out[:, A].copy(), act, adv, ret, old,
                                max_shift=True)
    d = dout.cpu().numpy()
    assert rel(d[:, :A], rdl) < 1e-5
    assert rel(d[:, A], rdv) < 1e-5
    assert np.all(d[:, A + 1:] == 7.0)


@pytest.mark.parametrize("n", [1, 257, 4096, 262144, 1000003])
def test_adv_normalize(gpu, n):
    x = rng.randf(0xAD7 + n, n, -3.0, 3.0)
    ref = np.zeros(n)
    O.lib().orc_adv_normalize(O.P(x), n, O.P(ref))
    g64 = D.adv_normalize(torch.from_numpy(x).cuda()).cpu().numpy()
    if n > 1:
        np.testing.assert_allclose(g64, ref, rtol=1e-10, atol=1e-12)
    g32 = D.adv_normalize(torch.from_numpy(x.astype(np.float32)).cuda()).cpu().numpy()
    if n > 1:
        assert rel(g32, ref) < 1e-5
    # deterministic: same bits on a second run
    assert np.array_equal(D.adv_normalize(torch.from_numpy(x).cuda()).cpu().numpy(), g64)


def test_colsum_deterministic(gpu):
    X = rng.normal(500, 65536 * 130).reshape(65536, 130).astype(np.float32)
    g = torch.from_numpy(X).cuda()
    s1 = D.colsum(g).cpu().numpy()
    s2 = D.colsum(g).cpu().numpy()
    assert np.array_equal(s1, s2)
    assert rel(s1, X.astype(np.float64).sum(0)) < 1e-5
