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
    old = (lg[np.arange(N), act] - lse + rng.normal(seed + 5, N, 0.0, 0.2)).astype(np.float32)
    ov = (v + rng.normal(seed + 6, N, 0.0, 0.5)).astype(np.float32)
    return lg, v, act, adv, ret, old, ov


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
    # Rows whose ratio lies within float rounding of a clip boundary may take the other branch of
    # the clipped surrogate in fp32; they are counted (must be rare) and left out of the tolerance.
    ratio = np.exp(rnlp - old.astype(np.float64))
    edge = (np.abs(ratio - 0.8) < 1e-5) | (np.abs(ratio - 1.2) < 1e-5)
    assert edge.sum() <= max(2, int(1e-4 * N))
    keep = ~edge
    assert rel(dl.cpu().numpy()[keep], rdl[keep]) < 1e-5
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
