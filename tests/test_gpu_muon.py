"""Muon / Newton-Schulz on the GPU vs the CPU oracle.

Exact tier: bit-exact with the reference-order f64 oracle (the reference's verify-muon-gpu shapes).
Fast tier: bf16 MFMA within 1e-2 relative Frobenius of the f64 oracle (and of the fp32-MFMA tier);
fp32 MFMA within 1e-4 of the f64 oracle.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import _lib
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


# (128, 28), (15, 128), (48, 48) ... run in one workgroup (2 n + min^2 <= 8192 doubles of LDS);
# (128, 128), (64, 64), (90, 40) run as the launch chain
@pytest.mark.parametrize("shape", [(16, 24), (24, 16), (20, 20), (128, 128), (6, 128), (128, 28), (28, 128),
                                   (15, 128), (128, 15), (48, 48), (64, 64), (90, 40), (1, 1)])
def test_exact_tier_bit_exact(gpu, shape):
    # verify-muon-gpu draw order: per element w U[-.5,.5), g U[-.3,.3), m U[-.2,.2) (Exe/Puffer.lean:1134-1138)
    rows, cols = shape
    n = rows * cols
    w = rng.uniform01(rng.words(0x3E7A + rows * 7 + cols, 3 * n)).reshape(n, 3)
    W = -0.5 + (0.5 - -0.5) * w[:, 0]
    G = -0.3 + (0.3 - -0.3) * w[:, 1]
    M = -0.2 + (0.2 - -0.2) * w[:, 2]
    lr, wd, mu, eps = 0.1, 0.01, 0.95, 1e-7
    nW = np.zeros(n); nM = np.zeros(n)
    c = O.coeffs_array(O.REF_COEFFS)
    O.lib().orc_muon_mat(rows, cols, O.P(W), O.P(G), O.P(M), O.P(nW), O.P(nM), 1.0, lr, wd, mu, eps,
                         O.P(c), 5, 0)
    t = lambda x: torch.from_numpy(x.reshape(rows, cols)).cuda()
    gW, gM = D.muon_mat_f64(t(W), t(G), t(M), lr=lr, wd=wd, mu=mu, eps=eps)
    assert np.array_equal(gM.cpu().numpy().ravel(), nM)
    got = gW.cpu().numpy().ravel()
    assert np.array_equal(got, nW), f"max|d| {np.abs(got - nW).max()}"


def test_stepvec_bit_exact(gpu):
    n = 300
    b, g, m = rng.normal(1, n), rng.normal(2, n), rng.normal(3, n)
    nb = np.zeros(n); nm = np.zeros(n)
    O.lib().orc_stepvec(n, O.P(b), O.P(g), O.P(m), O.P(nb), O.P(nm), 0.25, 0.1, 0.01, 0.95)
    t = lambda x: torch.from_numpy(x).cuda()
    gb, gm = D.stepvec_f64(t(b), t(g), t(m), gscale=0.25, lr=0.1, wd=0.01, mu=0.95)
    assert np.array_equal(gb.cpu().numpy(), nb) and np.array_equal(gm.cpu().numpy(), nm)


CONFIG3 = [(512, 512)] * 4 + [(512, 1024), (1024, 512)]


@pytest.mark.parametrize("shape", CONFIG3[3:] + [(128, 128), (96, 200), (200, 96)])
@pytest.mark.parametrize("coeffs", ["const", "ref"])
def test_fast_ns_vs_oracle(gpu, shape, coeffs):
    rows, cols = shape
    X0 = rng.normal(0x300 + rows + cols, rows * cols, 0.0, 0.02).reshape(rows, cols).astype(np.float32)
    cf = O.BASELINE_COEFFS if coeffs == "const" else O.REF_COEFFS
    ref = O.newton_schulz(X0.astype(np.float64), cf, 1e-7, form=1)
    xb = torch.from_numpy(X0).cuda()
    D.newton_schulz(xb, coeffs=cf, math="bf16")
    xf = torch.from_numpy(X0).cuda()
    D.newton_schulz(xf, coeffs=cf, math="f32")
    gb, gf = xb.cpu().numpy(), xf.cpu().numpy()
    assert rel(gf, ref) < 1e-4
    assert rel(gb, ref) < 1e-2
    assert rel(gb, gf.astype(np.float64)) < 1e-2


@pytest.mark.parametrize("math_", ["bf16", "f32"])
def test_ns_batch_equals_single_calls(gpu, math_):
    """The config-3 batch (4 x 512x512 + 2 x 512x1024, plus a tall and a small matrix, 8 matrices
    over 8 lanes, and 11 so that lanes are reused) through the batched entry equals one call per
    matrix, bit for bit (same kernels; the lanes only change where they run)."""
    shapes = CONFIG3 + [(1024, 512), (64, 32), (512, 512), (100, 300), (32, 32)]
    mats = [rng.normal(0x310 + i, r * c, 0.0, 0.02).reshape(r, c).astype(np.float32)
            for i, (r, c) in enumerate(shapes)]
    batch = [torch.from_numpy(m).cuda() for m in mats]
    D.newton_schulz_batch(batch, coeffs=O.BASELINE_COEFFS, math=math_)
    torch.cuda.synchronize()
    for m, b in zip(mats, batch):
        single = torch.from_numpy(m).cuda()
        D.newton_schulz(single, coeffs=O.BASELINE_COEFFS, math=math_)
        assert torch.equal(b, single)


def test_ns_fused_many_matrices(gpu):
    """More matrices than one fused launch takes (16), with empty, one-row and single-tile shapes:
    the batch equals one call per matrix bit for bit, and every result holds the 1e-2 bar."""
    shapes = [(64, 64), (1, 512), (0, 7), (130, 70), (512, 128), (16, 512), (200, 64), (64, 1)] * 3
    mats = [rng.normal(0x330 + i, r * c, 0.0, 0.02).reshape(r, c).astype(np.float32)
            for i, (r, c) in enumerate(shapes)]
    batch = [torch.from_numpy(m).cuda() for m in mats]
    D.newton_schulz_batch(batch, coeffs=O.BASELINE_COEFFS, math="bf16")
    torch.cuda.synchronize()
    for m, b in zip(mats, batch):
        single = torch.from_numpy(m).cuda()
        D.newton_schulz(single, coeffs=O.BASELINE_COEFFS, math="bf16")
        assert torch.equal(b, single)
        if m.size:
            ref = O.newton_schulz(m.astype(np.float64), O.BASELINE_COEFFS, 1e-7, form=1)
            assert rel(b.cpu().numpy(), ref) < 1e-2, m.shape


@pytest.mark.parametrize("nsteps", [1, 2, 7])
def test_ns_fused_step_counts(gpu, nsteps):
    # the per-step buffers and the last step's direct write to the caller's matrix, for other step
    # counts (constant coefficients: restarting the reference schedule's aggressive first triples
    # after its last one amplifies bf16 rounding past 1e-2 in any bf16 evaluation)
    X0 = rng.normal(0x340 + nsteps, 192 * 320, 0.0, 0.02).reshape(192, 320).astype(np.float32)
    cf = O.BASELINE_COEFFS[:1] * nsteps
    ref = O.newton_schulz(X0.astype(np.float64), cf, 1e-7, form=1)
    x = torch.from_numpy(X0).cuda()
    D.newton_schulz(x, coeffs=cf, math="bf16")
    assert rel(x.cpu().numpy(), ref) < 1e-2


def test_fast_ns_orthogonalises(gpu):
    # size-independent property at the full config-3 size: singular values pushed into the
    # quintic's fixed band (the constant-coefficient schedule leaves them in about [0.68, 1.2])
    X0 = rng.normal(0x301, 512 * 1024, 0.0, 0.02).reshape(512, 1024).astype(np.float32)
    x = torch.from_numpy(X0).cuda()
    D.newton_schulz(x, coeffs=O.BASELINE_COEFFS, math="bf16")
    s = np.linalg.svd(x.cpu().numpy().astype(np.float64), compute_uv=False)
    assert s.min() > 0.5 and s.max() < 1.3


def test_fast_muon_step_vs_oracle(gpu):
    rows, cols = 128, 128
    W = rng.normal(0x310, rows * cols, 0, 0.1).reshape(rows, cols).astype(np.float32)
    G = rng.normal(0x311, rows * cols).reshape(rows, cols).astype(np.float32)
    M = rng.normal(0x312, rows * cols, 0, 0.1).reshape(rows, cols).astype(np.float32)
    nW = np.zeros(rows * cols); nM = np.zeros(rows * cols)
    c = O.coeffs_array(O.BASELINE_COEFFS)
    O.lib().orc_muon_mat(rows, cols, O.P(O.f64(W)), O.P(O.f64(G)), O.P(O.f64(M)), O.P(nW), O.P(nM),
                         1 / 64, 0.015, 0.0, 0.95, 1e-7, O.P(c), 5, 1)
    gW, gM = torch.from_numpy(W).cuda(), torch.from_numpy(M).cuda()
    D.muon_mat(gW, torch.from_numpy(G).cuda(), gM, gscale=1 / 64, lr=0.015, wd=0.0, mu=0.95,
               coeffs=O.BASELINE_COEFFS, math="bf16")
    assert rel(gM.cpu().numpy().ravel(), nM) < 1e-6
    dW = gW.cpu().numpy().ravel() - W.ravel()
    assert rel(dW, nW - W.ravel().astype(np.float64)) < 1e-2


def test_gclip(gpu):
    g = rng.normal(0x320, 100000).astype(np.float32)
    ref = g.astype(np.float64).copy()
    O.lib().orc_gclip(O.P(ref), ref.size, 0.5, 10.0)
    t = torch.from_numpy(g).cuda()
    D.gclip(t, scale=0.5, max_norm=10.0)
    assert rel(t.cpu().numpy(), ref) < 1e-6


@pytest.mark.parametrize("shapes", [CONFIG3, CONFIG3 * 2 + [(1536, 512), (48, 700)], [(1536, 512)], [(64, 64), (512, 128)],
                                    [(128, 4), (128, 128), (2, 128), (1, 128), (200, 64)]],
                         ids=["config3", "queues-shared", "one", "two", "small"])
def test_ns_queue_placements_identical(gpu, shapes):
    """Per-XCD queues and the device-wide queue give the same matrices bit for bit (same tiles, same
    per-tile order; only where and how the items synchronise differs), including queues that hold
    several matrices (14 matrices on 8 queues), tall inputs and a batch with idle queues; no block ran
    off its queue's XCD."""
    mats = [rng.normal(0x350 + i, r * c, 0.0, 0.02).reshape(r, c).astype(np.float32)
            for i, (r, c) in enumerate(shapes)]
    D.ns_status()
    out = {}
    try:
        for mode in (1, 2):
            D.ns_set_queues(mode)
            batch = [torch.from_numpy(m).cuda() for m in mats]
            D.newton_schulz_batch(batch, coeffs=O.BASELINE_COEFFS, math="bf16")
            D.ns_status()
            out[mode] = [b.cpu() for b in batch]
    finally:
        D.ns_set_queues(0)
    for a, b in zip(out[2], out[1]):
        assert torch.equal(a, b)
    ref = O.newton_schulz(mats[0].astype(np.float64), O.BASELINE_COEFFS, 1e-7, form=1)
    assert rel(out[2][0].numpy(), ref) < 1e-2


def test_ns_wait_failure_is_reported(gpu):
    """A fused launch whose bounded waits give up (forced from the host with a one-poll bound) still
    ends normally, and ph_ns_status reports it once; with the default bound the record stays clear
    and the batch holds the 1e-2 bar."""
    mats = [rng.normal(0x340 + i, r * c, 0.0, 0.02).reshape(r, c).astype(np.float32)
            for i, (r, c) in enumerate(CONFIG3)]
    D.ns_status()  # clear anything an earlier test left
    D.ns_set_spin_limit(1)
    try:
        batch = [torch.from_numpy(m).cuda() for m in mats]
        D.newton_schulz_batch(batch, coeffs=O.BASELINE_COEFFS, math="bf16")
        with pytest.raises(_lib.PufferHipError, match="gave up"):
            D.ns_status()
    finally:
        D.ns_set_spin_limit(0)
    D.ns_status()  # the report cleared the record
    batch = [torch.from_numpy(m).cuda() for m in mats]
    D.newton_schulz_batch(batch, coeffs=O.BASELINE_COEFFS, math="bf16")
    D.ns_status()
    for m, b in zip(mats, batch):
        ref = O.newton_schulz(m.astype(np.float64), O.BASELINE_COEFFS, 1e-7, form=1)
        assert rel(b.cpu().numpy(), ref) < 1e-2
