"""Each bf16 product of the headline MinGRU step at its own shape, against the f64 product of the oracle.

The step (obs 128 -> encoder 512 -> 2 MinGRU layers of 512 -> 16-way + value head, 4096 segments x 64
steps, TB = 262,144 rows) runs these products, bf16 operands with fp32 accumulation:
  encoder forward   x0 = obs W_enc^T            262144 x 512  x 128     NT, bf16 out
  layer forward     cmb = x W_l^T               262144 x 1536 x 512     NT, bf16 out
  head forward      logits = x_L W_h^T          262144 x 32   x 512     NT, fp32 out
  data gradient     dx = dy W_l  (W_l^T copy)   262144 x 512  x 1536    NT, bf16 out
  layer weight grad gW = dy^T x                 1536   x 512  x 262144  TN, fp32 out (split-K)
  head weight grad  gWh = dl^T x_L              32     x 512  x 262144  TN, fp32 out (split-K)
  encoder weight    gWenc = dh^T [obs | 1 | 0]  512    x 136  x 262144  TN, fp32 out (split-K)
Every one holds the single-product bar of 1e-2 relative Frobenius against the f64 product of the
unrounded fp32 operands, and against the f64 product of the same bf16-rounded operands it is within
one output rounding (bf16 out: 4e-3) or the fp32 accumulation (fp32 out: 1e-4 at these reduction
lengths). Rows (NT forms, sampled 512 of 262,144) or output rows (TN forms, sampled 32) are checked,
so the oracle's work stays within seconds; the GPU computes the whole product.
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import device as D

pytestmark = pytest.mark.gpu

TB = 262144


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def bf16_round(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def normal(seed, shape, std=1.0):
    return (np.random.default_rng(seed).standard_normal(shape, dtype=np.float32) * np.float32(std))


NT = {  # name: (N, K, seed) of  C[TB][N] = A[TB][K] . B[N][K]^T
    "encoder_fwd": (512, 128, 0xE100),
    "layer_fwd": (1536, 512, 0xE200),
    "head_fwd": (32, 512, 0xE300),
    "data_grad": (512, 1536, 0xE400),
}


@pytest.mark.parametrize("name", list(NT))
def test_step_nt_product(gpu, name):
    N, K, seed = NT[name]
    print(f"step product {name}: {TB} x {N} x {K} NT", flush=True)
    a = normal(seed, (TB, K))
    b = normal(seed + 1, (N, K), 1.0 / np.sqrt(K))
    out_bf16 = N >= 128  # the head's logits stay fp32
    ga = torch.from_numpy(a).cuda().bfloat16()
    gb = torch.from_numpy(b).cuda().bfloat16()
    c = D.gemm(ga, gb, trans_b=True, out_dtype=torch.bfloat16 if out_bf16 else torch.float32)
    c = c.float().cpu().numpy()
    rows = np.sort(np.random.default_rng(seed + 2).choice(TB, 512, replace=False))
    ref = O.gemm(0, 1, a[rows], b, len(rows), N, K, threads=8)
    ref_r = O.gemm(0, 1, bf16_round(a[rows]), bf16_round(b), len(rows), N, K, threads=8)
    e, er = rel(c[rows], ref), rel(c[rows], ref_r)
    print(f"  vs f64: {e:.2e}  vs f64 of the bf16 operands: {er:.2e}", flush=True)
    assert e < 1e-2
    assert er < (4e-3 if out_bf16 else 1e-4)


TN = {  # name: (M, N, seed) of  C[M][N] = A[TB][M]^T . B[TB][N]
    "layer_wgrad": (1536, 512, 0xE500),
    "head_wgrad": (32, 512, 0xE600),
    "encoder_wgrad": (512, 136, 0xE700),
}


@pytest.mark.parametrize("name", list(TN))
def test_step_tn_product(gpu, name):
    M, N, seed = TN[name]
    print(f"step product {name}: {M} x {N} x {TB} TN", flush=True)
    a = normal(seed, (TB, M))
    b = normal(seed + 1, (TB, N))
    if name == "encoder_wgrad":  # [obs | 1 | 0]: the bias gradient rides in column 128
        b[:, 128] = 1.0
        b[:, 129:] = 0.0
    ga = torch.from_numpy(a).cuda().bfloat16()
    gb = torch.from_numpy(b).cuda().bfloat16()
    c = D.gemm(ga, gb, trans_a=True).cpu().numpy()
    assert np.array_equal(c, D.gemm(ga, gb, trans_a=True).cpu().numpy())  # deterministic split-K fold
    sel = np.sort(np.random.default_rng(seed + 2).choice(M, min(M, 32), replace=False))
    asel = np.ascontiguousarray(a[:, sel])
    ref = O.gemm(1, 0, asel, b, len(sel), N, TB, threads=8)
    ref_r = O.gemm(1, 0, bf16_round(asel), bf16_round(b), len(sel), N, TB, threads=8)
    e, er = rel(c[sel], ref), rel(c[sel], ref_r)
    print(f"  vs f64: {e:.2e}  vs f64 of the bf16 operands: {er:.2e}", flush=True)
    assert e < 1e-2
    assert er < 1e-4
