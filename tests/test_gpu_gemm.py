"""MFMA GEMMs vs the f64 oracle GEMM: all transpose forms, dtypes, epilogues, edge shapes.

Tolerances (relative Frobenius): fp32 math 1e-5 vs f64; bf16 math 1e-2 vs f64 on the unrounded
inputs, and 1e-5 vs f64 on the bf16-rounded inputs (isolates the fp32 accumulation).
"""
import numpy as np
import pytest
import torch

import oracle_lib as O
from pufferlean_amd import _lib as L
from pufferlean_amd import device as D
from pufferlean_amd import rng

pytestmark = pytest.mark.gpu


def rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / max(np.linalg.norm(b), 1e-30))


def bf16_round(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


def operands(M, N, K, ta, tb, seed):
    a = rng.normal(seed, M * K).reshape((K, M) if ta else (M, K)).astype(np.float32)
    b = (rng.normal(seed + 1, K * N) / np.sqrt(K)).reshape((N, K) if tb else (K, N)).astype(np.float32)
    return a, b


def oracle(a, b, ta, tb, M, N, K):
    return O.gemm(ta, tb, a, b, M, N, K, threads=8)


FORMS = [(0, 0), (0, 1), (1, 0), (1, 1)]


@pytest.mark.parametrize("ta,tb", FORMS)
@pytest.mark.parametrize("M,N,K", [(256, 128, 64), (300, 136, 72), (64, 64, 512), (512, 512, 2048)])
@pytest.mark.parametrize("math_", ["bf16", "f32"])
def test_gemm_forms(gpu, ta, tb, M, N, K, math_):
    a, b = operands(M, N, K, ta, tb, 100 + M + N + K)
    ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    c = D.gemm(ga, gb, trans_a=bool(ta), trans_b=bool(tb), math=math_).cpu().numpy()
    ref = oracle(a, b, ta, tb, M, N, K)
    if math_ == "f32":
        assert rel(c, ref) < 1e-5
    else:
        assert rel(c, ref) < 1e-2
        ref_r = oracle(bf16_round(a), bf16_round(b), ta, tb, M, N, K)
        assert rel(c, ref_r) < 1e-5


@pytest.mark.parametrize("ta,tb", FORMS)
def test_gemm_bf16_storage_and_output(gpu, ta, tb):
    M, N, K = 384, 256, 320
    a, b = operands(M, N, K, ta, tb, 7)
    ga = torch.from_numpy(a).cuda().to(torch.bfloat16)
    gb = torch.from_numpy(b).cuda().to(torch.bfloat16)
    c = D.gemm(ga, gb, trans_a=bool(ta), trans_b=bool(tb), out_dtype=torch.bfloat16).float().cpu().numpy()
    ref_r = oracle(bf16_round(a), bf16_round(b), ta, tb, M, N, K)
    assert rel(c, ref_r) < 4e-3  # one bf16 rounding of the output
    assert rel(c, oracle(a, b, ta, tb, M, N, K)) < 1e-2


def test_gemm_config2_full_size(gpu):
    """16384 x 512 x 512 in the three policy forms; checked against the oracle on sampled rows
    (forward/dgrad) and sampled columns (wgrad)."""
    M, K, N = 16384, 512, 512
    X = rng.normal(200, M * K).reshape(M, K).astype(np.float32)
    W = (rng.normal(201, K * N) / np.sqrt(512)).reshape(N, K).astype(np.float32)  # [out][in]
    dY = rng.normal(202, M * N).reshape(M, N).astype(np.float32)
    gX, gW, gdY = (torch.from_numpy(v).cuda() for v in (X, W, dY))
    rows = np.sort(rng.randint(203, 256, M))
    cols = np.sort(rng.randint(204, 64, N))
    for math_, tol in (("bf16", 1e-2), ("f32", 1e-5)):
        # forward Y = X W^T
        Y = D.gemm(gX, gW, trans_b=True, math=math_).cpu().numpy()
        assert rel(Y[rows], O.gemm(0, 1, X[rows], W, len(rows), N, K)) < tol
        # dgrad dX = dY W
        dX = D.gemm(gdY, gW, math=math_).cpu().numpy()
        assert rel(dX[rows], O.gemm(0, 0, dY[rows], W, len(rows), K, N)) < tol
        # wgrad dW = dY^T X  ([N x K], reduction over the 16384 rows; split-K path)
        dW = D.gemm(gdY, gX, trans_a=True, math=math_).cpu().numpy()
        ref = O.gemm(1, 0, dY, np.ascontiguousarray(X[:, cols]), N, len(cols), M, threads=8)
        assert rel(dW[:, cols], ref) < tol
        dW2 = D.gemm(gdY, gX, trans_a=True, math=math_).cpu().numpy()
        assert np.array_equal(dW, dW2)  # deterministic split-K fold


def test_gemm_epilogues(gpu):
    M, N, K = 200, 96, 64
    a, b = operands(M, N, K, 0, 1, 9)
    ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    bias = torch.from_numpy(rng.normal(10, N).astype(np.float32)).cuda()
    ref = oracle(a, b, 0, 1, M, N, K)
    bn = bias.cpu().numpy()
    c = D.gemm(ga, gb, trans_b=True, math="f32", epilogue=L.PH_EPI_BIAS, bias=bias).cpu().numpy()
    assert rel(c, ref + bn) < 1e-5
    c = D.gemm(ga, gb, trans_b=True, math="f32", epilogue=L.PH_EPI_BIAS_RELU, bias=bias).cpu().numpy()
    np.testing.assert_array_equal(c <= 0, (ref + bn) <= 0)
    assert rel(c, np.maximum(ref + bn, 0)) < 1e-5
    aux = torch.from_numpy(rng.normal(11, M * N).reshape(M, N).astype(np.float32)).cuda()
    auxn = aux.cpu().numpy()
    c = D.gemm(ga, gb, trans_b=True, math="f32", epilogue=L.PH_EPI_RELU_MASK, aux=aux).cpu().numpy()
    np.testing.assert_array_equal(c == 0, (auxn <= 0) | (ref == 0))
    assert rel(c, np.where(auxn > 0, ref, 0)) < 1e-5
    c2 = torch.empty((N, M), device="cuda", dtype=torch.bfloat16)
    c = D.gemm(ga, gb, trans_b=True, math="f32", epilogue=L.PH_EPI_AXPBY, aux=aux, alpha=-0.5,
               beta=2.0, out2=c2, out2_trans=True).cpu().numpy()
    assert rel(c, -0.5 * ref + 2.0 * auxn) < 1e-5
    assert rel(c2.float().cpu().numpy(), c.T) < 4e-3


@pytest.mark.parametrize("M,N,K", [(65536, 128, 4), (65536, 3, 128), (128, 4, 16384), (3, 128, 16384)])
def test_gemm_small_dims_padded_path(gpu, M, N, K):
    # the CartPole policy's 4-wide input layer and 3-wide head: operands staged zero-padded
    for ta, tb in FORMS:
        a, b = operands(M, N, K, ta, tb, 13 + ta * 2 + tb)
        ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        c = D.gemm(ga, gb, trans_a=bool(ta), trans_b=bool(tb), math="f32").cpu().numpy()
        assert rel(c, oracle(a, b, ta, tb, M, N, K)) < 1e-5


@pytest.mark.parametrize("M,N,K", [(32768, 128, 28), (32768, 28, 128), (128, 28, 32768), (32768, 15, 128),
                                   (15, 128, 32768), (32768, 128, 15), (300, 9, 21), (9, 300, 4097)])
@pytest.mark.parametrize("math_", ["bf16", "f32"])
def test_gemm_unaligned_env_shapes(gpu, M, N, K, math_):
    """The target/drone MLP products (obs 28 / 21, heads 15 / 9 wide): zero-padded staging, all forms."""
    print(f"gemm unaligned M={M} N={N} K={K} {math_}", flush=True)
    for ta, tb in FORMS:
        a, b = operands(M, N, K, ta, tb, 17 + M + N + K + 2 * ta + tb)
        ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
        c = D.gemm(ga, gb, trans_a=bool(ta), trans_b=bool(tb), math=math_).cpu().numpy()
        if math_ == "f32":
            assert rel(c, oracle(a, b, ta, tb, M, N, K)) < 1e-5, (ta, tb)
        else:
            assert rel(c, oracle(bf16_round(a), bf16_round(b), ta, tb, M, N, K)) < 1e-5, (ta, tb)


def test_gemm_unaligned_strided_bf16_storage_and_epilogue(gpu):
    """Unaligned leading dimensions (column views of wider rows), bf16-stored operands and the bias
    epilogue through the padded staging."""
    M, N, K = 4000, 15, 28
    a = rng.normal(21, M * 31).reshape(M, 31).astype(np.float32)
    b = (rng.normal(22, N * 29).reshape(N, 29) / np.sqrt(K)).astype(np.float32)
    ga = torch.from_numpy(a).cuda()[:, 1:1 + K]     # lda 31, base offset by one element
    gb = torch.from_numpy(b).cuda()[:, :K]          # ldb 29
    bias = torch.from_numpy(rng.normal(23, N).astype(np.float32)).cuda()
    ref = oracle(np.ascontiguousarray(a[:, 1:1 + K]), np.ascontiguousarray(b[:, :K]), 0, 1, M, N, K)
    c = D.gemm(ga, gb, trans_b=True, math="f32", epilogue=L.PH_EPI_BIAS, bias=bias).cpu().numpy()
    assert rel(c, ref + bias.cpu().numpy()) < 1e-5
    abf, bbf = ga.to(torch.bfloat16), gb.to(torch.bfloat16)  # contiguous bf16 copies, K = 28
    c = D.gemm(abf, bbf, trans_b=True, math="bf16").cpu().numpy()
    ref_r = oracle(abf.float().cpu().numpy(), bbf.float().cpu().numpy(), 0, 1, M, N, K)
    assert rel(c, ref_r) < 1e-5


def test_gemm_unaligned_mask_axpby_and_second_output(gpu):
    """The ReLU-mask and alpha*acc + beta*aux epilogues, with a transposed bf16 second output, on a
    15-wide reduction (the dgrad of a 15-wide head) through the padded staging."""
    M, N, K = 3000, 128, 15
    a, b = operands(M, N, K, 0, 0, 31)
    ga, gb = torch.from_numpy(a).cuda(), torch.from_numpy(b).cuda()
    ref = oracle(a, b, 0, 0, M, N, K)
    aux = torch.from_numpy(rng.normal(32, M * N).reshape(M, N).astype(np.float32)).cuda()
    auxn = aux.cpu().numpy()
    c = D.gemm(ga, gb, math="f32", epilogue=L.PH_EPI_RELU_MASK, aux=aux).cpu().numpy()
    assert rel(c, np.where(auxn > 0, ref, 0)) < 1e-5
    c2 = torch.empty((N, M), device="cuda", dtype=torch.bfloat16)
    c = D.gemm(ga, gb, math="f32", epilogue=L.PH_EPI_AXPBY, aux=aux, alpha=0.5, beta=-1.5, out2=c2,
               out2_trans=True).cpu().numpy()
    assert rel(c, 0.5 * ref - 1.5 * auxn) < 1e-5
    assert rel(c2.float().cpu().numpy(), c.T) < 4e-3


def _bf(x):
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda().to(torch.bfloat16)


@pytest.mark.parametrize("ta,tb", FORMS)
def test_gemm_big_tiles_ragged(gpu, ta, tb):
    """bf16 x bf16 with >= 512 tiles of 256x128 takes the 256x128 kernel (four 128x64 wavefronts,
    C staged in 64-row passes). Ragged M and N (not multiples of the tile) and a K tail (K % 32 = 8)."""
    M, N, K = 4136, 4104, 264
    a, b = operands(M, N, K, ta, tb, 300 + 2 * ta + tb)
    ar, br = bf16_round(a), bf16_round(b)
    ref = (ar.T if ta else ar).astype(np.float64) @ (br.T if tb else br).astype(np.float64)
    c = D.gemm(_bf(a), _bf(b), trans_a=bool(ta), trans_b=bool(tb)).cpu().numpy()
    assert rel(c, ref) < 1e-5
    cb = D.gemm(_bf(a), _bf(b), trans_a=bool(ta), trans_b=bool(tb), out_dtype=torch.bfloat16)
    assert rel(cb.float().cpu().numpy(), ref) < 4e-3


def test_gemm_big_tiles_epilogues(gpu):
    M, N, K = 4160, 4096, 128
    a, b = operands(M, N, K, 0, 1, 310)
    ar, br = bf16_round(a), bf16_round(b)
    ref = ar.astype(np.float64) @ br.T.astype(np.float64)
    ga, gb = _bf(a), _bf(b)
    bias = torch.from_numpy(rng.normal(311, N).astype(np.float32)).cuda()
    bn = bias.cpu().numpy()
    c = D.gemm(ga, gb, trans_b=True, epilogue=L.PH_EPI_BIAS, bias=bias).cpu().numpy()
    assert rel(c, ref + bn) < 1e-5
    aux = torch.from_numpy(rng.normal(312, M * N).reshape(M, N).astype(np.float32)).cuda()
    auxn = aux.cpu().numpy()
    c = D.gemm(ga, gb, trans_b=True, epilogue=L.PH_EPI_RELU_MASK, aux=aux).cpu().numpy()
    np.testing.assert_array_equal(c == 0, (auxn <= 0) | (ref == 0))
    assert rel(c, np.where(auxn > 0, ref, 0)) < 1e-5
    c2 = torch.empty((N, M), device="cuda", dtype=torch.bfloat16)
    c = D.gemm(ga, gb, trans_b=True, epilogue=L.PH_EPI_AXPBY, aux=aux, alpha=-0.5, beta=2.0,
               out2=c2, out2_trans=True).cpu().numpy()
    assert rel(c, -0.5 * ref + 2.0 * auxn) < 1e-5
    assert rel(c2.float().cpu().numpy(), c.T) < 4e-3


@pytest.mark.parametrize("ta,tb", [(1, 0), (0, 1)])
def test_gemm_big_tiles_split_k(gpu, ta, tb):
    """Few output tiles and a long reduction: split-K over 256x256 tiles (four 128x128 wavefronts,
    C staged in 64-row passes), deterministic fold."""
    M, N, K = 300, 520, 8232
    a, b = operands(M, N, K, ta, tb, 320 + ta)
    ar, br = bf16_round(a), bf16_round(b)
    ref = (ar.T if ta else ar).astype(np.float64) @ (br.T if tb else br).astype(np.float64)
    c = D.gemm(_bf(a), _bf(b), trans_a=bool(ta), trans_b=bool(tb)).cpu().numpy()
    assert rel(c, ref) < 1e-5
    c2 = D.gemm(_bf(a), _bf(b), trans_a=bool(ta), trans_b=bool(tb)).cpu().numpy()
    assert np.array_equal(c, c2)


def test_gemm_nt_big_tile_epilogue_paths(gpu):
    """The NT load-to-LDS kernel's epilogue paths at 256x128 tiles: AXPBY accumulating into its own
    bf16 output (the dgrad pattern), AXPBY without aux, BIAS into bf16 (the encoder pattern), explicit
    split-K partials, an odd N, and a second output, each against the f64 product."""
    M, N, K = 4136, 4104, 264
    a, b = operands(M, N, K, 0, 1, 330)
    ar, br = bf16_round(a), bf16_round(b)
    ref = ar.astype(np.float64) @ br.T.astype(np.float64)
    ga, gb = _bf(a), _bf(b)
    # AXPBY accumulating into its own output (the dgrad pattern), bf16
    x = rng.normal(331, M * N).reshape(M, N).astype(np.float32)
    out = _bf(x)
    xr = out.float().cpu().numpy()
    D.gemm(ga, gb, trans_b=True, out=out, epilogue=L.PH_EPI_AXPBY, aux=out, alpha=1.0, beta=1.0)
    assert rel(out.float().cpu().numpy(), ref + xr) < 4e-3
    # AXPBY without aux: alpha * acc
    c = D.gemm(ga, gb, trans_b=True, epilogue=L.PH_EPI_AXPBY, alpha=-0.5).cpu().numpy()
    assert rel(c, -0.5 * ref) < 1e-5
    # BIAS into bf16 (the encoder pattern)
    bias = torch.from_numpy(rng.normal(332, N).astype(np.float32)).cuda()
    cb = D.gemm(ga, gb, trans_b=True, out_dtype=torch.bfloat16, epilogue=L.PH_EPI_BIAS, bias=bias)
    assert rel(cb.float().cpu().numpy(), ref + bias.cpu().numpy()) < 4e-3
    # explicit split-K: fp32 partials from registers, deterministic fold
    c3 = D.gemm(ga, gb, trans_b=True, splits=3).cpu().numpy()
    assert rel(c3, ref) < 1e-5
    assert np.array_equal(c3, D.gemm(ga, gb, trans_b=True, splits=3).cpu().numpy())
    # odd N: LDS-staged path
    No = N - 7
    c = D.gemm(ga, gb[:No].contiguous(), trans_b=True).cpu().numpy()
    assert rel(c, ref[:, :No]) < 1e-5
    # a second output leaves the first unchanged
    c_one = D.gemm(ga, gb, trans_b=True).cpu().numpy()
    c2 = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
    c_two = D.gemm(ga, gb, trans_b=True, out2=c2).cpu().numpy()
    assert np.array_equal(c_one, c_two)
    assert rel(c2.float().cpu().numpy(), c_one) < 4e-3


@pytest.mark.parametrize("N", [64, 40, 32, 17])
def test_gemm_nt_narrow_output_big_tiles(gpu, N):
    """NT outputs at most 64 wide with >= 512 row tiles (the policy heads: 262144 x 32) take the
    256x64 load-to-LDS kernel: ragged M, a K tail, fp32 and bf16 C, the bias epilogue."""
    M, K = 131080, 264
    a, b = operands(M, N, K, 0, 1, 340 + N)
    ar, br = bf16_round(a), bf16_round(b)
    ref = ar.astype(np.float64) @ br.T.astype(np.float64)
    ga, gb = _bf(a), _bf(b)
    c = D.gemm(ga, gb, trans_b=True).cpu().numpy()
    assert rel(c, ref) < 1e-5
    bias = torch.from_numpy(rng.normal(341, N).astype(np.float32)).cuda()
    c = D.gemm(ga, gb, trans_b=True, epilogue=L.PH_EPI_BIAS, bias=bias).cpu().numpy()
    assert rel(c, ref + bias.cpu().numpy()) < 1e-5
    cb = D.gemm(ga, gb, trans_b=True, out_dtype=torch.bfloat16)
    assert rel(cb.float().cpu().numpy(), ref) < 4e-3


@pytest.mark.parametrize("M,N", [(4136, 4104), (131080, 64)])
def test_gemm_nt_bf16_staging_matches_fp32_staging(gpu, M, N):
    """bf16 C with no aux operand (NONE / BIAS / BIAS_RELU) rounds the accumulators in registers and
    stages the tile once as bf16; a second output forces the fp32 staging passes. Both give the same
    bits (ragged M and N, a K tail), and both match the f64 product."""
    K = 264
    a, b = operands(M, N, K, 0, 1, 350 + N)
    ar, br = bf16_round(a), bf16_round(b)
    ref = ar.astype(np.float64) @ br.T.astype(np.float64)
    ga, gb = _bf(a), _bf(b)
    bias = torch.from_numpy(rng.normal(351, N).astype(np.float32)).cuda()
    for epi in (L.PH_EPI_NONE, L.PH_EPI_BIAS, L.PH_EPI_BIAS_RELU):
        bb = None if epi == L.PH_EPI_NONE else bias
        c16 = D.gemm(ga, gb, trans_b=True, out_dtype=torch.bfloat16, epilogue=epi, bias=bb)
        two = torch.empty((M, N), device="cuda", dtype=torch.bfloat16)
        c32 = D.gemm(ga, gb, trans_b=True, out_dtype=torch.bfloat16, epilogue=epi, bias=bb, out2=two)
        assert torch.equal(c16, c32), epi
        assert torch.equal(two, c32), epi
        r = ref if bb is None else ref + bias.cpu().numpy()
        if epi == L.PH_EPI_BIAS_RELU:
            r = np.maximum(r, 0.0)
        assert rel(c16.float().cpu().numpy(), r) < 4e-3


@pytest.mark.parametrize("M,N,K", [(520, 264, 86024), (1536, 512, 45056), (2048, 2056, 512),
                                   (300, 132, 1032)])
def test_gemm_tn_matches_nt_on_transposed_copies(gpu, M, N, K):
    """The TN form (both operands m/n-contiguous: the weight gradients) transposes 4 x 8 register
    chunks into LDS; the NT form on transposed copies of the same operands runs the same tiles, LDS
    contents and MFMA order, so the two give the same bits. Split-K over 256x256 tiles (with a K
    tail), the weight-gradient shape's split count, 128x128 tiles with a ragged N, and a padded
    unaligned shape; the first also against the f64 product."""
    g = torch.Generator(device="cuda")
    g.manual_seed(M + N + K)
    aT = torch.randn(K, M, device="cuda", generator=g).bfloat16()
    b = torch.randn(K, N, device="cuda", generator=g).bfloat16()
    c_tn = D.gemm(aT, b, trans_a=True)
    c_nt = D.gemm(aT.t().contiguous(), b.t().contiguous(), trans_b=True)
    assert torch.equal(c_tn, c_nt)
    assert torch.equal(D.gemm(aT, b, trans_a=True), c_tn)  # deterministic split-K fold
    if M == 520:
        ref = aT.double().t() @ b.double()
        assert float((c_tn.double() - ref).norm() / ref.norm()) < 1e-5


@pytest.mark.parametrize("M,N,K", [(1024, 128, 131072), (512, 128, 262144)])
def test_gemm_split_k_tiles_of_a_split_on_one_xcd(gpu, M, N, K):
    """Weight-gradient reductions long enough for 64 / 128 splits of 2048 (a multiple of 8 splits,
    each at least 2048 of k) place every tile of one split on one XCD; the split index and tile come
    from that placement. Against the f64 product of the same bf16 operands, twice (same bits)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(M + K)
    aT = torch.randn(K, M, device="cuda", generator=g).bfloat16()
    b = torch.randn(K, N, device="cuda", generator=g).bfloat16()
    c = D.gemm(aT, b, trans_a=True)
    ref = aT.double().t() @ b.double()
    assert float((c.double() - ref).norm() / ref.norm()) < 1e-5
    assert torch.equal(D.gemm(aT, b, trans_a=True), c)


@pytest.mark.parametrize("M,N,K", [(512, 136, 262144), (300, 200, 8200), (136, 256, 65536)])
def test_gemm_tn_split_k_128x256_tiles(gpu, M, N, K):
    """TN bf16 split-K products 129..256 wide take 128x256 tiles, one block per CU (the encoder's
    weight and bias gradients over the observation copy with its ones column: 512 x 136). Ragged M
    and N and a K tail; against the f64 product of the same bf16 operands, twice (same bits)."""
    g = torch.Generator(device="cuda")
    g.manual_seed(M * N + K)
    aT = torch.randn(K, M, device="cuda", generator=g).bfloat16()
    b = torch.randn(K, N, device="cuda", generator=g).bfloat16()
    c = D.gemm(aT, b, trans_a=True)
    ref = aT.double().t() @ b.double()
    assert float((c.double() - ref).norm() / ref.norm()) < 1e-5
    assert torch.equal(D.gemm(aT, b, trans_a=True), c)


@pytest.mark.parametrize("epi", ["none", "none_f32", "bias", "bias_relu", "axpby"])
def test_gemm_long_k_nt(gpu, epi):
    """NT bf16 products with a long reduction (the MinGRU data gradient's form, k = 1536) on the
    load-to-LDS kernel: each epilogue against the f64 product of the bf16-rounded operands on sampled
    rows (one bf16 output rounding: 4e-3; fp32 output: 1e-5)."""
    M, N, K = 32768, 512, 1536
    rs = np.random.default_rng(0xF00 + len(epi))
    a = rs.standard_normal((M, K), dtype=np.float32)
    b = (rs.standard_normal((N, K), dtype=np.float32) / np.sqrt(K)).astype(np.float32)
    ga, gb = torch.from_numpy(a).cuda().bfloat16(), torch.from_numpy(b).cuda().bfloat16()
    ar, br = bf16_round(a), bf16_round(b)
    rows = np.sort(rs.choice(M, 384, replace=False))
    ref = O.gemm(0, 1, ar[rows], br, len(rows), N, K, threads=8)
    bias = torch.from_numpy(rs.standard_normal(N).astype(np.float32)).cuda()
    aux = torch.from_numpy(rs.standard_normal((M, N)).astype(np.float32)).cuda().bfloat16()
    kw = dict(trans_b=True, out_dtype=torch.float32 if epi == "none_f32" else torch.bfloat16)
    if epi == "bias":
        kw.update(epilogue=L.PH_EPI_BIAS, bias=bias)
        ref = ref + bias.cpu().numpy()
    elif epi == "bias_relu":
        kw.update(epilogue=L.PH_EPI_BIAS_RELU, bias=bias)
        ref = np.maximum(ref + bias.cpu().numpy(), 0.0)
    elif epi == "axpby":
        kw.update(epilogue=L.PH_EPI_AXPBY, aux=aux, alpha=0.75, beta=1.5)
        ref = 0.75 * ref + 1.5 * aux.float().cpu().numpy()[rows]
    c = D.gemm(ga, gb, **kw).float().cpu().numpy()
    assert np.isfinite(c).all()
    assert rel(c[rows], ref) < (1e-5 if epi == "none_f32" else 4e-3), rel(c[rows], ref)
    if epi == "bias_relu":  # zeros exactly where the product is <= 0 (up to fp32 accumulation at ~0)
        diff = (c[rows] == 0) != (ref <= 0)
        assert np.all(np.abs(ref[diff]) < 1e-4)
