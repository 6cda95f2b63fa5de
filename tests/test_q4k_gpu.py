"""Q4_K projections on the GPU against the oracle.

Dequantisation is integer/byte work plus the shader's f32 products: bit-exact
against the oracle.  The matvec sums in a different order than the shader
(per lane, then across lanes), so it is checked against the f64 product and
the shader-order oracle within the f32 rounding bound
1e-5 * sum_k (|w_k| + 2 |dmin*min_k|) |x_k| (the scale of the terms any
summation order adds up).  Shapes are the model's projections: temporal
in_proj [12288, 4096], out_proj [4096, 4096], FFN linear_in [22528, 4096],
linear_out [4096, 11264]; depformer in_proj [3072, 1024] and FFN linear_out
[1024, 2816] (scripts/quantize.py:24-42).
"""
import os

import numpy as np
import pytest
import torch

import oracle
import sts_attn
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def dev(x):
    return torch.from_numpy(np.ascontiguousarray(x)).to("cuda")


def host(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def bound(blocks, x, N):
    K = x.shape[1]
    w = oracle.q4k_dequant(blocks, N, K).astype(np.float64)
    zq = blocks.reshape(-1, 144).copy()
    zq[:, 16:] = 0
    mins = -oracle.q4k_dequant(zq.reshape(-1), N, K).astype(np.float64)
    return np.abs(x.astype(np.float64)) @ (np.abs(w) + 2 * np.abs(mins)).T


@pytest.mark.parametrize("name", ["q4k_random", "q4k_quantized"])
def test_golden_fixtures(gpu, name):
    f = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    N, K, B, seed = (int(f[k]) for k in ("N", "K", "B", "seed"))
    x = oracle.normal(seed + 1, (B, K))
    w = sts_attn.Q4KTensor.from_q4k_bytes(f["blocks"], (N, K))
    np.testing.assert_array_equal(host(w.dequant()), f["dequant"])
    got = host(sts_attn.q4k_matmul(dev(x[:, None, :]), w))[:, 0, :].astype(np.float64)
    tol = 1e-5 * bound(f["blocks"], x, N)
    assert (np.abs(got - f["out_f64"]) <= tol).all()
    assert (np.abs(got - f["out_wgsl"]) <= tol).all()


@pytest.mark.parametrize("N,K", [(1, 256), (7, 512), (64, 4096), (4096, 4096), (33, 11264),
                                 (3072, 1024), (5, 2816)])
def test_dequant_bit_exact(gpu, N, K):
    blocks = oracle.q4k_random_blocks(N * 31 + K, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    np.testing.assert_array_equal(host(w.dequant()), oracle.q4k_dequant(blocks, N, K))


def test_dequant_of_quantized_weights(gpu):
    """Blocks made by the reference's quantizer (scripts/quantize.py)."""
    x = oracle.normal(3, (256, 4096)) * 0.02
    blocks = oracle.q4k_quantize(x)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (256, 4096))
    np.testing.assert_array_equal(host(w.dequant()), oracle.q4k_dequant(blocks, 256, 4096))


@pytest.mark.parametrize("N,K,B", [(12288, 4096, 1), (4096, 4096, 1), (22528, 4096, 1),
                                   (4096, 11264, 1), (3072, 1024, 1), (1024, 2816, 1),
                                   (1001, 4096, 3), (5, 8192, 2), (17, 16384, 1), (1, 256, 1),
                                   (16000, 256, 2), (30000, 512, 1), (3000, 6144, 2),
                                   (700, 12288, 1), (9000, 11264, 1)])
def test_matvec_against_oracle(gpu, N, K, B):
    print(f"q4k matvec N={N} K={K} B={B}", flush=True)
    blocks = oracle.q4k_random_blocks(N + K + B, N, K)
    x = oracle.normal(N * 7 + B, (B, K))
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    got = host(sts_attn.q4k_matmul(dev(x[:, None, :]), w))[:, 0, :].astype(np.float64)
    ref64 = oracle.q4k_matvec_f64(blocks, x, N)
    tol = 1e-5 * bound(blocks, x, N)
    assert (np.abs(got - ref64) <= tol).all(), np.abs(got - ref64).max()
    if N * K <= 4096 * 4096:
        refw = oracle.q4k_matvec_wgsl(blocks, x, N).astype(np.float64)
        assert (np.abs(got - refw) <= tol).all()


def test_matvec_with_residual_and_quantized_weights(gpu):
    """q4k_matmul_with_residual on weights from the reference's quantizer."""
    N, K = 4096, 4096
    wf = oracle.normal(11, (N, K)) * 0.02
    blocks = oracle.q4k_quantize(wf)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    x = oracle.normal(12, (1, 1, K))
    res = oracle.normal(13, (1, 1, N))
    got = host(sts_attn.q4k_matmul_with_residual(dev(x), w, dev(res)))[0, 0].astype(np.float64)
    ref = oracle.q4k_matvec_f64(blocks, x[0], N)[0] + res[0, 0].astype(np.float64)
    tol = 1e-5 * bound(blocks, x[0], N)[0] + 1e-6 * np.abs(res[0, 0])
    assert (np.abs(got - ref) <= tol).all()
    lin = sts_attn.Q4KLinear(w)
    np.testing.assert_array_equal(host(lin.forward_with_residual(dev(x), dev(res))),
                                  host(sts_attn.q4k_matmul_with_residual(dev(x), w, dev(res))))


def test_matvec_bit_repeatable(gpu):
    N, K = 12288, 4096
    blocks = oracle.q4k_random_blocks(21, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    x = dev(oracle.normal(22, (1, 1, K)))
    first = host(sts_attn.q4k_matmul(x, w))
    for _ in range(5):
        np.testing.assert_array_equal(host(sts_attn.q4k_matmul(x, w)), first)


def test_matvec_argument_errors(gpu):
    blocks = oracle.q4k_random_blocks(1, 4, 512)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (4, 512))
    with pytest.raises(sts_attn.StsError):
        sts_attn.q4k_matmul(dev(oracle.normal(1, (1, 1, 256))), w)  # K mismatch
    lib = sts_attn.load()
    x = dev(oracle.normal(2, (1, 512)))
    y = torch.empty((1, 4), device="cuda")
    assert lib.sts_q4k_matvec(w.raw.data_ptr(), x.data_ptr(), None, y.data_ptr(), 1, 384, 4,
                              None) == sts_attn.STS_ERR_INVALID  # K not a multiple of 256
    assert lib.sts_q4k_matvec(w.raw.data_ptr() + 4, x.data_ptr(), None, y.data_ptr(), 1, 512, 4,
                              None) == sts_attn.STS_ERR_INVALID  # misaligned weights
    with pytest.raises(sts_attn.StsError):
        sts_attn.Q4KTensor.from_q4k_bytes(blocks[:-1], (4, 512))


@pytest.mark.parametrize("N,K,B,Mrows,residual", [(4096, 11264, 1, 5, True), (64, 11264, 2, 3, False),
                                                  (300, 1024, 1, 7, True)])
def test_matmul_many_rows(gpu, N, K, B, Mrows, residual):
    """q4k_matmul with M > 1 (the reference's prefill route, gguf.rs:810-897):
    the GEMM, K above 4096 (the temporal FFN's linear_out, K = 11264) as summed
    slices of 4096; within the f32 bound of the f64 product, with and without
    the residual (gguf.rs:899-905)."""
    blocks = oracle.q4k_random_blocks(N + K + Mrows, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    x = oracle.normal(N + 3 * Mrows, (B, Mrows, K))
    res = oracle.normal(N + 5, (B, Mrows, N)) if residual else None
    got = host(sts_attn.q4k_matmul(dev(x), w, residual=dev(res) if residual else None))
    assert got.shape == (B, Mrows, N)
    xf = x.reshape(B * Mrows, K)
    ref = oracle.q4k_matvec_f64(blocks, xf, N)
    tol = 1e-5 * bound(blocks, xf, N)
    if residual:
        r = res.reshape(B * Mrows, N).astype(np.float64)
        ref = ref + r
        tol = tol + 1e-6 * np.abs(r)
    assert (np.abs(got.reshape(B * Mrows, N).astype(np.float64) - ref) <= tol).all()


@pytest.mark.parametrize("N,K,B", [(4096, 11264, 2), (300, 8192, 3), (77, 16384, 1)])
def test_matvec_residual_split_rows(gpu, N, K, B):
    """q4k_matmul_with_residual (gguf.rs:899-905) where several waves share a
    row (K > 4096) and the batch has several rows: within the f32 bound of the
    f64 product plus residual."""
    print(f"q4k matvec+res N={N} K={K} B={B}", flush=True)
    blocks = oracle.q4k_random_blocks(3 * N + K + B, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    x = oracle.normal(N + 17 * B, (B, 1, K))
    res = oracle.normal(N + 19 * B, (B, 1, N))
    got = host(sts_attn.q4k_matmul_with_residual(dev(x), w, dev(res)))[:, 0].astype(np.float64)
    ref = oracle.q4k_matvec_f64(blocks, x[:, 0], N) + res[:, 0].astype(np.float64)
    tol = 1e-5 * bound(blocks, x[:, 0], N) + 1e-6 * np.abs(res[:, 0])
    assert (np.abs(got - ref) <= tol).all()


def test_gemm_split_k_padded_strides(gpu):
    """sts_q4k_gemm with k above 4096 (summed slices) and x, y and residual rows
    wider than the products (ldx > k, ldy > n, ldr > n): the padding is neither
    read into the sums nor written."""
    N, K, M = 200, 8704, 7
    ldx, ldy, ldr = K + 64, N + 40, N + 24
    blocks = oracle.q4k_random_blocks(91, N, K)
    w = sts_attn.Q4KTensor.from_q4k_bytes(blocks, (N, K))
    xf = oracle.normal(92, (M, K))
    rf = oracle.normal(93, (M, N))
    xp = np.full((M, ldx), np.nan, np.float32)
    xp[:, :K] = xf
    rp = np.full((M, ldr), np.nan, np.float32)
    rp[:, :N] = rf
    x, r = dev(xp), dev(rp)
    y = torch.full((M, ldy), -7.0, device="cuda")
    lib = sts_attn.load()
    assert lib.sts_q4k_gemm(w.raw.data_ptr(), x.data_ptr(), ldx, None, 0.0, r.data_ptr(), ldr,
                            y.data_ptr(), ldy, M, K, N, 0, None) == 0
    got = host(y)
    assert (got[:, N:] == -7.0).all()
    ref = oracle.q4k_matvec_f64(blocks, xf, N) + rf.astype(np.float64)
    tol = 1e-5 * bound(blocks, xf, N) + 1e-6 * np.abs(rf)
    assert (np.abs(got[:, :N].astype(np.float64) - ref) <= tol).all()
