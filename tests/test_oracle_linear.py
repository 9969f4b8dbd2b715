"""Pins the oracle's linear layer (vvo_linear: ggml_mul_mat(W, x) + bias,
src/qwen2.cpp:19-25) before it checks the projection kernels.

Every reference value here is computed by numpy alone, from the raw weight
bytes decoded independently of the oracle (f16 through numpy's float16, GGUF
Q8_0 blocks as an f16 scale followed by 32 int8 codes):
  * EXACT mode equals the fp64 matmul of the decoded weights with unrounded x;
  * GGML mode with F16 weights equals the fp64 sum of f16(x) * w (products
    exact in fp32), up to fp32 summation;
  * GGML mode with Q8_0 weights equals numpy's own Q8_0 quantization of x
    (d = amax / 127 stored as f16, codes round-half-away(x / d)) with integer
    block sums times d_w * d_x, up to fp32 summation;
  * the bias is added once per output; a transposed weight is caught.
"""
import numpy as np
import pytest


def _rand_w(vvo, rng, M, K, w_type, scale):
    w = (rng.standard_normal((M, K)) * scale).astype(np.float32)
    return vvo.from_f32(w, w_type)


def _decode_w(raw, w_type, M, K):
    """Independent numpy decoding of the weight bytes to fp64 [M, K]."""
    if w_type == 1:
        return raw.view(np.float16).reshape(M, K).astype(np.float64)
    blk = raw.reshape(M, K // 32, 34)
    d = blk[:, :, :2].copy().view(np.float16).astype(np.float64)          # [M, nb, 1]
    q = blk[:, :, 2:].view(np.int8).astype(np.float64)                    # [M, nb, 32]
    return (q * d).reshape(M, K)


def _q8_numpy(x):
    """GGUF Q8_0 of rows x [N, K] in numpy fp32: (codes int [N, nb, 32], d fp64 [N, nb, 1])."""
    N, K = x.shape
    xb = x.reshape(N, K // 32, 32).astype(np.float32)
    amax = np.abs(xb).max(axis=2, keepdims=True)
    d = (amax / np.float32(127.0)).astype(np.float32)
    inv = np.where(d != 0, np.float32(1.0) / np.where(d != 0, d, 1), 0).astype(np.float32)
    v = (xb * inv).astype(np.float32)
    codes = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)
    return codes, d.astype(np.float16).astype(np.float64)


@pytest.mark.parametrize("w_type", [1, 8])
@pytest.mark.parametrize("N,K,M", [(1, 896, 128), (7, 256, 96), (33, 3584, 64)])
def test_exact_mode_is_fp64_matmul(vvo, w_type, N, K, M):
    rng = np.random.default_rng(N * K + M + w_type)
    raw = _rand_w(vvo, rng, M, K, w_type, K ** -0.5)
    x = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(M).astype(np.float32)
    y = vvo.linear(x, raw, w_type, M, bias, mode=vvo.EXACT)
    ref = x.astype(np.float64) @ _decode_w(raw, w_type, M, K).T + bias
    assert np.abs(y - ref).max() <= 1e-6 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("N,K,M", [(1, 896, 128), (9, 3584, 64)])
def test_ggml_mode_f16_weights_rounds_x_to_f16(vvo, N, K, M):
    rng = np.random.default_rng(K + M)
    raw = _rand_w(vvo, rng, M, K, 1, K ** -0.5)
    x = (rng.standard_normal((N, K)) * 3.0).astype(np.float32)
    y = vvo.linear(x, raw, 1, M, None, mode=vvo.GGML)
    w = _decode_w(raw, 1, M, K)
    xr = x.astype(np.float16).astype(np.float64)
    ref = xr @ w.T
    mag = np.abs(xr) @ np.abs(w).T
    assert np.all(np.abs(y - ref) <= 2e-6 * mag + 1e-30)
    # rounding x matters: the unrounded product is measurably different
    assert np.abs(y - x.astype(np.float64) @ w.T).max() > 10 * np.abs(y - ref).max()


@pytest.mark.parametrize("N,K,M", [(1, 896, 128), (5, 3584, 64)])
def test_ggml_mode_q8_0_weights_quantizes_x_per_block(vvo, N, K, M):
    rng = np.random.default_rng(3 * K + M)
    raw = _rand_w(vvo, rng, M, K, 8, K ** -0.5)
    x = rng.standard_normal((N, K)).astype(np.float32)
    bias = rng.standard_normal(M).astype(np.float32)
    y = vvo.linear(x, raw, 8, M, bias, mode=vvo.GGML)
    blk = raw.reshape(M, K // 32, 34)
    dw = blk[:, :, :2].copy().view(np.float16).astype(np.float32)[:, :, 0]    # [M, nb]
    qw = blk[:, :, 2:].view(np.int8).astype(np.int64)                           # [M, nb, 32]
    qx, dx = _q8_numpy(x)                                                       # [N, nb, 32], [N, nb, 1]
    isum = np.einsum("nbi,mbi->nmb", qx, qw)                                    # exact integers
    scale = (dw[None, :, :] * dx[:, None, :, 0].astype(np.float32)).astype(np.float64)   # fp32 products
    ref = (isum * scale).sum(axis=2) + bias
    mag = (np.abs(isum) * np.abs(scale)).sum(axis=2) + np.abs(bias)
    assert np.all(np.abs(y - ref) <= 2e-6 * mag + 1e-30)


def test_transposed_weight_is_caught(vvo):
    rng = np.random.default_rng(5)
    K = M = 128
    raw = _rand_w(vvo, rng, M, K, 1, K ** -0.5)
    x = rng.standard_normal((4, K)).astype(np.float32)
    w = _decode_w(raw, 1, M, K)
    wt = vvo.from_f32(w.T.astype(np.float32), 1)
    good = vvo.linear(x, raw, 1, M, None, mode=vvo.EXACT)
    bad = vvo.linear(x, wt, 1, M, None, mode=vvo.EXACT)
    ref = x.astype(np.float64) @ w.T
    assert np.abs(good - ref).max() < 1e-5
    assert np.abs(bad - ref).max() > 0.1
