"""Conv2D, ConvTranspose2D and GEMM forward/backward on seeded random shapes (not
from the reference's tests): channel counts, sizes, kernels, strides and
paddings drawn over ranges that reach every dispatch path (three-role and
row-streaming kernels, channel slices, column tiles, widened rows, stride
phases, space-to-depth, the band and gather kernels), each against the oracle
at the tolerance of test_conv_gpu.py. The draws are fixed by the seed."""
import zlib

import numpy as np
import pytest

import oracle
from ml_framework_amd import capi
from oracle import fp16r
from tests.helpers import (assert_parity, hip_conv_bwd, hip_conv_fwd, hip_convT_bwd,
                           hip_convT_fwd, rel_fro)

pytestmark = pytest.mark.gpu
S = oracle.seera_cpp
STRICT = 1e-5


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    assert capi.gpu_available(), "no HIP device visible"


def _conv_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k = int(r.choice([1, 2, 3, 3, 3, 4, 5, 7]))
        s = int(r.choice([1, 1, 1, 2, 2, 3]))
        p = int(r.integers(0, k))
        N = int(r.integers(1, 4))
        C = int(r.choice([int(r.integers(1, 40)), 64, 128, int(r.integers(65, 200))]))
        F = int(r.choice([int(r.integers(1, 40)), 64, 96, int(r.integers(65, 150))]))
        H, W = int(r.integers(1, 40)), int(r.integers(1, 72))
        if (H + 2 * p - k) < 0 or (W + 2 * p - k) < 0:
            continue
        out.append((f"r{len(out):02d}", N, C, H, W, F, k, s, p))
    return out


def _convT_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k = int(r.choice([2, 3, 4, 4, 5]))
        s = int(r.choice([1, 2, 2, 3]))
        p = int(r.integers(0, k))
        N = int(r.integers(1, 4))
        Cin = int(r.choice([int(r.integers(1, 40)), 64, 128]))
        Cout = int(r.choice([int(r.integers(1, 40)), 32, 64]))
        H, W = int(r.integers(1, 20)), int(r.integers(1, 30))
        if (H - 1) * s - 2 * p + k < 1 or (W - 1) * s - 2 * p + k < 1:
            continue
        out.append((f"t{len(out):02d}", N, Cin, H, W, Cout, k, s, p))
    return out


CONV_CASES = _conv_cases(32, 20261202)
CONVT_CASES = _convT_cases(16, 20261203)


def _kaiming(r, shape, fan_in):
    lim = np.sqrt(6.0 / fan_in)
    return r.uniform(-lim, lim, shape).astype(np.float32)


@pytest.mark.parametrize("case", CONV_CASES, ids=[c[0] for c in CONV_CASES])
def test_conv2d_random_shape(case):
    name, N, C, H, W, F, k, s, p = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = _kaiming(r, (F, C, k, k), C * k * k)
    y = hip_conv_fwd(x, w, s, p)
    ry = S.conv2d_forward(fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(y, ry, f"{case} fwd")
    assert rel_fro(y, ry) <= STRICT
    dy = r.standard_normal(ry.shape).astype(np.float32)
    dx, dw = hip_conv_bwd(dy, x, w, s, p)
    rdx, rdw = S.conv2d_backward(fp16r(dy), fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(dx, rdx, f"{case} dX")
    assert_parity(dw, rdw, f"{case} dW")
    assert rel_fro(dx, rdx) <= STRICT and rel_fro(dw, rdw) <= STRICT


@pytest.mark.parametrize("case", CONVT_CASES, ids=[c[0] for c in CONVT_CASES])
def test_convT_random_shape(case):
    name, N, Cin, H, W, Cout, k, s, p = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = r.standard_normal((N, Cin, H, W)).astype(np.float32)
    w = _kaiming(r, (Cin, Cout, k, k), Cin * k * k)
    y = hip_convT_fwd(x, w, s, p)
    ry = S.conv_transpose2d_forward(fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(y, ry, f"{case} fwd")
    assert rel_fro(y, ry) <= STRICT
    dy = r.standard_normal(ry.shape).astype(np.float32)
    dx, dw = hip_convT_bwd(dy, x, w, s, p)
    rdx, rdw = S.conv_transpose2d_backward(fp16r(dy), fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(dx, rdx, f"{case} dX")
    assert_parity(dw, rdw, f"{case} dW")
    assert rel_fro(dx, rdx) <= STRICT and rel_fro(dw, rdw) <= STRICT


def _gemm_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        dims = [int(r.choice([int(r.integers(1, 64)), int(r.integers(64, 700)), int(r.integers(700, 2100))]))
                for _ in range(3)]
        nb = int(r.choice([1, 1, 1, 2, 3]))
        out.append((f"g{i:02d}", dims[0], dims[1], dims[2], nb))
    return out


GEMM_CASES = _gemm_cases(20, 20261204)


@pytest.mark.parametrize("case", GEMM_CASES, ids=[c[0] for c in GEMM_CASES])
def test_matmul_random_shape(case):
    """Seeded random GEMM shapes (every tile kernel, split-K, wave groups,
    pairs, scalar loads and the padded staging copies), forward and backward."""
    from tests.helpers import hip_matmul, hip_matmul_bwd
    name, M, K, N, nb = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()))
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    got = hip_matmul(a, b)
    ref = S.matmul_batched(fp16r(a), fp16r(b))
    assert_parity(got, ref, f"{case} fwd")
    assert rel_fro(got, ref) <= STRICT
    dc = r.uniform(-1, 1, (nb, M, N)).astype(np.float32)
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(fp16r(a), fp16r(b), fp16r(dc))
    assert_parity(da, rda, f"{case} dA")
    assert_parity(db, rdb, f"{case} dB")
    assert rel_fro(da, rda) <= STRICT and rel_fro(db, rdb) <= STRICT
