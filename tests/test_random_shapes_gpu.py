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


# The fused epilogues (bias + ReLU + mask in the forward stores; the ReLU
# gradient in the dA store and db from the dB GEMM's loads of dC, or from the
# dW pass's loads of dY) on their own seeded draws of the same ranges.
EPI_GEMM_CASES = _gemm_cases(12, 20261205)
EPI_CONV_CASES = _conv_cases(12, 20261206)


def _mask_clear_agrees(mask, pre, scale):
    """mask = (pre > 0) wherever the oracle's pre-activation is clear of 0 by
    more than the summation-order noise (values within it may fall either way)."""
    clear = np.abs(pre) > 1e-4 * scale
    return np.array_equal(mask[clear], (pre[clear] > 0).astype(np.float32))


@pytest.mark.parametrize("case", EPI_GEMM_CASES, ids=[c[0] for c in EPI_GEMM_CASES])
def test_matmul_epilogues_random_shape(case):
    """seera_hip_matmul_bias_act (ReLU) against the oracle's matmul + bias then
    ReLU (tensor_ops.cpp:9-15, broadcast.cu:12-64, activations.cu:9-15), its
    mask against the oracle's sign; seera_hip_matmul_bwd_relu_bias's dA and dB
    against the oracle's GEMM backward times the mask, db against an fp64 sum."""
    from ml_framework_amd.capi import DeviceBuffer
    name, M, K, N, nb = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()) + 1)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = r.uniform(-1, 1, N).astype(np.float32)
    dc = r.uniform(-1, 1, (nb, M, N)).astype(np.float32)
    with DeviceBuffer.from_array(a) as pa, DeviceBuffer.from_array(b) as pb, \
            DeviceBuffer.from_array(bias) as pbi, DeviceBuffer(nb * M * N * 4) as pc, \
            DeviceBuffer(nb * M * N * 4) as pm, DeviceBuffer.from_array(dc) as pdc, \
            DeviceBuffer(a.nbytes) as pda, DeviceBuffer(b.nbytes) as pdb, \
            DeviceBuffer(N * 4) as pdbias:
        capi.call("seera_hip_matmul_bias_act", pa.ptr, pb.ptr, pbi.ptr, pc.ptr, pm.ptr, M, N, K,
                  nb, capi.SEERA_ACT_RELU)
        got, mask = pc.to_array((nb, M, N)), pm.to_array((nb, M, N))
        # the backward of a layer whose input a went through a ReLU: its mask
        amask = (a > 0).astype(np.float32)
        with DeviceBuffer.from_array(amask) as pam:
            capi.call("seera_hip_matmul_bwd_relu_bias", pa.ptr, pb.ptr, pdc.ptr, pam.ptr, pda.ptr,
                      pdb.ptr, pdbias.ptr, M, N, K, nb)
        da, dbw, db = pda.to_array(a.shape), pdb.to_array(b.shape), pdbias.to_array((N,))
    pre = S.matmul_batched(fp16r(a), fp16r(b)) + bias
    assert_parity(got, np.where(pre > 0, pre, np.float32(0)), f"{case} fused fwd")
    assert _mask_clear_agrees(mask, pre, np.sqrt(K))
    rda, rdb = S.matmul_bwd(fp16r(a), fp16r(b), fp16r(dc))
    assert_parity(da, rda * amask, f"{case} fused dA")
    assert_parity(dbw, rdb, f"{case} dB")
    ref = dc.astype(np.float64).sum(axis=(0, 1))
    bound = 1e-6 * np.abs(dc).astype(np.float64).sum(axis=(0, 1)) + 1e-6
    assert np.all(np.abs(db - ref) <= bound), f"{case} db"


@pytest.mark.parametrize("case", EPI_CONV_CASES, ids=[c[0] for c in EPI_CONV_CASES])
def test_conv2d_epilogues_random_shape(case):
    """seera_hip_conv2d_fwd_bias_act (ReLU) against the oracle's conv2d_forward
    + bias then ReLU (conv_ops.cpp:95-122, broadcast.cu:12-64,
    activations.cu:9-15), its mask against the oracle's sign;
    seera_hip_conv2d_bwd_bias's dX and dW against the oracle's backward, db
    against an fp64 sum of dY over images and pixels."""
    from ml_framework_amd.capi import DeviceBuffer
    name, N, C, H, W, F, k, s, p = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()) + 1)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = _kaiming(r, (F, C, k, k), C * k * k)
    bias = r.uniform(-0.5, 0.5, F).astype(np.float32)
    Ho, Wo = (H + 2 * p - k) // s + 1, (W + 2 * p - k) // s + 1
    dy = r.standard_normal((N, F, Ho, Wo)).astype(np.float32)
    ny = N * F * Ho * Wo
    with DeviceBuffer.from_array(x) as px, DeviceBuffer.from_array(w) as pw, \
            DeviceBuffer.from_array(bias) as pbi, DeviceBuffer(ny * 4) as py, \
            DeviceBuffer(ny * 4) as pm, DeviceBuffer.from_array(dy) as pdy, \
            DeviceBuffer(x.nbytes) as pdx, DeviceBuffer(w.nbytes) as pdw, \
            DeviceBuffer(F * 4) as pdb:
        capi.call("seera_hip_conv2d_fwd_bias_act", px.ptr, pw.ptr, pbi.ptr, py.ptr, pm.ptr, N, C,
                  H, W, F, k, k, p, p, s, s, capi.SEERA_ACT_RELU)
        got, mask = py.to_array(dy.shape), pm.to_array(dy.shape)
        capi.call("seera_hip_conv2d_bwd_bias", pw.ptr, px.ptr, pdy.ptr, pdx.ptr, pdw.ptr, pdb.ptr,
                  N, C, H, W, F, k, k, s, s, p, p)
        dx, dw, db = pdx.to_array(x.shape), pdw.to_array(w.shape), pdb.to_array((F,))
    pre = S.conv2d_forward(fp16r(x), fp16r(w), s, s, p, p) + bias[None, :, None, None]
    assert_parity(got, np.where(pre > 0, pre, np.float32(0)), f"{case} fused fwd")
    assert _mask_clear_agrees(mask, pre, np.sqrt(C * k * k))
    rdx, rdw = S.conv2d_backward(fp16r(dy), fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(dx, rdx, f"{case} dX")
    assert_parity(dw, rdw, f"{case} dW")
    ref = dy.astype(np.float64).sum(axis=(0, 2, 3))
    bound = 1e-6 * np.abs(dy).astype(np.float64).sum(axis=(0, 2, 3)) + 1e-6
    assert np.all(np.abs(db - ref) <= bound), f"{case} db"


# The specialised kernels of the configs' layer types on random geometry:
# 3x3 stride-1 pad-1 convolutions of multiples of 64 channels (three-role
# forward, one-pass backward, channel slices, column tiles, widened rows) and
# 4x4 stride-2 pad-1 transposed convolutions (phase and stride-2 streaming
# kernels), with random batch, height and width.
def _hot_conv_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        C = int(r.choice([64, 64, 128, 192]))
        F = int(r.choice([64, 64, 128]))
        N = int(r.integers(1, 5))
        H, W = int(r.integers(1, 40)), int(r.integers(1, 130))
        out.append((f"h{i:02d}", N, C, H, W, F, 3, 1, 1))
    return out


def _hot_convT_cases(n, seed):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        Cin = int(r.choice([32, 64, 96, 128]))
        Cout = int(r.choice([16, 32, 64]))
        N = int(r.integers(1, 4))
        H, W = int(r.integers(1, 24)), int(r.integers(1, 40))
        out.append((f"u{i:02d}", N, Cin, H, W, Cout, 4, 2, 1))
    return out


HOT_CONV_CASES = _hot_conv_cases(12, 20261207)
HOT_CONVT_CASES = _hot_convT_cases(10, 20261208)


@pytest.mark.parametrize("case", HOT_CONV_CASES, ids=[c[0] for c in HOT_CONV_CASES])
def test_conv2d_hot_path_random_geometry(case):
    test_conv2d_random_shape(case)


@pytest.mark.parametrize("case", HOT_CONVT_CASES, ids=[c[0] for c in HOT_CONVT_CASES])
def test_convT_hot_path_random_geometry(case):
    test_convT_random_shape(case)
