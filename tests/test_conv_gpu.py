"""Conv2D and ConvTranspose2D forward/backward on the GPU, through the C ABI,
against the oracle (seera_cpp restatement) on the same seeded inputs: the
reference's own test shapes (Testing/test_1.py, test_3.py) and BASELINE
configs 4 and 5 at full size. Tolerance as in test_gemm_gpu.py."""
import zlib

import numpy as np
import pytest

import oracle
from ml_framework_amd import capi
from oracle import fp16r
from tests.helpers import (assert_parity, hip_conv_bwd, hip_conv_fwd, hip_convT_bwd,
                           hip_convT_fwd, rel_fro)
from tests.shapes import (CONV2D, CONV2D_EDGE, CONV2D_FUSED, CONV2D_PHASE2, CONV2D_STREAM,
                          CONVT, CONVT_PHASE2)

pytestmark = pytest.mark.gpu
S = oracle.seera_cpp
STRICT = 1e-5


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    assert capi.gpu_available(), "no HIP device visible"


def _kaiming(r, shape, fan_in):
    lim = np.sqrt(6.0 / fan_in)
    return r.uniform(-lim, lim, shape).astype(np.float32)


ALL_CONV2D = CONV2D + CONV2D_STREAM + CONV2D_EDGE + CONV2D_PHASE2 + CONV2D_FUSED
ALL_CONVT = CONVT + CONVT_PHASE2


@pytest.mark.parametrize("case", ALL_CONV2D, ids=[c[0] for c in ALL_CONV2D])
def test_conv2d_parity(case):
    name, N, C, H, W, F, KH, KW, s, p = case
    r = np.random.default_rng(zlib.crc32(name.encode()))
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    w = _kaiming(r, (F, C, KH, KW), C * KH * KW)
    y = hip_conv_fwd(x, w, s, p)
    ry = S.conv2d_forward(fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(y, ry, f"{name} fwd")
    assert rel_fro(y, ry) <= STRICT
    dy = r.standard_normal(ry.shape).astype(np.float32)
    dx, dw = hip_conv_bwd(dy, x, w, s, p)
    rdx, rdw = S.conv2d_backward(fp16r(dy), fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(dx, rdx, f"{name} dX")
    assert_parity(dw, rdw, f"{name} dW")
    assert rel_fro(dx, rdx) <= STRICT and rel_fro(dw, rdw) <= STRICT


@pytest.mark.parametrize("case", ALL_CONVT, ids=[c[0] for c in ALL_CONVT])
def test_convT_parity(case):
    name, N, Cin, H, W, Cout, KH, KW, s, p = case
    r = np.random.default_rng(zlib.crc32(name.encode()))
    x = r.standard_normal((N, Cin, H, W)).astype(np.float32)
    w = _kaiming(r, (Cin, Cout, KH, KW), Cin * KH * KW)
    y = hip_convT_fwd(x, w, s, p)
    ry = S.conv_transpose2d_forward(fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(y, ry, f"{name} fwd")
    assert rel_fro(y, ry) <= STRICT
    dy = r.standard_normal(ry.shape).astype(np.float32)
    dx, dw = hip_convT_bwd(dy, x, w, s, p)
    rdx, rdw = S.conv_transpose2d_backward(fp16r(dy), fp16r(x), fp16r(w), s, s, p, p)
    assert_parity(dx, rdx, f"{name} dX")
    assert_parity(dw, rdw, f"{name} dW")
    assert rel_fro(dx, rdx) <= STRICT and rel_fro(dw, rdw) <= STRICT


def _inner(a, b):
    return float(np.sum(np.asarray(a, np.float64) * np.asarray(b, np.float64)))


def test_conv2d_config4_full():
    """N=128, 64->64, 56x56, 3x3 s1 p1, seed 0."""
    r = np.random.default_rng(0)
    x = fp16r(r.standard_normal((128, 64, 56, 56)))
    w = fp16r(_kaiming(r, (64, 64, 3, 3), 576))
    dy = fp16r(r.standard_normal((128, 64, 56, 56)))
    y = hip_conv_fwd(x, w, 1, 1)
    assert_parity(y, S.conv2d_forward(x, w, 1, 1, 1, 1), "cfg4 fwd")
    dx, dw = hip_conv_bwd(dy, x, w, 1, 1)
    rdx, rdw = S.conv2d_backward(dy, x, w, 1, 1, 1, 1)
    assert_parity(dx, rdx, "cfg4 dX")
    assert_parity(dw, rdw, "cfg4 dW")
    ref = _inner(y, dy)
    assert abs(_inner(x, dx) - ref) <= 1e-4 * abs(ref) + 1.0
    assert abs(_inner(w, dw) - ref) <= 1e-4 * abs(ref) + 1.0


def test_convT_config5_full():
    """N=32, 128->64, 28x28 -> 56x56, 4x4 s2 p1, seed 0."""
    r = np.random.default_rng(0)
    x = fp16r(r.standard_normal((32, 128, 28, 28)))
    w = fp16r(_kaiming(r, (128, 64, 4, 4), 2048))
    dy = fp16r(r.standard_normal((32, 64, 56, 56)))
    y = hip_convT_fwd(x, w, 2, 1)
    assert_parity(y, S.conv_transpose2d_forward(x, w, 2, 2, 1, 1), "cfg5 fwd")
    dx, dw = hip_convT_bwd(dy, x, w, 2, 1)
    rdx, rdw = S.conv_transpose2d_backward(dy, x, w, 2, 2, 1, 1)
    assert_parity(dx, rdx, "cfg5 dX")
    assert_parity(dw, rdw, "cfg5 dW")
    ref = _inner(y, dy)
    assert abs(_inner(x, dx) - ref) <= 1e-4 * abs(ref) + 1.0
    assert abs(_inner(w, dw) - ref) <= 1e-4 * abs(ref) + 1.0


def test_outputs_are_overwritten_not_accumulated():
    """dX and dW are overwritten (the Python layer accumulates; Seera_Engine.py:339-340)."""
    from ml_framework_amd.capi import DeviceBuffer
    r = np.random.default_rng(9)
    x = r.standard_normal((2, 3, 8, 8)).astype(np.float32)
    w = r.standard_normal((4, 3, 3, 3)).astype(np.float32)
    dy = r.standard_normal((2, 4, 8, 8)).astype(np.float32)
    ref = hip_conv_bwd(dy, x, w, 1, 1)
    with DeviceBuffer.from_array(w) as pw, DeviceBuffer.from_array(x) as px, \
            DeviceBuffer.from_array(dy) as pdy, DeviceBuffer(x.nbytes) as pdx, \
            DeviceBuffer(w.nbytes) as pdw:
        pdx.fill(0x7F)
        pdw.fill(0x7F)
        for _ in range(2):
            capi.call("seera_hip_conv2d_bwd", pw.ptr, px.ptr, pdy.ptr, pdx.ptr, pdw.ptr,
                      2, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1)
        assert np.array_equal(pdx.to_array(x.shape), ref[0])
        assert np.array_equal(pdw.to_array(w.shape), ref[1])


@pytest.mark.parametrize("entry,C,F,K,s,p", [
    ("seera_hip_conv2d_bwd", 64, 64, 3, 1, 1),           # the one-pass backward's shape
    ("seera_hip_conv2d_bwd", 8, 16, 3, 2, 1),            # stride phases
    ("seera_hip_conv2d_bwd_bias", 64, 64, 3, 1, 1),      # with db
    ("seera_hip_conv2DTranspose_bwd", 128, 64, 4, 2, 1),  # config 5's layer
])
def test_empty_batch_backward_writes_zero_weight_gradient(entry, C, F, K, s, p):
    """batch = 0: dW (and db) are sums over no images, so exactly 0, and the
    activation pointers, which point at nothing, may be NULL. For the
    transposed convolution W is [Cin, Cout, K, K] (upsampling.cu:322-375)."""
    from ml_framework_amd.capi import DeviceBuffer
    wshape = (C, F, K, K) if "Transpose" in entry else (F, C, K, K)
    w = np.random.default_rng(C + F + K).standard_normal(wshape).astype(np.float32)
    nbias = F if "bias" in entry else 1
    with DeviceBuffer.from_array(w) as pw, DeviceBuffer(w.nbytes) as pdw, \
            DeviceBuffer(nbias * 4) as pdb:
        pdw.fill(0xFF)  # NaN everywhere until written
        pdb.fill(0xFF)
        extra = (pdb.ptr,) if "bias" in entry else ()
        capi.call(entry, pw.ptr, None, None, None, pdw.ptr, *extra, 0, C, 8, 8, F, K, K, s, s, p, p)
        assert np.array_equal(pdw.to_array(wshape), np.zeros(wshape, np.float32))
        if extra:
            assert np.array_equal(pdb.to_array((F,)), np.zeros(F, np.float32))


def test_empty_batch_forward_is_a_no_op():
    """batch = 0 forwards return success without touching memory: every
    activation pointer NULL, the weights a real buffer."""
    from ml_framework_amd.capi import DeviceBuffer
    with DeviceBuffer(128 * 64 * 16 * 4) as pw:
        pw.fill(0)
        capi.call("seera_hip_conv2d_fwd", None, pw.ptr, None, 0, 64, 56, 56, 64, 3, 3, 1, 1, 1, 1)
        capi.call("seera_hip_conv2d_fwd_bias_act", None, pw.ptr, None, None, None, 0, 64, 56, 56,
                  64, 3, 3, 1, 1, 1, 1, capi.SEERA_ACT_RELU)
        capi.call("seera_hip_conv2DTranpose_fwd", None, pw.ptr, None, 0, 128, 28, 28, 64, 4, 4,
                  2, 2, 1, 1)


def test_subnormal_fp16_operands_conv_identity_bit_exact():
    """A 1x1 identity convolution, and a 3x3 one with the identity on the
    centre tap (the config-4 forward and one-pass backward kernels), return
    fp16r(X) (and dX = fp16r(dY)) bit for bit on inputs full of fp16
    subnormals: the conv kernels round with subnormals kept, as
    __float2half does (convolution.cu:59, 68)."""
    from tests.test_gemm_gpu import _subnormals

    rng = np.random.default_rng(26)
    for N, C, H, W, k in [(2, 8, 9, 13, 1), (2, 64, 20, 16, 1), (3, 64, 56, 56, 3)]:
        x = _subnormals(N * C * H * W, rng).reshape(N, C, H, W)
        w = np.zeros((C, C, k, k), np.float32)
        w[np.arange(C), np.arange(C), k // 2, k // 2] = 1.0
        y = hip_conv_fwd(x, w, 1, k // 2)
        assert np.array_equal(y, fp16r(x)), ("fwd", N, C, H, W, k)
        dy = _subnormals(N * C * H * W, rng).reshape(N, C, H, W)
        dx, _ = hip_conv_bwd(dy, x, w, 1, k // 2)
        assert np.array_equal(dx, fp16r(dy)), ("dX", N, C, H, W, k)
