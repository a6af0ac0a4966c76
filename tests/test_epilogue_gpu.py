"""Fused Dense-layer forward (matmul + bias + ReLU in the GEMM's store) and
the bias gradient. The reference runs the forward as cuda_matmul,
broadcast_add_4d and cuda_relu_fwd (GEMM.cu:95-103, broadcast.cu:12-64,
activations.cu:9-15); the fused entry point must equal that sequence bit for
bit, which is checked against the unfused GPU GEMM with the fp32 bias add and
ReLU done in numpy. db is the reference's Reductionsum over the batch
(reductionKernels.cu:12-29; Seera_Engine.py:43-65)."""
import ctypes

import numpy as np
import pytest

from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer, check, load
from tests.helpers import assert_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    assert capi.gpu_available(), "no HIP device visible"


def _bits(x):
    return np.ascontiguousarray(x, np.float32).view(np.uint32)


SHAPES = [
    (256, 784, 512, 1),    # MLP cfg3 layer 1
    (256, 512, 256, 1),    # layer 2
    (256, 256, 10, 1),     # layer 3 (N = 10 edge tile)
    (64, 2048, 64, 1),     # few tiles: split-K, epilogue in the reduce
    (33, 65, 17, 2),       # odd dims, folded batch
    (7, 0, 5, 1),          # K = 0: C = act(bias)
    (4096, 4096, 512, 1),  # 256x256 warp-specialised tiles
    (2049, 2047, 1025, 1),  # unaligned and large: zero-padded staging copies of A and B
    (64, 1200, 64, 1),     # 32x32 tiles, 8 wave groups
    (50, 300, 30, 2),      # 32x32 tiles, scalar-load B, folded batch
]


@pytest.mark.parametrize("M,K,N,nb", SHAPES)
@pytest.mark.parametrize("act", [capi.SEERA_ACT_NONE, capi.SEERA_ACT_RELU])
@pytest.mark.parametrize("with_bias", [True, False])
def test_fused_bias_act_equals_unfused(M, K, N, nb, act, with_bias):
    r = np.random.default_rng(M * 31 + K * 7 + N + act)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = r.uniform(-1, 1, N).astype(np.float32)
    lib = load()
    with DeviceBuffer.from_array(a if a.size else np.zeros(1, np.float32)) as A, \
            DeviceBuffer.from_array(b if b.size else np.zeros(1, np.float32)) as B, \
            DeviceBuffer.from_array(bias) as Bi, DeviceBuffer(nb * M * N * 4) as C0, \
            DeviceBuffer(nb * M * N * 4) as C, DeviceBuffer(nb * M * N * 4) as Mk:
        check(lib.seera_hip_matmul(A.ptr, B.ptr, C0.ptr, M, N, K, nb))
        Mk.fill(0x7F)
        check(lib.seera_hip_matmul_bias_act(A.ptr, B.ptr, Bi.ptr if with_bias else None, C.ptr,
                                            Mk.ptr, M, N, K, nb, act))
        plain = C0.to_array((nb, M, N))
        pre = plain + (bias if with_bias else np.float32(0))
        want = np.where(pre > 0, pre, np.float32(0)) if act == capi.SEERA_ACT_RELU else pre
        got = C.to_array((nb, M, N))
        assert np.array_equal(_bits(got), _bits(want))
        mask = Mk.to_array((nb, M, N))
        if act == capi.SEERA_ACT_RELU:
            assert np.array_equal(mask, (pre > 0).astype(np.float32))
        else:  # mask untouched without ReLU
            assert (_bits(mask) == 0x7F7F7F7F).all()


def test_relu_mask_optional():
    r = np.random.default_rng(3)
    a = r.uniform(-1, 1, (64, 96)).astype(np.float32)
    b = r.uniform(-1, 1, (96, 48)).astype(np.float32)
    lib = load()
    with DeviceBuffer.from_array(a) as A, DeviceBuffer.from_array(b) as B, \
            DeviceBuffer(64 * 48 * 4) as C0, DeviceBuffer(64 * 48 * 4) as C:
        check(lib.seera_hip_matmul(A.ptr, B.ptr, C0.ptr, 64, 48, 96, 1))
        check(lib.seera_hip_matmul_bias_act(A.ptr, B.ptr, None, C.ptr, None, 64, 48, 96, 1,
                                            capi.SEERA_ACT_RELU))
        plain = C0.to_array((64, 48))
        assert np.array_equal(_bits(C.to_array((64, 48))), _bits(np.maximum(plain, 0)))


def test_unknown_activation_is_rejected():
    st = load().seera_hip_matmul_bias_act(None, None, None, None, None, 1, 1, 1, 1, 7)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT
    assert "activation" in load().seera_hip_last_error().decode()


@pytest.mark.parametrize("rows,N", [(256, 10), (256, 512), (1, 3), (1000, 65), (65536, 128), (5, 0)])
def test_bias_grad(rows, N):
    r = np.random.default_rng(rows + N)
    dy = r.standard_normal((rows, N)).astype(np.float32)
    lib = load()
    with DeviceBuffer.from_array(dy if dy.size else np.zeros(1, np.float32)) as D, \
            DeviceBuffer(max(N, 1) * 4) as db1, DeviceBuffer(max(N, 1) * 4) as db2:
        check(lib.seera_hip_bias_grad(D.ptr, db1.ptr, rows, N))
        check(lib.seera_hip_bias_grad(D.ptr, db2.ptr, rows, N))
        g1, g2 = db1.to_array((N,)), db2.to_array((N,))
        assert np.array_equal(_bits(g1), _bits(g2))  # fixed summation order
        ref = dy.astype(np.float64).sum(axis=0)
        # fp32 sums of up to rows/8 terms per group: the error grows with rows
        assert_parity(g1, ref, "db", rel=1e-5, mabs=max(1e-4, rows * 1e-7))


BWD_SHAPES = [
    (256, 784, 512, 1),    # MLP cfg3 layer 1 (dA is [256, 784])
    (256, 512, 256, 1),
    (64, 64, 4096, 1),     # long contraction over N: split-K, mask in the reduce
    (33, 65, 17, 2),       # odd dims, folded batch
    (2048, 2048, 2048, 1),  # 256x256 warp-specialised tiles
    (2049, 2047, 1025, 1),  # unaligned and large: zero-padded staging copies
    (5, 0, 7, 1),          # K = 0: empty dA and dB
    (160, 600, 72, 1),     # dA + dB as one launch on 32x32 tiles
]


@pytest.mark.parametrize("M,K,N,nb", BWD_SHAPES)
def test_fused_relu_backward_equals_unfused(M, K, N, nb):
    """dA = (dC . B^T) * mask against matmul_bwd followed by the multiply in
    numpy (fp32, exact for a 0/1 mask); dB unchanged."""
    r = np.random.default_rng(M + K + N)
    a = np.maximum(r.standard_normal((nb, M, K)), 0).astype(np.float32)
    b = r.standard_normal((K, N)).astype(np.float32)
    dc = r.standard_normal((nb, M, N)).astype(np.float32)
    mask = (r.uniform(0, 1, (nb, M, K)) > 0.4).astype(np.float32)
    n_a, n_b = max(a.size, 1), max(b.size, 1)
    with DeviceBuffer.from_array(a if a.size else np.zeros(1, np.float32)) as pa, \
            DeviceBuffer.from_array(b if b.size else np.zeros(1, np.float32)) as pb, \
            DeviceBuffer.from_array(dc) as pdc, \
            DeviceBuffer.from_array(mask if mask.size else np.zeros(1, np.float32)) as pm, \
            DeviceBuffer(n_a * 4) as pda, DeviceBuffer(n_b * 4) as pdb, \
            DeviceBuffer(n_a * 4) as pda2, DeviceBuffer(n_b * 4) as pdb2:
        capi.call("seera_hip_matmul_bwd", pa.ptr, pb.ptr, pdc.ptr, pda.ptr, pdb.ptr, M, N, K, nb)
        capi.call("seera_hip_matmul_bwd_relu", pa.ptr, pb.ptr, pdc.ptr, pm.ptr, pda2.ptr, pdb2.ptr,
                  M, N, K, nb)
        if a.size == 0:
            return
        da = pda.to_array(a.shape)
        want = da * mask
        got = pda2.to_array(a.shape)
        assert np.array_equal(_bits(got), _bits(want))
        assert np.array_equal(pdb2.to_array(b.shape), pdb.to_array(b.shape))


def _oracle_epilogue(pre, act):
    return np.where(pre > 0, pre, np.float32(0)) if act == capi.SEERA_ACT_RELU else pre


def _mask_agrees(mask, pre_ref, scale):
    """The mask must equal (pre > 0) of the oracle wherever the oracle's
    pre-activation is clear of 0 by more than the parity tolerance (the two
    sums differ in order, so values within rounding of 0 may fall either way)."""
    clear = np.abs(pre_ref) > 1e-4 * scale
    return np.array_equal(mask[clear], (pre_ref[clear] > 0).astype(np.float32))


@pytest.mark.parametrize("M,K,N,nb", [s for s in SHAPES if s[1] > 0])
@pytest.mark.parametrize("act", [capi.SEERA_ACT_NONE, capi.SEERA_ACT_RELU])
def test_fused_bias_act_against_oracle(M, K, N, nb, act):
    """The fused Dense forward against the oracle directly: the seera_cpp
    restatement's matmul on fp16-rounded operands (tensor_ops.cpp:9-15), then
    the bias add and ReLU in fp32 (broadcast.cu:12-64, activations.cu:9-15),
    at the north-star tolerance; the ReLU mask against the oracle's sign."""
    import oracle
    from oracle import fp16r

    r = np.random.default_rng(M * 13 + K + N + act)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    bias = r.uniform(-1, 1, N).astype(np.float32)
    lib = load()
    with DeviceBuffer.from_array(a) as A, DeviceBuffer.from_array(b) as B, \
            DeviceBuffer.from_array(bias) as Bi, DeviceBuffer(nb * M * N * 4) as C, \
            DeviceBuffer(nb * M * N * 4) as Mk:
        check(lib.seera_hip_matmul_bias_act(A.ptr, B.ptr, Bi.ptr, C.ptr, Mk.ptr, M, N, K, nb, act))
        got, mask = C.to_array((nb, M, N)), Mk.to_array((nb, M, N))
    pre = oracle.seera_cpp.matmul_batched(fp16r(a), fp16r(b)) + bias
    assert_parity(got, _oracle_epilogue(pre, act), f"fused fwd {M}x{K}x{N}x{nb}")
    if act == capi.SEERA_ACT_RELU:
        assert _mask_agrees(mask, pre, np.sqrt(K))


@pytest.mark.parametrize("M,K,N,nb", [s for s in BWD_SHAPES if s[1] > 0])
def test_fused_relu_backward_against_oracle(M, K, N, nb):
    """dA = (dC . B^T) * mask and dB = A^T . dC against the oracle's GEMM
    backward on fp16-rounded operands (Seera_Engine.py:557-564) times the
    mask (Seera_Engine.py:575-583), at the north-star tolerance."""
    import oracle
    from oracle import fp16r

    r = np.random.default_rng(M * 7 + K + N)
    a = np.maximum(r.standard_normal((nb, M, K)), 0).astype(np.float32)
    b = r.standard_normal((K, N)).astype(np.float32)
    dc = r.standard_normal((nb, M, N)).astype(np.float32)
    mask = (r.uniform(0, 1, (nb, M, K)) > 0.4).astype(np.float32)
    with DeviceBuffer.from_array(a) as pa, DeviceBuffer.from_array(b) as pb, \
            DeviceBuffer.from_array(dc) as pdc, DeviceBuffer.from_array(mask) as pm, \
            DeviceBuffer(a.nbytes) as pda, DeviceBuffer(b.nbytes) as pdb:
        capi.call("seera_hip_matmul_bwd_relu", pa.ptr, pb.ptr, pdc.ptr, pm.ptr, pda.ptr, pdb.ptr,
                  M, N, K, nb)
        da, db = pda.to_array(a.shape), pdb.to_array(b.shape)
    rda, rdb = oracle.seera_cpp.matmul_bwd(fp16r(a), fp16r(b), fp16r(dc))
    assert_parity(da, rda * mask, "fused dA")
    assert_parity(db, rdb, "dB")


BWD_BIAS_SHAPES = [
    (64, 784, 128, 1),     # BASELINE config 1 (dB [784, 128], contraction 64)
    (256, 784, 512, 1),    # MLP cfg3 layers
    (256, 256, 10, 1),     # N = 10: scalar B loads, a partial column tile
    (2048, 64, 64, 1),     # dB one tile, contraction 2048: split-K, sums reduced over splits
    (33, 65, 17, 2),       # odd dims, folded batch
    (7, 13, 5, 3),
    (2048, 2048, 2048, 1),  # 256x256 warp-specialised tiles, streaming stagers
    (1000, 4096, 4096, 1),  # contraction 1000 (not whole 32-slices): the other 256x256 kernel
    (1100, 512, 1024, 1),   # 64x64 tiles over a long contraction: two wave groups (dA: K 1024,
                            # dB with column sums: K 1100 with a tail)
    (400, 256, 256, 1),     # dB with column sums over wave groups in place of split-K (K 400)
    (1, 1, 1, 1),
    (5, 0, 7, 1),          # K = 0: no dB rows, db from its own pass
    (0, 4, 6, 1),          # no rows: dB = 0, db = 0
]


@pytest.mark.parametrize("M,K,N,nb", BWD_BIAS_SHAPES)
@pytest.mark.parametrize("relu", [False, True])
def test_matmul_bwd_bias(M, K, N, nb, relu):
    """seera_hip_matmul_bwd_bias (and with a ReLU mask on dA,
    seera_hip_matmul_bwd_relu_bias): dA and dB bit-identical to
    seera_hip_matmul_bwd (_relu); db against an fp64 sum of dC over the
    Nbatch*M rows (the reference's Reductionsum, reductionKernels.cu:12-29),
    and the same bits on a second call (fixed summation order)."""
    r = np.random.default_rng(M * 3 + K * 5 + N * 7 + nb)
    a = r.standard_normal((nb, M, K)).astype(np.float32)
    b = r.standard_normal((K, N)).astype(np.float32)
    dc = r.standard_normal((nb, M, N)).astype(np.float32)
    mask = (r.uniform(0, 1, (nb, M, K)) > 0.4).astype(np.float32)
    n_a, n_b = max(a.size, 1), max(b.size, 1)
    z1 = np.zeros(1, np.float32)
    with DeviceBuffer.from_array(a if a.size else z1) as pa, \
            DeviceBuffer.from_array(b if b.size else z1) as pb, \
            DeviceBuffer.from_array(dc if dc.size else z1) as pdc, \
            DeviceBuffer.from_array(mask if mask.size else z1) as pm, \
            DeviceBuffer(n_a * 4) as pda, DeviceBuffer(n_b * 4) as pdb, \
            DeviceBuffer(n_a * 4) as pda2, DeviceBuffer(n_b * 4) as pdb2, \
            DeviceBuffer(max(N, 1) * 4) as db1, DeviceBuffer(max(N, 1) * 4) as db2:
        if relu:
            capi.call("seera_hip_matmul_bwd_relu", pa.ptr, pb.ptr, pdc.ptr, pm.ptr, pda.ptr,
                      pdb.ptr, M, N, K, nb)
        else:
            capi.call("seera_hip_matmul_bwd", pa.ptr, pb.ptr, pdc.ptr, pda.ptr, pdb.ptr, M, N, K,
                      nb)
        db1.fill(0x7F)
        for out in (db1, db2):
            if relu:
                capi.call("seera_hip_matmul_bwd_relu_bias", pa.ptr, pb.ptr, pdc.ptr, pm.ptr,
                          pda2.ptr, pdb2.ptr, out.ptr, M, N, K, nb)
            else:
                capi.call("seera_hip_matmul_bwd_bias", pa.ptr, pb.ptr, pdc.ptr, pda2.ptr,
                          pdb2.ptr, out.ptr, M, N, K, nb)
        if a.size:
            assert np.array_equal(_bits(pda2.to_array(a.shape)), _bits(pda.to_array(a.shape)))
        if b.size:
            assert np.array_equal(_bits(pdb2.to_array(b.shape)), _bits(pdb.to_array(b.shape)))
        g1, g2 = db1.to_array((N,)), db2.to_array((N,))
    assert np.array_equal(_bits(g1), _bits(g2))
    ref = dc.reshape(-1, N).astype(np.float64).sum(axis=0)
    bound = 1e-6 * np.abs(dc.reshape(-1, N)).astype(np.float64).sum(axis=0) + 1e-6
    assert np.all(np.abs(g1 - ref) <= bound), float(np.max(np.abs(g1 - ref) / bound))


def test_config1_dense_on_its_own_inputs():
    """BASELINE config 1 on the GPU with its own inputs (seed 0: X ~ N(0,1)
    [64, 784], W Kaiming-uniform(fan_in 784) [784, 128], b = 0, dY ~ N(0,1)
    [64, 128]): the fused forward, the GEMM backward and db = sum of dY over
    the batch, each against the oracle (db against an fp64 sum)."""
    import oracle
    from oracle import fp16r

    r = np.random.default_rng(0)
    M, K, N = 64, 784, 128
    x = r.standard_normal((M, K)).astype(np.float32)
    lim = np.sqrt(6.0 / K)
    w = r.uniform(-lim, lim, (K, N)).astype(np.float32)
    bias = np.zeros(N, np.float32)
    dy = r.standard_normal((M, N)).astype(np.float32)
    S = oracle.seera_cpp
    lib = load()
    with DeviceBuffer.from_array(x) as px, DeviceBuffer.from_array(w) as pw, \
            DeviceBuffer.from_array(bias) as pb, DeviceBuffer.from_array(dy) as pdy, \
            DeviceBuffer(M * N * 4) as py, DeviceBuffer(M * K * 4) as pdx, \
            DeviceBuffer(K * N * 4) as pdw, DeviceBuffer(N * 4) as pdb:
        check(lib.seera_hip_matmul_bias_act(px.ptr, pw.ptr, pb.ptr, py.ptr, None, M, N, K, 1,
                                            capi.SEERA_ACT_NONE))
        check(lib.seera_hip_matmul_bwd(px.ptr, pw.ptr, pdy.ptr, pdx.ptr, pdw.ptr, M, N, K, 1))
        check(lib.seera_hip_bias_grad(pdy.ptr, pdb.ptr, M, N))
        y, dx, dw, db = (py.to_array((M, N)), pdx.to_array((M, K)), pdw.to_array((K, N)),
                         pdb.to_array((N,)))
        # the same layer's backward with db from the dB GEMM's pass
        check(lib.seera_hip_matmul_bwd_bias(px.ptr, pw.ptr, pdy.ptr, pdx.ptr, pdw.ptr, pdb.ptr,
                                            M, N, K, 1))
        dx2, dw2, db2 = pdx.to_array((M, K)), pdw.to_array((K, N)), pdb.to_array((N,))
    assert np.array_equal(_bits(dx2), _bits(dx)) and np.array_equal(_bits(dw2), _bits(dw))
    assert_parity(db2, dy.astype(np.float64).sum(axis=0), "cfg1 db (fused)", rel=1e-6, mabs=1e-4)
    assert_parity(y, S.matmul(fp16r(x), fp16r(w)) + bias, "cfg1 Y")
    rdx, rdw = S.matmul_bwd(fp16r(x), fp16r(w), fp16r(dy))
    assert_parity(dx, rdx, "cfg1 dX")
    assert_parity(dw, rdw, "cfg1 dW")
    assert_parity(db, dy.astype(np.float64).sum(axis=0), "cfg1 db", rel=1e-6, mabs=1e-4)
