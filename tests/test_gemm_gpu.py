"""GEMM forward / backward / transpose on the GPU, through the C ABI, against
the oracle (seera_cpp restatement) on the same seeded inputs.

Inputs go to the GPU as raw fp32; the GPU rounds them to fp16 internally
(GEMM.cu:41,52). The oracle receives the fp16-rounded values, as the
north-star parity rule prescribes. Tolerance: relative Frobenius error
<= 1e-3 and max abs error <= 2e-2; results are
also held to rel_fro <= 1e-5 (fp32 summation-order noise only).
"""
import json
import os

import numpy as np
import pytest

import oracle
from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer
from oracle import fp16r
from tests.helpers import assert_parity, hip_matmul, hip_matmul_bwd, rel_fro
from tests.shapes import MATMUL

pytestmark = pytest.mark.gpu
S = oracle.seera_cpp
STRICT = 1e-5


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    assert capi.gpu_available(), "no HIP device visible"


def _golden():
    g = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "demo_matmul.json")))
    a = np.array(g["a"], np.float32).reshape(g["a_shape"])
    b = np.array(g["b"], np.float32).reshape(g["b_shape"])
    c = np.array(g["c"], np.float32).reshape(g["c_shape"])
    return g, a, b, c


def test_demo_golden_vector_bit_exact():
    """demo.ipynb cells 1-3: cuda_matmul(A[3,2,2], B[2,2]) printed outputs."""
    _, a, b, c = _golden()
    assert np.array_equal(hip_matmul(a, b), c)


def test_known_answer_2x2():
    g, *_ = _golden()
    k = g["kat_2x2"]
    got = hip_matmul(np.array(k["a"], np.float32), np.array(k["b"], np.float32))
    assert np.array_equal(got, np.array(k["c"], np.float32))


def _ties(n, rng):
    """fp32 values exactly halfway between adjacent fp16 numbers, plus
    ordinary values: exercises round-to-nearest-even."""
    h = rng.uniform(-8, 8, n).astype(np.float16)
    nxt = np.nextafter(h, np.float16(np.inf))
    mid = (h.astype(np.float32) + nxt.astype(np.float32)) / 2
    out = rng.uniform(-8, 8, n).astype(np.float32)
    out[::2] = mid[::2]
    return out


def test_identity_returns_fp16_rounding_bit_exact():
    """A @ I == fp16r(A) (Testing/test_14.py:984-991), with RNE tie cases."""
    rng = np.random.default_rng(3)
    for M, K in [(5, 5), (37, 70), (256, 256)]:
        a = _ties(M * K, rng).reshape(M, K)
        got = hip_matmul(a, np.eye(K, dtype=np.float32))
        assert np.array_equal(got, fp16r(a)), (M, K)


def _subnormals(n, rng):
    """fp16 subnormals and the fp32 values around them, as __float2half
    rounds them (GEMM.cu:41,52 keep subnormals): exact subnormals k * 2^-24,
    fp32 values that round into [2^-24, 2^-14), ties between subnormals,
    values that round to 0 (below 2^-25, and 2^-25 itself: a tie to even),
    values just below 2^-14 that round up to the smallest normal, and
    ordinary values, all with random signs."""
    t = 2.0 ** -24
    k = rng.integers(1, 1024, n)
    parts = [
        k * t,                                                    # exact subnormals
        np.exp2(rng.uniform(-25, -14, n)),                        # round into the range
        (k + 0.5) * t,                                            # ties
        rng.uniform(0, 2.0 ** -25, n),                            # round to 0
        np.full(n, 2.0 ** -25),                                   # tie to 0
        2.0 ** -14 - rng.uniform(0, 2.0 ** -26, n),               # round up to 2^-14
        rng.uniform(-1, 1, n),                                    # ordinary
    ]
    v = np.stack(parts, 1).reshape(-1)[:n] * rng.choice([-1.0, 1.0], n)
    return v.astype(np.float32)


def test_subnormal_fp16_operands_kept_bit_exact():
    """fp16 subnormal operands pass through the in-kernel rounding and the
    MFMAs unflushed: A @ I == fp16r(A) and I @ B == fp16r(B) bit for bit, on
    shapes that take the 64x64, 128x128 and 256x256 tile kernels."""
    rng = np.random.default_rng(24)
    for M, K in [(37, 70), (256, 256), (2048, 2048), (4096, 4096)]:
        a = _subnormals(M * K, rng).reshape(M, K)
        assert np.count_nonzero(np.abs(fp16r(a)) < 2.0 ** -14) > M * K // 4
        eye = np.eye(K, dtype=np.float32)
        got = hip_matmul(a, eye)
        assert np.array_equal(got, fp16r(a)), ("A@I", M, K)
        got = hip_matmul(np.eye(M, dtype=np.float32), a)
        assert np.array_equal(got, fp16r(a)), ("I@B", M, K)


def test_subnormal_fp16_operands_backward_bit_exact():
    """The transposed-operand stagers of the backward keep subnormals too:
    with A = B = I, dA = dC @ I^T and dB = I^T @ dC both equal fp16r(dC)."""
    rng = np.random.default_rng(25)
    for n in (70, 256, 2048):
        dc = _subnormals(n * n, rng).reshape(n, n)
        eye = np.eye(n, dtype=np.float32)
        da, db = hip_matmul_bwd(eye, eye, dc)
        assert np.array_equal(da, fp16r(dc)), ("dA", n)
        assert np.array_equal(db, fp16r(dc)), ("dB", n)


def test_fp16_overflow_saturates_like_float2half():
    a = np.array([[65519.0, 65520.0, -70000.0]], np.float32)
    got = hip_matmul(a.reshape(3, 1, 1), np.ones((1, 1), np.float32)).reshape(-1)
    assert got[0] == 65504.0 and got[1] == np.inf and got[2] == -np.inf


@pytest.mark.parametrize("M,K,N,nb", MATMUL)
def test_matmul_parity(M, K, N, nb):
    r = np.random.default_rng(M * 7919 + K * 31 + N)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    got = hip_matmul(a, b)
    ref = S.matmul_batched(fp16r(a), fp16r(b))
    assert_parity(got, ref, f"fwd {M}x{K}x{N}x{nb}")
    assert rel_fro(got, ref) <= STRICT


@pytest.mark.parametrize("M,K,N,nb", MATMUL)
def test_matmul_bwd_parity(M, K, N, nb):
    r = np.random.default_rng(M * 104729 + K * 37 + N)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    dc = r.uniform(-1, 1, (nb, M, N)).astype(np.float32)
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(fp16r(a), fp16r(b), fp16r(dc))
    assert_parity(da, rda, "dA")
    assert_parity(db, rdb, "dB")
    assert rel_fro(da, rda) <= STRICT and rel_fro(db, rdb) <= STRICT


# Large GEMMs whose operands are not vector-aligned, or whose K is not a
# whole number of 32-deep slices, run on zero-padded staging copies of both
# operands (odd everything; aligned with K % 32 != 0; a folded batch).
PADDED = [(2049, 2047, 1025, 1), (1024, 4100, 1024, 1), (700, 2051, 1001, 3)]


@pytest.mark.parametrize("M,K,N,nb", PADDED)
def test_padded_large_gemm_parity(M, K, N, nb):
    r = np.random.default_rng(M + 3 * K + 7 * N + nb)
    a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    dc = r.uniform(-1, 1, (nb, M, N)).astype(np.float32)
    got = hip_matmul(a, b)
    ref = S.matmul_batched(fp16r(a), fp16r(b))
    assert_parity(got, ref, f"fwd {M}x{K}x{N}x{nb}")
    assert rel_fro(got, ref) <= STRICT
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(fp16r(a), fp16r(b), fp16r(dc))
    assert_parity(da, rda, "dA")
    assert_parity(db, rdb, "dB")
    assert rel_fro(da, rda) <= STRICT and rel_fro(db, rdb) <= STRICT


def test_padded_gemm_identity_bit_exact():
    """The zero-padded copies add only zero products: A @ I and I @ A return
    fp16r(A) bit for bit on a 2049 x 2047 operand."""
    r = np.random.default_rng(2049)
    a = r.uniform(-8, 8, (2049, 2047)).astype(np.float32)
    assert np.array_equal(hip_matmul(a, np.eye(2047, dtype=np.float32)), fp16r(a))
    assert np.array_equal(hip_matmul(np.eye(2049, dtype=np.float32), a), fp16r(a))


def test_matmul_2d_and_3d_entry_agree():
    """cuTen passes Nbatch=1 for 2-D A (cuTen.py:423-445)."""
    r = np.random.default_rng(5)
    a = r.uniform(-1, 1, (4, 24, 40)).astype(np.float32)
    b = r.uniform(-1, 1, (40, 12)).astype(np.float32)
    full = hip_matmul(a, b)
    for i in range(4):
        assert np.array_equal(hip_matmul(a[i], b), full[i])


@pytest.mark.parametrize("n", [1024, 2048, 4096])
def test_square_sweep_config2(n):
    """A, B, dC ~ U[-1,1] rounded to fp16, seed = n."""
    r = np.random.default_rng(n)
    a = fp16r(r.uniform(-1, 1, (n, n)))
    b = fp16r(r.uniform(-1, 1, (n, n)))
    dc = fp16r(r.uniform(-1, 1, (n, n)))
    got = hip_matmul(a, b)
    assert_parity(got, S.matmul(a, b), f"C n={n}")
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(a, b, dc)
    assert_parity(da, rda, f"dA n={n}")
    assert_parity(db, rdb, f"dB n={n}")
    # <A.B, dC> = <A, dA> = <B, dB> in fp64 on the GPU outputs
    ref = float(np.sum(got.astype(np.float64) * dc))
    for x, g in ((a, da), (b, db)):
        assert abs(float(np.sum(x.astype(np.float64) * g)) - ref) <= 1e-4 * abs(ref) + 1e-2


@pytest.mark.parametrize("M,K,N,nb", [(4000, 4096, 3900, 1), (2000, 4128, 4000, 2),
                                      (4096, 4100, 4096, 1)])
def test_large_tile_edges(M, K, N, nb):
    """256x256 tiles with partial edge tiles (M, N not multiples of 256); K a
    multiple of 32 (streaming producers) and not (register-staged producers);
    dB contracts over Nbatch*M."""
    r = np.random.default_rng(M + 3 * K + 7 * N)
    a = fp16r(r.uniform(-1, 1, (nb, M, K)))
    b = fp16r(r.uniform(-1, 1, (K, N)))
    dc = fp16r(r.uniform(-1, 1, (nb, M, N)))
    got = hip_matmul(a, b)
    assert_parity(got, S.matmul_batched(a, b), f"C {M}x{K}x{N}x{nb}")
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(a, b, dc)
    assert_parity(da, rda, "dA")
    assert_parity(db, rdb, "dB")


def test_square_8192_sampled_rows():
    """n = 8192: 64 sampled rows of C, dA and columns of dB against fp64."""
    n = 8192
    r = np.random.default_rng(n)
    a = fp16r(r.uniform(-1, 1, (n, n)))
    b = fp16r(r.uniform(-1, 1, (n, n)))
    dc = fp16r(r.uniform(-1, 1, (n, n)))
    got = hip_matmul(a, b)
    rows = np.sort(r.choice(n, 64, replace=False))
    assert_parity(got[rows], a[rows].astype(np.float64) @ b, "C rows")
    da, db = hip_matmul_bwd(a, b, dc)
    assert_parity(da[rows], dc[rows].astype(np.float64) @ b.T, "dA rows")
    cols = rows
    assert_parity(db[:, cols], a.T.astype(np.float64) @ dc[:, cols], "dB cols")


@pytest.mark.parametrize("rows,cols", [(1, 1), (3, 5), (64, 64), (65, 127), (1000, 3), (513, 2049),
                                       (4, 8), (1000, 12), (256, 4100), (4096, 4096)])
def test_transpose_2d_bit_exact(rows, cols):
    a = np.random.default_rng(rows + cols).standard_normal((rows, cols)).astype(np.float32)
    with DeviceBuffer.from_array(a) as pi, DeviceBuffer(a.nbytes) as po:
        capi.call("seera_hip_transpose_2d", pi.ptr, po.ptr, rows, cols)
        assert np.array_equal(po.to_array((cols, rows)), a.T)


@pytest.mark.parametrize("nb,M,K", [(1, 7, 9), (3, 64, 65), (5, 130, 33), (2, 128, 260), (3, 68, 4)])
def test_transpose_3d_bit_exact(nb, M, K):
    a = np.random.default_rng(M * K).standard_normal((nb, M, K)).astype(np.float32)
    with DeviceBuffer.from_array(a) as pi, DeviceBuffer(a.nbytes) as po:
        capi.call("seera_hip_transpose_3d", pi.ptr, po.ptr, nb, M, K)
        assert np.array_equal(po.to_array((nb, K, M)), a.transpose(0, 2, 1))


def test_zero_sized_and_empty_contraction():
    """M or N = 0 writes nothing; K = 0 gives C = 0 (the K loop never runs)."""
    with DeviceBuffer(64) as c:
        c.fill(0xFF)
        capi.call("seera_hip_matmul", c.ptr, c.ptr, c.ptr, 0, 4, 4, 1)
        assert np.all(np.isnan(c.to_array((16,))))
        capi.call("seera_hip_matmul", c.ptr, c.ptr, c.ptr, 2, 8, 0, 1)
        assert np.array_equal(c.to_array((16,)), np.zeros(16, np.float32))


def _softmax_ce_grad(logits, labels):
    z = logits - logits.max(1, keepdims=True)
    p = np.exp(z)
    p /= p.sum(1, keepdims=True)
    p[np.arange(len(labels)), labels] -= 1.0
    return (p / len(labels)).astype(np.float32)


def test_mlp_config3_fwd_bwd():
    """MLP 784->512->256->10, batch 256, ReLU, softmax-CE.
    The nine GEMMs run on the GPU; bias, ReLU and the loss gradient on the
    host. Each GPU GEMM output is compared with the oracle on the same
    (fp16-rounded) operands."""
    r = np.random.default_rng(0)
    x = r.uniform(0, 1, (256, 784)).astype(np.float32)
    dims = [784, 512, 256, 10]
    ws = [r.uniform(-np.sqrt(6 / i), np.sqrt(6 / i), (i, o)).astype(np.float32)
          for i, o in zip(dims[:-1], dims[1:])]
    labels = r.integers(0, 10, 256)
    acts, h = [x], x
    for li, w in enumerate(ws):
        z = hip_matmul(h, w)
        assert_parity(z, S.matmul(fp16r(h), fp16r(w)), f"fwd layer {li}")
        h = np.maximum(z, 0) if li < 2 else z
        acts.append(h)
    g = _softmax_ce_grad(acts[-1], labels)
    for li in (2, 1, 0):
        da, dw = hip_matmul_bwd(acts[li], ws[li], g)
        rda, rdw = S.matmul_bwd(fp16r(acts[li]), fp16r(ws[li]), fp16r(g))
        assert_parity(da, rda, f"dA layer {li}")
        assert_parity(dw, rdw, f"dW layer {li}")
        g = da * (acts[li] > 0)


@pytest.mark.parametrize("M,K,N,nb", [(5, 65536, 7, 1), (3, 40, 5, 4000), (1, 4096, 1, 1),
                                      (300, 1, 200, 1), (2, 3000, 3000, 1), (3000, 8, 2, 3)])
def test_extreme_aspect_ratios(M, K, N, nb):
    """Long contractions with tiny outputs (split-K), many tiny batches (dB
    contracts over Nbatch*M = 12000), K = 1, and skinny panels."""
    r = np.random.default_rng(M + 7 * K + 13 * N + nb)
    a = fp16r(r.uniform(-1, 1, (nb, M, K)))
    b = fp16r(r.uniform(-1, 1, (K, N)))
    dc = fp16r(r.uniform(-1, 1, (nb, M, N)))
    got = hip_matmul(a, b)
    assert_parity(got, S.matmul_batched(a, b), f"C {M}x{K}x{N}x{nb}")
    da, db = hip_matmul_bwd(a, b, dc)
    rda, rdb = S.matmul_bwd(a, b, dc)
    assert_parity(da, rda, "dA")
    assert_parity(db, rdb, "dB")


@pytest.mark.parametrize("rows,cols", [(5_000_000, 2), (2, 5_000_000), (4_194_305, 3)])
def test_transpose_2d_beyond_grid_limit(rows, cols):
    """Row tiles beyond the 65535 grid-y limit (the reference's 1-D grid
    accepts any count: GEMM.cu:229-235)."""
    a = np.random.default_rng(rows).standard_normal((rows, cols)).astype(np.float32)
    with DeviceBuffer.from_array(a) as pi, DeviceBuffer(a.nbytes) as po:
        capi.call("seera_hip_transpose_2d", pi.ptr, po.ptr, rows, cols)
        assert np.array_equal(po.to_array((cols, rows)), a.T)


def test_transpose_3d_many_slices():
    """More slices than the 65535 grid-z limit."""
    a = np.random.default_rng(9).standard_normal((70_000, 3, 2)).astype(np.float32)
    with DeviceBuffer.from_array(a) as pi, DeviceBuffer(a.nbytes) as po:
        capi.call("seera_hip_transpose_3d", pi.ptr, po.ptr, 70_000, 3, 2)
        assert np.array_equal(po.to_array((70_000, 2, 3)), a.transpose(0, 2, 1))
