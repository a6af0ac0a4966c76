"""Pins the oracle (CPU only).

Chain of evidence:
  * the reference's stored GEMM outputs (demo.ipynb) and its known answers
    (test_14.py 2x2 KAT, A@I == A) are reproduced bit for bit;
  * the C restatement of seera_cpp agrees with fp64 closed forms written tap
    by tap (no im2col) over the reference's own test shapes;
  * the closed forms agree with an independent implementation (PyTorch CPU,
    float64, autograd for the gradients) and with brute-force loops;
  * adjoint identities tie forward and backward together;
  * plausible mistakes planted in the oracle maths fail these checks.
"""
import json
import zlib
import os

import numpy as np
import pytest

import oracle
from oracle import closed_form as cf
from oracle import fp16r
from tests.shapes import CONV2D, CONV2D_EDGE, CONVT, MATMUL

S = oracle.seera_cpp
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "demo_matmul.json")


def _rng(seed):
    return np.random.default_rng(seed)


def _close(a, b, rtol=2e-5):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    scale = max(1.0, float(np.max(np.abs(b))) if b.size else 1.0)
    return float(np.max(np.abs(a - b))) <= rtol * scale if a.size else True


# ---------------------------------------------------------------- golden ---

def _golden():
    g = json.load(open(GOLDEN))
    a = np.array(g["a"], np.float32).reshape(g["a_shape"])
    b = np.array(g["b"], np.float32).reshape(g["b_shape"])
    c = np.array(g["c"], np.float32).reshape(g["c_shape"])
    return g, a, b, c


def test_demo_golden_vector_bit_exact():
    """demo.ipynb cells 1-3: printed a@b == fp32 GEMM of fp16-rounded operands."""
    _, a, b, c = _golden()
    got = S.matmul_batched(fp16r(a), fp16r(b))
    assert np.array_equal(got, c)
    assert np.array_equal(cf.gemm(fp16r(a), fp16r(b)).astype(np.float32), c)


def test_demo_golden_vector_requires_fp16_operands():
    """Without the fp16 operand rounding the stored outputs are NOT reproduced."""
    _, a, b, c = _golden()
    assert not np.array_equal(S.matmul_batched(a, b), c)
    assert abs(float(S.matmul_batched(a, b)[0, 0, 0]) - 0.47265625) > 1e-4


def test_known_answer_2x2():
    g, *_ = _golden()
    k = g["kat_2x2"]
    got = S.matmul(np.array(k["a"], np.float32), np.array(k["b"], np.float32))
    assert np.array_equal(got, np.array(k["c"], np.float32))


def test_identity_is_exact():
    a = fp16r(_rng(1).standard_normal((5, 5)))
    assert np.array_equal(S.matmul(a, np.eye(5, dtype=np.float32)), a)


# ------------------------------------------------- C oracle vs closed form ---

@pytest.mark.parametrize("M,K,N,nb", MATMUL)
def test_oracle_gemm_matches_closed_form(M, K, N, nb):
    r = _rng(M * 1000 + K * 10 + N)
    a = fp16r(r.uniform(-1, 1, (nb, M, K)))
    b = fp16r(r.uniform(-1, 1, (K, N)))
    dc = fp16r(r.uniform(-1, 1, (nb, M, N)))
    assert _close(S.matmul_batched(a, b), cf.gemm(a, b))
    da, db = S.matmul_bwd(a, b, dc)
    da2, db2 = cf.gemm_bwd(a, b, dc)
    assert _close(da, da2) and _close(db, db2)


@pytest.mark.parametrize("case", CONV2D + CONV2D_EDGE, ids=[c[0] for c in CONV2D + CONV2D_EDGE])
def test_oracle_conv2d_matches_closed_form(case):
    name, N, C, H, W, F, KH, KW, s, p = case
    r = _rng(zlib.crc32(name.encode()))
    x = fp16r(r.standard_normal((N, C, H, W)))
    w = fp16r(r.standard_normal((F, C, KH, KW)) * 0.2)
    y = S.conv2d_forward(x, w, s, s, p, p)
    assert _close(y, cf.conv2d_fwd(x, w, s, s, p, p))
    dy = fp16r(r.standard_normal(y.shape))
    dx, dw = S.conv2d_backward(dy, x, w, s, s, p, p)
    dx2, dw2 = cf.conv2d_bwd(dy, x, w, s, s, p, p)
    assert _close(dx, dx2) and _close(dw, dw2)


@pytest.mark.parametrize("case", CONVT, ids=[c[0] for c in CONVT])
def test_oracle_convT_matches_closed_form(case):
    name, N, Cin, H, W, Cout, KH, KW, s, p = case
    r = _rng(zlib.crc32(name.encode()))
    x = fp16r(r.standard_normal((N, Cin, H, W)))
    w = fp16r(r.standard_normal((Cin, Cout, KH, KW)) * 0.2)
    y = S.conv_transpose2d_forward(x, w, s, s, p, p)
    assert _close(y, cf.conv_transpose2d_fwd(x, w, s, s, p, p))
    dy = fp16r(r.standard_normal(y.shape))
    dx, dw = S.conv_transpose2d_backward(dy, x, w, s, s, p, p)
    dx2, dw2 = cf.conv_transpose2d_bwd(dy, x, w, s, s, p, p)
    assert _close(dx, dx2) and _close(dw, dw2)


def test_oracle_plain_sgemm_matches_openblas():
    """The fallback C sgemm and OpenBLAS give the same products."""
    lib = oracle.load()
    r = _rng(7)
    x = r.standard_normal((3, 5, 9, 7)).astype(np.float32)
    w = r.standard_normal((4, 5, 3, 3)).astype(np.float32)
    y_blas = S.conv2d_forward(x, w, 2, 2, 1, 1)
    dy = r.standard_normal(y_blas.shape).astype(np.float32)
    g_blas = S.conv2d_backward(dy, x, w, 2, 2, 1, 1)
    lib.oracle_init(None, 0)
    try:
        y_plain = S.conv2d_forward(x, w, 2, 2, 1, 1)
        g_plain = S.conv2d_backward(dy, x, w, 2, 2, 1, 1)
    finally:
        oracle._backend = None
        oracle.load()
    assert _close(y_plain, y_blas)
    assert _close(g_plain[0], g_blas[0]) and _close(g_plain[1], g_blas[1])


def test_dense_layer_config1():
    """Dense 64x784x128 fwd+bwd in fp32 on the CPU path."""
    r = np.random.default_rng(0)
    X = r.standard_normal((64, 784)).astype(np.float32)
    lim = np.sqrt(6.0 / 784)
    W = r.uniform(-lim, lim, (784, 128)).astype(np.float32)
    b = np.zeros(128, np.float32)
    dY = r.standard_normal((64, 128)).astype(np.float32)
    Y = S.matmul(X, W) + b
    dX, dW = S.matmul_bwd(X, W, dY)
    assert _close(Y, X.astype(np.float64) @ W)
    assert _close(dW, X.T.astype(np.float64) @ dY)
    assert _close(dX, dY.astype(np.float64) @ W.T)


# --------------------------------------- closed forms vs independent checks ---

torch = pytest.importorskip("torch")
F = torch.nn.functional


def _t(a):
    return torch.tensor(np.asarray(a, np.float64), requires_grad=True)


@pytest.mark.parametrize("case", CONV2D[:29:4], ids=[c[0] for c in CONV2D[:29:4]])
def test_closed_form_conv2d_vs_torch(case):
    name, N, C, H, W, Fo, KH, KW, s, p = case
    r = _rng(11)
    x = r.standard_normal((N, C, H, W))
    w = r.standard_normal((Fo, C, KH, KW))
    tx, tw = _t(x), _t(w)
    ty = F.conv2d(tx, tw, stride=s, padding=p)
    dy = r.standard_normal(tuple(ty.shape))
    (ty * torch.tensor(dy)).sum().backward()
    assert _close(cf.conv2d_fwd(x, w, s, s, p, p), ty.detach().numpy(), 1e-12)
    dx, dw = cf.conv2d_bwd(dy, x, w, s, s, p, p)
    assert _close(dx, tx.grad.numpy(), 1e-12) and _close(dw, tw.grad.numpy(), 1e-12)


@pytest.mark.parametrize("case", CONVT[:19:3], ids=[c[0] for c in CONVT[:19:3]])
def test_closed_form_convT_vs_torch(case):
    name, N, Cin, H, W, Cout, KH, KW, s, p = case
    r = _rng(12)
    x = r.standard_normal((N, Cin, H, W))
    w = r.standard_normal((Cin, Cout, KH, KW))
    tx, tw = _t(x), _t(w)
    ty = F.conv_transpose2d(tx, tw, stride=s, padding=p)
    dy = r.standard_normal(tuple(ty.shape))
    (ty * torch.tensor(dy)).sum().backward()
    assert _close(cf.conv_transpose2d_fwd(x, w, s, s, p, p), ty.detach().numpy(), 1e-12)
    dx, dw = cf.conv_transpose2d_bwd(dy, x, w, s, s, p, p)
    assert _close(dx, tx.grad.numpy(), 1e-12) and _close(dw, tw.grad.numpy(), 1e-12)


def _brute_conv(x, w, s, p):
    N, C, H, W = x.shape
    Fo, _, R, Sk = w.shape
    OH, OW = (H + 2 * p - R) // s + 1, (W + 2 * p - Sk) // s + 1
    y = np.zeros((N, Fo, OH, OW))
    for n in range(N):
        for f in range(Fo):
            for i in range(OH):
                for j in range(OW):
                    acc = 0.0
                    for c in range(C):
                        for r in range(R):
                            for q in range(Sk):
                                h, ww = i * s - p + r, j * s - p + q
                                if 0 <= h < H and 0 <= ww < W:
                                    acc += w[f, c, r, q] * x[n, c, h, ww]
                    y[n, f, i, j] = acc
    return y


def _brute_convT(x, w, s, p):
    N, Cin, H, W = x.shape
    _, Cout, KH, KW = w.shape
    OH, OW = (H - 1) * s - 2 * p + KH, (W - 1) * s - 2 * p + KW
    y = np.zeros((N, Cout, OH, OW))
    for n in range(N):
        for ci in range(Cin):
            for i in range(H):
                for j in range(W):
                    for co in range(Cout):
                        for kh in range(KH):
                            for kw in range(KW):
                                oh, ow = i * s - p + kh, j * s - p + kw
                                if 0 <= oh < OH and 0 <= ow < OW:
                                    y[n, co, oh, ow] += x[n, ci, i, j] * w[ci, co, kh, kw]
    return y


@pytest.mark.parametrize("s,p,k", [(1, 0, 3), (2, 1, 3), (3, 2, 2), (2, 1, 4)])
def test_closed_forms_vs_brute_force(s, p, k):
    r = _rng(13)
    x = r.standard_normal((2, 2, 6, 5))
    w = r.standard_normal((3, 2, k, k))
    assert _close(cf.conv2d_fwd(x, w, s, s, p, p), _brute_conv(x, w, s, p), 1e-12)
    wt = r.standard_normal((2, 3, k, k))
    assert _close(cf.conv_transpose2d_fwd(x, wt, s, s, p, p), _brute_convT(x, wt, s, p), 1e-12)


def _inner(a, b):
    return float(np.sum(np.asarray(a, np.float64) * np.asarray(b, np.float64)))


@pytest.mark.parametrize("s,p", [(1, 1), (2, 1), (3, 0)])
def test_adjoint_identities(s, p):
    """<conv(X,W), dY> = <X, dX> = <W, dW>, and the same for convT / GEMM."""
    r = _rng(14)
    x = fp16r(r.standard_normal((3, 4, 11, 9)))
    w = fp16r(r.standard_normal((5, 4, 3, 3)))
    y = S.conv2d_forward(x, w, s, s, p, p)
    dy = fp16r(r.standard_normal(y.shape))
    dx, dw = S.conv2d_backward(dy, x, w, s, s, p, p)
    ref = _inner(y, dy)
    assert abs(_inner(x, dx) - ref) <= 1e-4 * abs(ref) + 1e-3
    assert abs(_inner(w, dw) - ref) <= 1e-4 * abs(ref) + 1e-3
    wt = fp16r(r.standard_normal((4, 5, 3, 3)))
    yt = S.conv_transpose2d_forward(x, wt, s, s, p, p)
    dyt = fp16r(r.standard_normal(yt.shape))
    dxt, dwt = S.conv_transpose2d_backward(dyt, x, wt, s, s, p, p)
    ref = _inner(yt, dyt)
    assert abs(_inner(x, dxt) - ref) <= 1e-4 * abs(ref) + 1e-3
    assert abs(_inner(wt, dwt) - ref) <= 1e-4 * abs(ref) + 1e-3
    a = fp16r(r.uniform(-1, 1, (2, 7, 5)))
    b = fp16r(r.uniform(-1, 1, (5, 6)))
    dc = fp16r(r.uniform(-1, 1, (2, 7, 6)))
    da, db = S.matmul_bwd(a, b, dc)
    ref = _inner(S.matmul_batched(a, b), dc)
    assert abs(_inner(a, da) - ref) <= 1e-5 * abs(ref) + 1e-4
    assert abs(_inner(b, db) - ref) <= 1e-5 * abs(ref) + 1e-4


def test_finite_differences_conv():
    """Testing/test_1.py:1291-1344: central differences, EPS 1e-3, ATOL 2e-2."""
    r = np.random.RandomState(99)
    x = r.standard_normal((1, 2, 5, 5))
    w = r.standard_normal((2, 2, 3, 3))
    dy = r.standard_normal((1, 2, 3, 3))
    dx, dw = cf.conv2d_bwd(dy, x, w, 2, 2, 1, 1)
    eps = 1e-3
    for arr, grad in ((x, dx), (w, dw)):
        flat = arr.reshape(-1)
        for i in range(0, flat.size, 7):
            old = flat[i]
            flat[i] = old + eps
            up = _inner(cf.conv2d_fwd(x, w, 2, 2, 1, 1), dy)
            flat[i] = old - eps
            dn = _inner(cf.conv2d_fwd(x, w, 2, 2, 1, 1), dy)
            flat[i] = old
            assert abs((up - dn) / (2 * eps) - grad.reshape(-1)[i]) < 2e-2


# ------------------------------------------------------ planted mistakes ---

def test_planted_mistakes_fail_the_checks():
    """Plausible oracle mistakes must be rejected by the checks above."""
    r = _rng(15)
    x = r.standard_normal((2, 3, 8, 7))
    w = r.standard_normal((4, 3, 3, 3))
    ty = F.conv2d(torch.tensor(x), torch.tensor(w), stride=2, padding=1).numpy()
    # (1) true convolution (flipped kernel) instead of cross-correlation
    assert not _close(cf.conv2d_fwd(x, w[:, :, ::-1, ::-1], 2, 2, 1, 1), ty, 1e-6)
    # (2) stride and padding swapped (the reference's argument-order trap)
    assert not np.array_equal(cf.conv2d_fwd(x, w, 1, 1, 2, 2).shape, ty.shape) or \
        not _close(cf.conv2d_fwd(x, w, 1, 1, 2, 2), ty, 1e-6)
    # (3) ConvTranspose weight read as [Cout, Cin] instead of [Cin, Cout]
    wt = r.standard_normal((3, 3, 4, 4))
    tt = F.conv_transpose2d(torch.tensor(x), torch.tensor(wt), stride=2, padding=1).numpy()
    assert not _close(cf.conv_transpose2d_fwd(x, wt.transpose(1, 0, 2, 3), 2, 2, 1, 1), tt, 1e-6)
    # (4) dB without the batch sum (last slice only) breaks the adjoint identity
    a = r.uniform(-1, 1, (3, 4, 5))
    b = r.uniform(-1, 1, (5, 2))
    dc = r.uniform(-1, 1, (3, 4, 2))
    ref = _inner(a @ b, dc)
    assert abs(_inner(b, a[-1].T @ dc[-1]) - ref) > 1e-3
    # (5) operands kept in fp32 (no fp16 rounding) miss the stored golden vector
    _, ga, gb, gc = _golden()
    assert not np.array_equal((ga.astype(np.float64) @ gb).astype(np.float32), gc)
