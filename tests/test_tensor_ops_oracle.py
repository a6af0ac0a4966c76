"""Pins oracle/tensor_ops.py (the NumPy restatement of the reference's
element-wise, activation, softmax, broadcast, unpooling and reduction
kernels) on the CPU:

* against torch's CPU operators and autograd (an independent implementation
  of the same mathematics: values, and the local gradients / backward rules);
* against closed forms for the cases the reference fixes by its own order
  (ties in argmax / argmin / max backward, sums in index order, ReLU / abs /
  clip at their kinks);
* against brute-force scalar loops on tiny inputs (axis and index mapping);
* by planted mistakes that these checks must reject.
"""
import numpy as np
import pytest
import torch

from oracle import tensor_ops as T

f32 = np.float32
R = np.random.default_rng(7)


def _t(x):
    return torch.from_numpy(np.array(x, dtype=np.float64))


def _grad_of(fn, x):
    xt = _t(x).requires_grad_(True)
    fn(xt).sum().backward()
    return xt.grad.numpy()


KINKS = np.array([-2.0, -1.0, -0.5, 0.0, 0.5, 1.0, 2.0], f32)


@pytest.mark.parametrize("kind,tfn,dom", [
    ("relu", torch.relu, "any"),
    ("sigmoid", torch.sigmoid, "any"),
    ("tanh", torch.tanh, "any"),
    ("log", torch.log, "pos"),
    ("exp", torch.exp, "any"),
    ("abs", torch.abs, "any"),
    ("sqrt", torch.sqrt, "pos"),
])
def test_activation_values_and_local_grads(kind, tfn, dom):
    x = R.standard_normal(4099).astype(f32) * 3
    if dom == "pos":
        x = np.abs(x) + f32(0.05)
    else:
        x = np.concatenate([x, KINKS])
    out, grad = T.activation(kind, x)
    np.testing.assert_allclose(out, tfn(_t(x)).numpy(), rtol=3e-6, atol=1e-7)
    np.testing.assert_allclose(grad, _grad_of(tfn, x), rtol=2e-5, atol=1e-6)
    assert out.dtype == f32 and grad.dtype == f32


def test_activation_kinks_follow_the_reference():
    """At 0: relu grad 0 (x > 0), abs grad 0 (sign), clip bounds inclusive."""
    out, g = T.activation("relu", KINKS)
    assert g[3] == 0 and out[3] == 0 and np.all(g[4:] == 1) and np.all(g[:3] == 0)
    _, g = T.activation("abs", KINKS)
    assert list(g) == [-1, -1, -1, 0, 1, 1, 1]
    out, g = T.activation("clip", KINKS, -1.0, 1.0)
    assert list(out) == [-1, -1, -0.5, 0, 0.5, 1, 1]
    assert list(g) == [0, 1, 1, 1, 1, 1, 0]
    # sqrt grad carries the +1e-12 of activations.cu:65 (finite at 0)
    _, g = T.activation("sqrt", np.array([0.0, 4.0], f32))
    assert g[0] == f32(0.5) / f32(1e-12) and g[1] == f32(0.25)


@pytest.mark.parametrize("p", [2.0, 3.0, 0.5, -1.5])
def test_activation_pow_and_clip(p):
    x = np.abs(R.standard_normal(1000).astype(f32)) + f32(0.1)
    out, grad = T.activation("pow", x, p)
    np.testing.assert_allclose(out, torch.pow(_t(x), p).numpy(), rtol=3e-6)
    np.testing.assert_allclose(grad, _grad_of(lambda t: torch.pow(t, p), x), rtol=3e-5)
    out, grad = T.activation("clip", x - 1, -0.3, 0.7)
    np.testing.assert_array_equal(out, np.clip(x - 1, f32(-0.3), f32(0.7)))
    np.testing.assert_allclose(grad, _grad_of(lambda t: torch.clamp(t, -0.3, 0.7), x - 1))


@pytest.mark.parametrize("shape", [(1, 1), (3, 10), (64, 10), (5, 257), (2, 1000)])
def test_softmax_and_vjp_against_torch(shape):
    x = R.standard_normal(shape).astype(f32) * 4
    s = T.softmax(x)
    np.testing.assert_allclose(s, torch.softmax(_t(x), 1).numpy(), rtol=2e-6, atol=1e-8)
    d = R.standard_normal(shape).astype(f32)
    xt = _t(x).requires_grad_(True)
    torch.softmax(xt, 1).backward(_t(d))
    np.testing.assert_allclose(T.softmax_vjp(s, d), xt.grad.numpy(), rtol=2e-4, atol=2e-6)


def test_softmax_is_shift_invariant_and_sums_to_one():
    x = R.standard_normal((7, 33)).astype(f32)
    np.testing.assert_allclose(T.softmax(x).sum(1), 1.0, rtol=1e-6)
    np.testing.assert_allclose(T.softmax(x + f32(50)), T.softmax(x), rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("op,fn", [("add", np.add), ("sub", np.subtract), ("mul", np.multiply),
                                   ("div", np.divide)])
def test_elementwise_and_scalar(op, fn):
    a = R.standard_normal(1001).astype(f32)
    b = R.standard_normal(1001).astype(f32) + f32(3)
    np.testing.assert_array_equal(T.elementwise(op, a, b),
                                  torch_ops(op, torch.from_numpy(a), torch.from_numpy(b)).numpy())


def torch_ops(op, a, b):
    return {"add": torch.add, "sub": torch.sub, "mul": torch.mul, "div": torch.div}[op](a, b)


def test_scalar_inplace_against_torch():
    a = np.abs(R.standard_normal(513).astype(f32)) + f32(0.1)
    ta = torch.from_numpy(a)
    np.testing.assert_array_equal(T.scalar_inplace("mul", a, -1.5), (ta * -1.5).numpy())
    np.testing.assert_array_equal(T.scalar_inplace("add", a, 0.25), (ta + 0.25).numpy())
    np.testing.assert_allclose(T.scalar_inplace("pow", a, 2.5), torch.pow(ta, 2.5).numpy(),
                               rtol=3e-7)


BCAST = [((2, 3, 4, 5), (1, 3, 1, 1)), ((1, 1, 64, 128), (1, 1, 1, 128)),
         ((2, 1, 4, 1), (1, 3, 1, 5)), ((1, 1, 1, 1), (2, 3, 4, 5)), ((2, 3, 4, 5), (2, 3, 4, 5))]


@pytest.mark.parametrize("a4,b4", BCAST)
@pytest.mark.parametrize("op", ["add", "mul"])
def test_broadcast_against_numpy(a4, b4, op):
    a = R.standard_normal(a4).astype(f32)
    b = R.standard_normal(b4).astype(f32)
    want = a + b if op == "add" else a * b
    np.testing.assert_array_equal(T.broadcast_4d(op, a, b, a4, b4), want)


def test_broadcast_rejects_mismatch():
    assert T.broadcast_shape((2, 3, 4, 5), (1, 2, 1, 1)) is None
    with pytest.raises(ValueError):
        T.broadcast_4d("add", np.zeros((2, 3, 4, 5)), np.zeros((1, 2, 1, 1)), (2, 3, 4, 5),
                       (1, 2, 1, 1))


@pytest.mark.parametrize("sh,sw", [(2, 2), (1, 3), (3, 2)])
def test_unpool_against_torch(sh, sw):
    x = R.standard_normal((2, 3, 5, 4)).astype(f32)
    out = T.unpool_fwd(x, sh, sw)
    up = torch.nn.functional.interpolate(_t(x), scale_factor=(sh, sw), mode="nearest")
    np.testing.assert_array_equal(out, up.numpy().astype(f32))
    d = R.standard_normal(out.shape).astype(f32)
    xt = _t(x).requires_grad_(True)
    torch.nn.functional.interpolate(xt, scale_factor=(sh, sw), mode="nearest").backward(_t(d))
    np.testing.assert_allclose(T.unpool_bwd(d, sh, sw), xt.grad.numpy(), rtol=1e-6, atol=1e-6)


def test_unpool_bwd_adds_row_by_row_from_zero():
    """Brute force: the scalar float32 loop of unpooling.cu:38-47."""
    d = R.standard_normal((1, 2, 6, 9)).astype(f32)
    got = T.unpool_bwd(d, 3, 3)
    for c in range(2):
        for h in range(2):
            for w in range(3):
                s = f32(0)
                for ii in range(3):
                    for jj in range(3):
                        s = f32(s + d[0, c, h * 3 + ii, w * 3 + jj])
                assert got[0, c, h, w] == s


DIMS = [((4, 5, 6), 0), ((4, 5, 6), 1), ((4, 5, 6), 2), ((64, 128), 0), ((3,), 0),
        ((2, 3, 4, 5), 3), ((2, 3, 4, 5), 1)]


@pytest.mark.parametrize("dims,dim", DIMS)
def test_reductions_against_torch(dims, dim):
    a = R.standard_normal(dims).astype(f32)
    t = _t(a)
    np.testing.assert_allclose(T.reduce_fwd("sum", a, dims, dim), t.sum(dim).numpy(), rtol=1e-5,
                               atol=1e-5)
    np.testing.assert_allclose(T.reduce_fwd("mean", a, dims, dim), t.mean(dim).numpy(),
                               rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(T.reduce_fwd("max", a, dims, dim), t.amax(dim).numpy())
    np.testing.assert_array_equal(T.reduce_fwd("min", a, dims, dim), t.amin(dim).numpy())
    np.testing.assert_array_equal(T.reduce_fwd("argmax", a, dims, dim), t.argmax(dim).numpy())
    np.testing.assert_array_equal(T.reduce_fwd("argmin", a, dims, dim), t.argmin(dim).numpy())
    d = R.standard_normal(T.reduce_fwd("sum", a, dims, dim).shape).astype(f32)
    for kind, fn in [("sum", lambda x: x.sum(dim)), ("mean", lambda x: x.mean(dim)),
                     ("max", lambda x: x.max(dim).values), ("min", lambda x: x.min(dim).values)]:
        xt = _t(a).requires_grad_(True)
        fn(xt).backward(_t(d))
        y = T.reduce_fwd(kind, a, dims, dim) if kind in ("max", "min") else None
        got = T.reduce_bwd(kind, d, dims, dim, a, y)
        np.testing.assert_allclose(got, xt.grad.numpy(), rtol=1e-6, atol=1e-7)


def test_reduction_sum_is_serial_from_zero():
    """Brute force over axis 1 of a [3, 5, 4] tensor: float32 adds in index
    order starting at +0 (reductionKernels.cu:19-28)."""
    a = (R.standard_normal((3, 5, 4)) * 1e3).astype(f32)
    got = T.reduce_fwd("sum", a, (3, 5, 4), 1)
    for o in range(3):
        for i in range(4):
            s = f32(0)
            for k in range(5):
                s = f32(s + a[o, k, i])
            assert got[o, i] == s
    neg0 = np.full((2, 1), -0.0, f32)
    assert not np.signbit(T.reduce_fwd("sum", neg0, (2, 1), 0)[0])  # 0 + -0 = +0


def test_ties_follow_the_reference():
    """argmax/argmin keep the LAST tied index (>=, <=: reductionKernels.cu:
    80, 103); max/min backward route to the FIRST equal element (:242-253)."""
    a = np.array([[1, 3, 3, 0, 3], [2, 2, 2, 2, 2]], f32)
    assert list(T.reduce_fwd("argmax", a, (2, 5), 1)) == [4, 4]
    b = np.array([[1, 0, 5, 0], [7, 7, 7, 7]], f32)
    assert list(T.reduce_fwd("argmin", b, (2, 4), 1)) == [3, 3]
    y = T.reduce_fwd("max", a, (2, 5), 1)
    g = T.reduce_bwd("max", np.array([10, 20], f32), (2, 5), 1, a, y)
    np.testing.assert_array_equal(g, [[0, 10, 0, 0, 0], [20, 0, 0, 0, 0]])


def test_planted_mistakes_are_caught():
    a = np.array([[1, 3, 3, 0, 3]], f32)
    # strict > instead of >= picks the first tie
    strict = int(np.argmax(a[0]))
    assert strict != T.reduce_fwd("argmax", a, (1, 5), 1)[0]
    # relu grad with >= would be 1 at 0
    _, g = T.activation("relu", np.array([0.0], f32))
    assert g[0] != f32(1)
    # reducing the wrong axis changes the result
    x = R.standard_normal((5, 5)).astype(f32)
    assert not np.allclose(T.reduce_fwd("sum", x, (5, 5), 0), x.sum(1))
    # mean divided by the wrong extent
    y = R.standard_normal((4, 5)).astype(f32)
    assert not np.allclose(T.reduce_fwd("mean", y, (4, 5), 0), y.sum(0) / 5)
    # unpool backward without the block sum (a plain subsample) is wrong
    d = R.standard_normal((1, 1, 4, 4)).astype(f32)
    assert not np.allclose(T.unpool_bwd(d, 2, 2), d[:, :, ::2, ::2])
