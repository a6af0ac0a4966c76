"""TEST INFRASTRUCTURE ONLY -- the reference GPU engine's element-wise,
activation, softmax, broadcast, unpooling and reduction functions in NumPy.

Restatements of the kernels behind the seera_cuda names that cuTen.py and
Seera_Engine.py call around the GEMM / convolution path, used only as the
checker of the HIP kernels (tests/test_tensor_ops_gpu.py). Every function
computes in float32 in the reference's operation order where that order fixes
the bits (serial sums along the reduced axis from +0, the unpooling window
row by row); tests/test_tensor_ops_oracle.py pins each one against torch's
CPU operators, closed forms, brute force on tiny inputs and planted mistakes.

  activation      activations.cu:9-85        out = f(x), grad = f'(x)
  softmax         activations.cu:87-127      row softmax, max-shifted
  softmax_vjp     activations.cu:129-161     s * (dout - <s, dout>)
  elementwise     elemops.cu:14-40           A op B
  scalar_inplace  cuTen_essentails.cu:8-58   arr * k, arr + k, arr ** k
  broadcast_4d    broadcast.cu:12-153        4-D broadcast add / multiply
  unpool_fwd/bwd  unpooling.cu:7-50          nearest upsample, block sums
  reduce_*        reductionKernels.cu:12-380 one-axis reductions + backward
"""
from __future__ import annotations

import numpy as np

f32 = np.float32


def _f(x):
    return np.asarray(x, dtype=f32)


# ---- activations (activations.cu:9-85) ----
def activation(kind: str, x, p0: float = 0.0, p1: float = 0.0):
    """(out, grad) of one activation, float32 throughout."""
    x = _f(x)
    with np.errstate(all="ignore"):
        if kind == "relu":  # :9-15
            return np.where(x > 0, x, f32(0)), np.where(x > 0, f32(1), f32(0))
        if kind == "sigmoid":  # :17-24
            s = f32(1) / (f32(1) + np.exp(-x))
            return s, s * (f32(1) - s)
        if kind == "tanh":  # :26-33
            t = np.tanh(x)
            return t, f32(1) - t * t
        if kind == "log":  # :35-41
            return np.log(x), f32(1) / x
        if kind == "exp":  # :43-50
            e = np.exp(x)
            return e, e.copy()
        if kind == "abs":  # :52-58
            return np.abs(x), np.where(x > 0, f32(1), np.where(x < 0, f32(-1), f32(0)))
        if kind == "sqrt":  # :60-67
            s = np.sqrt(x)
            return s, f32(0.5) / (s + f32(1e-12))
        if kind == "pow":  # :69-75
            e = f32(p0)
            return np.power(x, e), e * np.power(x, e - f32(1))
        if kind == "clip":  # :77-83
            lo, hi = f32(p0), f32(p1)
            return (np.fmin(np.fmax(x, lo), hi),
                    np.where((x >= lo) & (x <= hi), f32(1), f32(0)))
    raise ValueError(kind)


# ---- softmax (activations.cu:87-161) ----
def softmax(x):
    """Row softmax of x [N, C]: exp(x - rowmax) * (1 / rowsum)."""
    x = _f(x)
    m = np.max(x, axis=1, keepdims=True)
    e = np.exp(x - m)
    return e * (f32(1) / np.sum(e, axis=1, keepdims=True, dtype=f32))


def softmax_vjp(s, dout):
    s, d = _f(s), _f(dout)
    dot = np.sum(s * d, axis=1, keepdims=True, dtype=f32)
    return s * (d - dot)


# ---- element-wise and scalar (elemops.cu:14-40; cuTen_essentails.cu:8-58) ----
def elementwise(op: str, a, b):
    a, b = _f(a), _f(b)
    with np.errstate(all="ignore"):
        return {"add": np.add, "sub": np.subtract, "mul": np.multiply,
                "div": np.divide}[op](a, b)


def scalar_inplace(op: str, a, k: float):
    a, k = _f(a), f32(k)
    with np.errstate(all="ignore"):
        return {"mul": np.multiply, "add": np.add, "pow": np.power}[op](a, k)


# ---- 4-D broadcast (broadcast.cu:12-153) ----
def broadcast_shape(a4, b4):
    """Output extents per axis, or None when the shapes do not broadcast
    (compute_out_shape_4d, broadcast.cu:71-91)."""
    out = []
    for x, y in zip(a4, b4):
        if x == y or y == 1:
            out.append(x)
        elif x == 1:
            out.append(y)
        else:
            return None
    return tuple(out)


def broadcast_4d(op: str, a, b, a4, b4):
    """C[n,c,h,w] = A[...] op B[...] with extent-1 axes read at index 0
    (broadcast_kernel_4d's index mapping, broadcast.cu:28-60), by explicit
    index arithmetic over every output element."""
    o = broadcast_shape(a4, b4)
    if o is None:
        raise ValueError("shapes do not broadcast")
    A = _f(a).reshape(-1)
    B = _f(b).reshape(-1)
    idx = np.indices(o).reshape(4, -1)
    def flat(ext, ix):
        sel = [np.zeros_like(ix[i]) if ext[i] == 1 else ix[i] for i in range(4)]
        return ((sel[0] * ext[1] + sel[1]) * ext[2] + sel[2]) * ext[3] + sel[3]
    av, bv = A[flat(a4, idx)], B[flat(b4, idx)]
    c = av + bv if op == "add" else av * bv
    return c.reshape(o)


# ---- unpooling (unpooling.cu:7-50) ----
def unpool_fwd(x, sh: int, sw: int):
    x = _f(x)
    return np.repeat(np.repeat(x, sh, axis=2), sw, axis=3)


def unpool_bwd(dout, sh: int, sw: int):
    """dx[h, w] = sum over ii < sh, jj < sw (ii outer) of dout[h*sh+ii, w*sw+jj],
    added in that order from +0 (unpooling.cu:38-47)."""
    d = _f(dout)
    B, C, Ho, Wo = d.shape
    H, W = Ho // sh, Wo // sw
    acc = np.zeros((B, C, H, W), f32)
    for ii in range(sh):
        for jj in range(sw):
            acc = acc + d[:, :, ii::sh, jj::sw][:, :, :H, :W]
    return acc


# ---- reductions (reductionKernels.cu:12-380) ----
def _axis_view(a, dims, dim):
    """[outer, len, inner] view of a row-major tensor with extents dims."""
    dims = [int(v) for v in dims]
    outer = int(np.prod(dims[:dim], dtype=np.int64))
    inner = int(np.prod(dims[dim + 1:], dtype=np.int64))
    return _f(a).reshape(outer, dims[dim], inner)


def _out_shape(dims, dim):
    return tuple(int(v) for i, v in enumerate(dims) if i != dim)


def reduce_fwd(kind: str, a, dims, dim):
    """sum / mean (serial float32 sum from +0, :12-29; mean divides by the
    extent, cuda_mean_fwd :177-181), max / min (fmax / fmin from the first
    element, :31-65), argmax / argmin (last index whose value is >= / <= the
    running best, :67-111)."""
    v = _axis_view(a, dims, dim)
    n = v.shape[1]
    if kind in ("sum", "mean"):
        acc = np.zeros((v.shape[0], v.shape[2]), f32)
        for i in range(n):
            acc = acc + v[:, i, :]
        if kind == "mean":
            with np.errstate(all="ignore"):
                acc = acc / f32(n)
        return acc.reshape(_out_shape(dims, dim))
    if kind in ("max", "min"):
        acc = v[:, 0, :].copy()
        fn = np.fmax if kind == "max" else np.fmin
        for i in range(n):
            acc = fn(acc, v[:, i, :])
        return acc.reshape(_out_shape(dims, dim))
    if kind in ("argmax", "argmin"):
        best = v[:, 0, :].copy()
        arg = np.zeros(best.shape, np.int32)
        for i in range(n):
            x = v[:, i, :]
            hit = x >= best if kind == "argmax" else x <= best
            best = np.where(hit, x, best)
            arg = np.where(hit, np.int32(i), arg)
        return arg.reshape(_out_shape(dims, dim))
    raise ValueError(kind)


def reduce_bwd(kind: str, dout, dims, dim, fwd_in=None, fwd_out=None):
    """sum / mean: dA = dOut (/ extent) along the axis (:209-225, :349-364);
    max / min: dOut at the first element equal to the forward output, 0
    elsewhere (:229-284)."""
    dims = [int(v) for v in dims]
    outer = int(np.prod(dims[:dim], dtype=np.int64))
    inner = int(np.prod(dims[dim + 1:], dtype=np.int64))
    n = dims[dim]
    d = _f(dout).reshape(outer, 1, inner)
    if kind in ("sum", "mean"):
        g = d / f32(n) if kind == "mean" else d / f32(1)
        return np.broadcast_to(g, (outer, n, inner)).reshape(dims).copy()
    if kind in ("max", "min"):
        x = _f(fwd_in).reshape(outer, n, inner)
        y = _f(fwd_out).reshape(outer, 1, inner)
        eq = x == y
        first = np.cumsum(eq, axis=1) == 1
        hit = eq & first
        return np.where(hit, d, f32(0)).reshape(dims)
    raise ValueError(kind)
