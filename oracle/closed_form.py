"""TEST INFRASTRUCTURE ONLY -- fp64 closed forms that pin the C oracle.

Each function is the defining sum of the reference operation written tap by
tap in float64 NumPy (no im2col, no col2im, no BLAS call ordering), so that a
mistake shared by the C restatement and the HIP kernels (a transposed operand,
a wrong tap sign, a swapped stride/pad) cannot cancel out.

  gemm / gemm_bwd        GEMM.cu:13-103, 164-225 (C = A.B, dA = dC.B^T,
                         dB = sum_b A_b^T.dC_b)
  conv2d_fwd             convolution.cu:15-101 (cross-correlation,
                         out = floor((H + 2p - R)/s) + 1)
  conv2d_bwd             convolution.cu:393-453 (dX = adjoint of conv2d_fwd in
                         X, dW = adjoint in W)
  conv_transpose2d_fwd   upsampling.cu:376-401 (Hout = (H-1)s - 2p + KH,
                         W laid out [Cin, Cout, KH, KW])
  conv_transpose2d_bwd   upsampling.cu:322-375
"""
from __future__ import annotations

import numpy as np


def _f64(a):
    return np.asarray(a, dtype=np.float64)


def gemm(a, b):
    """C[b] = A[b].B with A [Nbatch,M,K] or [M,K] and B [K,N]."""
    return _f64(a) @ _f64(b)


def gemm_bwd(a, b, dc):
    """Returns (dA, dB): dA = dC.B^T, dB = sum over slices of A_b^T.dC_b."""
    a, b, dc = _f64(a), _f64(b), _f64(dc)
    da = dc @ b.T
    a2 = a.reshape(-1, a.shape[-1])
    dc2 = dc.reshape(-1, dc.shape[-1])
    return da, a2.T @ dc2


def _out(h, p, k, s):
    return (h + 2 * p - k) // s + 1


def conv2d_fwd(x, w, sh=1, sw=1, ph=0, pw=0):
    """Y[n,f,i,j] = sum_{c,r,s} W[f,c,r,s] X[n,c,i*sh-ph+r, j*sw-pw+s]."""
    x, w = _f64(x), _f64(w)
    N, C, H, W = x.shape
    F, _, R, S = w.shape
    OH, OW = _out(H, ph, R, sh), _out(W, pw, S, sw)
    xp = np.zeros((N, C, H + 2 * ph + sh * OH, W + 2 * pw + sw * OW))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    y = np.zeros((N, F, OH, OW))
    for r in range(R):
        for s in range(S):
            patch = xp[:, :, r:r + sh * OH:sh, s:s + sw * OW:sw]
            y += np.einsum("nchw,fc->nfhw", patch, w[:, :, r, s])
    return y


def conv2d_bwd(dy, x, w, sh=1, sw=1, ph=0, pw=0):
    """Returns (dX, dW) of conv2d_fwd for upstream gradient dY."""
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    N, C, H, W = x.shape
    F, _, R, S = w.shape
    OH, OW = dy.shape[2], dy.shape[3]
    Hp, Wp = H + 2 * ph + sh * OH, W + 2 * pw + sw * OW
    xp = np.zeros((N, C, Hp, Wp))
    xp[:, :, ph:ph + H, pw:pw + W] = x
    dxp = np.zeros((N, C, Hp, Wp))
    dw = np.zeros_like(w)
    for r in range(R):
        for s in range(S):
            sl = (slice(None), slice(None), slice(r, r + sh * OH, sh),
                  slice(s, s + sw * OW, sw))
            dw[:, :, r, s] = np.einsum("nfhw,nchw->fc", dy, xp[sl])
            dxp[sl] += np.einsum("nfhw,fc->nchw", dy, w[:, :, r, s])
    return dxp[:, :, ph:ph + H, pw:pw + W], dw


def conv_transpose2d_fwd(x, w, sh=1, sw=1, ph=0, pw=0):
    """out[n,o,i*sh-ph+kh, j*sw-pw+kw] += X[n,c,i,j] W[c,o,kh,kw]."""
    x, w = _f64(x), _f64(w)
    N, Cin, H, W = x.shape
    _, Cout, KH, KW = w.shape
    Hout, Wout = (H - 1) * sh - 2 * ph + KH, (W - 1) * sw - 2 * pw + KW
    full = np.zeros((N, Cout, (H - 1) * sh + KH, (W - 1) * sw + KW))
    for kh in range(KH):
        for kw in range(KW):
            full[:, :, kh:kh + sh * (H - 1) + 1:sh, kw:kw + sw * (W - 1) + 1:sw] += \
                np.einsum("nchw,co->nohw", x, w[:, :, kh, kw])
    return full[:, :, ph:ph + Hout, pw:pw + Wout]


def conv_transpose2d_bwd(dy, x, w, sh=1, sw=1, ph=0, pw=0):
    """Returns (dX, dW) of conv_transpose2d_fwd for upstream gradient dY."""
    dy, x, w = _f64(dy), _f64(x), _f64(w)
    N, Cin, H, W = x.shape
    _, Cout, KH, KW = w.shape
    Hf, Wf = (H - 1) * sh + KH, (W - 1) * sw + KW
    Hout, Wout = dy.shape[2], dy.shape[3]
    full = np.zeros((N, Cout, Hf, Wf))
    full[:, :, ph:ph + Hout, pw:pw + Wout] = dy
    dx = np.zeros_like(x)
    dw = np.zeros_like(w)
    for kh in range(KH):
        for kw in range(KW):
            patch = full[:, :, kh:kh + sh * (H - 1) + 1:sh, kw:kw + sw * (W - 1) + 1:sw]
            dx += np.einsum("nohw,co->nchw", patch, w[:, :, kh, kw])
            dw[:, :, kh, kw] = np.einsum("nchw,nohw->co", x, patch)
    return dx, dw
