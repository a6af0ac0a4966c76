"""TEST INFRASTRUCTURE ONLY -- MaxPool2D as the reference GPU engine computes it.

A plain-loop NumPy restatement of engine_cuda/src/maxPool.cu (the kernels the
`seera_cuda` names cuda_maxpool_fwd / cuda_maxpool_bwd run; cuTen.py:578-606
and Seera_Engine.py:117-136 call them), used only as the checker of the HIP
kernels. Pinned in tests/test_oracle.py against torch's CPU max_pool2d
(values; gradients where windows do not overlap and values are distinct),
against brute force on tiny inputs, and by planted mistakes it must reject.

  maxpool_fwd   maxPool.cu:9-53   the running max starts at the window origin
                                  (0 when the origin is padding, :16-26); an
                                  in-window element >= it replaces it and
                                  becomes the argmax (ties: later element,
                                  :29-40); mask [B, C, H, W] is 1 at argmaxes
  maxpool_bwd   maxPool.cu:56-77  dX[i] = sum over covering windows of
                                  dout * mask[i]

Two places where the reference is not deterministic or not memory-safe are
given one fixed outcome, as the HIP kernels give it: an element that is the
argmax of one window and loses in another (overlapping windows, thread order
decides in the reference) has mask 1; a window whose origin is padding and
whose elements are all below 0 marks nothing (the reference writes the mask
at the origin's out-of-range address).
"""
from __future__ import annotations

import numpy as np


def out_extent(h, p, k, s):
    return (h + 2 * p - k) // s + 1


def maxpool_fwd(x, R, S, ph=0, pw=0, sh=1, sw=1, ties_later=True, origin_zero=True):
    """Returns (out [B,C,Ho,Wo] float32, mask [B,C,H,W] int32).

    ties_later / origin_zero exist to plant mistakes in tests (False flips the
    rule); the reference's rules are the defaults."""
    x = np.asarray(x, np.float32)
    B, C, H, W = x.shape
    Ho, Wo = out_extent(H, ph, R, sh), out_extent(W, pw, S, sw)
    out = np.zeros((B, C, Ho, Wo), np.float32)
    mask = np.zeros((B, C, H, W), np.int32)
    for ho in range(Ho):
        for wo in range(Wo):
            h0, w0 = ho * sh - ph, wo * sw - pw
            if 0 <= h0 < H and 0 <= w0 < W:
                best = x[:, :, h0, w0].copy()
            else:
                best = np.full((B, C), 0.0 if origin_zero else -np.inf, np.float32)
            arg = np.full((B, C), -1, np.int64)  # in-plane index of the argmax
            for r in range(R):
                for s in range(S):
                    h, w = h0 + r, w0 + s
                    if not (0 <= h < H and 0 <= w < W):
                        continue
                    v = x[:, :, h, w]
                    take = (best <= v) if ties_later else (best < v)
                    best = np.where(take, v, best)
                    arg = np.where(take, h * W + w, arg)
            out[:, :, ho, wo] = best
            bi, ci = np.nonzero(arg >= 0)
            mask.reshape(B, C, H * W)[bi, ci, arg[bi, ci]] = 1
    return out, mask


def maxpool_bwd(dout, mask, R, S, ph=0, pw=0, sh=1, sw=1):
    """dX [B,C,H,W] = sum over the windows covering each element of dout * mask,
    windows in (ho, wo) order, summed in float32 like the kernels."""
    dout = np.asarray(dout, np.float32)
    mask = np.asarray(mask)
    B, C, H, W = mask.shape
    Ho, Wo = dout.shape[2], dout.shape[3]
    dx = np.zeros((B, C, H, W), np.float32)

    def covering(i, p, k, s, n_out):
        # windows o with o*s - p <= i <= o*s - p + k - 1, within [0, n_out)
        lo = max(0, -(-(i + p - k + 1) // s))
        return range(lo, min(n_out - 1, (i + p) // s) + 1)

    for h in range(H):
        for w in range(W):
            m = mask[:, :, h, w].astype(np.float32)
            acc = np.zeros((B, C), np.float32)
            for ho in covering(h, ph, R, sh, Ho):
                for wo in covering(w, pw, S, sw, Wo):
                    acc = (acc + dout[:, :, ho, wo] * m).astype(np.float32)
            dx[:, :, h, w] = acc
    return dx
