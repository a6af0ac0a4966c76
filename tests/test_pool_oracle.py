"""Pins oracle/pool.py (the reference GPU engine's MaxPool2D, maxPool.cu:9-77)
on the CPU, before it is used to check the HIP kernels:

* values against torch's max_pool2d, which pads with -inf: equal wherever the
  window origin is inside the image; max(torch, 0) where it is padding
  (maxPool.cu:16-26 starts the running max at 0 there);
* the mask against torch's argmax indices when values are distinct;
* ties against a closed form: the argmax is the last in-window element equal
  to the window max (maxPool.cu:37 compares with <=);
* the backward against mask * conv_transpose2d(dout, ones) -- the sum of dout
  over every window covering an element (maxPool.cu:65-75) -- and against
  torch's max_pool2d gradient where windows do not overlap;
* planted mistakes (strict ties, a -inf start, swapped padding) that these
  checks must reject.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import pool
from tests.shapes import MAXPOOL

CPU_CASES = [c for c in MAXPOOL if c[1] * c[2] * c[3] * c[4] <= 4096]


def _origin_inside(H, W, Ho, Wo, s, p):
    hs = np.arange(Ho) * s - p
    ws = np.arange(Wo) * s - p
    return ((hs >= 0) & (hs < H))[:, None] & ((ws >= 0) & (ws < W))[None, :]


def _torch_pool(x, k, s, p):
    t = torch.from_numpy(x)
    # torch requires pad <= kernel / 2; pad the input with -inf by hand.
    t = F.pad(t, (p, p, p, p), value=float("-inf"))
    v, idx = F.max_pool2d(t, k, stride=s, return_indices=True)
    return v.numpy(), idx.numpy()


@pytest.mark.parametrize("case", CPU_CASES, ids=[c[0] for c in CPU_CASES])
def test_values_and_mask_vs_torch(case):
    _, N, C, H, W, KH, KW, s, p = case
    x = np.random.default_rng(H * W + KH).standard_normal((N, C, H, W)).astype(np.float32)
    out, mask = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    tv, tidx = _torch_pool(x, (KH, KW), s, p)
    Ho, Wo = out.shape[2:]
    inside = _origin_inside(H, W, Ho, Wo, s, p)
    expect = np.where(inside, tv, np.maximum(tv, 0)).astype(np.float32)
    assert np.array_equal(out, expect)
    # torch's indices address the padded plane; map them back and mark the
    # windows that take an in-image argmax (origin inside, or max >= 0).
    Wp = W + 2 * p
    ref = np.zeros_like(mask)
    for b in range(N):
        for c in range(C):
            for ho in range(Ho):
                for wo in range(Wo):
                    if not (inside[ho, wo] or tv[b, c, ho, wo] >= 0):
                        continue
                    hp, wp = divmod(int(tidx[b, c, ho, wo]), Wp)
                    ref[b, c, hp - p, wp - p] = 1
    assert np.array_equal(mask, ref)


def _tie_closed_form(x, KH, KW, p, s):
    """argmax = last in-window element equal to max(start, window)."""
    N, C, H, W = x.shape
    Ho, Wo = pool.out_extent(H, p, KH, s), pool.out_extent(W, p, KW, s)
    out = np.zeros((N, C, Ho, Wo), np.float32)
    mask = np.zeros(x.shape, np.int32)
    for ho in range(Ho):
        for wo in range(Wo):
            h0, w0 = ho * s - p, wo * s - p
            hs = [h for h in range(h0, h0 + KH) if 0 <= h < H]
            ws = [w for w in range(w0, w0 + KW) if 0 <= w < W]
            cells = [(h, w) for h in hs for w in ws]
            if not cells:  # window wholly in the padding: 0, nothing marked
                continue
            vals = np.stack([x[:, :, h, w] for h, w in cells], -1)  # [N, C, cells]
            start = x[:, :, h0, w0] if (0 <= h0 < H and 0 <= w0 < W) else np.zeros((N, C))
            m = np.maximum(vals.max(-1), start)
            out[:, :, ho, wo] = m
            hit = vals == m[..., None]
            any_hit = hit.any(-1)
            last = len(cells) - 1 - np.argmax(hit[..., ::-1], -1)
            for b in range(N):
                for c in range(C):
                    if any_hit[b, c]:
                        h, w = cells[last[b, c]]
                        mask[b, c, h, w] = 1
    return out, mask


TIE_CASES = [(2, 2, 0, 2), (3, 3, 1, 2), (2, 3, 1, 1), (3, 2, 2, 1)]


@pytest.mark.parametrize("KH,KW,p,s", TIE_CASES)
def test_ties_go_to_the_later_element(KH, KW, p, s):
    x = np.random.default_rng(KH * 10 + KW + p).integers(-2, 3, (2, 3, 7, 6)).astype(np.float32)
    out, mask = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    eo, em = _tie_closed_form(x, KH, KW, p, s)
    assert np.array_equal(out, eo) and np.array_equal(mask, em)


def test_constant_input_marks_last_of_each_window():
    """Testing/test_1.py:358-372: all-equal windows; every window marks its
    last element, so the gradient mass equals the number of outputs."""
    x = np.ones((2, 4, 8, 8), np.float32)
    out, mask = pool.maxpool_fwd(x, 2, 2, 0, 0, 2, 2)
    assert np.array_equal(mask[:, :, 1::2, 1::2], np.ones((2, 4, 4, 4), np.int32))
    assert mask.sum() == out.size
    dx = pool.maxpool_bwd(np.ones_like(out), mask, 2, 2, 0, 0, 2, 2)
    assert dx.min() >= 0 and dx.sum() == out.size


def _bwd_closed_form(dout, mask, KH, KW, p, s):
    N, C, H, W = mask.shape
    Ho = dout.shape[2]
    Wo = dout.shape[3]
    oph = H - ((Ho - 1) * s - 2 * p + KH)
    opw = W - ((Wo - 1) * s - 2 * p + KW)
    cover = F.conv_transpose2d(torch.from_numpy(dout).double(),
                               torch.ones(C, 1, KH, KW, dtype=torch.float64), stride=s,
                               padding=p, output_padding=(oph, opw), groups=C).numpy()
    return mask * cover


@pytest.mark.parametrize("case", CPU_CASES, ids=[c[0] for c in CPU_CASES])
def test_backward_is_mask_times_window_cover(case):
    _, N, C, H, W, KH, KW, s, p = case
    r = np.random.default_rng(N * C + H)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    out, mask = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    dout = r.standard_normal(out.shape).astype(np.float32)
    dx = pool.maxpool_bwd(dout, mask, KH, KW, p, p, s, s)
    np.testing.assert_allclose(dx, _bwd_closed_form(dout, mask, KH, KW, p, s), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("case", [c for c in CPU_CASES if c[7] == c[5] == c[6] and c[8] == 0],
                         ids=lambda c: c[0])
def test_backward_vs_torch_non_overlapping(case):
    _, N, C, H, W, KH, KW, s, p = case
    r = np.random.default_rng(H + 7)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    out, mask = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    dout = r.standard_normal(out.shape).astype(np.float32)
    t = torch.from_numpy(x).requires_grad_()
    (F.max_pool2d(t, (KH, KW), stride=s) * torch.from_numpy(dout)).sum().backward()
    assert np.array_equal(pool.maxpool_bwd(dout, mask, KH, KW, p, p, s, s), t.grad.numpy())


def test_planted_mistakes_are_caught():
    x = np.random.default_rng(1).integers(-2, 3, (1, 2, 6, 6)).astype(np.float32)
    eo, em = _tie_closed_form(x, 2, 2, 1, 1)
    _, m_strict = pool.maxpool_fwd(x, 2, 2, 1, 1, 1, 1, ties_later=False)
    assert not np.array_equal(m_strict, em)
    xn = -np.abs(np.random.default_rng(2).standard_normal((1, 2, 6, 6))).astype(np.float32) - 0.1
    o_inf, _ = pool.maxpool_fwd(xn, 2, 2, 1, 1, 2, 2, origin_zero=False)
    eo, _ = _tie_closed_form(xn, 2, 2, 1, 2)
    assert not np.array_equal(o_inf, eo)
    # Padding swapped between the axes in the backward of an asymmetric case.
    x = np.random.default_rng(3).standard_normal((1, 1, 7, 9)).astype(np.float32)
    out, mask = pool.maxpool_fwd(x, 3, 3, 1, 1, 1, 1)
    mask = np.ones_like(mask)
    dout = np.random.default_rng(4).standard_normal(out.shape).astype(np.float32)
    ref = _bwd_closed_form(dout, mask, 3, 3, 1, 1)
    assert np.allclose(pool.maxpool_bwd(dout, mask, 3, 3, 1, 1, 1, 1), ref, atol=1e-6)
    assert not np.allclose(pool.maxpool_bwd(dout, mask, 3, 3, 0, 2, 1, 1), ref, atol=1e-6)
