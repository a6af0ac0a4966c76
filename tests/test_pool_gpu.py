"""MaxPool2D forward / backward on the GPU, through the C ABI, against the
oracle (oracle/pool.py, the reference engine's maxPool.cu:9-77 restated).

Bar: bit-exact. The forward only compares and copies; the backward adds, per
input element, dout * mask over the covering windows in the same (ho, wo)
order as the oracle, in float32, and mask is 0 or 1 so every product is
exact. At CNN sizes, too large for the oracle's loops, the kernels are held
to closed forms computed with torch on the CPU: values against max_pool2d on
the -inf-padded input, the mask against its argmax indices (distinct
values), the gradient against mask * conv_transpose2d(dout, ones).
"""
import zlib

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer
from oracle import pool
from tests.shapes import MAXPOOL

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True, scope="module")
def _gpu():
    assert capi.gpu_available(), "no HIP device visible"


def hip_maxpool(x, KH, KW, p, s):
    N, C, H, W = x.shape
    Ho, Wo = pool.out_extent(H, p, KH, s), pool.out_extent(W, p, KW, s)
    with DeviceBuffer.from_array(x) as px, DeviceBuffer(max(N * C * Ho * Wo, 1) * 4) as po, \
            DeviceBuffer(x.nbytes) as pm:
        pm.fill(0x7F)  # every mask element is written
        capi.call("seera_hip_maxpool_fwd", px.ptr, po.ptr, pm.ptr, N, C, H, W, KH, KW, p, p, s, s)
        return po.to_array((N, C, Ho, Wo)), pm.to_array(x.shape, np.int32)


def hip_maxpool_bwd(dout, mask, KH, KW, p, s):
    N, C, H, W = mask.shape
    with DeviceBuffer.from_array(dout) as pg, DeviceBuffer.from_array(mask) as pm, \
            DeviceBuffer(mask.size * 4) as pd:
        pd.fill(0x7F)  # every element is written
        capi.call("seera_hip_maxpool_bwd", pg.ptr, pm.ptr, pd.ptr, N, C, H, W, KH, KW, p, p, s, s)
        return pd.to_array(mask.shape)


@pytest.mark.parametrize("case", MAXPOOL, ids=[c[0] for c in MAXPOOL])
def test_parity_reference_shapes(case):
    _, N, C, H, W, KH, KW, s, p = case
    r = np.random.default_rng(N * 1000 + C * 100 + H + KH)
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    out, mask = hip_maxpool(x, KH, KW, p, s)
    ro, rm = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    assert np.array_equal(out, ro) and np.array_equal(mask, rm)
    dout = r.standard_normal(out.shape).astype(np.float32)
    assert np.array_equal(hip_maxpool_bwd(dout, mask, KH, KW, p, s),
                          pool.maxpool_bwd(dout, rm, KH, KW, p, p, s, s))


@pytest.mark.parametrize("KH,KW,p,s", [(2, 2, 0, 2), (3, 3, 1, 2), (2, 3, 1, 1), (3, 2, 2, 1)])
def test_ties_and_padded_origins(KH, KW, p, s):
    """Small integers: many ties (the later element wins), windows whose
    origin is padding with every element below 0 (output 0, nothing marked)."""
    x = np.random.default_rng(KH * 7 + KW + p).integers(-3, 2, (2, 3, 9, 7)).astype(np.float32)
    out, mask = hip_maxpool(x, KH, KW, p, s)
    ro, rm = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    assert np.array_equal(out, ro) and np.array_equal(mask, rm)
    dout = np.random.default_rng(5).standard_normal(out.shape).astype(np.float32)
    assert np.array_equal(hip_maxpool_bwd(dout, mask, KH, KW, p, s),
                          pool.maxpool_bwd(dout, rm, KH, KW, p, p, s, s))


def test_constant_input_gradient_mass():
    """Testing/test_1.py:358-372: all-ones input, 2x2 stride 2."""
    x = np.ones((2, 4, 8, 8), np.float32)
    out, mask = hip_maxpool(x, 2, 2, 0, 2)
    dx = hip_maxpool_bwd(np.ones_like(out), mask, 2, 2, 0, 2)
    assert dx.min() >= 0 and dx.sum() == out.size


@pytest.mark.parametrize("N,C,H,W,K,s,p", [(16, 64, 112, 112, 3, 2, 1),   # ResNet stem pool
                                           (32, 128, 56, 56, 2, 2, 0),
                                           (8, 96, 55, 55, 3, 2, 0)])     # AlexNet-style overlap
def test_cnn_sizes_closed_forms(N, C, H, W, K, s, p):
    n = N * C * H * W
    assert n < 2 ** 24  # every integer below 2^24 is a float32: the values stay distinct
    x = torch.randperm(n, generator=torch.Generator().manual_seed(H)) - n // 2
    x = (x.float() * 2.0 ** -20).reshape(N, C, H, W).numpy()  # distinct, both signs, exact
    out, mask = hip_maxpool(x, K, K, p, s)
    tv, tidx = F.max_pool2d(F.pad(torch.from_numpy(x), (p,) * 4, value=float("-inf")),
                            K, stride=s, return_indices=True)
    Ho, Wo = out.shape[2:]
    hs = torch.arange(Ho) * s - p
    ws = torch.arange(Wo) * s - p
    inside = ((hs >= 0) & (hs < H))[:, None] & ((ws >= 0) & (ws < W))[None, :]
    expect = torch.where(inside, tv, tv.clamp(min=0))
    assert np.array_equal(out, expect.numpy())
    marked = inside | (tv >= 0)
    Wp = W + 2 * p
    hi, wi = tidx // Wp - p, tidx % Wp - p
    # Count the windows that mark each element (unmarked windows add 0 at
    # index 0); the mask is 1 where the count is positive.
    hits = torch.zeros(N, C, H * W, dtype=torch.int32)
    flat = torch.where(marked, hi * W + wi, 0).reshape(N, C, -1)
    hits.scatter_add_(2, flat, marked.reshape(N, C, -1).int())
    assert np.array_equal(mask, (hits > 0).int().reshape(N, C, H, W).numpy())
    dout = torch.randn(N, C, Ho, Wo, generator=torch.Generator().manual_seed(1))
    oph = H - ((Ho - 1) * s - 2 * p + K)
    opw = W - ((Wo - 1) * s - 2 * p + K)
    cover = F.conv_transpose2d(dout.double(), torch.ones(C, 1, K, K, dtype=torch.float64),
                               stride=s, padding=p, output_padding=(oph, opw), groups=C)
    dx = hip_maxpool_bwd(dout.numpy(), mask, K, K, p, s)
    # The kernel rounds each of at most ceil(K/s)^2 = 4 partial sums of N(0,1)
    # terms to float32: a few 1e-7 relative to the terms.
    np.testing.assert_allclose(dx, mask * cover.numpy(), rtol=1e-6, atol=1e-5)


def test_async_entry_points_on_a_stream():
    """seera_hip_maxpool_{fwd,bwd}_async on a created stream give the same
    bits as the synchronous entry points (cells and general kernels)."""
    import ctypes

    lib = capi.load()
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    try:
        for K, s, p in [(2, 2, 0), (3, 2, 1)]:
            x = np.random.default_rng(K).standard_normal((3, 5, 17, 19)).astype(np.float32)
            out, mask = hip_maxpool(x, K, K, p, s)
            dout = np.random.default_rng(9).standard_normal(out.shape).astype(np.float32)
            dx = hip_maxpool_bwd(dout, mask, K, K, p, s)
            N, C, H, W = x.shape
            with DeviceBuffer.from_array(x) as px, DeviceBuffer(out.nbytes) as po, \
                    DeviceBuffer(x.nbytes) as pm, DeviceBuffer.from_array(dout) as pg, \
                    DeviceBuffer(x.nbytes) as pd:
                args = (N, C, H, W, K, K, p, p, s, s, st.value)
                capi.check(lib.seera_hip_maxpool_fwd_async(px.ptr, po.ptr, pm.ptr, *args))
                capi.check(lib.seera_hip_maxpool_bwd_async(pg.ptr, pm.ptr, pd.ptr, *args))
                capi.check(lib.seera_hip_stream_synchronize(st.value))
                assert np.array_equal(po.to_array(out.shape), out)
                assert np.array_equal(pm.to_array(x.shape, np.int32), mask)
                assert np.array_equal(pd.to_array(x.shape), dx)
    finally:
        lib.seera_hip_stream_destroy(st.value)


def test_unaligned_pointers_match_aligned():
    """2x2 stride 2 moves element pairs as 8-byte accesses when x, mask and dX
    are 8-byte aligned; 4-byte-aligned pointers take the element-wise kernels
    and give the same bits."""
    x = np.random.default_rng(11).standard_normal((2, 3, 10, 12)).astype(np.float32)
    out, mask = hip_maxpool(x, 2, 2, 0, 2)
    dout = np.random.default_rng(12).standard_normal(out.shape).astype(np.float32)
    dx = hip_maxpool_bwd(dout, mask, 2, 2, 0, 2)
    N, C, H, W = x.shape
    n = x.size
    with DeviceBuffer(4 * n + 4) as px, DeviceBuffer(out.nbytes) as po, \
            DeviceBuffer(4 * n + 4) as pm, DeviceBuffer.from_array(dout) as pg, \
            DeviceBuffer(4 * n + 4) as pd:
        capi.check(capi.load().seera_hip_memcpy_h2d(px.ptr + 4, x.ctypes.data, x.nbytes))
        args = (N, C, H, W, 2, 2, 0, 0, 2, 2)
        capi.call("seera_hip_maxpool_fwd", px.ptr + 4, po.ptr, pm.ptr + 4, *args)
        capi.call("seera_hip_maxpool_bwd", pg.ptr, pm.ptr + 4, pd.ptr + 4, *args)
        got_m = pm.to_array((n + 1,), np.int32)[1:].reshape(x.shape)
        got_dx = pd.to_array((n + 1,))[1:].reshape(x.shape)
        assert np.array_equal(po.to_array(out.shape), out)
        assert np.array_equal(got_m, mask) and np.array_equal(got_dx, dx)


@pytest.mark.parametrize("H,W", [(9, 12), (8, 8), (1, 4), (13, 20), (31, 8), (40, 12)])
def test_3x3_s2_p1_vector_path_matches_general(H, W):
    """3x3 stride 2 padding 1 with W % 4 == 0 and 16-byte aligned tensors runs
    the 16-byte kernels (the forward in segments of 7 output rows: H = 31 and
    40 give 3 segments); 4-byte-aligned pointers take the general kernels.
    Small integers (many ties, padded origins with every element below 0):
    both give the oracle's bits."""
    x = np.random.default_rng(H * 31 + W).integers(-3, 2, (2, 3, H, W)).astype(np.float32)
    out, mask = hip_maxpool(x, 3, 3, 1, 2)
    ro, rm = pool.maxpool_fwd(x, 3, 3, 1, 1, 2, 2)
    assert np.array_equal(out, ro) and np.array_equal(mask, rm)
    dout = np.random.default_rng(H + W).standard_normal(out.shape).astype(np.float32)
    dx = hip_maxpool_bwd(dout, mask, 3, 3, 1, 2)
    assert np.array_equal(dx, pool.maxpool_bwd(dout, rm, 3, 3, 1, 1, 2, 2))
    N, C = x.shape[:2]
    n = x.size
    with DeviceBuffer(4 * n + 4) as px, DeviceBuffer(out.nbytes) as po, \
            DeviceBuffer(4 * n + 4) as pm, DeviceBuffer.from_array(dout) as pg, \
            DeviceBuffer(4 * n + 4) as pd:
        capi.check(capi.load().seera_hip_memcpy_h2d(px.ptr + 4, x.ctypes.data, x.nbytes))
        args = (N, C, H, W, 3, 3, 1, 1, 2, 2)
        capi.call("seera_hip_maxpool_fwd", px.ptr + 4, po.ptr, pm.ptr + 4, *args)
        capi.call("seera_hip_maxpool_bwd", pg.ptr, pm.ptr + 4, pd.ptr + 4, *args)
        assert np.array_equal(po.to_array(out.shape), out)
        assert np.array_equal(pm.to_array((n + 1,), np.int32)[1:].reshape(x.shape), mask)
        assert np.array_equal(pd.to_array((n + 1,))[1:].reshape(x.shape), dx)


def _random_pool_cases(n, seed):
    """Seeded random pooling shapes: window, stride and padding combinations
    that reach the pair, cell, 3x3-s2-p1 and general kernels, including
    overlapping windows, odd sizes and padding up to half the window."""
    r = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        KH, KW = int(r.choice([1, 2, 3, 3, 4, 5])), int(r.choice([1, 2, 3, 3, 4]))
        s = int(r.choice([1, 2, 2, 3]))
        p = int(r.integers(0, min(KH, KW) // 2 + 1))
        N, C = int(r.integers(1, 4)), int(r.integers(1, 20))
        H, W = int(r.integers(1, 30)), int(r.choice([int(r.integers(1, 30)), 4 * int(r.integers(1, 10))]))
        if pool.out_extent(H, p, KH, s) < 1 or pool.out_extent(W, p, KW, s) < 1:
            continue
        out.append((f"q{len(out):02d}", N, C, H, W, KH, KW, s, p))
    return out


RANDOM_POOL = _random_pool_cases(24, 20261205)


@pytest.mark.parametrize("case", RANDOM_POOL, ids=[c[0] for c in RANDOM_POOL])
def test_parity_random_shapes(case):
    _, N, C, H, W, KH, KW, s, p = case
    r = np.random.default_rng(zlib.crc32(repr(case).encode()))
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    out, mask = hip_maxpool(x, KH, KW, p, s)
    ro, rm = pool.maxpool_fwd(x, KH, KW, p, p, s, s)
    assert np.array_equal(out, ro) and np.array_equal(mask, rm), case
    dout = r.standard_normal(out.shape).astype(np.float32)
    assert np.array_equal(hip_maxpool_bwd(dout, mask, KH, KW, p, s),
                          pool.maxpool_bwd(dout, rm, KH, KW, p, p, s, s)), case
