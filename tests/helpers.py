"""Shared test helpers: run the HIP path through the C ABI and compare with
the oracle at the north-star tolerance."""
from __future__ import annotations

import numpy as np

from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer

# relative Frobenius error <= 1e-3 and max abs
# error <= 2e-2 against the fp32 CPU result on identical fp16-rounded operands.
REL_FRO = 1e-3
MAX_ABS = 2e-2


def rel_fro(got, ref) -> float:
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(got - ref) / (den if den > 0 else 1.0))


def assert_parity(got, ref, what: str = "", rel: float = REL_FRO, mabs: float = MAX_ABS):
    got = np.asarray(got)
    ref = np.asarray(ref)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    r = rel_fro(got, ref)
    m = float(np.max(np.abs(got.astype(np.float64) - ref))) if got.size else 0.0
    assert r <= rel and m <= mabs, f"{what}: rel_fro={r:.3e} max_abs={m:.3e}"
    return r, m


def _dev(a):
    return DeviceBuffer.from_array(np.ascontiguousarray(a, np.float32))


def _out(shape):
    return DeviceBuffer(max(int(np.prod(shape)), 1) * 4)


def hip_matmul(a, b):
    a3 = a if a.ndim == 3 else a[None]
    nb, M, K = a3.shape
    N = b.shape[1]
    with _dev(a3) as da, _dev(b) as db, _out((nb, M, N)) as dc:
        capi.call("seera_hip_matmul", da.ptr, db.ptr, dc.ptr, M, N, K, nb)
        c = dc.to_array((nb, M, N))
    return c if a.ndim == 3 else c[0]


def hip_matmul_bwd(a, b, dc):
    a3 = a if a.ndim == 3 else a[None]
    nb, M, K = a3.shape
    N = b.shape[1]
    with _dev(a3) as pa, _dev(b) as pb, _dev(dc.reshape(nb, M, N)) as pdc, \
            _out((nb, M, K)) as pda, _out((K, N)) as pdb:
        capi.call("seera_hip_matmul_bwd", pa.ptr, pb.ptr, pdc.ptr, pda.ptr, pdb.ptr,
                  M, N, K, nb)
        da = pda.to_array((nb, M, K))
        dbv = pdb.to_array((K, N))
    return (da if a.ndim == 3 else da[0]), dbv


def out_hw(H, W, KH, KW, s, p):
    return (H + 2 * p - KH) // s + 1, (W + 2 * p - KW) // s + 1


def hip_conv_fwd(x, w, s, p):
    N, C, H, W = x.shape
    F, _, KH, KW = w.shape
    OH, OW = out_hw(H, W, KH, KW, s, p)
    with _dev(x) as px, _dev(w) as pw, _out((N, F, OH, OW)) as py:
        # cuda_conv2d_fwd argument order: pad before stride (cuTen.py:562-564)
        capi.call("seera_hip_conv2d_fwd", px.ptr, pw.ptr, py.ptr, N, C, H, W, F, KH, KW,
                  p, p, s, s)
        return py.to_array((N, F, OH, OW))


def hip_conv_bwd(dy, x, w, s, p):
    N, C, H, W = x.shape
    F, _, KH, KW = w.shape
    with _dev(w) as pw, _dev(x) as px, _dev(dy) as pdy, _out(x.shape) as pdx, \
            _out(w.shape) as pdw:
        # cuda_conv2d_bwd argument order: stride before pad (Seera_Engine.py:76-81)
        capi.call("seera_hip_conv2d_bwd", pw.ptr, px.ptr, pdy.ptr, pdx.ptr, pdw.ptr,
                  N, C, H, W, F, KH, KW, s, s, p, p)
        return pdx.to_array(x.shape), pdw.to_array(w.shape)


def convT_hw(H, W, KH, KW, s, p):
    return (H - 1) * s - 2 * p + KH, (W - 1) * s - 2 * p + KW


def hip_convT_fwd(x, w, s, p):
    N, Cin, H, W = x.shape
    _, Cout, KH, KW = w.shape
    OH, OW = convT_hw(H, W, KH, KW, s, p)
    with _dev(x) as px, _dev(w) as pw, _out((N, Cout, OH, OW)) as po:
        capi.call("seera_hip_conv2DTranpose_fwd", px.ptr, pw.ptr, po.ptr, N, Cin, H, W,
                  Cout, KH, KW, s, s, p, p)
        return po.to_array((N, Cout, OH, OW))


def hip_convT_bwd(dy, x, w, s, p):
    N, Cin, H, W = x.shape
    _, Cout, KH, KW = w.shape
    with _dev(w) as pw, _dev(x) as px, _dev(dy) as pdy, _out(x.shape) as pdx, \
            _out(w.shape) as pdw:
        capi.call("seera_hip_conv2DTranspose_bwd", pw.ptr, px.ptr, pdy.ptr, pdx.ptr,
                  pdw.ptr, N, Cin, H, W, Cout, KH, KW, s, s, p, p)
        return pdx.to_array(x.shape), pdw.to_array(w.shape)
