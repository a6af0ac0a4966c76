"""TEST INFRASTRUCTURE ONLY -- the parity oracle and CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package. The product (``ml_framework_amd``) never does.

Two independent CPU restatements of the reference's arithmetic:

* ``seera_cpp`` -- ctypes wrappers over ``seera_cpp_oracle.c``, a C + OpenMP
  restatement of the reference's CPU engine (engine/src/tensor_ops.cpp:9-15,
  engine/src/conv_ops.cpp:10-287) calling OpenBLAS sgemm. This is what the
  GPU is compared with and what the CPU baseline times.
* ``closed_form`` -- fp64 NumPy formulas written tap by tap (no im2col), used
  to pin the C restatement.

``fp16r`` reproduces the operand rounding of the reference GPU engine
(``__float2half``, round-to-nearest-even; GEMM.cu:41,52).
"""
from __future__ import annotations

import ctypes
import glob
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle_seera.so")
_lib = None
_backend = None


def fp16r(x) -> np.ndarray:
    """Round to fp16 (RNE) and return as fp32 -- the reference's __float2half."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def openblas_path() -> str | None:
    """numpy's bundled OpenBLAS (ILP64, symbols prefixed ``scipy_``)."""
    libdir = os.path.join(os.path.dirname(os.path.dirname(np.__file__)), "numpy.libs")
    hits = sorted(glob.glob(os.path.join(libdir, "libscipy_openblas64_*.so")))
    return hits[0] if hits else None


def load(nthreads: int = 0):
    """Load the compiled oracle (built by ``oracle/build.sh``)."""
    global _lib, _backend
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"oracle library missing: {LIB_PATH}; run oracle/build.sh "
                "(or __graft_entry__.build())")
        lib = ctypes.CDLL(LIB_PATH)
        lib.oracle_init.argtypes = [ctypes.c_char_p, ctypes.c_int]
        lib.oracle_init.restype = ctypes.c_int
        _declare(lib)
        _lib = lib
    if _backend is None or nthreads:
        path = openblas_path()
        _backend = _lib.oracle_init(path.encode() if path else None, int(nthreads))
    return _lib


def backend() -> str:
    load()
    return "openblas" if _backend else "plain-c"


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class seera_cpp:  # noqa: N801 -- mirrors the reference module name
    """ctypes mirror of the reference's ``seera_cpp`` GEMM/conv entry points
    (engine/src/bindings.cpp:14-21, 102-128, 174-201), plus the batched
    GEMM forward/backward the GPU entry points define."""

    @staticmethod
    def matmul(a, b):
        """bindings.cpp:14-21 -> tensor_ops.cpp:9-15 (2-D only)."""
        a, b = _f32(a), _f32(b)
        M, K = a.shape
        K2, N = b.shape
        assert K == K2
        c = np.empty((M, N), np.float32)
        load().oracle_matmul(_p(a), _p(b), _p(c), M, K, N)
        return c

    @staticmethod
    def matmul_batched(a, b):
        """C[b] = A[b].B for A [Nbatch,M,K] (or 2-D), B [K,N] (GEMM.cu:95-103)."""
        a, b = _f32(a), _f32(b)
        a3 = a if a.ndim == 3 else a[None]
        nb, M, K = a3.shape
        N = b.shape[1]
        c = np.empty((nb, M, N), np.float32)
        load().oracle_matmul_batched(_p(np.ascontiguousarray(a3)), _p(b), _p(c),
                                     M, N, K, nb)
        return c if a.ndim == 3 else c[0]

    @staticmethod
    def matmul_bwd(a, b, dc):
        """dA = dC.B^T per slice, dB = sum_b A_b^T.dC_b (Seera_Engine.py:557-564)."""
        a, b, dc = _f32(a), _f32(b), _f32(dc)
        a3 = a if a.ndim == 3 else a[None]
        nb, M, K = a3.shape
        N = b.shape[1]
        dc3 = np.ascontiguousarray(dc.reshape(nb, M, N))
        da = np.empty((nb, M, K), np.float32)
        db = np.empty((K, N), np.float32)
        load().oracle_matmul_bwd(_p(np.ascontiguousarray(a3)), _p(b), _p(dc3),
                                 _p(da), _p(db), M, N, K, nb)
        return (da if a.ndim == 3 else da[0]), db

    @staticmethod
    def im2col_batch(x, KH, KW, sh, sw, ph, pw):
        x = _f32(x)
        N, C, H, W = x.shape
        OH = (H + 2 * ph - KH) // sh + 1
        OW = (W + 2 * pw - KW) // sw + 1
        col = np.empty((N, C * KH * KW, OH * OW), np.float32)
        load().oracle_im2col_batch(_p(x), _p(col), N, C, H, W, KH, KW, sh, sw, ph, pw)
        return col

    @staticmethod
    def col2im_batch(col, shape, KH, KW, sh, sw, ph, pw):
        col = _f32(col)
        N, C, H, W = shape
        x = np.empty((N, C, H, W), np.float32)
        load().oracle_col2im_batch(_p(col), _p(x), N, C, H, W, KH, KW, sh, sw, ph, pw)
        return x

    @staticmethod
    def conv2d_forward(x, w, sh=1, sw=1, ph=0, pw=0):
        """bindings.cpp:102-113 -> conv_ops.cpp:95-122."""
        x, w = _f32(x), _f32(w)
        N, C, H, W = x.shape
        F, C2, KH, KW = w.shape
        assert C == C2
        OH = (H + 2 * ph - KH) // sh + 1
        OW = (W + 2 * pw - KW) // sw + 1
        out = np.empty((N, F, OH, OW), np.float32)
        load().oracle_conv2d_forward(_p(x), _p(w), _p(out), N, C, H, W, F, KH, KW,
                                     sh, sw, ph, pw)
        return out

    @staticmethod
    def conv2d_backward(dout, x, w, sh=1, sw=1, ph=0, pw=0):
        """bindings.cpp:116-128 -> conv_ops.cpp:127-185. Returns (dX, dW)."""
        dout, x, w = _f32(dout), _f32(x), _f32(w)
        N, C, H, W = x.shape
        F, _, KH, KW = w.shape
        dx = np.empty_like(x)
        dw = np.empty_like(w)
        load().oracle_conv2d_backward(_p(dout), _p(x), _p(w), _p(dx), _p(dw), N, C,
                                      H, W, F, KH, KW, sh, sw, ph, pw)
        return dx, dw

    @staticmethod
    def conv_transpose2d_forward(x, w, sh=1, sw=1, ph=0, pw=0):
        """bindings.cpp:174-186 -> conv_ops.cpp:197-228. W is [Cin,Cout,KH,KW]."""
        x, w = _f32(x), _f32(w)
        N, Cin, H, W = x.shape
        Cin2, Cout, KH, KW = w.shape
        assert Cin == Cin2
        Hout = (H - 1) * sh - 2 * ph + KH
        Wout = (W - 1) * sw - 2 * pw + KW
        out = np.empty((N, Cout, Hout, Wout), np.float32)
        load().oracle_conv_transpose2d_fwd(_p(x), _p(w), _p(out), N, Cin, H, W,
                                           Cout, KH, KW, sh, sw, ph, pw)
        return out

    @staticmethod
    def conv_transpose2d_backward(dout, x, w, sh=1, sw=1, ph=0, pw=0):
        """bindings.cpp:189-201 -> conv_ops.cpp:233-287. Returns (dX, dW)."""
        dout, x, w = _f32(dout), _f32(x), _f32(w)
        N, Cin, H, W = x.shape
        _, Cout, KH, KW = w.shape
        dx = np.empty_like(x)
        dw = np.empty_like(w)
        load().oracle_conv_transpose2d_bwd(_p(dout), _p(x), _p(w), _p(dx), _p(dw),
                                           N, Cin, H, W, Cout, KH, KW, sh, sw, ph, pw)
        return dx, dw


def _declare(lib):
    vp, i = ctypes.c_void_p, ctypes.c_int
    sig = {
        "oracle_matmul": [vp, vp, vp, i, i, i],
        "oracle_matmul_batched": [vp, vp, vp, i, i, i, i],
        "oracle_matmul_bwd": [vp, vp, vp, vp, vp, i, i, i, i],
        "oracle_im2col_batch": [vp, vp] + [i] * 10,
        "oracle_col2im_batch": [vp, vp] + [i] * 10,
        "oracle_conv2d_forward": [vp, vp, vp] + [i] * 11,
        "oracle_conv2d_backward": [vp] * 5 + [i] * 11,
        "oracle_conv_transpose2d_fwd": [vp, vp, vp] + [i] * 11,
        "oracle_conv_transpose2d_bwd": [vp] * 5 + [i] * 11,
    }
    for name, args in sig.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = None
    lib.oracle_backend.restype = ctypes.c_int

