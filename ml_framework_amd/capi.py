"""ctypes binding of the C ABI in ``include/seera_hip.h`` (``libseera_hip.so``).

This is the path tests and ``bench.py`` drive. It never falls back to
anything: a missing or unloadable library raises ``RuntimeError``.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG, "libseera_hip.so")
HEADER = os.path.join(os.path.dirname(PKG), "include", "seera_hip.h")

SEERA_OK = 0
SEERA_ACT_NONE, SEERA_ACT_RELU = 0, 1
SEERA_ERR_INVALID_ARGUMENT = 1
SEERA_ERR_HIP = 2
SEERA_ERR_OUT_OF_MEMORY = 3

_vp, _i, _sz, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float
_conv14 = [_vp, _vp, _vp] + [_i] * 11
_conv16 = [_vp] * 5 + [_i] * 11

# name -> (argtypes, restype); mirrors include/seera_hip.h one for one.
PROTOTYPES: dict[str, tuple[list, object]] = {
    "seera_hip_last_error": ([], ctypes.c_char_p),
    "seera_hip_version": ([], ctypes.c_char_p),
    "seera_hip_device_count": ([], _i),
    "seera_hip_malloc": ([ctypes.POINTER(_vp), _sz], _i),
    "seera_hip_free": ([_vp], _i),
    "seera_hip_malloc_async": ([ctypes.POINTER(_vp), _sz, _vp], _i),
    "seera_hip_free_async": ([_vp, _vp], _i),
    "seera_hip_empty_cache": ([], _i),
    "seera_hip_memory_stats": ([ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i),
    "seera_hip_fill_f32": ([_vp, ctypes.c_float, _sz], _i),
    "seera_hip_memset": ([_vp, _i, _sz], _i),
    "seera_hip_memcpy_d2d": ([_vp, _vp, _sz], _i),
    "seera_hip_memcpy_h2d": ([_vp, _vp, _sz], _i),
    "seera_hip_memcpy_d2h": ([_vp, _vp, _sz], _i),
    "seera_hip_synchronize": ([], _i),
    "seera_hip_matmul": ([_vp, _vp, _vp, _i, _i, _i, _i], _i),
    "seera_hip_matmul_async": ([_vp, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "seera_hip_matmul_noalloc": ([_vp, _vp, _vp, _i, _i, _i, _i, _vp], _i),
    "seera_hip_matmul_bias_act": ([_vp] * 5 + [_i] * 5, _i),
    "seera_hip_matmul_bias_act_async": ([_vp] * 5 + [_i] * 5 + [_vp], _i),
    "seera_hip_bias_grad": ([_vp, _vp, _i, _i], _i),
    "seera_hip_maxpool_fwd": ([_vp] * 3 + [_i] * 10, _i),
    "seera_hip_maxpool_bwd": ([_vp] * 3 + [_i] * 10, _i),
    "seera_hip_maxpool_fwd_async": ([_vp] * 3 + [_i] * 10 + [_vp], _i),
    "seera_hip_maxpool_bwd_async": ([_vp] * 3 + [_i] * 10 + [_vp], _i),
    "seera_hip_bias_grad_async": ([_vp, _vp, _i, _i, _vp], _i),
    "seera_hip_matmul_bwd": ([_vp] * 5 + [_i] * 4, _i),
    "seera_hip_matmul_bwd_async": ([_vp] * 5 + [_i] * 4 + [_vp], _i),
    "seera_hip_matmul_bwd_bias": ([_vp] * 6 + [_i] * 4, _i),
    "seera_hip_matmul_bwd_bias_async": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "seera_hip_matmul_bwd_relu_bias": ([_vp] * 7 + [_i] * 4, _i),
    "seera_hip_matmul_bwd_relu_bias_async": ([_vp] * 7 + [_i] * 4 + [_vp], _i),
    "seera_hip_matmul_bwd_relu": ([_vp] * 6 + [_i] * 4, _i),
    "seera_hip_matmul_bwd_relu_async": ([_vp] * 6 + [_i] * 4 + [_vp], _i),
    "seera_hip_transpose_2d": ([_vp, _vp, _i, _i], _i),
    "seera_hip_transpose_3d": ([_vp, _vp, _i, _i, _i], _i),
    "seera_hip_conv2d_fwd": (_conv14, _i),
    "seera_hip_conv2d_fwd_bias_act": ([_vp] * 5 + [_i] * 12, _i),
    "seera_hip_conv2d_fwd_bias_act_async": ([_vp] * 5 + [_i] * 12 + [_vp], _i),
    "seera_hip_conv_bias_grad": ([_vp, _vp, _i, _i, _i], _i),
    "seera_hip_conv_bias_grad_async": ([_vp, _vp, _i, _i, _i, _vp], _i),
    "seera_hip_conv2d_fwd_async": (_conv14 + [_vp], _i),
    "seera_hip_conv2d_bwd": (_conv16, _i),
    "seera_hip_conv2d_bwd_async": (_conv16 + [_vp], _i),
    "seera_hip_conv2d_bwd_bias": ([_vp] * 6 + [_i] * 11, _i),
    "seera_hip_conv2d_bwd_bias_async": ([_vp] * 6 + [_i] * 11 + [_vp], _i),
    "seera_hip_conv2DTranpose_fwd": (_conv14, _i),
    "seera_hip_conv2DTranpose_fwd_async": (_conv14 + [_vp], _i),
    "seera_hip_conv2DTranspose_bwd": (_conv16, _i),
    "seera_hip_conv2DTranspose_bwd_async": (_conv16 + [_vp], _i),
    "seera_hip_event_create": ([ctypes.POINTER(_vp)], _i),
    "seera_hip_event_record": ([_vp, _vp], _i),
    "seera_hip_event_elapsed_ms": ([_vp, _vp, ctypes.POINTER(_f)], _i),
    "seera_hip_event_destroy": ([_vp], _i),
    "seera_hip_stream_create": ([ctypes.POINTER(_vp)], _i),
    "seera_hip_stream_destroy": ([_vp], _i),
    "seera_hip_stream_release_workspace": ([_vp], _i),
    "seera_hip_stream_synchronize": ([_vp], _i),
    "seera_hip_graph_capture_begin": ([_vp], _i),
    "seera_hip_graph_capture_end": ([_vp, ctypes.POINTER(_vp)], _i),
    "seera_hip_graph_launch": ([_vp, _vp], _i),
    "seera_hip_graph_destroy": ([_vp], _i),
    "seera_hip_workspace_stats": ([ctypes.POINTER(_sz), ctypes.POINTER(_sz)], _i),
    # activations, softmax, unpooling, reductions, scalar, element-wise, broadcast
    **{f"seera_hip_{n}_fwd": ([_vp, _vp, _vp, _i], _i)
       for n in ("relu", "sigmoid", "tanh", "log", "exp", "abs", "sqrt")},
    "seera_hip_pow_fwd": ([_vp, _f, _vp, _vp, _i], _i),
    "seera_hip_clip_fwd": ([_vp, _f, _f, _vp, _vp, _i], _i),
    "seera_hip_softmax_fwd": ([_vp, _vp, _i, _i], _i),
    "seera_hip_softmax_vjp": ([_vp, _vp, _vp, _i, _i], _i),
    "seera_hip_unpooling_fwd": ([_vp, _vp] + [_i] * 6, _i),
    "seera_hip_unpooling_bwd": ([_vp, _vp] + [_i] * 6, _i),
    **{f"seera_hip_{n}": ([_vp, _vp, _i, _i, _vp], _i)
       for n in ("sum_fwd", "mean_fwd", "max_fwd", "min_fwd", "argmax_fwd", "argmin_fwd",
                 "sum_bwd", "mean_bwd")},
    "seera_hip_max_bwd": ([_vp] * 4 + [_i, _i, _vp], _i),
    "seera_hip_min_bwd": ([_vp] * 4 + [_i, _i, _vp], _i),
    **{f"seera_hip_{n}": ([_vp, _f, _i], _i)
       for n in ("scaler_multiply_f", "scaler_add_f", "power_of")},
    **{f"seera_hip_{n}": ([_vp, _vp, _vp, _i], _i)
       for n in ("elemadd", "elemsub", "elemdiv", "elemmult")},
    "seera_hip_broadcast_add_4d": ([_vp] * 3 + [_i] * 8, _i),
    "seera_hip_broadcast_mul_4d": ([_vp] * 3 + [_i] * 8, _i),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libseera_hip.so and attach the prototypes (raises if missing)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is not built; run `python -m ml_framework_amd.build`")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in PROTOTYPES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = res
        _lib = lib
    return _lib


class SeeraError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"seera_hip status {status}: {msg}")
        self.status = status


def check(status: int) -> None:
    if status != SEERA_OK:
        raise SeeraError(status, load().seera_hip_last_error().decode())


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise on failure."""
    check(getattr(load(), name)(*args))


def gpu_available() -> bool:
    return load().seera_hip_device_count() > 0


class DeviceBuffer:
    """A device allocation made through seera_hip_malloc, freed on close()."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = ctypes.c_void_p()
        check(load().seera_hip_malloc(ctypes.byref(p), self.nbytes))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        buf = cls(a.nbytes)
        check(load().seera_hip_memcpy_h2d(buf.ptr, a.ctypes.data, a.nbytes))
        return buf

    def to_array(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(load().seera_hip_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def fill(self, byte: int) -> None:
        check(load().seera_hip_memset(self.ptr, byte, self.nbytes))

    def close(self) -> None:
        if self.ptr:
            check(load().seera_hip_free(self.ptr))
            self.ptr = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = ctypes.c_void_p()
        check(load().seera_hip_event_create(ctypes.byref(p)))
        self.ptr = p.value

    def record(self, stream=None) -> None:
        check(load().seera_hip_event_record(self.ptr, stream))

    def elapsed_ms(self, end: "Event") -> float:
        ms = ctypes.c_float()
        check(load().seera_hip_event_elapsed_ms(self.ptr, end.ptr, ctypes.byref(ms)))
        return ms.value

    def __del__(self):
        try:
            load().seera_hip_event_destroy(self.ptr)
        except Exception:
            pass
