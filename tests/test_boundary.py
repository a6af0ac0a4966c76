"""The drop-in boundary, checked on the CPU (no kernel is launched).

* libseera_hip.so loads and exports every function include/seera_hip.h
  declares, with the arity the ctypes binding uses;
* the seera_cuda module loads without a GPU (cuTen.py:3 imports it
  unconditionally) and carries the reference's names and argument counts
  (restated from engine_cuda/src/cuda_bindings.cpp);
* argument validation rejects bad calls with a status and a message before
  any device work.
"""
import ctypes
import os
import re

import pytest

from ml_framework_amd import capi

HEADER = capi.HEADER


def _header_prototypes():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    protos = {}
    for m in re.finditer(r"\b(seera_hip_\w+)\s*\(([^)]*)\)\s*;", text):
        params = [p for p in m.group(2).split(",") if p.strip() and p.strip() != "void"]
        protos[m.group(1)] = len(params)
    return protos


def test_header_declares_the_hot_path():
    protos = _header_prototypes()
    for name in ["seera_hip_matmul", "seera_hip_matmul_bwd", "seera_hip_transpose_2d",
                 "seera_hip_transpose_3d", "seera_hip_conv2d_fwd", "seera_hip_conv2d_bwd",
                 "seera_hip_conv2DTranpose_fwd", "seera_hip_conv2DTranspose_bwd"]:
        assert name in protos


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    raw = ctypes.CDLL(capi.LIB_PATH)
    for name in _header_prototypes():
        assert hasattr(raw, name), f"{name} declared in seera_hip.h but not exported"
    assert lib.seera_hip_version().decode().startswith("seera-hip")


def test_ctypes_prototypes_match_header():
    protos = _header_prototypes()
    assert set(protos) == set(capi.PROTOTYPES)
    for name, nargs in protos.items():
        assert len(capi.PROTOTYPES[name][0]) == nargs, name


# name -> argument count, restated from cuda_bindings.cpp (line in comment)
REFERENCE_SIGNATURES = {
    "cuda_malloc": 1,                    # 23
    "cuda_malloc_f16": 1,                # 30
    "cuda_malloc_f32": 1,                # 37
    "cuda_malloc_i32": 1,                # 44
    "cuda_malloc_i16": 1,                # 51
    "cuda_free": 1,                      # 58
    "cuda_memcopy_devicetodevice": 3,    # 61
    "cuda_memset": 3,                    # 65
    "to_device_f16": 1,                  # 73
    "to_host_f16": 2,                    # 82
    "to_device_f32": 1,                  # 98
    "to_host_f32": 2,                    # 107
    "to_host_i32": 2,                    # 123
    "to_host_i16": 2,                    # 139
    "to_device_i16": 1,                  # 155
    "to_device_i32": 1,                  # 164
    "cuda_matmul": 7,                    # 260 (A, B, C, M, N, K, Nbatch)
    "cuda_matmul_bwd": 9,                # 267 (A, B, dC, dA, dB, M, N, K, Nbatch)
    "cuda_transpose_2d": 4,              # 276 (in, out, rows, cols)
    "cuda_transpose_3d": 5,              # 283 (in, out, Nbatch, M, K)
    "cuda_conv2d_fwd": 14,               # 294 (..., pad_h, pad_w, stride_h, stride_w)
    "cuda_conv2d_bwd": 16,               # 302 (..., strideh, stridew, padh, padw)
    "cuda_conv2DTranpose_fwd": 14,       # 316 [sic]
    "cuda_conv2DTranspose_bwd": 16,      # 324
    "cuda_ones_f": 1,                    # 467 (total_elements) -> device pointer
    "cuda_zeros_f": 1,                   # 474 (total_elements) -> device pointer
    "cuda_maxpool_fwd": 13,              # 338 (image, out, mask, N, C, H, W, R, S, ph, pw, sh, sw)
    "cuda_maxpool_bwd": 13,              # 346 (dout, mask, dX, N, C, H, W, R, S, ph, pw, sh, sw)
    "cuda_relu_fwd": 4,                  # 176 (x, out, grad, size)
    "cuda_sigmoid_fwd": 4,               # 183
    "cuda_tanh_fwd": 4,                  # 190
    "cuda_log_fwd": 4,                   # 197
    "cuda_exp_fwd": 4,                   # 204
    "cuda_abs_fwd": 4,                   # 211
    "cuda_sqrt_fwd": 4,                  # 218
    "cuda_pow_fwd": 5,                   # 225 (x, exponent, out, grad, size)
    "cuda_clip_fwd": 6,                  # 232 (x, lo, hi, out, grad, size)
    "cuda_softmax_fwd": 4,               # 243 (x, out, N, C)
    "cuda_softmax_vjp": 5,               # 249 (s, dout, dx, N, C)
    "cuda_unpooling_fwd": 8,             # 358 (inp, out, batchN, C, H, W, sh, sw)
    "cuda_unpooling_bwd": 8,             # 365 (dout, dx, batchN, C, H, W, sh, sw)
    "cuda_sum_fwd": 5,                   # 376 (A, out, ndims, dim, dimarr)
    "cuda_mean_fwd": 5,                  # 384
    "cuda_max_fwd": 5,                   # 392
    "cuda_min_fwd": 5,                   # 400
    "cuda_argmax_fwd": 5,                # 408
    "cuda_argmin_fwd": 5,                # 416
    "cuda_sum_bwd": 5,                   # 426 (dOut, dA, ndims, dim, dimarr)
    "cuda_mean_bwd": 5,                  # 434
    "cuda_max_bwd": 7,                   # 442 (dOut, fwdInput, fwdOutput, dA, ndims, dim, dimarr)
    "cuda_min_bwd": 7,                   # 452
    "cuda_scaler_multiply_f": 3,         # 461 (arr, k, total_elements)
    "cuda_scaler_add_f": 3,              # 464
    "cuda_power_of": 3,                  # 479
    "cuda_elemadd": 4,                   # 486 (A, B, C, size)
    "cuda_elemsub": 4,                   # 493
    "cuda_elemdiv": 4,                   # 500
    "cuda_elemmult": 4,                  # 507
    "broadcast_add_4d": 11,              # 518 (A, B, C, aN, aC, aH, aW, bN, bC, bH, bW)
    "broadcast_mul_4d": 11,              # 526
}


def test_reference_signature_table_is_complete():
    """Every name cuda_bindings.cpp defines (60) is in the table."""
    assert len(REFERENCE_SIGNATURES) == 60


def _arity(fn):
    first = fn.__doc__.strip().splitlines()[0]
    inner = first[first.index("(") + 1:first.rindex(")")]
    return 0 if not inner.strip() else inner.count(":")


def test_seera_cuda_module_signatures():
    import ml_framework_amd

    mod = ml_framework_amd.seera_cuda()
    for name, n in REFERENCE_SIGNATURES.items():
        assert hasattr(mod, name), name
        assert _arity(getattr(mod, name)) == n, name


def _status(name, *args):
    lib = capi.load()
    st = getattr(lib, name)(*args)
    return st, lib.seera_hip_last_error().decode()


def test_validation_negative_dims():
    st, msg = _status("seera_hip_matmul", None, None, None, -1, 4, 4, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "dims" in msg


def test_validation_null_pointers():
    st, msg = _status("seera_hip_matmul", None, None, None, 4, 4, 4, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "null" in msg
    st, _ = _status("seera_hip_conv2d_fwd", None, None, None, 1, 3, 8, 8, 4, 3, 3, 1, 1, 1, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT


@pytest.mark.parametrize("args,what", [
    ((2, 3, 8, 8, 4, 3, 3, 1, 1, 0, 1), "stride"),      # stride_h = 0
    ((2, 3, 8, 8, 4, 3, 3, -1, 1, 1, 1), "padding"),    # pad_h < 0
    ((2, 3, 8, 8, 4, 0, 3, 1, 1, 1, 1), "kernel"),      # R = 0
    ((2, 3, 2, 8, 4, 5, 3, 0, 1, 1, 1), "larger"),      # R > H + 2 pad
])
def test_validation_conv_geometry(args, what):
    st, msg = _status("seera_hip_conv2d_fwd", 1, 1, 1, *args)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and what in msg, msg


def test_validation_convT_output_extent():
    # Hout = (1 - 1) * 1 - 2 * 3 + 3 < 1
    st, msg = _status("seera_hip_conv2DTranpose_fwd", 1, 1, 1, 1, 2, 1, 1, 2, 3, 3, 1, 1, 3, 3)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "extent" in msg


def test_no_device_is_a_clean_error():
    if capi.gpu_available():
        pytest.skip("a GPU is present")
    assert capi.load().seera_hip_device_count() <= 0
    p = ctypes.c_void_p()
    st = capi.load().seera_hip_malloc(ctypes.byref(p), 1024)
    assert st != capi.SEERA_OK and capi.load().seera_hip_last_error()


@pytest.mark.parametrize("args,what", [
    ((2, 3, 8, 8, 2, 2, 0, 0, 0, 2), "stride"),          # stride_h = 0
    ((2, 3, 8, 8, 2, 2, -1, 0, 2, 2), "padding"),        # pad_h < 0
    ((2, 3, 2, 8, 5, 2, 1, 0, 1, 1), "larger"),          # R > H + 2 pad
    ((2, 0, 8, 8, 2, 2, 0, 0, 2, 2), "dims"),            # C = 0
    ((1, 1, 8, 8, 2, 2, 1 << 21, 0, 1, 1), "2^20"),      # pad near int overflow
])
def test_validation_maxpool(args, what):
    for name in ("seera_hip_maxpool_fwd", "seera_hip_maxpool_bwd"):
        st, msg = _status(name, 1, 1, 1, *args)
        assert st == capi.SEERA_ERR_INVALID_ARGUMENT and what in msg, (name, msg)


def test_validation_fused_entry_points():
    """Argument checks of the entry points with no reference counterpart run
    before any device work."""
    st, msg = _status("seera_hip_conv2d_fwd_bias_act", 1, 1, None, 1, None, 1, 1, 4, 4, 1, 3, 3,
                      1, 1, 1, 1, 5)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "activation" in msg, msg
    st, msg = _status("seera_hip_conv2d_fwd_bias_act", 1, 1, None, 1, None, 1, 1, 2, 4, 1, 5, 3,
                      0, 1, 1, 1, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "larger" in msg, msg
    st, msg = _status("seera_hip_conv2d_bwd_bias", 1, 1, 1, 1, 1, None, 2, 3, 8, 8, 4, 3, 3,
                      1, 1, 1, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "db" in msg, msg
    st, msg = _status("seera_hip_conv2d_bwd_bias", 1, 1, 1, 1, 1, 1, 2, 3, 8, 8, 4, 3, 3,
                      0, 1, 1, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "stride" in msg, msg
    st, msg = _status("seera_hip_conv_bias_grad", 1, 1, -1, 4, 9)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "dims" in msg, msg
    st, msg = _status("seera_hip_matmul_bwd_relu", 1, 1, 1, None, 1, 1, 4, 4, 4, 1)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "null" in msg, msg
    st, msg = _status("seera_hip_matmul_bias_act", 1, 1, None, 1, None, 4, 4, 4, 1, 3)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "activation" in msg, msg
    st, msg = _status("seera_hip_graph_capture_begin", None)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT, msg
    st, msg = _status("seera_hip_graph_launch", None, None)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT, msg


@pytest.mark.parametrize("name,args,what", [
    ("seera_hip_relu_fwd", (1, 1, 1, -1), "size"),
    ("seera_hip_clip_fwd", (1, 0.0, 1.0, 1, 1, -3), "size"),
    ("seera_hip_elemadd", (1, 1, 1, -1), "size"),
    ("seera_hip_elemadd", (None, 1, 1, 4), "null"),
    ("seera_hip_scaler_add_f", (1, 1.0, -2), "total_elements"),
    ("seera_hip_softmax_fwd", (1, 1, -1, 4), "N and C"),
    ("seera_hip_unpooling_fwd", (1, 1, 1, 1, 2, 2, 0, 2), "scale"),
    ("seera_hip_unpooling_bwd", (1, 1, 1, -1, 2, 2, 2, 2), "negative"),
    ("seera_hip_broadcast_add_4d", (1, 1, 1, 2, 3, 4, 5, 1, 2, 1, 1), "broadcast"),
    ("seera_hip_broadcast_mul_4d", (1, 1, 1, 2, 3, 4, -5, 1, 1, 1, 1), "negative"),
])
def test_validation_tensor_ops(name, args, what):
    st, msg = _status(name, *args)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and what in msg, (name, msg)


def test_validation_reductions():
    dims = (ctypes.c_int * 2)(2, 3)
    st, msg = _status("seera_hip_sum_fwd", 1, 1, 2, 2, dims)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "dim" in msg, msg
    st, msg = _status("seera_hip_max_fwd", 1, 1, 2, -1, dims)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "dim" in msg, msg
    st, msg = _status("seera_hip_mean_bwd", 1, 1, 2, 0, None)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "extents" in msg, msg
    empty = (ctypes.c_int * 2)(2, 0)
    st, msg = _status("seera_hip_argmax_fwd", 1, 1, 2, 1, empty)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "empty" in msg, msg
    st, msg = _status("seera_hip_max_bwd", 1, 1, None, 1, 2, 0, dims)
    assert st == capi.SEERA_ERR_INVALID_ARGUMENT and "null" in msg, msg


def test_seera_cuda_reduction_checks_dimarr_length():
    import ml_framework_amd
    import numpy as np

    mod = ml_framework_amd.seera_cuda()
    with pytest.raises(ValueError, match="dimarr"):
        mod.cuda_sum_fwd(1, 1, 3, 0, np.array([2, 3], np.int32))
