"""seera_hip_matmul_noalloc: the GEMM forward whose split-K partials go to the
library's fixed device array instead of an allocated workspace. Checked
through the C ABI against seera_hip_matmul_async (the same kernels and plan,
so the same bits) on calls in a row, each next one smaller, including a
GEMM with no split-K, and once under HIP graph capture."""
import ctypes

import numpy as np
import pytest

from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    assert capi.gpu_available(), "no HIP device visible"
    return capi.load()


def _run(lib, name, a, b, M, N, K, nb, stream):
    with DeviceBuffer.from_array(a) as pa, DeviceBuffer.from_array(b) as pb, \
            DeviceBuffer(nb * M * N * 4) as pc:
        pc.fill(0x7F)
        capi.check(getattr(lib, name)(pa.ptr, pb.ptr, pc.ptr, M, N, K, nb, stream))
        capi.check(lib.seera_hip_stream_synchronize(stream))
        return pc.to_array((nb, M, N))


def test_noalloc_matches_async_twice_then_smaller(lib):
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    try:
        r = np.random.default_rng(17)
        # (M, N, K, Nbatch): split-K with large partials, then a smaller one,
        # then a shape with no split (no scratch use) and odd edges.
        for M, N, K, nb in [(256, 256, 8192, 1), (64, 96, 2048, 1), (33, 65, 17, 2),
                            (512, 512, 1024, 1)]:
            a = r.uniform(-1, 1, (nb, M, K)).astype(np.float32)
            b = r.uniform(-1, 1, (K, N)).astype(np.float32)
            want = _run(lib, "seera_hip_matmul_async", a, b, M, N, K, nb, st.value)
            got = _run(lib, "seera_hip_matmul_noalloc", a, b, M, N, K, nb, st.value)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (M, N, K, nb)
            ref = a.astype(np.float16).astype(np.float64) @ b.astype(np.float16).astype(np.float64)
            assert np.linalg.norm(got - ref) <= 1e-3 * np.linalg.norm(ref)
    finally:
        lib.seera_hip_stream_destroy(st.value)


def test_noalloc_under_graph_capture(lib):
    """Captured on a fresh stream (no workspace to size first; only the
    array's address is resolved by one eager call on the device), replayed
    twice: each replay equals the allocating entry point's result."""
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    r = np.random.default_rng(23)
    M, N, K = 64, 128, 4096  # split-K: the partials live in the fixed array
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = r.uniform(-1, 1, (K, N)).astype(np.float32)
    try:
        want = _run(lib, "seera_hip_matmul_async", a, b, M, N, K, 1, st.value)
        _run(lib, "seera_hip_matmul_noalloc", a, b, M, N, K, 1, st.value)  # first call on the device
        with DeviceBuffer.from_array(a) as pa, DeviceBuffer.from_array(b) as pb, \
                DeviceBuffer(M * N * 4) as pc:
            capi.check(lib.seera_hip_graph_capture_begin(st.value))
            status = lib.seera_hip_matmul_noalloc(pa.ptr, pb.ptr, pc.ptr, M, N, K, 1, st.value)
            g = ctypes.c_void_p()
            capi.check(lib.seera_hip_graph_capture_end(st.value, ctypes.byref(g)))
            capi.check(status)
            try:
                for _ in range(2):
                    pc.fill(0x7F)
                    capi.check(lib.seera_hip_synchronize())
                    capi.check(lib.seera_hip_graph_launch(g.value, st.value))
                    capi.check(lib.seera_hip_stream_synchronize(st.value))
                    got = pc.to_array((1, M, N))
                    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
            finally:
                capi.check(lib.seera_hip_graph_destroy(g.value))
    finally:
        lib.seera_hip_stream_destroy(st.value)


def test_noalloc_argument_checks(lib):
    assert lib.seera_hip_matmul_noalloc(None, None, None, -1, 2, 2, 1, None) == \
        capi.SEERA_ERR_INVALID_ARGUMENT
    assert lib.seera_hip_matmul_noalloc(None, None, None, 2, 2, 2, 1, None) == \
        capi.SEERA_ERR_INVALID_ARGUMENT
