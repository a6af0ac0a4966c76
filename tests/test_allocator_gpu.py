"""The caching allocator behind seera_hip_malloc / seera_hip_free (the
reference cudaMallocs and cudaFrees every buffer: cuTen.py:77-84,
cuda_bindings.cpp:23-59) and the allocate-and-fill entry points cuda_ones_f /
cuda_zeros_f (cuda_bindings.cpp:467-477)."""
import ctypes

import numpy as np
import pytest

import oracle
from ml_framework_amd import capi
from ml_framework_amd.capi import DeviceBuffer, Event, check, load
from oracle import fp16r
from tests.helpers import assert_parity

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def sc():
    import ml_framework_amd

    assert capi.gpu_available(), "no HIP device visible"
    return ml_framework_amd.seera_cuda()


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000, 4097, 1 << 20])
def test_ones_and_zeros(sc, n):
    p1, p0 = sc.cuda_ones_f(n), sc.cuda_zeros_f(n)
    assert (sc.to_host_f32(p1, (n,)) == 1.0).all()
    assert (sc.to_host_f32(p0, (n,)) == 0.0).all()
    sc.cuda_free(p1)
    sc.cuda_free(p0)


@pytest.mark.parametrize("off,count", [(0, 37), (1, 37), (2, 3), (3, 64), (1, 0)])
def test_fill_stays_in_range(off, count):
    """Unaligned starts and short counts: exactly [off, off + count) changes."""
    with DeviceBuffer(128 * 4) as buf:
        buf.fill(0x7F)  # sentinel bytes
        check(load().seera_hip_fill_f32(buf.ptr + 4 * off, ctypes.c_float(2.5), count))
        got = buf.to_array((128,))
        sentinel = np.frombuffer(b"\x7f" * 4, np.float32)[0]
        want = np.full(128, sentinel, np.float32)
        want[off:off + count] = 2.5
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _stats():
    live, cached = ctypes.c_size_t(), ctypes.c_size_t()
    check(load().seera_hip_memory_stats(ctypes.byref(live), ctypes.byref(cached)))
    return live.value, cached.value


def test_freed_block_is_reused_by_its_size_class(sc):
    sc.cuda_empty_cache()
    assert _stats()[1] == 0
    p = sc.cuda_malloc_f32(1000)        # 4000 B: the 4096 B class
    live0 = _stats()[0]
    sc.cuda_free(p)
    assert _stats() == (live0 - 4096, 4096)
    q = sc.cuda_malloc_f32(900)         # 3600 B: same class, same block
    assert q == p
    r = sc.cuda_malloc_f32(3 << 20)     # 12 MiB: a class of its own
    assert r != q
    big = 3 << 22                       # 12 MiB in bytes
    sc.cuda_free(r)
    assert _stats()[1] == big
    r2 = sc.cuda_malloc(big - 100)      # rounds to the same 2 MiB multiple
    assert r2 == r
    for x in (q, r2):
        sc.cuda_free(x)
    sc.cuda_empty_cache()
    assert _stats()[1] == 0


def test_reused_block_holds_the_new_contents(sc):
    a = np.arange(256, dtype=np.float32)
    p = sc.to_device_f32(a)
    sc.cuda_free(p)
    b = -np.arange(256, dtype=np.float32)
    q = sc.to_device_f32(b)
    assert q == p
    assert np.array_equal(sc.to_host_f32(q, (256,)), b)
    sc.cuda_free(q)


def test_free_after_async_work_waits_for_it():
    """A free that follows an *_async launch synchronizes the device before the
    block can be handed out again (cudaFree semantics): the work queued on a
    user stream has finished by the time the free returns."""
    lib = load()
    n = 4096
    r = np.random.default_rng(7)
    a = r.uniform(-1, 1, (n, n)).astype(np.float32)
    b = r.uniform(-1, 1, (n, n)).astype(np.float32)
    st = ctypes.c_void_p()
    check(lib.seera_hip_stream_create(ctypes.byref(st)))
    try:
        A, B, C = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b), DeviceBuffer(a.nbytes)
        e0, e1 = Event(), Event()
        e0.record(st.value)
        check(lib.seera_hip_matmul_async(A.ptr, B.ptr, C.ptr, n, n, n, 1, st.value))
        e1.record(st.value)
        A.close()  # must wait for the matmul still reading A
        assert e0.elapsed_ms(e1) > 0.0  # both events complete: no hipErrorNotReady
        rows = np.arange(0, n, 257)
        got = C.to_array((n, n))[rows]
        assert_parity(got, fp16r(a[rows]).astype(np.float64) @ fp16r(b), "C rows")
        B.close()
        C.close()
    finally:
        check(lib.seera_hip_stream_destroy(st.value))


def _malloc_async(n, st):
    p = ctypes.c_void_p()
    check(load().seera_hip_malloc_async(ctypes.byref(p), n, st))
    return p.value


def _matmul_into(c_ptr, a, b, st):
    """C = A.B queued on st (A, B uploaded to fresh buffers kept alive by the caller)."""
    A, B = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b)
    check(load().seera_hip_matmul_async(A.ptr, B.ptr, c_ptr, a.shape[0], b.shape[1], a.shape[1], 1, st))
    return A, B


def test_stream_ordered_reuse_on_one_stream():
    """seera_hip_free_async then seera_hip_malloc_async on the same stream hands
    the block back at once, and work queued after it sees its own results."""
    lib = load()
    r = np.random.default_rng(3)
    n = 512
    a1, b1, a2, b2 = (r.uniform(-1, 1, (n, n)).astype(np.float32) for _ in range(4))
    st = ctypes.c_void_p()
    check(lib.seera_hip_stream_create(ctypes.byref(st)))
    try:
        p = _malloc_async(n * n * 4, st.value)
        keep1 = _matmul_into(p, a1, b1, st.value)
        check(lib.seera_hip_free_async(p, st.value))
        q = _malloc_async(n * n * 4, st.value)
        assert q == p
        keep2 = _matmul_into(q, a2, b2, st.value)
        check(lib.seera_hip_stream_synchronize(st.value))
        got = np.empty((n, n), np.float32)
        check(lib.seera_hip_memcpy_d2h(got.ctypes.data, q, got.nbytes))
        assert_parity(got, fp16r(a2).astype(np.float64) @ fp16r(b2), "C after reuse")
        check(lib.seera_hip_free_async(q, st.value))
        del keep1, keep2
    finally:
        check(lib.seera_hip_stream_destroy(st.value))


def test_stream_ordered_free_waits_for_other_streams():
    """A block freed on one stream with work still queued there is not handed
    to another stream until that work has completed; afterwards it is."""
    lib = load()
    n = 4096
    r = np.random.default_rng(5)
    a = r.uniform(-1, 1, (n, n)).astype(np.float32)
    b = r.uniform(-1, 1, (n, n)).astype(np.float32)
    s1, s2 = ctypes.c_void_p(), ctypes.c_void_p()
    check(lib.seera_hip_stream_create(ctypes.byref(s1)))
    check(lib.seera_hip_stream_create(ctypes.byref(s2)))
    try:
        A, B = DeviceBuffer.from_array(a), DeviceBuffer.from_array(b)
        p = _malloc_async(n * n * 4, s1.value)
        e0, e1 = Event(), Event()
        e0.record(s1.value)
        for _ in range(8):  # ~1 ms of work writing p
            check(lib.seera_hip_matmul_async(A.ptr, B.ptr, p, n, n, n, 1, s1.value))
        check(lib.seera_hip_free_async(p, s1.value))
        e1.record(s1.value)
        q = _malloc_async(n * n * 4, s2.value)
        try:
            e0.elapsed_ms(e1)
            s1_done = True
        except capi.SeeraError:
            s1_done = False  # the GEMMs are still running
        if not s1_done:
            assert q != p
        check(lib.seera_hip_free_async(q, s2.value))
        check(lib.seera_hip_stream_synchronize(s1.value))
        check(lib.seera_hip_stream_synchronize(s2.value))
        p2 = _malloc_async(n * n * 4, s2.value)
        assert p2 in (p, q)  # both frees have completed: either block may come back
        got = np.empty((n, n), np.float32)
        check(lib.seera_hip_memcpy_d2h(got.ctypes.data, p, got.nbytes))
        rows = np.arange(0, n, 511)
        assert_parity(got[rows], fp16r(a[rows]).astype(np.float64) @ fp16r(b), "C rows")
        check(lib.seera_hip_free_async(p2, s2.value))
        A.close()
        B.close()
    finally:
        check(lib.seera_hip_stream_destroy(s1.value))
        check(lib.seera_hip_stream_destroy(s2.value))


def test_free_async_rejects_foreign_pointers_and_counts_pending_bytes():
    lib = load()
    check(lib.seera_hip_empty_cache())
    p = _malloc_async(1 << 20, None)
    assert lib.seera_hip_free_async(p + 256, None) == capi.SEERA_ERR_INVALID_ARGUMENT
    live0, cached0 = _stats()
    check(lib.seera_hip_free_async(p, None))
    live1, cached1 = _stats()
    assert live1 == live0 - (1 << 20) and cached1 == cached0 + (1 << 20)
    check(lib.seera_hip_empty_cache())
    assert _stats()[1] == 0
