"""HIP-graph capture and replay of the _async entry points: a Dense MLP step
(fused forward, backward GEMMs, bias gradients) and a Conv2D + MaxPool layer
pair. Each graph is replayed several times with new inputs written between the
replays, with eager calls of the same sequence in between, and every replay
must equal the eager result bit for bit (every kernel here is deterministic).
"""
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


@pytest.fixture
def stream(lib):
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    yield st.value
    lib.seera_hip_stream_destroy(st.value)


def _capture(lib, stream, seq):
    capi.check(lib.seera_hip_graph_capture_begin(stream))
    try:
        seq()
    finally:
        g = ctypes.c_void_p()
        st = lib.seera_hip_graph_capture_end(stream, ctypes.byref(g))
    capi.check(st)
    return g.value


def _upload(buf, a):
    capi.check(capi.load().seera_hip_memcpy_h2d(buf.ptr, np.ascontiguousarray(a).ctypes.data,
                                                a.nbytes))


def _replays_match_eager(lib, stream, seq, inputs, outputs, make_inputs, replays=3):
    """seq() queues the sequence on `stream`; inputs: [(buf, shape)];
    outputs: [(buf, shape, dtype)]."""
    seq()  # eager warm-up: the workspace reaches its size outside capture
    capi.check(lib.seera_hip_stream_synchronize(stream))
    g = _capture(lib, stream, seq)
    try:
        for rep in range(replays):
            vals = make_inputs(rep)
            for (buf, _), v in zip(inputs, vals):
                _upload(buf, v)
            capi.check(lib.seera_hip_graph_launch(g, stream))
            capi.check(lib.seera_hip_stream_synchronize(stream))
            got = [b.to_array(shape, dt) for b, shape, dt in outputs]
            for b, _, _ in outputs:
                b.fill(0x7F)
            seq()  # the same inputs, eagerly
            capi.check(lib.seera_hip_stream_synchronize(stream))
            want = [b.to_array(shape, dt) for b, shape, dt in outputs]
            for i, (x, y) in enumerate(zip(got, want)):
                assert np.array_equal(x, y, equal_nan=True), (rep, i)
    finally:
        lib.seera_hip_graph_destroy(g)


def test_mlp_step_graph(lib, stream):
    r = np.random.default_rng(0)
    dims, B = [784, 512, 256, 10], 256
    acts = [DeviceBuffer(B * d * 4) for d in dims]
    masks = [DeviceBuffer(B * d * 4) for d in dims[1:]]
    ws = [DeviceBuffer.from_array(r.uniform(-0.05, 0.05, (i, o)).astype(np.float32))
          for i, o in zip(dims[:-1], dims[1:])]
    bs = [DeviceBuffer.from_array(r.uniform(-0.1, 0.1, o).astype(np.float32)) for o in dims[1:]]
    grads = [DeviceBuffer(B * d * 4) for d in dims]
    dws = [DeviceBuffer(i * o * 4) for i, o in zip(dims[:-1], dims[1:])]
    dbs = [DeviceBuffer(o * 4) for o in dims[1:]]

    def seq():
        for li in range(3):
            act = capi.SEERA_ACT_RELU if li < 2 else capi.SEERA_ACT_NONE
            capi.check(lib.seera_hip_matmul_bias_act_async(
                acts[li].ptr, ws[li].ptr, bs[li].ptr, acts[li + 1].ptr, masks[li].ptr, B,
                dims[li + 1], dims[li], 1, act, stream))
        for li in (2, 1, 0):
            capi.check(lib.seera_hip_bias_grad_async(grads[li + 1].ptr, dbs[li].ptr, B,
                                                     dims[li + 1], stream))
            capi.check(lib.seera_hip_matmul_bwd_async(acts[li].ptr, ws[li].ptr,
                                                      grads[li + 1].ptr, grads[li].ptr,
                                                      dws[li].ptr, B, dims[li + 1], dims[li], 1,
                                                      stream))

    def make_inputs(rep):
        g = np.random.default_rng(rep + 10)
        return [g.uniform(0, 1, (B, 784)).astype(np.float32),
                g.standard_normal((B, 10)).astype(np.float32)]

    outputs = [(acts[3], (B, 10), np.float32), (masks[0], (B, 512), np.float32),
               (grads[0], (B, 784), np.float32)] + \
        [(dws[i], (dims[i], dims[i + 1]), np.float32) for i in range(3)] + \
        [(dbs[i], (dims[i + 1],), np.float32) for i in range(3)]
    _replays_match_eager(lib, stream, seq, [(acts[0], None), (grads[3], None)], outputs,
                         make_inputs)


def test_conv_pool_layer_graph(lib, stream):
    r = np.random.default_rng(1)
    N, C, H, W, F = 8, 32, 28, 28, 64
    px = DeviceBuffer(N * C * H * W * 4)
    pw = DeviceBuffer.from_array((r.standard_normal((F, C, 3, 3)) * 0.1).astype(np.float32))
    pb = DeviceBuffer.from_array(r.uniform(-0.1, 0.1, F).astype(np.float32))
    py, pm = DeviceBuffer(N * F * H * W * 4), DeviceBuffer(N * F * H * W * 4)
    pp, ppm = DeviceBuffer(N * F * 14 * 14 * 4), DeviceBuffer(N * F * H * W * 4)
    pq, ppm3 = DeviceBuffer(N * F * 14 * 14 * 4), DeviceBuffer(N * F * H * W * 4)
    pg, pdx, pdx3 = DeviceBuffer(N * F * 14 * 14 * 4), DeviceBuffer(N * F * H * W * 4), \
        DeviceBuffer(N * F * H * W * 4)
    pdb = DeviceBuffer(F * 4)

    def seq():
        capi.check(lib.seera_hip_conv2d_fwd_bias_act_async(
            px.ptr, pw.ptr, pb.ptr, py.ptr, pm.ptr, N, C, H, W, F, 3, 3, 1, 1, 1, 1,
            capi.SEERA_ACT_RELU, stream))
        pool = (N, F, H, W, 2, 2, 0, 0, 2, 2, stream)
        capi.check(lib.seera_hip_maxpool_fwd_async(py.ptr, pp.ptr, ppm.ptr, *pool))
        capi.check(lib.seera_hip_maxpool_bwd_async(pg.ptr, ppm.ptr, pdx.ptr, *pool))
        pool3 = (N, F, H, W, 3, 3, 1, 1, 2, 2, stream)  # overlapping: mask cleared by a kernel
        capi.check(lib.seera_hip_maxpool_fwd_async(py.ptr, pq.ptr, ppm3.ptr, *pool3))
        capi.check(lib.seera_hip_maxpool_bwd_async(pg.ptr, ppm3.ptr, pdx3.ptr, *pool3))
        capi.check(lib.seera_hip_conv_bias_grad_async(pdx.ptr, pdb.ptr, N, F, H * W, stream))

    def make_inputs(rep):
        g = np.random.default_rng(rep + 20)
        return [g.standard_normal((N, C, H, W)).astype(np.float32),
                g.standard_normal((N, F, 14, 14)).astype(np.float32)]

    sh = (N, F, H, W)
    outputs = [(py, sh, np.float32), (pm, sh, np.float32), (pp, (N, F, 14, 14), np.float32),
               (ppm, sh, np.int32), (pdx, sh, np.float32), (pq, (N, F, 14, 14), np.float32),
               (ppm3, sh, np.int32), (pdx3, sh, np.float32), (pdb, (F,), np.float32)]
    _replays_match_eager(lib, stream, seq, [(px, None), (pg, None)], outputs, make_inputs)


def test_capture_needs_a_created_stream(lib):
    assert lib.seera_hip_graph_capture_begin(None) == capi.SEERA_ERR_INVALID_ARGUMENT
