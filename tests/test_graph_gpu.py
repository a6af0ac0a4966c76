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


def _stats(lib):
    held, retired = ctypes.c_size_t(), ctypes.c_size_t()
    capi.check(lib.seera_hip_workspace_stats(ctypes.byref(held), ctypes.byref(retired)))
    return held.value, retired.value


def _splitk_gemm(lib, a, b, c, M, N, K, stream):
    # M, N small against K: the planner splits K and the partials go to the
    # stream's workspace.
    capi.check(lib.seera_hip_matmul_async(a.ptr, b.ptr, c.ptr, M, N, K, 1, stream))


def test_replay_after_workspace_growth(lib, stream):
    """A graph keeps the workspace address it was captured with. An eager
    call that grows the stream's workspace between replays must not free that
    buffer: the old one is retired until the graph is destroyed, and every
    replay still equals the eager result bit for bit."""
    r = np.random.default_rng(3)
    K = 8192
    a = DeviceBuffer.from_array(r.uniform(-1, 1, (64, K)).astype(np.float32))
    b = DeviceBuffer.from_array(r.uniform(-1, 1, (K, 64)).astype(np.float32))
    c = DeviceBuffer(64 * 64 * 4)
    a2 = DeviceBuffer.from_array(r.uniform(-1, 1, (256, K)).astype(np.float32))
    b2 = DeviceBuffer.from_array(r.uniform(-1, 1, (K, 256)).astype(np.float32))
    c2 = DeviceBuffer(256 * 256 * 4)
    _splitk_gemm(lib, a, b, c, 64, 64, K, stream)  # sizes the workspace
    capi.check(lib.seera_hip_stream_synchronize(stream))
    want = c.to_array((64, 64))
    _, retired0 = _stats(lib)
    g = _capture(lib, stream, lambda: _splitk_gemm(lib, a, b, c, 64, 64, K, stream))
    try:
        for rep in range(3):
            # 16x the partials of the captured call: the workspace grows.
            _splitk_gemm(lib, a2, b2, c2, 256, 256, K, stream)
            capi.check(lib.seera_hip_stream_synchronize(stream))
            if rep == 0:
                assert _stats(lib)[1] >= retired0 + 1, "old workspace was not retired"
            c.fill(0x7F)
            capi.check(lib.seera_hip_graph_launch(g, stream))
            capi.check(lib.seera_hip_stream_synchronize(stream))
            assert np.array_equal(c.to_array((64, 64)), want), rep
    finally:
        capi.check(lib.seera_hip_graph_destroy(g))
    assert _stats(lib)[1] == retired0, "retired workspaces not released with the graph"


def test_release_workspace_of_a_callers_stream(lib):
    """seera_hip_stream_release_workspace frees a stream's workspace once its
    queued work is done (the held bytes drop by what the stream held); a
    later call on the stream starts a new workspace and still computes the
    same result; releasing twice, or a stream that never had one, is a no-op."""
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    r = np.random.default_rng(6)
    K = 8192
    a = DeviceBuffer.from_array(r.uniform(-1, 1, (64, K)).astype(np.float32))
    b = DeviceBuffer.from_array(r.uniform(-1, 1, (K, 64)).astype(np.float32))
    c = DeviceBuffer(64 * 64 * 4)
    try:
        held0, _ = _stats(lib)
        _splitk_gemm(lib, a, b, c, 64, 64, K, st.value)  # queued: the release must wait for it
        held1, _ = _stats(lib)
        assert held1 > held0, "the split-K call took no workspace"
        capi.check(lib.seera_hip_stream_release_workspace(st.value))
        assert _stats(lib)[0] == held0
        want = c.to_array((64, 64))
        c.fill(0x7F)
        _splitk_gemm(lib, a, b, c, 64, 64, K, st.value)
        capi.check(lib.seera_hip_stream_synchronize(st.value))
        assert np.array_equal(c.to_array((64, 64)), want)
        capi.check(lib.seera_hip_stream_release_workspace(st.value))
        capi.check(lib.seera_hip_stream_release_workspace(st.value))
        assert _stats(lib)[0] == held0
        capi.check(lib.seera_hip_stream_release_workspace(None))
    finally:
        capi.check(lib.seera_hip_stream_destroy(st.value))


def test_growth_under_capture_is_a_clean_error(lib):
    """A call that would have to grow its stream's workspace during capture
    fails with SEERA_ERR_INVALID_ARGUMENT instead of recording a buffer a
    later call could free."""
    st = ctypes.c_void_p()
    capi.check(lib.seera_hip_stream_create(ctypes.byref(st)))
    r = np.random.default_rng(4)
    K = 4096
    a = DeviceBuffer.from_array(r.uniform(-1, 1, (32, K)).astype(np.float32))
    b = DeviceBuffer.from_array(r.uniform(-1, 1, (K, 32)).astype(np.float32))
    c = DeviceBuffer(32 * 32 * 4)
    try:
        capi.check(lib.seera_hip_graph_capture_begin(st.value))
        status = lib.seera_hip_matmul_async(a.ptr, b.ptr, c.ptr, 32, 32, K, 1, st.value)
        msg = lib.seera_hip_last_error().decode()
        g = ctypes.c_void_p()
        end = lib.seera_hip_graph_capture_end(st.value, ctypes.byref(g))
        if end == capi.SEERA_OK:
            capi.check(lib.seera_hip_graph_destroy(g.value))
        assert status == capi.SEERA_ERR_INVALID_ARGUMENT and "capture" in msg, msg
        # The same call outside capture sizes the workspace and succeeds.
        capi.check(lib.seera_hip_matmul_async(a.ptr, b.ptr, c.ptr, 32, 32, K, 1, st.value))
        capi.check(lib.seera_hip_stream_synchronize(st.value))
    finally:
        lib.seera_hip_stream_destroy(st.value)


def test_async_calls_on_two_streams(lib):
    """Split-K GEMMs and conv backward passes (dW partials) queued on two
    streams at once: each stream has its own workspace, so both results equal
    the same calls run one at a time."""
    streams = []
    for _ in range(2):
        s = ctypes.c_void_p()
        capi.check(lib.seera_hip_stream_create(ctypes.byref(s)))
        streams.append(s.value)
    r = np.random.default_rng(5)
    K = 8192
    gem = [(DeviceBuffer.from_array(r.uniform(-1, 1, (m, K)).astype(np.float32)),
            DeviceBuffer.from_array(r.uniform(-1, 1, (K, m)).astype(np.float32)),
            DeviceBuffer(m * m * 4), m) for m in (64, 96)]
    N, C, H, W, F = 4, 16, 20, 20, 32
    conv = []
    for _ in range(2):
        conv.append([DeviceBuffer.from_array(r.standard_normal(s).astype(np.float32))
                     for s in ((F, C, 3, 3), (N, C, H, W), (N, F, H, W))] +
                    [DeviceBuffer(N * C * H * W * 4), DeviceBuffer(F * C * 9 * 4)])

    def queue(i, st):
        a, b, c, m = gem[i]
        capi.check(lib.seera_hip_matmul_async(a.ptr, b.ptr, c.ptr, m, m, K, 1, st))
        w, x, dy, dx, dw = conv[i]
        capi.check(lib.seera_hip_conv2d_bwd_async(w.ptr, x.ptr, dy.ptr, dx.ptr, dw.ptr, N, C, H,
                                                  W, F, 3, 3, 1, 1, 1, 1, st))

    def results(i):
        return [gem[i][2].to_array((gem[i][3],) * 2), conv[i][3].to_array((N, C, H, W)),
                conv[i][4].to_array((F, C, 3, 3))]

    try:
        want = []
        for i in range(2):  # one at a time
            queue(i, streams[i])
            capi.check(lib.seera_hip_stream_synchronize(streams[i]))
            want.append(results(i))
        for rep in range(3):
            for i in range(2):
                for buf in (gem[i][2], conv[i][3], conv[i][4]):
                    buf.fill(0x7F)
            capi.check(lib.seera_hip_synchronize())
            for i in range(2):  # both queued before either is waited for
                queue(i, streams[i])
            for s in streams:
                capi.check(lib.seera_hip_stream_synchronize(s))
            for i in range(2):
                for j, (x, y) in enumerate(zip(results(i), want[i])):
                    assert np.array_equal(x, y), (rep, i, j)
    finally:
        for s in streams:
            lib.seera_hip_stream_destroy(s)


def test_convT_backward_graph(lib, stream):
    """ConvTranspose2D config 5 backward (weight prep, stride-2 dX, stride-2 dW
    partials and their reduce) captured and replayed."""
    r = np.random.default_rng(4)
    N, Ci, H, W, Co = 32, 128, 28, 28, 64
    x = DeviceBuffer(N * Ci * H * W * 4)
    dy = DeviceBuffer(N * Co * 56 * 56 * 4)
    w = DeviceBuffer.from_array((r.standard_normal((Ci, Co, 4, 4)) * 0.05).astype(np.float32))
    dx, dw = DeviceBuffer(N * Ci * H * W * 4), DeviceBuffer(Ci * Co * 16 * 4)

    def seq():
        capi.check(lib.seera_hip_conv2DTranspose_bwd_async(w.ptr, x.ptr, dy.ptr, dx.ptr, dw.ptr, N,
                                                           Ci, H, W, Co, 4, 4, 2, 2, 1, 1, stream))

    def make_inputs(rep):
        g = np.random.default_rng(10 + rep)
        return [g.standard_normal((N, Ci, H, W)).astype(np.float32),
                g.standard_normal((N, Co, 56, 56)).astype(np.float32)]

    _replays_match_eager(lib, stream, seq, [(x, None), (dy, None)],
                         [(dx, (N, Ci, H, W), np.float32), (dw, (Ci, Co, 4, 4), np.float32)],
                         make_inputs)


def test_staged_layouts_graph(lib, stream):
    """Convolutions that stage a re-laid-out operand in the second per-stream
    buffer: a 14x14 layer (rows widened to 16 floats for the forward, dX and
    dW) and a 7x7 stride-2 stem (space-to-depth) forward and backward, with
    bias and ReLU on the stem, captured and replayed."""
    r = np.random.default_rng(5)
    N, C, H, W, F = 4, 64, 14, 14, 64
    x = DeviceBuffer(N * C * H * W * 4)
    w = DeviceBuffer.from_array((r.standard_normal((F, C, 3, 3)) * 0.05).astype(np.float32))
    y, dx = DeviceBuffer(N * F * H * W * 4), DeviceBuffer(N * C * H * W * 4)
    dy, dw = DeviceBuffer(N * F * H * W * 4), DeviceBuffer(F * C * 9 * 4)
    Ns, Cs, Hs, Fs = 2, 3, 32, 16  # stem: 32x32 -> 16x16
    xs = DeviceBuffer(Ns * Cs * Hs * Hs * 4)
    ws = DeviceBuffer.from_array((r.standard_normal((Fs, Cs, 7, 7)) * 0.1).astype(np.float32))
    bs = DeviceBuffer.from_array(r.uniform(-0.1, 0.1, Fs).astype(np.float32))
    ys, ms = DeviceBuffer(Ns * Fs * 16 * 16 * 4), DeviceBuffer(Ns * Fs * 16 * 16 * 4)
    dys = DeviceBuffer(Ns * Fs * 16 * 16 * 4)
    dxs, dws = DeviceBuffer(Ns * Cs * Hs * Hs * 4), DeviceBuffer(Fs * Cs * 49 * 4)

    def seq():
        capi.check(lib.seera_hip_conv2d_fwd_async(x.ptr, w.ptr, y.ptr, N, C, H, W, F, 3, 3, 1, 1,
                                                  1, 1, stream))
        capi.check(lib.seera_hip_conv2d_bwd_async(w.ptr, x.ptr, dy.ptr, dx.ptr, dw.ptr, N, C, H, W,
                                                  F, 3, 3, 1, 1, 1, 1, stream))
        capi.check(lib.seera_hip_conv2d_fwd_bias_act_async(
            xs.ptr, ws.ptr, bs.ptr, ys.ptr, ms.ptr, Ns, Cs, Hs, Hs, Fs, 7, 7, 3, 3, 2, 2,
            capi.SEERA_ACT_RELU, stream))
        capi.check(lib.seera_hip_conv2d_bwd_async(ws.ptr, xs.ptr, dys.ptr, dxs.ptr, dws.ptr, Ns, Cs,
                                                  Hs, Hs, Fs, 7, 7, 2, 2, 3, 3, stream))

    def make_inputs(rep):
        g = np.random.default_rng(30 + rep)
        return [g.standard_normal((N, C, H, W)).astype(np.float32),
                g.standard_normal((N, F, H, W)).astype(np.float32),
                g.standard_normal((Ns, Cs, Hs, Hs)).astype(np.float32),
                g.standard_normal((Ns, Fs, 16, 16)).astype(np.float32)]

    outputs = [(y, (N, F, H, W), np.float32), (dx, (N, C, H, W), np.float32),
               (dw, (F, C, 3, 3), np.float32), (ys, (Ns, Fs, 16, 16), np.float32),
               (ms, (Ns, Fs, 16, 16), np.float32), (dxs, (Ns, Cs, Hs, Hs), np.float32),
               (dws, (Fs, Cs, 7, 7), np.float32)]
    _replays_match_eager(lib, stream, seq, [(x, None), (dy, None), (xs, None), (dys, None)],
                         outputs, make_inputs)
