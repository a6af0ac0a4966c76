"""The pybind11 `seera_cuda` module driven the way the reference's Python
front end drives it (cuTen.py and Seera_Engine.py call sites)."""
import numpy as np
import pytest

import oracle
from ml_framework_amd import capi
from oracle import fp16r
from tests.helpers import assert_parity

pytestmark = pytest.mark.gpu
S = oracle.seera_cpp


@pytest.fixture(scope="module")
def sc():
    import ml_framework_amd

    assert capi.gpu_available(), "no HIP device visible"
    return ml_framework_amd.seera_cuda()


def test_cuten_matmul_call_sequence(sc):
    """cuTen.matmul (cuTen.py:412-455): upload, cuda_malloc_f32 the output,
    cuda_matmul(A, B, C, M, N, K, Nbatch), download, free."""
    r = np.random.default_rng(1)
    a = r.standard_normal((3, 33, 65)).astype(np.float32)
    b = r.standard_normal((65, 17)).astype(np.float32)
    pa, pb = sc.to_device_f32(a), sc.to_device_f32(b)
    pc = sc.cuda_malloc_f32(3 * 33 * 17)
    sc.cuda_matmul(pa, pb, pc, 33, 17, 65, 3)
    c = sc.to_host_f32(pc, (3, 33, 17))
    assert_parity(c, S.matmul_batched(fp16r(a), fp16r(b)))
    for p in (pa, pb, pc):
        sc.cuda_free(p)


def test_engine_matmul_bwd_call_sequence(sc):
    """Seera_Engine.py:527-543: fresh dA/dB buffers, cuda_matmul_bwd."""
    r = np.random.default_rng(2)
    M, K, N = 4, 3, 2
    a = (r.standard_normal((M, K)) * 0.1).astype(np.float32)
    b = (r.standard_normal((K, N)) * 0.1).astype(np.float32)
    dc = np.ones((M, N), np.float32)
    pa, pb, pdc = sc.to_device_f32(a), sc.to_device_f32(b), sc.to_device_f32(dc)
    pda, pdb = sc.cuda_malloc_f32(M * K), sc.cuda_malloc_f32(K * N)
    sc.cuda_matmul_bwd(pa, pb, pdc, pda, pdb, M, N, K, 1)
    da, db = S.matmul_bwd(fp16r(a), fp16r(b), dc)
    assert_parity(sc.to_host_f32(pda, (M, K)), da)
    assert_parity(sc.to_host_f32(pdb, (K, N)), db)
    for p in (pa, pb, pdc, pda, pdb):
        sc.cuda_free(p)


def test_conv_and_convT_call_sequences(sc):
    r = np.random.default_rng(3)
    x = r.standard_normal((2, 3, 9, 8)).astype(np.float32)
    w = r.standard_normal((4, 3, 3, 3)).astype(np.float32)
    px, pw = sc.to_device_f32(x), sc.to_device_f32(w)
    OH, OW = 5, 4  # (9 + 2 - 3)//2 + 1, (8 + 2 - 3)//2 + 1
    py = sc.cuda_malloc_f32(2 * 4 * OH * OW)
    # cuTen.py:562-564: (..., padh, padw, strideh, stridew)
    sc.cuda_conv2d_fwd(px, pw, py, 2, 3, 9, 8, 4, 3, 3, 1, 1, 2, 2)
    y = sc.to_host_f32(py, (2, 4, OH, OW))
    assert_parity(y, S.conv2d_forward(fp16r(x), fp16r(w), 2, 2, 1, 1))
    dy = r.standard_normal(y.shape).astype(np.float32)
    pdy = sc.to_device_f32(dy)
    pdx, pdw = sc.cuda_malloc_f32(x.size), sc.cuda_malloc_f32(w.size)
    # Seera_Engine.py:76-81: (..., strideh, stridew, padh, padw)
    sc.cuda_conv2d_bwd(pw, px, pdy, pdx, pdw, 2, 3, 9, 8, 4, 3, 3, 2, 2, 1, 1)
    rdx, rdw = S.conv2d_backward(fp16r(dy), fp16r(x), fp16r(w), 2, 2, 1, 1)
    assert_parity(sc.to_host_f32(pdx, x.shape), rdx)
    assert_parity(sc.to_host_f32(pdw, w.shape), rdw)

    wt = r.standard_normal((3, 5, 4, 4)).astype(np.float32)
    pwt = sc.to_device_f32(wt)
    Ho, Wo = (9 - 1) * 2 - 2 + 4, (8 - 1) * 2 - 2 + 4
    pyt = sc.cuda_malloc_f32(2 * 5 * Ho * Wo)
    sc.cuda_conv2DTranpose_fwd(px, pwt, pyt, 2, 3, 9, 8, 5, 4, 4, 2, 2, 1, 1)
    yt = sc.to_host_f32(pyt, (2, 5, Ho, Wo))
    assert_parity(yt, S.conv_transpose2d_forward(fp16r(x), fp16r(wt), 2, 2, 1, 1))
    dyt = r.standard_normal(yt.shape).astype(np.float32)
    pdyt = sc.to_device_f32(dyt)
    pdwt = sc.cuda_malloc_f32(wt.size)
    sc.cuda_conv2DTranspose_bwd(pwt, px, pdyt, pdx, pdwt, 2, 3, 9, 8, 5, 4, 4, 2, 2, 1, 1)
    rdx, rdw = S.conv_transpose2d_backward(fp16r(dyt), fp16r(x), fp16r(wt), 2, 2, 1, 1)
    assert_parity(sc.to_host_f32(pdx, x.shape), rdx)
    assert_parity(sc.to_host_f32(pdwt, wt.shape), rdw)
    for p in (px, pw, py, pdy, pdx, pdw, pwt, pyt, pdyt, pdwt):
        sc.cuda_free(p)


def test_memory_helpers(sc):
    a = np.arange(12, dtype=np.float32).reshape(3, 4)
    p = sc.to_device_f32(a)
    q = sc.cuda_malloc_f32(12)
    sc.cuda_memcopy_devicetodevice(q, p, 12)
    assert np.array_equal(sc.to_host_f32(q, (3, 4)), a)
    sc.cuda_memset(q, 0, 48)
    assert not sc.to_host_f32(q, (12,)).any()
    t = sc.cuda_malloc_f32(12)
    sc.cuda_transpose_2d(p, t, 3, 4)
    assert np.array_equal(sc.to_host_f32(t, (4, 3)), a.T)
    i = np.arange(6, dtype=np.int32)
    pi = sc.to_device_i32(i)
    assert np.array_equal(sc.to_host_i32(pi, (6,)), i)
    for x in (p, q, t, pi):
        sc.cuda_free(x)


def test_errors_raise(sc):
    with pytest.raises(RuntimeError, match="stride"):
        sc.cuda_conv2d_fwd(0, 0, 0, 1, 3, 8, 8, 4, 3, 3, 1, 1, 0, 1)


def test_maxpool_call_sequence(sc):
    """cuTen.maxpool2d (cuTen.py:578-606): cuda_malloc_f32 the output,
    cuda_malloc_i32 the mask, cuda_maxpool_fwd; Seera_Engine.py:117-136:
    cuda_malloc_f32 + cuda_memset dX, cuda_maxpool_bwd."""
    from oracle import pool

    r = np.random.default_rng(6)
    N, C, H, W, K, s, p = 2, 3, 9, 8, 3, 2, 1
    x = r.standard_normal((N, C, H, W)).astype(np.float32)
    OH, OW = 5, 4
    px = sc.to_device_f32(x)
    pout, pmask = sc.cuda_malloc_f32(N * C * OH * OW), sc.cuda_malloc_i32(x.size)
    sc.cuda_maxpool_fwd(px, pout, pmask, N, C, H, W, K, K, p, p, s, s)
    ro, rm = pool.maxpool_fwd(x, K, K, p, p, s, s)
    assert np.array_equal(sc.to_host_f32(pout, (N, C, OH, OW)), ro)
    assert np.array_equal(sc.to_host_i32(pmask, x.shape), rm)
    dout = r.standard_normal((N, C, OH, OW)).astype(np.float32)
    pg = sc.to_device_f32(dout)
    pdx = sc.cuda_malloc_f32(x.size)
    sc.cuda_memset(pdx, 0, x.size * 4)
    sc.cuda_maxpool_bwd(pg, pmask, pdx, N, C, H, W, K, K, p, p, s, s)
    assert np.array_equal(sc.to_host_f32(pdx, x.shape), pool.maxpool_bwd(dout, rm, K, K, p, p, s, s))
    for q in (px, pout, pmask, pg, pdx):
        sc.cuda_free(q)


def test_fused_layer_entry_points(sc):
    """The module's fused Dense / Conv2D entry points equal the reference's
    call sequences (matmul + bias + relu; conv + bias + relu; the ReLU
    chain rule on dA) bit for bit, and the bias gradients match fp64 sums."""
    r = np.random.default_rng(8)
    a = r.standard_normal((64, 48)).astype(np.float32)
    b = r.standard_normal((48, 32)).astype(np.float32)
    bias = r.standard_normal(32).astype(np.float32)
    pa, pb, pbias = sc.to_device_f32(a), sc.to_device_f32(b), sc.to_device_f32(bias)
    pc, pm, pz = (sc.cuda_malloc_f32(64 * 32) for _ in range(3))
    sc.cuda_matmul(pa, pb, pz, 64, 32, 48, 1)
    sc.cuda_matmul_bias_act(pa, pb, pbias, pc, pm, 64, 32, 48, 1, 1)
    z = sc.to_host_f32(pz, (64, 32)) + bias
    assert np.array_equal(sc.to_host_f32(pc, (64, 32)), np.where(z > 0, z, np.float32(0)))
    assert np.array_equal(sc.to_host_f32(pm, (64, 32)), (z > 0).astype(np.float32))
    dc = r.standard_normal((64, 32)).astype(np.float32)
    mask_a = (r.uniform(0, 1, (64, 48)) > 0.5).astype(np.float32)
    pdc, pma = sc.to_device_f32(dc), sc.to_device_f32(mask_a)
    pda, pdb, pda2, pdb2 = (sc.cuda_malloc_f32(n) for n in (64 * 48, 48 * 32, 64 * 48, 48 * 32))
    sc.cuda_matmul_bwd(pa, pb, pdc, pda, pdb, 64, 32, 48, 1)
    sc.cuda_matmul_bwd_relu(pa, pb, pdc, pma, pda2, pdb2, 64, 32, 48, 1)
    assert np.array_equal(sc.to_host_f32(pda2, (64, 48)), sc.to_host_f32(pda, (64, 48)) * mask_a)
    pdbias = sc.cuda_malloc_f32(32)
    sc.cuda_bias_grad(pdc, pdbias, 64, 32)
    assert np.allclose(sc.to_host_f32(pdbias, (32,)), dc.astype(np.float64).sum(0), atol=1e-4)
    pdbias2 = sc.cuda_malloc_f32(32)
    sc.cuda_matmul_bwd_bias(pa, pb, pdc, pda2, pdb2, pdbias2, 64, 32, 48, 1)
    assert np.array_equal(sc.to_host_f32(pdb2, (48, 32)), sc.to_host_f32(pdb, (48, 32)))
    assert np.allclose(sc.to_host_f32(pdbias2, (32,)), dc.astype(np.float64).sum(0), atol=1e-4)
    sc.cuda_matmul_bwd_relu_bias(pa, pb, pdc, pma, pda2, pdb2, pdbias2, 64, 32, 48, 1)
    assert np.array_equal(sc.to_host_f32(pda2, (64, 48)), sc.to_host_f32(pda, (64, 48)) * mask_a)
    assert np.allclose(sc.to_host_f32(pdbias2, (32,)), dc.astype(np.float64).sum(0), atol=1e-4)
    x = r.standard_normal((2, 8, 10, 12)).astype(np.float32)
    w = (r.standard_normal((16, 8, 3, 3)) * 0.2).astype(np.float32)
    cb = r.standard_normal(16).astype(np.float32)
    px, pw, pcb = sc.to_device_f32(x), sc.to_device_f32(w), sc.to_device_f32(cb)
    py, py2, pym = (sc.cuda_malloc_f32(2 * 16 * 10 * 12) for _ in range(3))
    sc.cuda_conv2d_fwd(px, pw, py, 2, 8, 10, 12, 16, 3, 3, 1, 1, 1, 1)
    sc.cuda_conv2d_fwd_bias_act(px, pw, pcb, py2, pym, 2, 8, 10, 12, 16, 3, 3, 1, 1, 1, 1, 1)
    zc = sc.to_host_f32(py, (2, 16, 10, 12)) + cb[None, :, None, None]
    assert np.array_equal(sc.to_host_f32(py2, (2, 16, 10, 12)), np.where(zc > 0, zc, np.float32(0)))
    pcdb = sc.cuda_malloc_f32(16)
    sc.cuda_conv_bias_grad(py2, pcdb, 2, 16, 120)
    ref = sc.to_host_f32(py2, (2, 16, 10, 12)).astype(np.float64).sum((0, 2, 3))
    assert np.allclose(sc.to_host_f32(pcdb, (16,)), ref, rtol=1e-5, atol=1e-4)
    for q in (pa, pb, pbias, pc, pm, pz, pdc, pma, pda, pdb, pda2, pdb2, pdbias, px, pw, pcb, py,
              py2, pym, pcdb):
        sc.cuda_free(q)
