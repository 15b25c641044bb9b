"""mtg_q8_mul_mat_dev_noalloc (static device scratch, no allocation) against
mtg_q8_mul_mat_dev (per-call allocation) on the same packed weights and inputs:
two calls in a row, the second with a smaller input (fewer rows, shorter K), so
the second call runs on a scratch array that still holds the first call's panel.
Bit-identical results are required (same kernels, same canonical order); the
oracle's q8_0 GEMM is checked too."""
import ctypes

import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _packed(k, n, rng):
    w = rng.standard_normal((n, k)).astype(np.float32)
    raw = np.empty(n * (k // 32) * 34, np.uint8)
    mtg.lib().mtg_quantize_q8_0_weight(mtg.ptr(w), w.size, mtg.ptr(raw))
    p = ctypes.c_void_p()
    assert mtg.lib().mtg_q8_pack(mtg.ptr(raw), k, n, ctypes.byref(p)) == 0
    return raw, p


def _run(fn, packed, x, n, *extra):
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    yd = torch.full((x.shape[0], n), float("nan"), dtype=torch.float32, device="cuda")
    rc = fn(packed, ctypes.c_void_p(xd.data_ptr()), x.shape[0], ctypes.c_void_p(yd.data_ptr()), *extra)
    torch.cuda.synchronize()
    assert rc == 0, mtg.lib().mtg_last_error(None)
    return yd.cpu().numpy()


def test_noalloc_matches_allocating_entry_point():
    rng = np.random.default_rng(4242)
    cases = [(3072, 1024, 16), (1024, 2048, 5)]  # second call: fewer rows and a shorter K
    for k, n, T in cases:
        print("no-alloc q8_0 GEMM: K=%d N=%d T=%d" % (k, n, T), flush=True)
        raw, packed = _packed(k, n, rng)
        x = rng.standard_normal((T, k)).astype(np.float32)
        try:
            y_alloc = _run(mtg.lib().mtg_q8_mul_mat_dev, packed, x, n)
            y_static = _run(mtg.lib().mtg_q8_mul_mat_dev_noalloc, packed, x, n, None)
        finally:
            mtg.lib().mtg_q8_free(packed)
        assert np.isfinite(y_static).all()
        assert np.array_equal(y_static.view(np.uint32), y_alloc.view(np.uint32)), (k, n, T)
        ref = oracle_py.mul_mat(mtg.TYPE_Q8_0, raw, k, n, x)
        assert np.array_equal(y_static, ref), (k, n, T)


def test_noalloc_on_a_torch_stream_and_capacity_error():
    rng = np.random.default_rng(4343)
    raw, packed = _packed(2048, 1024, rng)
    x = rng.standard_normal((9, 2048)).astype(np.float32)
    try:
        s = torch.cuda.Stream()
        xd = torch.from_numpy(x).cuda()
        yd = torch.empty((9, 1024), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        rc = mtg.lib().mtg_q8_mul_mat_dev_noalloc(packed, ctypes.c_void_p(xd.data_ptr()), 9,
                                                  ctypes.c_void_p(yd.data_ptr()),
                                                  ctypes.c_void_p(s.cuda_stream))
        s.synchronize()
        assert rc == 0
        y_alloc = _run(mtg.lib().mtg_q8_mul_mat_dev, packed, x, 1024)
        assert np.array_equal(yd.cpu().numpy(), y_alloc)
    finally:
        mtg.lib().mtg_q8_free(packed)
    # K beyond the static scratch: rejected before any launch, with the reason
    raw, packed = _packed(8192, 16, rng)
    try:
        xd = torch.zeros((1, 8192), dtype=torch.float32, device="cuda")
        yd = torch.zeros((1, 16), dtype=torch.float32, device="cuda")
        rc = mtg.lib().mtg_q8_mul_mat_dev_noalloc(packed, ctypes.c_void_p(xd.data_ptr()), 1,
                                                  ctypes.c_void_p(yd.data_ptr()), None)
    finally:
        mtg.lib().mtg_q8_free(packed)
    assert rc == mtg.ERR_CAPACITY
    assert b"exceeds the static scratch" in mtg.lib().mtg_last_error(None)
