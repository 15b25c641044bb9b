"""Kernel-level parity on the GPU: the q8_0 MFMA GEMM (cpu_decode_mul_mat's
replacement) and the causal-context op, through the C ABI on device pointers."""
import ctypes

import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _q8_weights(n, k, dist, rng):
    """n rows of k as q8_0 blocks (tests/test_cpu_q8.cpp:37-46 distributions)."""
    blocks = np.zeros((n, k // 32), oracle_py.Q8_BLOCK)
    if dist == "normal":
        w = rng.standard_normal((n, k)).astype(np.float32)
        raw = np.empty(n * (k // 32) * 34, np.uint8)
        mtg.lib().mtg_quantize_q8_0_weight(mtg.ptr(w), w.size, mtg.ptr(raw))
        return raw
    codes = np.array([-128, -127, 0, 127], np.int8)
    b = np.arange(n * (k // 32)).reshape(n, k // 32)
    if dist == "zero":
        blocks["d"] = 0
        blocks["qs"] = 0
    else:
        d = (1.0 / (1 + b % 9)).astype(np.float32)
        blocks["d"] = d.astype(np.float16).view(np.uint16)
        j = np.arange(32)
        blocks["qs"] = codes[(b[..., None] + j) % 4]
    return blocks.view(np.uint8).reshape(-1).copy()


def _input(k, T, dist, rng):
    if dist == "normal":
        return rng.standard_normal((T, k)).astype(np.float32)
    if dist == "zero":
        return np.zeros((T, k), np.float32)
    vals = np.array([-1000.0, 1000.0, -0.0, 1e-12, -1e-12], np.float32)
    return np.tile(vals[np.arange(k) % 5], (T, 1)).astype(np.float32)


@pytest.mark.parametrize("k,n", [(1024, 1024), (1024, 2048), (3072, 1024), (1024, 3072),
                                 (2048, 1024), (1024, 151936)])
@pytest.mark.parametrize("T", [1, 4, 8, 9, 16])
def test_q8_gemm_matches_oracle(k, n, T):
    rng = np.random.default_rng(20261009 + k + n + T)
    dists = ["normal", "extreme", "zero"] if n <= 3072 else ["normal"]
    for dist in dists:
        raw = _q8_weights(n, k, dist, rng)
        x = _input(k, T, dist, rng)
        ref = oracle_py.mul_mat(mtg.TYPE_Q8_0, raw, k, n, x)
        packed = ctypes.c_void_p()
        assert mtg.lib().mtg_q8_pack(mtg.ptr(raw), k, n, ctypes.byref(packed)) == 0
        xd = _dev(x)
        yd = torch.empty((T, n), dtype=torch.float32, device="cuda")
        rc = mtg.lib().mtg_q8_mul_mat_dev(packed, ctypes.c_void_p(xd.data_ptr()), T,
                                          ctypes.c_void_p(yd.data_ptr()))
        mtg.lib().mtg_q8_free(packed)
        assert rc == 0
        y = yd.cpu().numpy()
        assert np.isfinite(y).all()
        # per-block int32 dots are exact and the cross-block float order is the
        # canonical one on both sides: bit-identical
        err = np.abs(y.astype(np.float64) - ref)
        assert np.array_equal(y, ref), (dist, int((y != ref).sum()), err.max())


def test_q8_gemm_exact_when_sums_are_exact():
    """Power-of-two scales and small codes make every float operation exact, so
    the device result must equal the oracle bit for bit: this pins the per-block
    int8 dot, the block/row/column placement and the scale pairing."""
    rng = np.random.default_rng(7)
    k, n = 1024, 2048
    blocks = np.zeros((n, k // 32), oracle_py.Q8_BLOCK)
    # |block dot| <= 32*4*127, 32 blocks, scales 2^-2..2^0: every partial sum is a
    # multiple of 2^-4 below 2^19, i.e. exactly representable in f32
    e = rng.integers(-2, 1, size=(n, k // 32))
    blocks["d"] = (2.0 ** e).astype(np.float16).view(np.uint16)
    blocks["qs"] = rng.integers(-4, 5, size=(n, k // 32, 32)).astype(np.int8)
    raw = blocks.view(np.uint8).reshape(-1).copy()
    for T in (3, 8, 13):
        # activations: amax of every block is 127 * 2^j, codes exact integers
        xe = rng.integers(-2, 1, size=(T, k // 32, 1))
        codes = rng.integers(-126, 127, size=(T, k // 32, 32)).astype(np.float32)
        codes[..., 0] = 127.0
        x = (codes * 2.0 ** xe).reshape(T, k).astype(np.float32)
        ref = oracle_py.mul_mat(mtg.TYPE_Q8_0, raw, k, n, x)
        exact = (blocks["qs"].astype(np.float64) * 2.0 ** e[..., None]).reshape(n, k) @ x.T.astype(np.float64)
        assert np.array_equal(ref, exact.T.astype(np.float32)), "oracle not exact"
        packed = ctypes.c_void_p()
        assert mtg.lib().mtg_q8_pack(mtg.ptr(raw), k, n, ctypes.byref(packed)) == 0
        xd = _dev(x)
        yd = torch.empty((T, n), dtype=torch.float32, device="cuda")
        assert mtg.lib().mtg_q8_mul_mat_dev(packed, ctypes.c_void_p(xd.data_ptr()), T,
                                            ctypes.c_void_p(yd.data_ptr())) == 0
        mtg.lib().mtg_q8_free(packed)
        assert np.array_equal(yd.cpu().numpy(), ref)


@pytest.mark.parametrize("prefix,queries", [(1, 2), (31, 4), (33, 8), (513, 8), (1025, 4)])
def test_causal_context_matches_oracle_and_ignores_poison(prefix, queries):
    rng = np.random.default_rng(20261010 + prefix)
    hd, heads, kvh = 128, 16, 8
    kv = prefix + queries
    v = rng.uniform(-0.2, 0.2, size=(kvh, kv, hd)).astype(np.float32)
    p = np.zeros((heads, queries, kv), np.float32)
    for q in range(queries):
        p[:, q, : prefix + q + 1] = rng.uniform(0, 0.25, size=(heads, prefix + q + 1))
        p[:, q, prefix + q + 1:] = np.nan  # future probabilities are never read
    ref = oracle_py.causal_context(v, p, kvh, heads, queries, kv, hd)
    out = torch.empty((heads, queries, hd), dtype=torch.float32, device="cuda")
    vd, pd = _dev(v), _dev(p)
    assert mtg.lib().mtg_causal_context_dev(ctypes.c_void_p(vd.data_ptr()), ctypes.c_void_p(pd.data_ptr()),
                                            hd, kvh, heads, queries, kv,
                                            ctypes.c_void_p(out.data_ptr())) == 0
    got = out.cpu().numpy()
    assert np.isfinite(got).all()
    assert np.array_equal(got, ref)  # same key order, no contraction: bit-exact


def test_causal_context_rejects_unsupported_layouts():
    z = ctypes.c_void_p(1)
    L = mtg.lib()
    assert L.mtg_causal_context_dev(z, z, 128, 8, 16, 1, 10, z) == mtg.ERR_UNSUPPORTED  # one query
    assert L.mtg_causal_context_dev(z, z, 128, 8, 12, 4, 10, z) == mtg.ERR_UNSUPPORTED  # heads % kv
    assert L.mtg_causal_context_dev(z, z, 128, 8, 16, 4, 4, z) == mtg.ERR_UNSUPPORTED   # no prefix


@pytest.mark.parametrize("k,n", [(1024, 64), (3072, 1024), (1024, 151936)])
def test_q8_pack_is_lossless(k, n):
    """PackedQ8::round_trip_exact (src/cpu_q8.hpp:17): the tiles hold exactly the
    q8_0 blocks they were packed from."""
    rng = np.random.default_rng(k + n)
    raw = _q8_weights(n, k, "normal" if n < 100000 else "extreme", rng)
    packed = ctypes.c_void_p()
    assert mtg.lib().mtg_q8_pack(mtg.ptr(raw), k, n, ctypes.byref(packed)) == 0
    back = np.zeros_like(raw)
    rc = mtg.lib().mtg_q8_unpack(packed, mtg.ptr(back))
    mtg.lib().mtg_q8_free(packed)
    assert rc == 0
    assert np.array_equal(back, raw)
    assert mtg.lib().mtg_q8_pack(mtg.ptr(raw), 1000, 64, ctypes.byref(packed)) == mtg.ERR_UNSUPPORTED
