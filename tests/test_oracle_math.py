"""The oracle's primitives against what the mathematics fixes, on the CPU.

Each check is chosen so that a plausible slip in the oracle (a dropped term, a
wrong index, a swapped operand, the wrong rounding rule) fails it: exhaustive
f16 conversion against numpy, brute-force integer block dots, exactly
representable GEMMs compared bit for bit with float64, and float64 closed forms
of RMSNorm, NEOX RoPE, softmax and the causal context."""
import ctypes

import numpy as np
import pytest

import mtg
import oracle_py

L = oracle_py.lib


def test_f16_conversion_matches_ieee_rne_exhaustively():
    # every half -> float is exact
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = np.array([L().orc_f16_to_f32(int(x)) for x in h[::7]], np.float32)
    r = ref[::7]
    assert np.array_equal(np.isnan(got), np.isnan(r))
    ok = ~np.isnan(r)
    assert np.array_equal(got[ok].view(np.uint32), r[ok].view(np.uint32))
    # float -> half, round to nearest even, incl. midpoints, subnormals, overflow
    rng = np.random.default_rng(1)
    mids = (h[:-1].view(np.float16).astype(np.float64) + h[1:].view(np.float16).astype(np.float64)) / 2
    xs = np.concatenate([rng.standard_normal(3000) * 10.0 ** rng.integers(-9, 6, 3000),
                         mids[np.isfinite(mids)][::13], [0.0, -0.0, 65504.0, 65520.0, 1e9, 6e-8, 3e-8]])
    xs = xs.astype(np.float32)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([L().orc_f32_to_f16(float(x)) for x in xs], np.uint16)
    assert np.array_equal(got, want)


def test_q8_0_block_dot_is_the_exact_integer_sum():
    rng = np.random.default_rng(2)
    for trial in range(200):
        a = np.zeros(1, oracle_py.Q8_BLOCK)
        b = np.zeros(1, oracle_py.Q8_BLOCK)
        a["qs"] = rng.integers(-128, 128, 32)
        b["qs"] = rng.integers(-128, 128, 32)
        want = int((a["qs"].astype(np.int64) * b["qs"].astype(np.int64)).sum())
        assert L().orc_q8_0_block_dot(mtg.ptr(a), mtg.ptr(b)) == want
    # extremes: -128 * -128 * 32 = 524288
    a["qs"] = -128
    b["qs"] = -128
    assert L().orc_q8_0_block_dot(mtg.ptr(a), mtg.ptr(b)) == 524288


def test_q8_0_gemm_block_dots_are_the_exact_integer_sums():
    """The GEMM's eight-blocks-at-a-time int8 dots (|w| x sign(w) x in 16-bit pair
    sums) against the exact sums: weights over the whole int8 range (-128 included),
    activation codes in [-127, 127] as the q8_0 quantizer makes them, block counts
    around the eight-block step, and the largest pair sums."""
    rng = np.random.default_rng(3)
    for nb in (1, 7, 8, 9, 16, 31, 32, 33, 96):
        for trial in range(20):
            w = rng.integers(-128, 128, 32 * nb).astype(np.int8)
            x = rng.integers(-127, 128, 32 * nb).astype(np.int8)
            if trial == 0:
                w[:] = -128
                x[:] = np.where(np.arange(32 * nb) % 2 == 0, 127, -127)
            if trial == 1:
                w[:] = -128
                x[:] = -127
            out = np.zeros(nb, np.int32)
            L().orc_q8_0_block_dots(mtg.ptr(w), mtg.ptr(x), nb, mtg.ptr(out))
            want = (w.astype(np.int64) * x.astype(np.int64)).reshape(nb, 32).sum(axis=1)
            assert np.array_equal(out.astype(np.int64), want), (nb, trial)


def test_q8_0_activation_quantizer_rules():
    """d = amax/127 stored as f16; codes = round-half-even(x * 127/amax); zero
    blocks give d = 0 and zero codes; |code| <= 127 and the amax element maps to
    +-127."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal(32 * 64) * 10.0 ** rng.integers(-6, 4, 32 * 64)).astype(np.float32)
    x[:32] = 0.0
    q = oracle_py.quantize_q8_0_act(x)
    b = x.reshape(-1, 32)
    amax = np.abs(b).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    assert np.array_equal(q["d"], d.astype(np.float16).view(np.uint16))
    assert (q["qs"][0] == 0).all() and q["d"][0] == 0
    assert np.abs(q["qs"].astype(int)).max() <= 127
    nz = amax > 0
    am = np.abs(b).argmax(axis=1)
    assert (np.abs(q["qs"][nz, am[nz]].astype(int)) == 127).all()
    # ties: x * 127/amax landing exactly on k + 0.5 rounds to even
    blk = np.zeros(32, np.float32)
    blk[0] = 127.0
    blk[1:6] = [0.5, 1.5, 2.5, -0.5, -3.5]
    qt = oracle_py.quantize_q8_0_act(blk)
    assert qt["qs"][0][:6].tolist() == [127, 0, 2, 2, 0, -4]
    # the multiplier: x * (127 / amax) (ggml's x86 quantize_row_q8_0) and x * (1 / d)
    # with d = amax / 127 (ggml's generic rule) round apart on this block: -81.49999
    # against -81.5, so the oracle's code tells the two rules apart
    f = np.float32
    amax, xv = f(0.5413191), f(-0.3473819)
    x86 = np.rint(xv * (f(127) / amax))
    generic = np.rint(xv * (f(1) / (amax / f(127))))
    assert (x86, generic) == (-81.0, -82.0)
    blk = np.zeros(32, np.float32)
    blk[0], blk[1] = amax, xv
    qn = oracle_py.quantize_q8_0_act(blk)
    assert qn["qs"][0][:2].tolist() == [127, -81]


def _q8_matrix(n, k, rng, exp_range=(-2, 1), code_range=(-4, 5)):
    blocks = np.zeros((n, k // 32), oracle_py.Q8_BLOCK)
    e = rng.integers(exp_range[0], exp_range[1], size=(n, k // 32))
    blocks["d"] = (2.0 ** e).astype(np.float16).view(np.uint16)
    blocks["qs"] = rng.integers(code_range[0], code_range[1], size=(n, k // 32, 32)).astype(np.int8)
    w = (blocks["qs"].astype(np.float64) * (2.0 ** e)[..., None]).reshape(n, k)
    return blocks.view(np.uint8).reshape(-1).copy(), w


def test_q8_0_mul_mat_exact_when_every_sum_is_representable():
    """Power-of-two scales, small codes, activations whose block amax is 127*2^j:
    every partial sum is exact in f32, so the oracle must equal the float64
    product bit for bit whatever its summation order. A wrong block pairing,
    row/column placement or scale product cannot pass."""
    rng = np.random.default_rng(4)
    for k, n in ((1024, 48), (2048, 32), (3072, 16)):
        raw, w = _q8_matrix(n, k, rng)
        T = 5
        xe = rng.integers(-2, 1, size=(T, k // 32, 1))
        codes = rng.integers(-126, 127, size=(T, k // 32, 32)).astype(np.float32)
        codes[..., 3] = 127.0
        x = (codes * 2.0 ** xe).reshape(T, k).astype(np.float32)
        got = oracle_py.mul_mat(mtg.TYPE_Q8_0, raw, k, n, x)
        want = (x.astype(np.float64) @ w.T).astype(np.float32)
        assert np.array_equal(got, want)


def test_q8_0_mul_mat_close_to_float64_of_quantized_operands():
    rng = np.random.default_rng(5)
    k, n, T = 1024, 64, 4
    wf = rng.standard_normal((n, k)).astype(np.float32) * np.float32(0.02)
    raw = np.empty(n * (k // 32) * 34, np.uint8)
    mtg.lib().mtg_quantize_q8_0_weight(mtg.ptr(wf), wf.size, mtg.ptr(raw))
    wq = np.empty((n, k), np.float32)
    mtg.lib().mtg_dequantize(mtg.TYPE_Q8_0, mtg.ptr(raw), wf.size, mtg.ptr(wq))
    x = rng.standard_normal((T, k)).astype(np.float32)
    xq = oracle_py.quantize_q8_0_act(x)
    xd = (xq["qs"].astype(np.float64) *
          xq["d"].view(np.float16).astype(np.float64)[:, None]).reshape(T, k)
    want = xd @ wq.astype(np.float64).T
    got = oracle_py.mul_mat(mtg.TYPE_Q8_0, raw, k, n, x).astype(np.float64)
    assert np.abs(got - want).max() <= 1e-5 * np.abs(want).max()


@pytest.mark.parametrize("wtype", [mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K])
def test_f16_f32_and_q4k_mul_mat_close_to_float64_of_quantized_operands(wtype):
    rng = np.random.default_rng(6)
    k, n, T = 1024, 32, 3
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    nb = mtg.lib().mtg_row_bytes(wtype, k) * n
    raw = np.empty(nb, np.uint8)
    if wtype == mtg.TYPE_F16:
        raw[:] = wf.astype(np.float16).view(np.uint8).reshape(-1)
    elif wtype == mtg.TYPE_F32:
        raw[:] = wf.view(np.uint8).reshape(-1)
    else:
        mtg.lib().mtg_quantize_q4_k(mtg.ptr(wf), wf.size, mtg.ptr(raw))
    wq = np.empty((n, k), np.float32)
    mtg.lib().mtg_dequantize(wtype, mtg.ptr(raw), wf.size, mtg.ptr(wq))
    x = rng.standard_normal((T, k)).astype(np.float32)
    got = oracle_py.mul_mat(wtype, raw, k, n, x).astype(np.float64)
    if wtype == mtg.TYPE_F16:
        xa = x.astype(np.float16).astype(np.float64)  # vec_dot_type F16
        tol = 1e-5
    elif wtype == mtg.TYPE_F32:
        xa = x.astype(np.float64)  # vec_dot_type F32: x as it is
        tol = 1e-5
    else:
        # q8_K activations: 256-blocks, scale max/-127, codes nearest
        b = x.reshape(T, -1, 256).astype(np.float32)
        idx = np.abs(b).argmax(axis=2)
        mx = np.take_along_axis(b, idx[..., None], 2)
        iscale = np.float32(-127.0) / mx
        codes = np.minimum(127, np.rint(iscale * b))
        xa = (codes * (np.float32(1.0) / iscale).astype(np.float64)).reshape(T, k)
        tol = 1e-4
    want = xa @ wq.astype(np.float64).T
    assert np.abs(got - want).max() <= tol * np.abs(want).max()
    # the dequantized weights themselves are close to the float input
    bound = {mtg.TYPE_F16: 1e-3, mtg.TYPE_F32: 0.0}.get(wtype, 0.25)
    assert np.abs(wq - wf).max() <= bound * np.abs(wf).max()


def test_f16_mul_mat_exact_on_small_integers():
    """Small-integer f16 weights and activations: every product and partial sum is
    exact in f32, so any summation order gives the float64 value bit for bit; a
    dropped, repeated or misplaced element does not."""
    rng = np.random.default_rng(16)
    for k in (1024, 2048, 3072):
        n, T = 24, 5
        w = rng.integers(-8, 9, (n, k)).astype(np.float16)
        x = rng.integers(-8, 9, (T, k)).astype(np.float32)
        got = oracle_py.mul_mat(mtg.TYPE_F16, w.view(np.uint8).reshape(-1).copy(), k, n, x)
        want = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.array_equal(got.astype(np.float64), want)


def test_f32_mul_mat_exact_on_small_integers():
    """f32 weights: small-integer operands make every fma exact, so the result is
    the float64 dot bit for bit whatever the order; an element dropped, repeated,
    misplaced or taken from the wrong operand changes it."""
    rng = np.random.default_rng(17)
    for k in (1024, 2048, 3072):
        n, T = 24, 5
        w = rng.integers(-64, 65, (n, k)).astype(np.float32)
        x = rng.integers(-64, 65, (T, k)).astype(np.float32)
        got = oracle_py.mul_mat(mtg.TYPE_F32, w.view(np.uint8).reshape(-1).copy(), k, n, x)
        want = x.astype(np.float64) @ w.astype(np.float64).T
        assert np.array_equal(got.astype(np.float64), want)


def _f32_planted(k, cells):
    """A one-row f32 matrix and activation with w[i] * x[i] planted at the given
    elements (i: (w, x)), zeros elsewhere."""
    w = np.zeros((1, k), np.float32)
    x = np.zeros((1, k), np.float32)
    for i, (a, b) in cells.items():
        w[0, i], x[0, i] = a, b
    return oracle_py.mul_mat(mtg.TYPE_F32, w.view(np.uint8).reshape(-1).copy(), k, 1, x)[0, 0]


def test_f32_mul_mat_order_planted():
    """Planted rows where the candidate orders give different floats:
    * one fused multiply-add per element: -(1 + 2^-11) then (1 + 2^-12)^2 in one
      segment gives 2^-24 with fma, 0 with a rounded product then an add;
    * segments of K/64 consecutive elements: 2^24 and 1 in segment 0 and -2^24 in
      segment 1 give 0 (2^24 + 1 rounds to 2^24 inside the chain); with elements
      dealt to the lanes in turn the 1 would meet the cancelled pair last: 1;
    * the xor butterfly: partials 2^24, 1, -2^24 in segments 0, 1, 2 give 1
      (segments 0 and 2 meet before segment 1 joins); a sequential sum gives 0."""
    one = np.float32(1.0)
    a = np.float32(1.0 + 2.0 ** -12)
    for k in (1024, 2048, 3072):
        seg = k // 64
        assert _f32_planted(k, {0: (one, -np.float32(1.0 + 2.0 ** -11)), 1: (a, a)}) == np.float32(2.0 ** -24)
        # the same pair in the last segment, at its last two elements
        assert _f32_planted(k, {k - 2: (one, -np.float32(1.0 + 2.0 ** -11)), k - 1: (a, a)}) == np.float32(2.0 ** -24)
        big = np.float32(2.0 ** 24)
        assert _f32_planted(k, {0: (one, big), 1: (one, one), seg: (one, -big)}) == 0.0
        assert _f32_planted(k, {0: (one, big), seg: (one, one), 2 * seg: (one, -big)}) == 1.0
        # pairs at distance 32 segments meet first: 2^24 in segment 5, -2^24 in 37, 1 in 4
        assert _f32_planted(k, {5 * seg: (one, big), 37 * seg: (one, -big), 4 * seg: (one, one)}) == 1.0


def test_rms_norm_matches_float64_closed_form():
    rng = np.random.default_rng(7)
    for n in (1024, 128, 96):
        x = rng.standard_normal(n).astype(np.float32) * np.float32(3)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        got = oracle_py.rms_norm(x, w, 1e-6).astype(np.float64)
        x64 = x.astype(np.float64)
        want = x64 / np.sqrt((x64 * x64).mean() + 1e-6) * w
        assert np.abs(got - want).max() <= 4 * np.finfo(np.float32).eps * np.abs(want).max()
    # a zero row stays zero (eps keeps the scale finite)
    z = oracle_py.rms_norm(np.zeros(1024, np.float32), np.ones(1024, np.float32), 1e-6)
    assert (z == 0).all()


def test_rope_neox_matches_closed_form_and_invariants():
    """NEOX pairs (i, i+64) rotated by theta_i = pos * base^(-2i/128). ggml builds
    theta_i by repeated float multiplication (theta_{i+1} = theta_i * powf(base,
    -2/d)), so the angles are those of that float32 recurrence; given them, the
    rotation is checked in float64 (a swapped sign, pair index or cos/sin fails)."""
    rng = np.random.default_rng(8)
    x = rng.standard_normal(128).astype(np.float32)
    assert np.array_equal(oracle_py.rope_neox(x, 0, 1e6), x)  # position 0: identity
    scale = np.float32(np.power(np.float32(1e6), np.float32(-2.0 / 128)))
    x0, x1 = x[:64].astype(np.float64), x[64:].astype(np.float64)
    for pos in (1, 7, 511, 1600, 16383):
        theta = np.empty(64, np.float32)
        t = np.float32(pos)
        for i in range(64):
            theta[i] = t
            t = np.float32(t * scale)
        th = theta.astype(np.float64)
        want = np.concatenate([x0 * np.cos(th) - x1 * np.sin(th), x0 * np.sin(th) + x1 * np.cos(th)])
        got = oracle_py.rope_neox(x, pos, 1e6).astype(np.float64)
        assert np.abs(got - want).max() <= 4 * np.finfo(np.float32).eps * np.abs(x).max(), pos
        # and the float angles stay within the recurrence's error of the exact ones
        exact = pos * 1e6 ** (-2.0 * np.arange(64) / 128)
        assert np.abs(th - exact).max() <= 64 * 2 * np.finfo(np.float32).eps * pos
        n0, n1 = np.hypot(x0, x1), np.hypot(got[:64], got[64:])
        assert np.abs(n0 - n1).max() <= 1e-5


def test_softmax_rows_including_extreme_values():
    """Rows of tests/test_cpu_softmax.cpp:40-46: lengths 1..4096, +-10000 and
    -inf spikes; the result equals exp(w - max) / sum in float64 and sums to 1."""
    rng = np.random.default_rng(9)
    for n in (1, 2, 31, 64, 255, 1024, 4096):
        s = rng.standard_normal(n).astype(np.float32) * np.float32(4)
        if n > 2:
            s[n // 3] = 10000.0
            s[n // 2] = -10000.0
        mask = np.zeros(n, np.float32)
        if n > 3:
            mask[-1] = -np.inf
        scale = 1.0 / np.sqrt(128.0)
        got = oracle_py.softmax(s, scale, mask).astype(np.float64)
        w = s.astype(np.float64) * np.float32(scale) + mask
        e = np.exp(w - w.max())
        want = e / e.sum()
        assert np.abs(got - want).max() <= 1e-6
        assert abs(got.sum() - 1.0) <= 1e-5
        if n > 3:
            assert got[-1] == 0.0


def test_causal_context_sums_exactly_the_valid_prefix():
    """out[h][q][f] = sum over k <= past+q of v[h/groups][k][f] * p[h][q][k]
    (src/cpu_context.cpp:13-32), accumulated key by key in f32: numpy's
    sequential float32 accumulate gives the same bits. Future probabilities are
    NaN: reading one would poison the output (tests/test_cpu_context.cpp:41-47)."""
    rng = np.random.default_rng(10)
    for past, queries, heads, kvh, hd in ((1, 2, 4, 2, 3), (31, 4, 16, 8, 128), (33, 8, 3, 1, 16),
                                          (128, 8, 16, 8, 128)):
        kv = past + queries
        v = rng.uniform(-0.2, 0.2, size=(kvh, kv, hd)).astype(np.float32)
        p = np.full((heads, queries, kv), np.nan, np.float32)
        for q in range(queries):
            p[:, q, :past + q + 1] = rng.uniform(0, 0.25, size=(heads, past + q + 1))
        got = oracle_py.causal_context(v, p, kvh, heads, queries, kv, hd)
        assert np.isfinite(got).all()
        g = heads // kvh
        want = np.empty_like(got)
        for h in range(heads):
            for q in range(queries):
                n = past + q + 1
                prod = (v[h // g, :n, :] * p[h, q, :n, None]).astype(np.float32)
                want[h, q] = np.add.accumulate(prod, axis=0, dtype=np.float32)[-1]
        assert np.array_equal(got, want)


def test_exp_is_within_two_ulps_of_float64():
    """The exp of attention and SiLU (Cody-Waite reduction, degree-7 Taylor
    polynomial): at most 2 ulps from the float64 exponential on [-87, 88.7], exact
    at 0, 0 below -87 and inf above 88.7."""
    xs = np.concatenate([np.linspace(-87, 88.7, 20001), [-1e-30, 1e-30, -0.5, 0.5, -1e-8]])
    xs = xs.astype(np.float32)
    got = np.array([L().orc_exp(float(x)) for x in xs], np.float64)
    want = np.exp(xs.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert (np.abs(got - want) <= 2 * ulp).all()
    assert L().orc_exp(0.0) == 1.0
    assert L().orc_exp(-87.5) == 0.0 and L().orc_exp(-1000.0) == 0.0
    assert L().orc_exp(89.0) == np.inf


def test_q8_k_activation_quantizer_rules():
    """ggml's quantize_row_q8_K (the vec_dot_type of q4_K): the scale comes from the
    SIGNED value of the first element of largest magnitude (strict '>' scan), so
    that element always maps to -127 and d = 1/iscale carries the opposite sign;
    codes are round-half-even of iscale * x, at most +127; bsums are the sums of
    16-code groups; an all-zero block gives d = 0 and zero codes. Each planted case
    tells the rule apart from a plausible alternative (amax/127 scaling, last
    occurrence on ties, half-away rounding)."""
    def q(block):
        return oracle_py.quantize_q8_k_act(np.asarray(block, np.float32))[0]
    # signed max: the largest |x| is negative -> iscale > 0, d < 0 ... and positive
    b = np.zeros(256, np.float32)
    b[7], b[20] = -4.0, 3.0
    r = q(b)
    assert r["qs"][7] == -127 and r["d"] == np.float32(1.0) / (np.float32(-127.0) / np.float32(-4.0))
    assert r["d"] > 0 and r["qs"][20] == int(np.rint(np.float32(31.75) * np.float32(3.0)))  # 95.25 -> 95
    b[7], b[20] = 4.0, -3.0
    r = q(b)
    assert r["qs"][7] == -127 and r["qs"][20] == 95 and r["d"] < 0
    # a tie in magnitude: the FIRST occurrence sets the sign; the opposite-sign
    # extreme lands on +127 exactly (the clamp's bound, never 128)
    b = np.zeros(256, np.float32)
    b[3], b[10] = -5.0, 5.0
    r = q(b)
    assert r["qs"][3] == -127 and r["qs"][10] == 127
    b[3], b[10] = 5.0, -5.0
    r = q(b)
    assert r["qs"][3] == -127 and r["qs"][10] == 127
    # rounding ties: max = -127 gives iscale = 1 exactly, so x = k + 0.5 is a tie
    b = np.zeros(256, np.float32)
    b[0] = -127.0
    b[1:8] = [0.5, 1.5, 2.5, -0.5, -3.5, 126.5, -126.5]
    r = q(b)
    assert r["qs"][:8].tolist() == [-127, 0, 2, 2, 0, -4, 126, -126]
    # bsums = sums of the 16-code groups (int16), on random blocks
    rng = np.random.default_rng(31)
    x = (rng.standard_normal(256 * 32) * 10.0 ** rng.integers(-4, 3, 256 * 32)).astype(np.float32)
    x[256:512] = 0.0
    blocks = oracle_py.quantize_q8_k_act(x)
    qs = blocks["qs"].astype(np.int64)
    assert np.array_equal(blocks["bsums"], qs.reshape(-1, 16, 16).sum(axis=2))
    assert blocks["d"][1] == 0 and (blocks["qs"][1] == 0).all()
    assert qs.max() <= 127 and qs.min() >= -127
    # the codes are the nearest integers: |x - d * code| <= |d| / 2 (+ rounding of
    # the float product), and the extreme element of every block is -127
    xb = x.reshape(-1, 256).astype(np.float64)
    d = blocks["d"].astype(np.float64)[:, None]
    err = np.abs(xb - d * qs)
    assert (err <= np.abs(d) * (0.5 + 1e-5) + 1e-30).all()
    nz = np.abs(xb).max(axis=1) > 0
    first = np.abs(xb).argmax(axis=1)  # numpy: first occurrence
    assert (qs[nz, first[nz]] == -127).all()


def _attention_f64(q, k, v, past):
    """Causal softmax attention in float64: q [T][H][D], k, v [G][S][D]."""
    T, H, D = q.shape
    G = k.shape[0]
    out = np.empty((T, H, D))
    for h in range(H):
        g = h // (H // G)
        kk = k[g, :past + T].astype(np.float64)
        vv = v[g, :past + T].astype(np.float64)
        s = q[:, h, :].astype(np.float64) @ kk.T / np.sqrt(D)
        for t in range(T):
            s[t, past + t + 1:] = -np.inf
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[:, h, :] = (p / p.sum(axis=1, keepdims=True)) @ vv
    return out


# (cached prefix, T): 26 chunks; 33 chunks, the last one reached by the last rows
# only; 63, 96, 97, 140 and 194 chunks (the step kernel's attention items take 2 to
# 7 chunks of a kv head each beyond 32 chunks; the per-op kernels stride over them)
LONG_CASES = [(1650, 8), (2040, 16), (4000, 16), (6140, 4), (6200, 4), (8950, 9), (12400, 16)]


@pytest.mark.parametrize("past,T", LONG_CASES)
@pytest.mark.parametrize("kv", ["f32", "f16"])
def test_attention_long_context_close_to_float64(past, T, kv):
    """The step's attention in the canonical order (chunks of 64 keys, each with its
    own maximum, merged in order with f = exp(m_c - M)) against float64 causal
    softmax attention. The keys of each chunk are scaled by a factor between 0.3
    and 3, so that the chunk maxima differ and every merge factor matters: a factor
    taken the wrong way round, a chunk dropped or counted twice, or a mask off by
    one row moves the result far beyond the bound."""
    rng = np.random.default_rng(past + T)
    G, H, D = 2, 4, 128
    S = past + T + 7
    q = rng.standard_normal((T, H, D)).astype(np.float32)
    k = rng.standard_normal((G, S, D)).astype(np.float32)
    nch = (past + T + 63) // 64
    k *= np.repeat(rng.uniform(0.3, 3.0, (G, nch + 1)), 64, axis=1)[:, :S, None].astype(np.float32)
    v = rng.standard_normal((G, S, D)).astype(np.float32)
    if kv == "f16":
        q16, k, v = q.astype(np.float16).astype(np.float32), k.astype(np.float16), v.astype(np.float16)
        ref = _attention_f64(q16, k.astype(np.float32), v.astype(np.float32), past)
        tol = 3e-3  # probabilities rounded to f16
    else:
        ref = _attention_f64(q, k, v, past)
        tol = 2e-5
    got = oracle_py.attention(q, k, v, past).astype(np.float64)
    err = np.abs(got - ref).max() / np.abs(ref).max()
    assert err <= tol, err


@pytest.mark.parametrize("past,T", LONG_CASES)
def test_attention_long_context_exact_on_planted_keys(past, T):
    """Scores of exactly +50 ("hot" keys) or -150 (probability exp(-200), which
    flushes to 0): every chunk maximum that holds a hot key is 50, so every merge
    factor is 1 or 0, l is the count of hot keys and O the sum of their
    small-integer v rows: all exact, so the output is (sum / count) rounded once,
    in any order. A chunk missing from the merge or counted twice, or a key past a
    row's causal limit changes it."""
    rng = np.random.default_rng(7 * past + T)
    G, H, D = 2, 4, 128
    S = past + T
    a = np.float32(np.sqrt(128.0))  # q = a e0 and k[0] = +-50 or -150: score k[0]
    q = np.zeros((T, H, D), np.float32)
    q[:, :, 0] = a
    k = np.zeros((G, S, D), np.float32)
    hot = rng.random((G, S)) < 0.05
    hot[:, rng.integers(0, S, 3)] = True
    k[:, :, 0] = np.where(hot, 50.0, -150.0)
    v = rng.integers(-8, 9, (G, S, D)).astype(np.float32)
    got = oracle_py.attention(q, k, v, past)
    for t in range(T):
        for h in range(H):
            g = h // (H // G)
            sel = hot[g, :past + t + 1]
            if not sel.any():
                continue  # a row without a hot key: every p is 0 (0 / 0)
            want = (v[g, :past + t + 1][sel].astype(np.float64).sum(axis=0) / sel.sum()).astype(np.float32)
            assert np.array_equal(got[t, h], want), (t, h)
