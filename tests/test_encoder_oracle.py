"""The oracle's Whisper encoder + audio adaptor (oracle/oracle.cpp, encoder
section; reference src/whisper_encoder.cpp:103-209, src/audio_adaptor.cpp:38-97)
pinned against float64 restatements in numpy: each part (GELU-erf, LayerNorm,
the conv stem's conv1d, the bidirectional attention) to float rounding, and the
whole encoder + adaptor on a small configuration with the q8_0 activation
rounding of ggml's mul_mat reproduced exactly (integer block dots), so only
float summation order separates the two."""
import ctypes
import math

import numpy as np
import pytest

import mtg
import oracle_py


def test_gelu_erf_matches_float64():
    """ggml's float formula (0.5 x)(1 + erf(x c)), c = 1/sqrt(2) as a float, with
    erf correctly rounded from float64: the oracle's series erf may differ from
    that by an ulp of erf, so the result agrees to 2 ulp, and exactly almost
    always; against exact GELU, to float rounding plus the absolute error of the
    formula's 1 + erf (an ulp of 1, times 0.5 |x|)."""
    xs = np.concatenate([np.linspace(-12, 12, 6001), [0.0, -0.0, 1e-30, -1e-30, 1e-6, 5.65685, -5.65686, 20, -20]])
    xs = xs.astype(np.float32)
    c = np.float32(0.70710678118654752440)
    exact_hits = 0
    for x in xs:
        z = np.float32(x * c)
        e = np.float32(math.erf(float(z)))
        ref = np.float32(np.float32(np.float32(0.5) * x) * np.float32(np.float32(1) + e))
        got = np.float32(oracle_py.gelu_erf(x))
        ulp = np.spacing(np.float32(max(abs(ref), 1e-37)))
        assert abs(float(got) - float(ref)) <= 2 * ulp, (x, got, ref)
        exact_hits += int(got == ref)
        true = 0.5 * float(x) * (1.0 + math.erf(float(x) / math.sqrt(2.0)))
        assert abs(float(got) - true) <= 2e-6 * abs(true) + 6e-8 * abs(float(x)) + 1e-37, (x, got, true)
    assert exact_hits >= 0.999 * len(xs)
    assert oracle_py.gelu_erf(0.0) == 0.0 and oracle_py.gelu_erf(-30.0) == 0.0 and oracle_py.gelu_erf(30.0) == 30.0


@pytest.mark.parametrize("n,eps", [(1024, 1e-5), (128, 1e-6), (64, 0.5)])
def test_layer_norm_matches_float64(n, eps):
    rng = np.random.default_rng(n)
    for scale, shift in ((1.0, 0.0), (0.01, 3.0), (40.0, -7.0)):
        x = (rng.standard_normal(n) * scale + shift).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
        b = (0.1 * rng.standard_normal(n)).astype(np.float32)
        got = oracle_py.layer_norm(x, w, b, eps)
        # ggml_norm's float steps: the mean rounded to float, x - mean in float,
        # the squares in float, the sums in double
        mean = np.float32(x.astype(np.float64).sum() / n)
        v = (x - mean).astype(np.float32)
        var = np.float32((v * v).astype(np.float64).sum() / n)
        inv = np.float32(1) / np.sqrt(np.float32(var + np.float32(eps)))
        ref = v.astype(np.float64) * float(inv) * w + b
        np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-7)
        # and the exact normalization, to the float rounding of the mean's subtraction
        x64 = x.astype(np.float64)
        exact = (x64 - x64.mean()) / np.sqrt(x64.var() + eps) * w + b
        np.testing.assert_allclose(got, exact, rtol=0, atol=4e-7 * (abs(shift) + 1) / scale + 2e-6)


@pytest.mark.parametrize("stride", [1, 2])
def test_conv1d_matches_float64(stride):
    rng = np.random.default_rng(stride)
    ic, oc, L = 16, 32, 37
    w = rng.standard_normal((oc, ic, 3)).astype(np.float32)
    x = rng.standard_normal((ic, L)).astype(np.float32)
    got = oracle_py.conv1d(w, x, stride)
    xp = np.pad(x.astype(np.float64), ((0, 0), (1, 1)))
    OL = (L - 1) // stride + 1
    ref = np.empty((OL, oc))
    for t in range(OL):
        ref[t] = np.einsum("oik,ik->o", w.astype(np.float64), xp[:, t * stride: t * stride + 3])
    assert got.shape == (OL, oc)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("T", [1, 63, 64, 150])
def test_encoder_attention_matches_float64(T):
    rng = np.random.default_rng(T)
    H, D = 2, 64
    q, k, v = (rng.standard_normal((T, H * D)).astype(np.float32) for _ in range(3))
    got = oracle_py.enc_attention(q, k, v, H)
    ref = np.empty((T, H * D))
    for h in range(H):
        sl = slice(h * D, (h + 1) * D)
        s = q[:, sl].astype(np.float64) @ k[:, sl].astype(np.float64).T / math.sqrt(D)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        p /= p.sum(axis=1, keepdims=True)
        ref[:, sl] = p @ v[:, sl].astype(np.float64)
    np.testing.assert_allclose(got, ref, rtol=1e-5, atol=1e-6)


# ---- the whole encoder + adaptor against numpy float64 -----------------------
def _f32(addr, n):
    return np.frombuffer(ctypes.string_at(addr, 4 * n), np.float32).astype(np.float64)


def _q8(addr, n, k):
    raw = np.frombuffer(ctypes.string_at(addr, n * (k // 32) * 34), np.uint8).reshape(n, k // 32, 34)
    d = raw[:, :, :2].copy().view(np.float16).astype(np.float64)  # [n][k/32][1]
    q = raw[:, :, 2:].view(np.int8).astype(np.float64)
    return q, d


def _act_q8(x):
    """ggml's q8_0 activation rounding, per row and 32-block (float32 arithmetic)."""
    x = x.astype(np.float32)
    xb = x.reshape(x.shape[0], -1, 32)
    amax = np.abs(xb).max(axis=2, keepdims=True)
    d = (amax / np.float32(127)).astype(np.float16).astype(np.float64)
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = np.where(amax != 0, np.float32(127) / amax, np.float32(0)).astype(np.float32)
    codes = np.rint((xb * iscale).astype(np.float32)).astype(np.float64)
    return codes, d


def _act_q8k(x):
    """ggml's q8_K activation (the vec_dot_type of q4_K): per 256-block the signed
    first-largest element gives iscale = -127 / max, codes round to nearest, at
    most 127, d = 1 / iscale; returned dequantized (float64)."""
    b = x.astype(np.float32).reshape(x.shape[0], -1, 256)
    idx = np.abs(b).argmax(axis=2)
    mx = np.take_along_axis(b, idx[..., None], 2)
    with np.errstate(divide="ignore", invalid="ignore"):
        iscale = np.where(mx != 0, np.float32(-127.0) / mx, np.float32(0)).astype(np.float32)
        codes = np.minimum(127, np.rint(iscale * b))
        d = np.where(iscale != 0, np.float32(1.0) / iscale, np.float32(0)).astype(np.float64)
    return (codes * d).reshape(x.shape)


def _weights(wtype, addr, n, k):
    """A matrix of the synthetic encoder: q8_0 as (codes, scales) for the exact
    block dots, f16, f32 and q4_K dequantized to float64 by the library's decoder."""
    if wtype == mtg.TYPE_Q8_0:
        return wtype, _q8(addr, n, k)
    nbytes = mtg.lib().mtg_row_bytes(wtype, k) * n
    raw = np.frombuffer(ctypes.string_at(addr, nbytes), np.uint8).copy()
    w = np.empty((n, k), np.float32)
    mtg.lib().mtg_dequantize(wtype, mtg.ptr(raw), n * k, mtg.ptr(w))
    return wtype, w.astype(np.float64)


def _linear(W, b, x):
    wtype, m = W
    if wtype == mtg.TYPE_Q8_0:
        q, dw = m
        cx, dx = _act_q8(x)
        # exact integer block dots, then (d_w d_x) per block, summed in float64
        dots = np.einsum("nbj,tbj->tnb", q, cx)
        y = np.einsum("tnb,nb,tb->tn", dots, dw[:, :, 0], dx[:, :, 0])
    elif wtype == mtg.TYPE_F16:
        y = x.astype(np.float32).astype(np.float16).astype(np.float64) @ m.T  # vec_dot_type F16
    elif wtype == mtg.TYPE_F32:
        y = x.astype(np.float32).astype(np.float64) @ m.T  # vec_dot_type F32
    else:
        y = _act_q8k(x) @ m.T
    return y if b is None else y + b


def _ln(x, w, b, eps):
    m = x.mean(axis=1, keepdims=True)
    return (x - m) / np.sqrt(x.var(axis=1, keepdims=True) + eps) * w + b


def _gelu(x):
    from scipy.special import erf
    return 0.5 * x * (1 + erf(x / math.sqrt(2)))


def _reference(syn, mel):
    h, d = syn.hp, syn.desc
    D, F, M, H, NF = h.d_model, h.ffn, h.n_mels, h.hidden, h.n_frames
    R = syn.rows
    wt = syn.wtype
    c1w = _f32(d.conv1_w, D * M * 3).reshape(D, M, 3)
    c2w = _f32(d.conv2_w, D * D * 3).reshape(D, D, 3)

    def conv(w, x, s):
        xp = np.pad(x, ((0, 0), (1, 1)))
        OL = (x.shape[1] - 1) // s + 1
        return np.stack([np.einsum("oik,ik->o", w, xp[:, t * s: t * s + 3]) for t in range(OL)])

    x1 = _gelu(conv(c1w, mel.astype(np.float64), 1) + _f32(d.conv1_b, D))
    x = _gelu(conv(c2w, x1.T, 2) + _f32(d.conv2_b, D)) + _f32(d.pos_embd, R * D).reshape(R, D)
    NH, hd = h.n_heads, D // h.n_heads
    for i in range(h.n_layers):
        L = d.layers[i]
        xn = _ln(x, _f32(L.attn_ln_w, D), _f32(L.attn_ln_b, D), 1e-5)
        q = _linear(_weights(wt, L.q_w, D, D), _f32(L.q_b, D), xn)
        k = _linear(_weights(wt, L.k_w, D, D), None, xn)
        v = _linear(_weights(wt, L.v_w, D, D), _f32(L.v_b, D), xn)
        a = np.empty_like(q)
        for hh in range(NH):
            sl = slice(hh * hd, (hh + 1) * hd)
            s = q[:, sl] @ k[:, sl].T / math.sqrt(hd)
            p = np.exp(s - s.max(axis=1, keepdims=True))
            a[:, sl] = (p / p.sum(axis=1, keepdims=True)) @ v[:, sl]
        x = x + _linear(_weights(wt, L.o_w, D, D), _f32(L.o_b, D), a)
        xn = _ln(x, _f32(L.ffn_ln_w, D), _f32(L.ffn_ln_b, D), 1e-5)
        f = _gelu(_linear(_weights(wt, L.fc1_w, F, D), _f32(L.fc1_b, F), xn))
        x = x + _linear(_weights(wt, L.fc2_w, D, F), _f32(L.fc2_b, D), f)
    enc = _ln(x, _f32(d.ln_post_w, D), _f32(d.ln_post_b, D), 1e-5)
    return enc


def _adapt_reference(syn, enc, T):
    h, d = syn.hp, syn.desc
    D, H, IN = h.d_model, h.hidden, h.d_model * h.merge
    N = T // h.merge
    x = enc[: N * h.merge].reshape(N, IN)
    y = _linear(_weights(syn.wtype, d.ad_fc1_w, H, IN), _f32(d.ad_fc1_b, H), x)
    y = y / (1 + np.exp(-y))
    y = _linear(_weights(syn.wtype, d.ad_fc2_w, H, H), _f32(d.ad_fc2_b, H), y)
    return _ln(y, _f32(d.ad_ln_w, H), _f32(d.ad_ln_b, H), h.adaptor_eps)


def _rel_rms(a, b):
    return float(np.sqrt(np.mean((a - b) ** 2)) / np.sqrt(np.mean(b ** 2)))


# (weight type, seed, d): d 256 for q4_K so that every matrix's K is a whole number
# of superblocks. The seeds are ones whose activations have no q8_0 / q8_K code
# within float32 rounding of a rounding boundary: a code that flips between the
# float32 and the float64 evaluation moves a row by one quantization step, and
# attention spreads it to every row (another seed's second layer shows 2e-3).
ENC_CASES = [(mtg.TYPE_Q8_0, 5, 128), (mtg.TYPE_F16, 6, 256), (mtg.TYPE_F32, 6, 256), (mtg.TYPE_Q4_K, 6, 256)]


@pytest.mark.parametrize("wtype,seed,d", ENC_CASES, ids=["q8_0", "f16", "f32", "q4_K"])
def test_small_encoder_and_adaptor_match_float64(wtype, seed, d):
    syn = mtg.SynthEncoder(seed=seed, wtype=wtype, n_mels=16, n_frames=96, d_model=d, n_layers=2,
                           n_heads=d // 64, ffn=2 * d, merge=4, hidden=d)
    orc = oracle_py.OracleEncoder(syn)
    mel = syn.mel(seed=9)
    got = orc.encode(mel)
    ref = _reference(syn, mel)
    assert got.shape == ref.shape == (48, d)
    err = _rel_rms(got, ref)
    print("encoder vs float64: relative rms %.2e" % err)
    assert err < 2e-4
    T = 46  # trimmed to 44 rows -> 11 adaptor rows
    ad = orc.adapt(T)
    ad_ref = _adapt_reference(syn, got.astype(np.float64), T)
    assert ad.shape == (11, d)
    err = _rel_rms(ad, ad_ref)
    print("adaptor vs float64: relative rms %.2e" % err)
    assert err < 2e-4
    # rows given by the caller instead of the last encode
    np.testing.assert_array_equal(orc.adapt(T, rows=got), ad)
    orc.close()
