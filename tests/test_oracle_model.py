"""The oracle's decoder step on the CPU.

* Against an independent float64 numpy model written from the Qwen3 definition
  (tests/numpy_ref.py): checks the composition of the ops (norm placement, q/k
  norm before RoPE, GQA head mapping, causal mask, SwiGLU, residuals, tied
  lm_head).
* The reference's state invariants (cpu-lab/moss_target_batch_gate.cpp:204-303):
  a verify batch of T rows equals T serial single-row steps bit for bit (hidden,
  logits, KV), a rewind makes the discarded rows unreachable (NaN-poisoned KV
  past past_len is never read), and invalid rewinds / capacity overflows fail.
"""
import numpy as np
import pytest

import mtg
import numpy_ref
import oracle_py


@pytest.fixture(scope="module")
def model():
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=20261010, std=0.02, gain_jitter=0.05, n_layers=2,
                       vocab=2048)
    yield m
    m.close()


def _prefilled(model, n, kv_type=mtg.TYPE_F32, max_seq=160, seed=1):
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    ids = np.random.default_rng(seed).integers(0, model.hp.vocab, n)
    orc.prefill(orc.embed(ids))
    return orc, ids


def test_embed_rows_are_dequantized_token_embd_rows(model):
    orc = oracle_py.Oracle(model, 16)
    ids = [0, 5, 2047, 5]
    got = orc.embed(ids)
    want = model.dequant_rows(model.desc.contents.token_embd, model.hp.hidden, ids)
    assert np.array_equal(got, want)
    with pytest.raises(AssertionError):
        orc.embed([2048])


def test_oracle_matches_independent_float64_model(model):
    hp = model.hp
    ref = numpy_ref.NumpyQwen3(model, numpy_ref.layer_weights(model))
    orc = oracle_py.Oracle(model, 64)
    rng = np.random.default_rng(2)
    out_norm = np.ctypeslib.as_array(
        (mtg.c_float * hp.hidden).from_address(model.desc.contents.output_norm)).astype(np.float64)
    embd = model.dequant_rows(model.desc.contents.token_embd, hp.hidden, range(hp.vocab)).astype(np.float64)
    for T in (5, 1, 8):  # prefix of 5 rows, then a single row, then a verify batch of 8
        ids = rng.integers(0, hp.vocab, T)
        x = orc.embed(ids)
        h_orc = orc.run(x).astype(np.float64)
        h_ref = numpy_ref.rms(ref.step(x), out_norm, hp.rms_eps)
        err = np.abs(h_orc - h_ref)
        # activation codes of the two models may differ by one at rounding
        # boundaries; the bulk agrees to ~1e-5 relative
        assert np.sqrt((err ** 2).mean()) <= 2e-4 * np.sqrt((h_ref ** 2).mean())
        assert err.max() <= 5e-3 * np.abs(h_ref).max()
        lg = orc.logits(h_orc.astype(np.float32)).astype(np.float64)
        lr = numpy_ref.q8_act(h_orc) @ embd.T
        assert np.abs(lg - lr).max() <= 1e-5 * np.abs(lr).max()


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16])
def test_batch_equals_serial_bit_for_bit(model, kv_type):
    """The reference's exactness gate: one append of T rows equals T single-row
    appends (hidden, logits and every active KV element)."""
    a, _ = _prefilled(model, 70, kv_type)
    b, _ = _prefilled(model, 70, kv_type)
    rng = np.random.default_rng(3)
    for T in (2, 8, 16):
        toks = rng.integers(0, model.hp.vocab, T)
        ca, ma, ha, la = a.verify(toks, want_hidden=True, want_logits=True)
        hs, ls = [], []
        for t in toks:
            _, _, h1, l1 = b.verify([t], want_hidden=True, want_logits=True)
            hs.append(h1[0])
            ls.append(l1[0])
        assert np.array_equal(ha, np.stack(hs))
        assert np.array_equal(la, np.stack(ls))
        ka, va = a.kv_read(a.past_len)
        kb, vb = b.kv_read(b.past_len)
        assert np.array_equal(ka.view(np.uint8), kb.view(np.uint8))
        assert np.array_equal(va.view(np.uint8), vb.view(np.uint8))
        # verify's choices are the first maxima of the returned logits
        assert ca.tolist() == [int(np.argmax(r)) for r in la]


def test_rewind_hides_discarded_rows_from_later_steps(model):
    """After a rewind, a step reads only positions < past_len: poisoning every
    position from past_len on with NaN changes nothing
    (cpu-lab/moss_speculative_gate.cpp:216-229)."""
    a, _ = _prefilled(model, 40)
    b, _ = _prefilled(model, 40)
    rng = np.random.default_rng(4)
    toks = rng.integers(0, model.hp.vocab, 8)
    a.verify(toks)
    a.rewind(43)                       # keep 3 of the 8 rows
    k, v = a.kv_read(43)
    L, NKV, _, D = k.shape
    kp = np.full((L, NKV, 160, D), np.nan, np.float32)
    vp = np.full((L, NKV, 160, D), np.nan, np.float32)
    kp[:, :, :43], vp[:, :, :43] = k, v
    b.kv_write(kp, vp)
    b.rewind(43)
    nxt = rng.integers(0, model.hp.vocab, 6)
    c1, m1, h1, l1 = a.verify(nxt, want_hidden=True, want_logits=True)
    c2, m2, h2, l2 = b.verify(nxt, want_hidden=True, want_logits=True)
    assert np.isfinite(l2).all()
    assert np.array_equal(h1, h2) and np.array_equal(l1, l2) and np.array_equal(c1, c2)


def test_acceptance_counts_leading_drafts_equal_to_the_previous_choice(model):
    orc, _ = _prefilled(model, 20)
    rng = np.random.default_rng(5)
    seed = int(rng.integers(0, model.hp.vocab))
    # learn the greedy continuation row by row, then verify it as drafts
    chain = [seed]
    for _ in range(6):
        past = orc.past_len
        c, _, _, _ = orc.verify(chain + [0])
        orc.rewind(past)
        chain.append(int(c[len(chain) - 1]))
    past = orc.past_len
    c, m, _, _ = orc.verify(chain)
    assert m == 6 and c[:6].tolist() == chain[1:]
    orc.rewind(past)
    bad = list(chain)
    bad[3] = (bad[3] + 1) % model.hp.vocab
    c, m, _, _ = orc.verify(bad)
    assert m == 2


def test_state_errors(model):
    orc, _ = _prefilled(model, 10, max_seq=16)
    L = oracle_py.lib()
    assert L.orc_rewind(orc.m, 11) == mtg.ERR_STATE
    assert L.orc_rewind(orc.m, -1) == mtg.ERR_STATE
    with pytest.raises(RuntimeError):
        orc.run(orc.embed([1] * 7))  # 10 + 7 > 16
    assert orc.past_len == 10
    orc.run(orc.embed([1] * 6))
    assert orc.past_len == 16


def test_f16_kv_cache_stays_close_to_f32(model):
    a, _ = _prefilled(model, 60, mtg.TYPE_F32)
    b, _ = _prefilled(model, 60, mtg.TYPE_F16)
    toks = np.random.default_rng(6).integers(0, model.hp.vocab, 8)
    _, _, ha, _ = a.verify(toks, want_hidden=True)
    _, _, hb, _ = b.verify(toks, want_hidden=True)
    assert np.sqrt(((ha - hb) ** 2).mean()) <= 2e-2 * np.sqrt((ha ** 2).mean())
    kb, _ = b.kv_read(68)
    ka, _ = a.kv_read(68)
    assert kb.dtype == np.float16
    # K written at positions 60..67 by the two runs differ only by f16 rounding
    # plus the propagated differences of the earlier layers
    assert np.abs(kb[0, :, 60:].astype(np.float32) - ka[0, :, 60:]).max() <= 1e-2 * np.abs(ka).max()
