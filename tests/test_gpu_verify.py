"""Verify-step parity on the GPU against the oracle (same weights, same KV)."""
import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu


def _setup(n_layers, prefix, kv_type=mtg.TYPE_F32, vocab=4096, seed=0, max_seq=256, jitter=0.05):
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=seed, std=0.02, gain_jitter=jitter, n_layers=n_layers,
                           vocab=vocab)
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    dec = mtg.Decoder(model, max_seq, kv_type)
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, vocab, prefix)
    orc.prefill(orc.embed(ids))
    k, v = orc.kv_read(prefix)
    dec.kv_write(k, v)
    return model, orc, dec, rng


def _close(got, ref, what):
    tol = 1e-4 + 1e-3 * np.abs(ref)
    err = np.abs(got - ref)
    assert (err <= tol).all(), "%s: max err %.3g at %s" % (what, err.max(), np.unravel_index(err.argmax(), err.shape))


@pytest.mark.parametrize("T", [1, 4, 8, 16])
def test_verify_matches_oracle(T):
    print("verify parity: 2 layers, prefix 40, T=%d" % T, flush=True)
    model, orc, dec, rng = _setup(2, 40)
    tokens = rng.integers(0, model.hp.vocab, T)
    c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
    c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
    _close(h1, h0, "hidden")
    _close(l1, l0, "logits")
    assert np.array_equal(c1, c0)
    assert m1 == m0
    assert dec.past_len == orc.past_len == 40 + T
    # the appended KV rows match too
    k0, v0 = orc.kv_read(40 + T)
    k1, v1 = dec.kv_read(40 + T)
    _close(k1, k0, "K cache")
    _close(v1, v0, "V cache")
