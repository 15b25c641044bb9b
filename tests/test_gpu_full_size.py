"""Full-size parity: the Qwen3-0.6B shape (28 layers, hidden 1024, 16 / 8 heads,
151,936-row tied vocabulary) at the row counts and contexts of the benchmark
workloads, two verify steps each (the second with the repetition penalty), device
against the oracle bit for bit.

The cached prefix is seeded random K/V written to both sides, different in every
layer: the verify arithmetic does not depend on how the cache was filled, and
prefill parity is covered at small sizes (test_gpu_verify.py) and on the full
1,600-row prompt (test_gpu_streams.py)."""
import os

import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

# (id, weights, KV type, verify rows T, cached prefix, execution path)
CASES = [
    ("q8_0-f32kv-T8-ctx1600-step", mtg.TYPE_Q8_0, mtg.TYPE_F32, 8, 1600, mtg.EXEC_STEP_KERNEL),
    ("q8_0-f32kv-T4-ctx512-step", mtg.TYPE_Q8_0, mtg.TYPE_F32, 4, 512, mtg.EXEC_STEP_KERNEL),
    ("q8_0-f16kv-T16-ctx4000-step", mtg.TYPE_Q8_0, mtg.TYPE_F16, 16, 4000, mtg.EXEC_STEP_KERNEL),
    ("q8_0-f32kv-T8-ctx1600-graph", mtg.TYPE_Q8_0, mtg.TYPE_F32, 8, 1600, mtg.EXEC_GRAPH),
    ("f16-f16kv-T8-ctx8000-step", mtg.TYPE_F16, mtg.TYPE_F16, 8, 8000, mtg.EXEC_STEP_KERNEL),
    ("f16-f16kv-T8-ctx8000-graph", mtg.TYPE_F16, mtg.TYPE_F16, 8, 8000, mtg.EXEC_GRAPH),
    ("q4_K-f16kv-T16-ctx16384-graph", mtg.TYPE_Q4_K, mtg.TYPE_F16, 16, 16384, mtg.EXEC_GRAPH),
    # the converter's default dtype: every matrix f32 (2.4 GB of weights)
    ("f32-f32kv-T8-ctx1600-graph", mtg.TYPE_F32, mtg.TYPE_F32, 8, 1600, mtg.EXEC_GRAPH),
    ("f32-f32kv-T8-ctx1600-step", mtg.TYPE_F32, mtg.TYPE_F32, 8, 1600, mtg.EXEC_STEP_KERNEL),
]


def _same(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g at %s"
                         % (what, int((got != ref).sum()), err.max(), np.unravel_index(err.argmax(), err.shape)))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_full_size_verify_matches_oracle(case):
    name, wtype, kv, T, prefix, exec_mode = case
    print("full-size parity: %s" % name, flush=True)
    oracle_py.lib().orc_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    model = mtg.SynthModel(wtype, seed=3, std=0.02, gain_jitter=0.05)
    hp = model.hp
    assert (hp.n_layers, hp.hidden, hp.n_heads, hp.n_kv_heads, hp.vocab) == (28, 1024, 16, 8, 151936)
    max_seq = prefix + 2 * T + 16
    orc = oracle_py.Oracle(model, max_seq, kv)
    dec = mtg.Decoder(model, max_seq, kv)
    dec.set_exec(exec_mode)
    dec.set_step_max_keys(1 << 30)  # the step cases run the persistent kernel at every context
    rng = np.random.default_rng(prefix + T)
    dt = np.float32 if kv == mtg.TYPE_F32 else np.float16
    # distinct seeded rows in every layer, so that a layer reading another layer's
    # cache (a wrong layer stride or table entry) changes the result
    shape = (hp.n_layers, hp.n_kv_heads, prefix, hp.head_dim)
    k = rng.standard_normal(shape, dtype=np.float32).astype(dt)
    v = (0.5 * rng.standard_normal(shape, dtype=np.float32)).astype(dt)
    orc.kv_write(k, v)
    dec.kv_write(k, v)
    del k, v
    tokens = rng.integers(0, hp.vocab, T)
    c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
    c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
    _same(h1, h0, "hidden")
    _same(l1, l0, "logits")
    assert np.array_equal(c1, c0) and m1 == m0
    assert dec.past_len == orc.past_len == prefix + T
    if prefix <= 4000:  # the appended rows, and the prefix left as it was
        k0, v0 = orc.kv_read(prefix + T)
        k1, v1 = dec.kv_read(prefix + T)
        _same(k1, k0, "K cache")
        _same(v1, v0, "V cache")
    # a second step with the repetition penalty over a 120-token history
    hist = rng.integers(0, hp.vocab, 120)
    tokens = rng.integers(0, hp.vocab, T)
    c0, m0, _, l0 = orc.verify(tokens, history=hist, penalty=1.3, want_logits=True)
    c1, m1, _, l1 = dec.verify(tokens, history=hist, penalty=1.3, want_logits=True)
    _same(l1, l0, "logits, second step")
    assert np.array_equal(c1, c0) and m1 == m0
    dec.close()
    orc.close()
    model.close()
