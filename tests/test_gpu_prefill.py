"""The block prefill (csrc/prefill.hip for q8_0 weights, csrc/prefill_wt.hip for f16
and q4_K): S prompt rows through the decoder with each weight matrix streamed once
per block of up to 2,048 rows, against the oracle's prefill
(src/qwen3_decoder.cpp:162-166 runs the prompt as one batch) and against the
verify-size batch path. Hidden rows and the whole KV cache must be bit-identical:
the block kernels keep the canonical order of every reduction."""
import os

import numpy as np
import pytest

import mtg
import oracle_py
from workloads import WORKLOADS, build_prompt, prompt_rows

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _same(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g at %s"
                         % (what, int((got != ref).sum()), err.max(), np.unravel_index(err.argmax(), err.shape)))


WTYPES = [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K]
WT_IDS = ["q8_0", "f16", "f32", "q4_K"]


@pytest.mark.parametrize("wtype", WTYPES, ids=WT_IDS)
@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
@pytest.mark.parametrize("S", [1, 37, 64, 100, 333])
def test_block_prefill_matches_oracle(kv_type, S, wtype):
    print("block prefill vs oracle: S=%d kv %d weights %d" % (S, kv_type, wtype), flush=True)
    oracle_py.lib().orc_set_threads(THREADS)
    model = mtg.SynthModel(wtype, seed=5, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    hp = model.hp
    max_seq = S + 40
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    dec = mtg.Decoder(model, max_seq, kv_type)
    rng = np.random.default_rng(S)
    rows = orc.embed(rng.integers(0, hp.vocab, S))
    rows[: S // 2] = rng.standard_normal((S // 2, hp.hidden)).astype(np.float32) * np.float32(0.05)
    h0 = orc.prefill(rows)
    h1 = dec.prefill(rows)
    _same(h1, h0, "hidden rows")
    k0, v0 = orc.kv_read(S)
    k1, v1 = dec.kv_read(S)
    _same(k1, k0, "K cache")
    _same(v1, v0, "V cache")
    assert dec.past_len == S
    tokens = rng.integers(0, hp.vocab, 8)
    c0, m0, _, l0 = orc.verify(tokens, want_logits=True)
    c1, m1, _, l1 = dec.verify(tokens, want_logits=True)
    _same(l1, l0, "logits of the verify step after the prefill")
    assert np.array_equal(c1, c0) and m1 == m0
    dec.close()
    orc.close()
    model.close()


@pytest.mark.parametrize("wtype", WTYPES, ids=WT_IDS)
@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
def test_block_prefill_equals_verify_batches_over_two_blocks(kv_type, wtype):
    """2,100 rows: a full block of 2,048 and a second block of 52 that attends
    over the first one's cache rows; against the same prompt in 16-row batches."""
    print("block prefill vs batches: S=2100 kv %d weights %d" % (kv_type, wtype), flush=True)
    model = mtg.SynthModel(wtype, seed=6, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    hp = model.hp
    S = 2100
    a = mtg.Decoder(model, S + 8, kv_type)
    b = mtg.Decoder(model, S + 8, kv_type)
    b.prefill_mode(False)
    rows = mtg.normal(11, 0, S * hp.hidden).reshape(S, hp.hidden) * np.float32(0.03)
    ha = a.prefill(rows)
    hb = b.prefill(rows)
    _same(ha, hb, "hidden rows")
    ka, va = a.kv_read(S)
    kb, vb = b.kv_read(S)
    _same(ka, kb, "K cache")
    _same(va, vb, "V cache")
    a.close()
    b.close()
    model.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg_id", [2, 4, 5], ids=["q8_0-1600rows", "f16-8000rows", "q4_K-16384rows"])
def test_full_size_prefill_paths_and_time(cfg_id):
    """A workload's prompt at full size (the 1,600-row q8_0 one, the 8,000-row f16
    one, the 16,384-row q4_K one): block prefill and 16-row batches give the same
    hidden rows and KV cache; both are timed."""
    import time
    cfg = WORKLOADS[cfg_id]
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n = prompt_rows(cfg)
    a = mtg.Decoder(model, n + 64, cfg["kv"])
    b = mtg.Decoder(model, n + 64, cfg["kv"])
    b.prefill_mode(False)
    rows, _, _ = build_prompt(model, a.embed, cfg)
    a.prefill(rows)  # warm
    t0 = time.perf_counter()
    ha = a.prefill(rows)
    t_block = time.perf_counter() - t0
    t0 = time.perf_counter()
    hb = b.prefill(rows)
    t_batch = time.perf_counter() - t0
    print("full-size %d-row prefill (weights %d): block path %.2f ms (device %.2f ms), 16-row batches %.1f ms"
          % (n, cfg["wtype"], 1e3 * t_block, a.last_prefill_ms, 1e3 * t_batch), flush=True)
    _same(ha, hb, "hidden rows")
    ka, va = a.kv_read(n)
    kb, vb = b.kv_read(n)
    _same(ka, kb, "K cache")
    _same(va, vb, "V cache")
    a.close()
    b.close()
    model.close()
