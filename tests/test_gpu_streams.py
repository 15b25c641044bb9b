"""Full-size token streams on the GPU against the oracle, and the reference's
softmax stress rows through the device attention.

* The 1,600-row prompt of the K=8 q8_0 workload (4 x 375 audio rows + 100 text
  ids) is prefilled on the device and by the oracle: hidden rows and the whole KV
  cache bit-identical. Then all 256 greedy steps of the workload with the stream
  drafter on both sides: identical ids and counters. The top-2 logit margins of the committed stream are
  printed, and the choices of the oracle in ggml's generic order are compared with
  the device's on the first 64 committed rows (they must agree wherever the margin
  exceeds the largest logit difference between the two orders, and they agree on
  every one of those rows).
* The K=16 f16-KV workload at a 4,000-row prompt: all 128 greedy steps from the same
  KV state on both sides, identical ids and counters.
* The f16-weight workload (8,000-row prompt, K=8, 128 steps) and the q4_K workload
  (16,384-row prompt, K=16, 64 steps), both with an f16 cache, on the per-op kernels:
  the prompt prefilled on the device, every greedy step of the workload on both sides
  from that KV state, identical ids, counters and appended KV rows.
* The 1,600-row workload with f16 and with f32 weights on the persistent kernel's row
  variants: 128 greedy steps through the host loop and the device loop, identical to
  the oracle.
* Attention on scores of +-10000 and -inf (tests/test_cpu_softmax.cpp:40-46), made
  by planting keys of magnitude 10^4 in the cache: bit-identical to the oracle.
"""
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
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g"
                         % (what, int((got != ref).sum()), err.max()))


def _log(msg):
    print(msg, flush=True)


@pytest.mark.timeout(600)
def test_full_size_prefill_and_stream_k8_q8_0_ctx1600():
    cfg = WORKLOADS[2]
    oracle_py.lib().orc_set_threads(THREADS)
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    hp = model.hp
    n_prompt, steps, K = prompt_rows(cfg), cfg["steps"], cfg["K"]
    assert steps == 256
    max_seq = n_prompt + (steps + 4) * K
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    orc = oracle_py.Oracle(model, max_seq, cfg["kv"])
    rows, text, stream = build_prompt(model, dec.embed, cfg)
    assert np.array_equal(rows[-cfg["text"]:], orc.embed(text))
    _log("config-2 stream: device prefill of %d rows" % n_prompt)
    hid_gpu = dec.prefill(rows)
    _log("config-2 stream: oracle prefill of %d rows (%d threads)" % (n_prompt, THREADS))
    hid_orc = orc.prefill(rows)
    _same(hid_gpu, hid_orc, "prefill hidden rows")
    k0, v0 = orc.kv_read(n_prompt)
    k1, v1 = dec.kv_read(n_prompt)
    _same(k1, k0, "K cache after prefill")
    _same(v1, v0, "V cache after prefill")
    del k0, v0, k1, v1
    l_gpu = dec.logits(hid_gpu[-1:])
    l_orc = orc.logits(hid_orc[-1:])
    _same(l_gpu, l_orc, "logits of the last prompt row")
    first = int(np.argmax(l_gpu[0]))
    fn, user, _keep = mtg.stream_drafter(text, stream)
    _log("config-2 stream: %d greedy steps on both sides" % steps)
    ids1, st1 = dec.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    ids0, st0 = orc.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    assert ids1.tolist() == ids0.tolist()
    for f in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds"):
        assert getattr(st1, f) == getattr(st0, f), f
    assert dec.past_len == orc.past_len
    _log("config-2 stream: %d ids, %d accepted drafts over %d steps" % (len(ids1), st1.accepted, st1.target_calls))
    # top-2 margins along the committed stream, and the generic-order oracle
    gen = oracle_py.Oracle(model, max_seq, cfg["kv"])
    k, v = dec.kv_read(n_prompt)
    gen.kv_write(k, v)
    del k, v
    gen.set_order(gen.ORDER_GGML_GENERIC)
    dec.rewind(n_prompt)
    # the input at position n_prompt + i is committed id i (the first seed is id 0),
    # and the row of input i chooses id i + 1
    seq = ids1.astype(np.int32)
    assert seq[0] == first
    margins, agree, diffs = [], 0, []
    windows = min(8, len(seq) // K)
    for wi in range(windows):
        tok = seq[wi * K:(wi + 1) * K]
        hist = seq[:wi * K]
        c1, _, _, lg = dec.verify(tok, history=hist, want_logits=True)
        c2, _, _, lr = gen.verify(tok, history=hist, want_logits=True)
        top = np.sort(lg, axis=1)
        m = top[:, -1] - top[:, -2]
        d = np.abs(lg.astype(np.float64) - lr).max()
        diffs.append(d)
        margins.extend(m.tolist())
        safe = m > 2 * d
        assert np.array_equal(c1[safe], c2[safe]), (wi, c1.tolist(), c2.tolist(), m.tolist(), d)
        # the device's choices are the committed stream's next ids
        n = min(K, len(seq) - 1 - wi * K)
        assert np.array_equal(c1[:n], seq[wi * K + 1:wi * K + 1 + n]), wi
        agree += int((c1 == c2).sum())
    gen.close()
    m = np.array(margins)
    _log("config-2 margins over %d rows: min %.3g, p1 %.3g, p5 %.3g, p50 %.3g; rows below 0.04: %d; "
         "device vs generic order: max |dlogit| %.3g, choices equal in %d of %d rows"
         % (len(m), m.min(), np.percentile(m, 1), np.percentile(m, 5), np.median(m), int((m < 0.04).sum()),
            max(diffs), agree, len(m)))
    # The generic-order oracle run over the whole stream from the same prefill
    # (tests/order_stream.py, on the CPU) commits the same ids as the canonical
    # order up to id 165, so every row replayed here chooses the same id in both.
    assert agree == len(m) == windows * K
    dec.close()
    orc.close()
    model.close()


STREAMS = [(3, "k16-q8_0-f16kv-ctx4000-step"), (4, "k8-f16-f16kv-ctx8000-graph"),
           (5, "k16-q4_K-f16kv-ctx16384-graph")]


@pytest.mark.timeout(600)
@pytest.mark.parametrize("cfg_id", [c for c, _ in STREAMS], ids=[n for _, n in STREAMS])
def test_full_size_stream_all_steps(cfg_id):
    """Every greedy step of a workload (128, 128 and 64) at full size from the
    device's prefilled KV state, on the device and on the oracle: identical ids,
    counters and appended KV rows. The q8_0 workload runs the persistent step kernel;
    the f16 workload (8,000 keys, past the persistent kernel's default limit for f16
    weights) and the q4_K workload the per-op kernels from a graph."""
    cfg = WORKLOADS[cfg_id]
    oracle_py.lib().orc_set_threads(THREADS)
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n_prompt, steps, K = prompt_rows(cfg), cfg["steps"], cfg["K"]
    max_seq = n_prompt + (steps + 4) * K
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    want_exec = mtg.EXEC_STEP_KERNEL if cfg["wtype"] == mtg.TYPE_Q8_0 else mtg.EXEC_GRAPH
    dec.set_exec(want_exec)
    assert dec.exec_mode == want_exec
    rows, text, stream = build_prompt(model, dec.embed, cfg)
    _log("config-%d stream: device prefill of %d rows" % (cfg_id, n_prompt))
    hid = dec.prefill(rows)
    first = int(np.argmax(dec.logits(hid[-1:])[0]))
    orc = oracle_py.Oracle(model, max_seq, cfg["kv"])
    k, v = dec.kv_read(n_prompt)
    orc.kv_write(k, v)
    del k, v
    fn, user, _keep = mtg.stream_drafter(text, stream)
    _log("config-%d stream: %d greedy steps on both sides" % (cfg_id, steps))
    ids1, st1 = dec.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    ids0, st0 = orc.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    assert ids1.tolist() == ids0.tolist()
    for f in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds"):
        assert getattr(st1, f) == getattr(st0, f), f
    assert st1.target_calls == steps
    assert dec.past_len == orc.past_len
    k0, v0 = orc.kv_read(orc.past_len)
    k1, v1 = dec.kv_read(dec.past_len)
    _same(k1[:, :, n_prompt:], k0[:, :, n_prompt:], "K rows appended by the steps")
    _same(v1[:, :, n_prompt:], v0[:, :, n_prompt:], "V rows appended by the steps")
    _log("config-%d stream: %d ids, %d accepted drafts" % (cfg_id, len(ids1), st1.accepted))
    dec.close()
    orc.close()
    model.close()


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
@pytest.mark.parametrize("exec_mode", [mtg.EXEC_STEP_KERNEL, mtg.EXEC_GRAPH], ids=["step", "graph"])
def test_attention_on_extreme_scores(kv_type, exec_mode):
    """Keys of magnitude 10^4 planted at positions 0, 65 and 130 of every head give
    scores of roughly +-10^4 (a row dominated by one key, or one key whose
    probability underflows to exactly 0); the rest of the keys give N(0, 12)-sized
    scores and the causal mask gives -inf. Hidden, logits and choices must be
    finite and bit-identical to the oracle's."""
    print("extreme attention scores: kv %d exec %d" % (kv_type, exec_mode), flush=True)
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=9, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    hp = model.hp
    prefix, max_seq = 200, 256
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    dec = mtg.Decoder(model, max_seq, kv_type)
    dec.set_exec(exec_mode)
    rng = np.random.default_rng(77)
    dt = np.float32 if kv_type == mtg.TYPE_F32 else np.float16
    shape = (hp.n_layers, hp.n_kv_heads, prefix, hp.head_dim)
    k = rng.normal(0.0, 12.0, shape).astype(np.float32)
    for pos in (0, 65, 130):
        k[:, :, pos, :] = np.sign(rng.standard_normal((hp.n_layers, hp.n_kv_heads, hp.head_dim))) * 1e4
    v = rng.standard_normal(shape).astype(np.float32)
    k, v = k.astype(dt), v.astype(dt)
    orc.kv_write(k, v)
    dec.kv_write(k, v)
    for T in (8, 3):
        tokens = rng.integers(0, hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        assert np.isfinite(h1).all() and np.isfinite(l1).all()
        _same(h1, h0, "hidden")
        _same(l1, l0, "logits")
        assert np.array_equal(c1, c0) and m1 == m0
    dec.close()
    orc.close()
    model.close()


@pytest.mark.timeout(600)
@pytest.mark.parametrize("wtype", [mtg.TYPE_F16, mtg.TYPE_F32], ids=["f16", "f32"])
def test_full_size_stream_f16_weights_step_kernel(wtype):
    """f16 and f32 weights on the persistent kernel's row variants at full size: the
    1,600-row prompt of the K=8 workload prefilled on the device, then 128 greedy steps
    with the stream drafter through the host loop and through the device loop (a
    second decoder from the same KV state), against the oracle: identical ids,
    counters and appended KV rows, every step on the persistent kernel (within its
    key limit)."""
    cfg = dict(WORKLOADS[2])
    cfg["wtype"] = wtype
    steps, K = 128, cfg["K"]
    oracle_py.lib().orc_set_threads(THREADS)
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n_prompt = prompt_rows(cfg)
    max_seq = n_prompt + (steps + 4) * K
    assert max_seq <= 5120
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    assert dec.exec_mode == mtg.EXEC_STEP_KERNEL
    rows, text, stream = build_prompt(model, dec.embed, cfg)
    _log("row-weight stream: device prefill of %d rows" % n_prompt)
    hid = dec.prefill(rows)
    first = int(np.argmax(dec.logits(hid[-1:])[0]))
    k, v = dec.kv_read(n_prompt)
    orc = oracle_py.Oracle(model, max_seq, cfg["kv"])
    orc.kv_write(k, v)
    dev = mtg.Decoder(model, max_seq, cfg["kv"])
    dev.kv_write(k, v)
    del k, v
    fn, user, _keep = mtg.stream_drafter(text, stream)
    drafter = mtg.stream_drafter(text, stream)
    _log("row-weight stream: %d greedy steps, host loop, device loop and oracle" % steps)
    runs0 = dec.step_kernel_runs
    ids1, st1 = dec.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    ids2, st2 = dev.generate_device(first, 1 << 20, max_steps=steps, max_draft=K - 1, stream=drafter)
    ids0, st0 = orc.generate_from(first, 1 << 20, max_steps=steps, max_draft=K - 1, draft=fn, user=user)
    assert ids1.tolist() == ids0.tolist()
    assert ids2.tolist() == ids0.tolist()
    for f in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds"):
        assert getattr(st1, f) == getattr(st0, f), f
        assert getattr(st2, f) == getattr(st0, f), f
    assert st1.target_calls == steps
    assert dec.step_kernel_runs - runs0 == steps and dev.step_kernel_runs == steps
    assert dec.step_fallbacks == 0 and dev.step_fallbacks == 0
    assert dec.past_len == dev.past_len == orc.past_len
    k0, v0 = orc.kv_read(orc.past_len)
    for d, what in ((dec, "host loop"), (dev, "device loop")):
        k1, v1 = d.kv_read(d.past_len)
        _same(k1[:, :, n_prompt:], k0[:, :, n_prompt:], "K rows appended by the steps (%s)" % what)
        _same(v1[:, :, n_prompt:], v0[:, :, n_prompt:], "V rows appended by the steps (%s)" % what)
    _log("row-weight stream: %d ids, %d accepted drafts" % (len(ids1), st1.accepted))
    for x in (dec, dev, orc, model):
        x.close()
