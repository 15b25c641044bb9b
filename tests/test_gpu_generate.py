"""Whole generation on the device (mtg_generate_device: the controller of
cpu_speculative_generate, src/cpu_speculative.cpp:68-147, with the n-gram
drafter of :27-38, as a kernel between the verify steps) against the host
controller on a second decoder from the same KV state (mtg_generate_from,
draft == NULL) and the oracle's controller: the same ids, counters, stop reason,
next seed and KV position, for every stop rule."""
import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

COUNTERS = ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds",
            "stop_reason", "next_seed")


def _setup(prefix, max_seq, kv_type=mtg.TYPE_F32, seed=3, vocab=4096, wtype=mtg.TYPE_Q8_0):
    model = mtg.SynthModel(wtype, seed=seed, std=0.02, gain_jitter=0.05, n_layers=2, vocab=vocab)
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, vocab, prefix)
    orc.prefill(orc.embed(ids))
    k, v = orc.kv_read(prefix)
    a = mtg.Decoder(model, max_seq, kv_type)
    b = mtg.Decoder(model, max_seq, kv_type)
    a.kv_write(k, v)
    b.kv_write(k, v)
    return model, orc, a, b, rng


def _prior(rng, vocab):
    # committed ids with repeats, so that the n-gram drafter finds matches
    motif = rng.integers(0, vocab, 6)
    return np.concatenate([rng.integers(0, vocab, 10), motif, rng.integers(0, vocab, 5), motif, motif[:3]])


def _same_run(a_run, b_run, what):
    (ia, sa), (ib, sb) = a_run, b_run
    assert ia.tolist() == ib.tolist(), "%s: ids differ" % what
    for k in COUNTERS:
        assert getattr(sa, k) == getattr(sb, k), "%s: %s %s != %s" % (what, k, getattr(sa, k), getattr(sb, k))


@pytest.mark.parametrize("penalty,max_draft,kv_type", [(1.0, 4, mtg.TYPE_F32), (1.25, 7, mtg.TYPE_F32),
                                                       (1.0, 7, mtg.TYPE_F16)], ids=["p1-d4", "p1.25-d7", "f16kv-d7"])
def test_device_loop_equals_host_loop_and_oracle(penalty, max_draft, kv_type):
    print("device loop: penalty %.2f max_draft %d kv %d" % (penalty, max_draft, kv_type), flush=True)
    model, orc, a, b, rng = _setup(40, 600, kv_type)
    prior = _prior(rng, model.hp.vocab)
    first = int(prior[-1])
    kw = dict(max_steps=0, eos=-1, penalty=penalty, max_draft=max_draft, prior=prior)
    dev = a.generate_device(first, 300, **kw)
    host = b.generate_from(first, 300, **kw)
    ref = orc.generate_from(first, 300, **kw)
    print("  %d ids in %d steps, %d drafted steps, %d proposed, %d accepted" % (
        len(dev[0]), dev[1].target_calls, dev[1].drafted_calls, dev[1].proposed, dev[1].accepted), flush=True)
    _same_run(dev, host, "device vs host")
    _same_run(dev, ref, "device vs oracle")
    assert dev[1].drafted_calls > 0
    assert a.past_len == b.past_len == orc.past_len
    # the loop continues from where it stopped, on both paths
    nxt = int(dev[1].next_seed)
    prior2 = np.concatenate([prior, dev[0]])
    dev2 = a.generate_device(nxt, 40, max_draft=max_draft, penalty=penalty, prior=prior2)
    host2 = b.generate_from(nxt, 40, max_draft=max_draft, penalty=penalty, prior=prior2)
    _same_run(dev2, host2, "second run")
    assert a.past_len == b.past_len


@pytest.mark.parametrize("penalty,max_draft,kv_type", [(1.0, 15, mtg.TYPE_F32), (1.25, 15, mtg.TYPE_F16),
                                                       (1.0, 11, mtg.TYPE_F16)], ids=["p1-d15", "p1.25-d15-f16kv",
                                                                                      "p1-d11-f16kv"])
def test_device_loop_16_rows_equals_host_loop_and_oracle(penalty, max_draft, kv_type):
    """More than 7 drafts per step: every step of the device loop runs the 16-row
    step kernel, whatever its row count; ids, counters and KV position equal the
    host loop's and the oracle's."""
    print("device loop, 16 rows: penalty %.2f max_draft %d kv %d" % (penalty, max_draft, kv_type), flush=True)
    model, orc, a, b, rng = _setup(40, 800, kv_type)
    prior = _prior(rng, model.hp.vocab)
    first = int(prior[-1])
    kw = dict(max_steps=0, eos=-1, penalty=penalty, max_draft=max_draft, prior=prior)
    dev = a.generate_device(first, 300, **kw)
    host = b.generate_from(first, 300, **kw)
    ref = orc.generate_from(first, 300, **kw)
    _same_run(dev, host, "device vs host")
    _same_run(dev, ref, "device vs oracle")
    assert dev[1].drafted_calls > 0
    assert a.past_len == b.past_len == orc.past_len


@pytest.mark.parametrize("max_draft,period", [(7, 37), (15, 37), (15, 0), (5, 11)],
                         ids=["d7-p37", "d15-p37", "d15-ngram", "d5-p11"])
def test_device_stream_drafter_equals_host_hook_and_oracle(max_draft, period):
    """The draft hook of the reference loop (called every step,
    src/cpu_speculative.cpp:105) as the long-context workloads use it: the stream
    drafter (n-gram over prompt ++ ids, completed from a periodic stream) run by
    the device controller, against the host loop and the oracle's controller
    calling mtg_stream_draft as their hook."""
    print("device stream drafter: max_draft %d period %d" % (max_draft, period), flush=True)
    model, orc, a, b, rng = _setup(50, 900)
    vocab = model.hp.vocab
    prompt = rng.integers(0, vocab, 30).astype(np.int32)
    stream = rng.integers(0, vocab, max(period, 1)).astype(np.int32)[:period]
    drafter = mtg.stream_drafter(prompt, stream)
    fn, user, _keep = drafter
    first = int(rng.integers(0, vocab))
    for penalty in (1.0, 1.2):
        a.rewind(50)
        b.rewind(50)
        orc.rewind(50)
        kw = dict(max_steps=24, eos=-1, penalty=penalty, max_draft=max_draft)
        dev = a.generate_device(first, 400, stream=drafter, **kw)
        host = b.generate_from(first, 400, draft=fn, user=user, **kw)
        ref = orc.generate_from(first, 400, draft=fn, user=user, **kw)
        _same_run(dev, host, "device vs host, penalty %.1f" % penalty)
        _same_run(dev, ref, "device vs oracle, penalty %.1f" % penalty)
        assert a.past_len == b.past_len == orc.past_len
        if period:
            assert dev[1].proposed == dev[1].target_calls * max_draft


def test_device_loop_stop_rules():
    """eos (stop 1), the token limit (2), a full KV cache (3) and a step limit (0)."""
    print("device loop: stop rules", flush=True)
    model, orc, a, b, rng = _setup(30, 400)
    prior = _prior(rng, model.hp.vocab)
    first = int(prior[-1])
    k, v = a.kv_read(30)

    def both(max_new, **kw):
        a.rewind(30)
        b.rewind(30)
        a.kv_write(k, v)
        b.kv_write(k, v)
        dev = a.generate_device(first, max_new, prior=prior, max_draft=7, **kw)
        host = b.generate_from(first, max_new, prior=prior, max_draft=7, **kw)
        _same_run(dev, host, str(kw))
        assert a.past_len == b.past_len
        return dev

    ids, st = both(60)
    assert st.stop_reason == 2 and len(ids) == 60
    eos = int(ids[17])
    ids_e, st_e = both(60, eos=eos)
    assert st_e.stop_reason == 1 and ids_e[-1] == eos and eos not in ids_e[:-1].tolist()
    ids_s, st_s = both(60, max_steps=3)
    assert st_s.stop_reason == 0 and st_s.target_calls == 3
    ids_1, st_1 = both(1)
    assert st_1.stop_reason == 2 and ids_1.tolist() == [first] and st_1.target_calls == 0
    # a cache with 12 free rows
    small_o = oracle_py.Oracle(model, 42, mtg.TYPE_F32)
    small_a = mtg.Decoder(model, 42, mtg.TYPE_F32)
    small_b = mtg.Decoder(model, 42, mtg.TYPE_F32)
    for d in (small_a, small_b):
        d.kv_write(k, v)
    small_o.kv_write(k, v)
    dev = small_a.generate_device(first, 200, prior=prior, max_draft=7)
    host = small_b.generate_from(first, 200, prior=prior, max_draft=7)
    ref = small_o.generate_from(first, 200, prior=prior, max_draft=7)
    _same_run(dev, host, "full cache")
    _same_run(dev, ref, "full cache vs oracle")
    assert dev[1].stop_reason == 3 and small_a.past_len == small_b.past_len == 42


def test_device_loop_finishes_on_the_host_after_an_abandoned_step():
    """A step whose bounded wait runs out (a 1-poll limit set from the host) ends
    the device loop with that step undone; the host controller finishes from the
    same state (its steps on the per-op fallback), with the same result."""
    print("device loop: abandoned step", flush=True)
    model, orc, a, b, rng = _setup(30, 400)
    prior = _prior(rng, model.hp.vocab)
    first = int(prior[-1])
    before = a.step_fallbacks
    a.debug_wait_limit(1)
    try:
        dev = a.generate_device(first, 40, prior=prior, max_draft=7)
    finally:
        a.debug_wait_limit(0)
    host = b.generate_from(first, 40, prior=prior, max_draft=7)
    _same_run(dev, host, "after the abandoned step")
    assert a.step_fallbacks > before
    assert a.past_len == b.past_len


@pytest.mark.parametrize("wtype,kv_type", [(mtg.TYPE_F16, mtg.TYPE_F32), (mtg.TYPE_F16, mtg.TYPE_F16),
                                           (mtg.TYPE_F32, mtg.TYPE_F32), (mtg.TYPE_F32, mtg.TYPE_F16)],
                         ids=["f16-f32kv", "f16-f16kv", "f32-f32kv", "f32-f16kv"])
def test_device_loop_f16_weights_equals_host_loop_and_oracle(wtype, kv_type):
    """f16 and f32 weights on the step kernel's row variants (8-row steps): the device
    loop, the host loop and the oracle's controller agree with the penalty on; a
    device loop with more than 7 drafts (16-row steps) is refused."""
    print("device loop, weights %d: kv %d" % (wtype, kv_type), flush=True)
    model, orc, a, b, rng = _setup(40, 600, kv_type, wtype=wtype)
    assert a.exec_mode == mtg.EXEC_STEP_KERNEL
    prior = _prior(rng, model.hp.vocab)
    first = int(prior[-1])
    kw = dict(max_steps=0, eos=-1, penalty=1.25, max_draft=7, prior=prior)
    dev = a.generate_device(first, 200, **kw)
    host = b.generate_from(first, 200, **kw)
    ref = orc.generate_from(first, 200, **kw)
    _same_run(dev, host, "device vs host")
    _same_run(dev, ref, "device vs oracle")
    assert dev[1].drafted_calls > 0
    assert a.past_len == b.past_len == orc.past_len
    assert a.step_fallbacks == 0 and b.step_fallbacks == 0
    assert a.step_kernel_runs == dev[1].target_calls and b.step_kernel_runs == host[1].target_calls
    with pytest.raises(mtg.MtgError) as e:
        a.generate_device(int(dev[1].next_seed), 10, max_draft=8)
    assert e.value.code == mtg.ERR_UNSUPPORTED


def test_device_loop_unsupported_cases():
    model, orc, a, b, rng = _setup(10, 100)
    a.set_exec(mtg.EXEC_GRAPH)
    with pytest.raises(mtg.MtgError) as e:
        a.generate_device(5, 10)
    assert e.value.code == mtg.ERR_UNSUPPORTED


def test_full_size_device_loop_k8_ctx1600():
    """The K=8 workload at full size (28 layers, 151,936-row vocabulary, q8_0, f32
    KV, the 1,600-row prompt): 64 steps of the device loop against the host loop,
    the same ids and counters; both are timed."""
    import time
    from workloads import WORKLOADS, build_prompt, prompt_rows
    cfg = WORKLOADS[2]
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n = prompt_rows(cfg)
    a = mtg.Decoder(model, n + 600, cfg["kv"])
    b = mtg.Decoder(model, n + 600, cfg["kv"])
    rows, text, _ = build_prompt(model, a.embed, cfg)
    hid = a.prefill(rows)
    b.prefill(rows)
    first = int(np.argmax(a.logits(hid[-1:])[0]))
    times = {}
    runs = {}
    for name, d, fn in (("device", a, a.generate_device), ("host", b, b.generate_from)):
        t0 = time.perf_counter()
        runs[name] = fn(first, 400, max_steps=64, max_draft=cfg["K"] - 1, prior=text)
        times[name] = (time.perf_counter() - t0) / max(1, runs[name][1].target_calls)
    _same_run(runs["device"], runs["host"], "full size")
    st = runs["device"][1]
    assert a.past_len == b.past_len
    # the same with the workload's own drafter (the stream drafter) on both loops
    _, text2, stream = build_prompt(model, a.embed, cfg)
    drafter = mtg.stream_drafter(text2, stream)
    fn, user, _keep = drafter
    for d in (a, b):
        d.rewind(n)
    runs["device_stream"] = a.generate_device(first, 1 << 12, max_steps=64, max_draft=cfg["K"] - 1, stream=drafter)
    runs["host_stream"] = b.generate_from(first, 1 << 12, max_steps=64, max_draft=cfg["K"] - 1, draft=fn, user=user)
    _same_run(runs["device_stream"], runs["host_stream"], "full size, stream drafter")
    print("full-size K=8 loop: %d steps, %d ids, %d accepted; %.1f us/step on the device loop, %.1f on the host loop"
          % (st.target_calls, len(runs["device"][0]), st.accepted, 1e6 * times["device"], 1e6 * times["host"]),
          flush=True)
    assert a.past_len == b.past_len


def test_full_size_device_loop_k16_f16kv_ctx4000():
    """The K=16 f16-KV workload at full size on the device loop with its stream
    drafter (the 16-row step kernel): 16 steps against the host loop and the
    oracle from the same prefilled KV state."""
    import os
    from workloads import WORKLOADS, build_prompt, prompt_rows
    cfg = WORKLOADS[3]
    oracle_py.lib().orc_set_threads(max(1, min(16, len(os.sched_getaffinity(0)))))
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n = prompt_rows(cfg)
    max_seq = n + 20 * cfg["K"]
    a = mtg.Decoder(model, max_seq, cfg["kv"])
    b = mtg.Decoder(model, max_seq, cfg["kv"])
    rows, text, stream = build_prompt(model, a.embed, cfg)
    hid = a.prefill(rows)
    first = int(np.argmax(a.logits(hid[-1:])[0]))
    k, v = a.kv_read(n)
    b.kv_write(k, v)
    orc = oracle_py.Oracle(model, max_seq, cfg["kv"])
    orc.kv_write(k, v)
    del k, v
    drafter = mtg.stream_drafter(text, stream)
    fn, user, _keep = drafter
    kw = dict(max_steps=16, max_draft=cfg["K"] - 1)
    dev = a.generate_device(first, 1 << 12, stream=drafter, **kw)
    host = b.generate_from(first, 1 << 12, draft=fn, user=user, **kw)
    ref = orc.generate_from(first, 1 << 12, draft=fn, user=user, **kw)
    _same_run(dev, host, "K=16 device vs host")
    _same_run(dev, ref, "K=16 device vs oracle")
    assert dev[1].target_calls == 16 and a.past_len == b.past_len == orc.past_len
    print("full-size K=16 device loop: %d ids, %d accepted drafts" % (len(dev[0]), dev[1].accepted), flush=True)
