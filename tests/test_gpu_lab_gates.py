"""The reference's two CPU parity gates, restated on the GPU against the oracle.

* Speculative gate (cpu-lab/moss_speculative_gate.cpp:163-229): prefixes 31, 128,
  513 and 1,024 of seeded token ids x repetition penalties 1.0, 1.1 and 1.5 x ten
  scenarios: a first draft of four gold tokens with the token at position 0..3
  changed (a rejection there) or none changed (all accepted), token limits 1, 2
  and 5, eos on the first token, and eos on a token inside the first accepted
  batch. The gold stream is the plain greedy decode (no drafts). After every
  commit the decoder's whole discarded capacity is NaN-poisoned before the next
  step; every step's hidden rows, logits and appended KV equal the oracle's bit
  for bit, and the committed ids equal the gold prefix and the oracle
  controller's ids and counters.
* Target-batch gate (cpu-lab/moss_target_batch_gate.cpp:183-286): two prefix
  kinds (seeded random rows, and embeddings of seeded ids) x prefixes 31, 32, 33,
  127, 128, 129, 511, 512, 513, 1,023, 1,024, 1,025 x batches of 1, 2, 4 and 8
  appended rows: the batch append equals row-by-row appends and the oracle bit for
  bit (hidden rows, logits of every row, greedy choices, KV); rewinding to
  prefix + count / 2, poisoning the discarded suffix with NaN and appending a
  changed token gives the same hidden row, logits and KV as the row-by-row
  decoder; invalid rewinds fail and leave the position unchanged.

The model is the 2-layer Qwen3-0.6B-width synthetic decoder (vocabulary 4,096),
max_seq 1,088 as in the gates.
"""
import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

MAX_SEQ = 1088
VOCAB = 4096


def _same(got, ref, what):
    got, ref = np.asarray(got), np.asarray(ref)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g"
                         % (what, int((got != ref).sum()), np.nanmax(err)))


def _lcg_ids(n, vocab):
    seed, out = 0x12345678, []
    for _ in range(n):
        seed = (seed * 1664525 + 1013904223) & 0xffffffff
        out.append(seed % vocab)
    return np.array(out, np.int32)


def _lcg_rows(n, hidden):
    seed, out = 0x12345678, np.empty(n * hidden, np.float32)
    for i in range(n * hidden):
        seed = (seed * 1664525 + 1013904223) & 0xffffffff
        out[i] = np.float32((int(seed >> 8) - 8388608) * (0.2 / 8388608.0))
    return out.reshape(n, hidden)


def _poison_beyond(dec, past):
    """NaN in every cache position from past on (all layers, heads, both sides)."""
    k, v = dec.kv_read(past)
    shape = (k.shape[0], k.shape[1], MAX_SEQ, k.shape[3])
    kf = np.full(shape, np.nan, k.dtype)
    vf = np.full(shape, np.nan, v.dtype)
    kf[:, :, :past] = k
    vf[:, :, :past] = v
    dec.kv_write(kf, vf)
    dec.rewind(past)


@pytest.fixture(scope="module")
def model():
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=5, std=0.02, gain_jitter=0.05, n_layers=2, vocab=VOCAB)
    yield m
    m.close()


@pytest.mark.parametrize("penalty", [1.0, 1.1, 1.5])
@pytest.mark.parametrize("prefix", [31, 128, 513, 1024])
def test_speculative_gate(model, prefix, penalty):
    print("speculative gate: prefix %d penalty %.1f" % (prefix, penalty), flush=True)
    hp = model.hp
    gold_orc = oracle_py.Oracle(model, MAX_SEQ, mtg.TYPE_F32)
    rows = gold_orc.embed(_lcg_ids(prefix, hp.vocab))
    hid = gold_orc.prefill(rows)
    first = int(np.argmax(gold_orc.logits(hid[-1:])[0]))
    gold, _ = gold_orc.generate_from(first, 10, penalty=penalty, max_draft=0)
    gold = [int(x) for x in gold]
    assert len(gold) == 10 and gold[0] == first
    gold_orc.close()
    distinct = next((i for i in range(1, 5) if gold[i] not in gold[:i]), -1)
    dec = mtg.Decoder(model, MAX_SEQ, mtg.TYPE_F32)
    orc = oracle_py.Oracle(model, MAX_SEQ, mtg.TYPE_F32)   # the step-by-step reference
    ctl = oracle_py.Oracle(model, MAX_SEQ, mtg.TYPE_F32)   # the oracle's own controller
    hd = dec.prefill(rows)
    _same(hd, orc.prefill(rows), "prefill hidden rows")
    ctl.prefill(rows)
    k_prefix, v_prefix = orc.kv_read(prefix)
    cases = 0
    for scenario in range(10):
        if scenario == 9 and distinct < 0:
            continue
        forced = scenario if scenario < 5 else 4
        limit = {5: 1, 6: 2, 7: 5}.get(scenario, 10)
        eos = gold[0] if scenario == 8 else gold[distinct] if scenario == 9 else -1
        for m in (dec, orc, ctl):
            m.rewind(prefix)
        state = {"first": True}

        def draft(ids, budget, state=state):
            if not state["first"]:
                return []
            state["first"] = False
            count = min(4, budget, len(gold) - len(ids))
            prop = gold[len(ids):len(ids) + count]
            if forced < count:
                prop[forced] = (prop[forced] + 1) % hp.vocab
            return prop

        steps = []

        def verify(tokens, history, pen, past):
            _poison_beyond(dec, past)
            orc.rewind(past)
            c1, m1, h1, l1 = dec.verify(tokens, history=history, penalty=pen, want_hidden=True, want_logits=True)
            c0, m0, h0, l0 = orc.verify(tokens, history=history, penalty=pen, want_hidden=True, want_logits=True)
            tag = "prefix %d penalty %.1f scenario %d step %d" % (prefix, pen, scenario, len(steps))
            assert np.isfinite(h1).all() and np.isfinite(l1).all(), tag + ": a poisoned position was read"
            _same(h1, h0, tag + " hidden")
            _same(l1, l0, tag + " logits")
            assert np.array_equal(c1, c0) and m1 == m0, tag
            k1, v1 = dec.kv_read(past + len(tokens))
            k0, v0 = orc.kv_read(past + len(tokens))
            _same(k1[:, :, past:], k0[:, :, past:], tag + " appended K")
            _same(v1[:, :, past:], v0[:, :, past:], tag + " appended V")
            steps.append(len(tokens))
            return c1, m1

        ids, st, past = mtg.speculative_run(verify, first, limit, eos=eos, penalty=penalty, max_draft=4,
                                            past=prefix, max_seq=MAX_SEQ, vocab=hp.vocab, draft=draft)
        expected = []
        for i in range(limit):
            expected.append(gold[i])
            if gold[i] == eos:
                break
        assert ids == expected, (scenario, ids, expected)
        state["first"] = True
        fn, keep = mtg._draft_pointer(draft)
        ids0, st0 = ctl.generate_from(first, limit, eos=eos, penalty=penalty, max_draft=4, draft=fn)
        del keep
        assert [int(x) for x in ids0] == ids, scenario
        for f in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens", "rewinds",
                  "stop_reason"):
            assert getattr(st, f) == getattr(st0, f), (scenario, f)
        assert past == ctl.past_len, scenario
        if scenario < 5 and steps:
            assert steps[0] == 5  # the seed and the four drafted tokens in one batch
        # the prefix stays as prefilled
        k1, v1 = dec.kv_read(prefix)
        _same(k1, k_prefix, "prefix K after scenario %d" % scenario)
        _same(v1, v_prefix, "prefix V after scenario %d" % scenario)
        cases += 1
    assert cases >= 9
    dec.close()
    orc.close()
    ctl.close()


PREFIXES = [31, 32, 33, 127, 128, 129, 511, 512, 513, 1023, 1024, 1025]


@pytest.mark.parametrize("prefix", PREFIXES)
@pytest.mark.parametrize("mode", [0, 1], ids=["random-rows", "token-rows"])
def test_target_batch_gate(model, mode, prefix):
    print("target-batch gate: mode %d prefix %d" % (mode, prefix), flush=True)
    hp = model.hp
    orc = oracle_py.Oracle(model, MAX_SEQ, mtg.TYPE_F32)
    rows = _lcg_rows(prefix, hp.hidden) if mode == 0 else orc.embed(_lcg_ids(prefix, hp.vocab))
    tail_ids = np.array([(i * 104729 + 41) % hp.vocab for i in range(8)], np.int32)
    tail = orc.embed(tail_ids)
    serial = mtg.Decoder(model, MAX_SEQ, mtg.TYPE_F32)
    batch = mtg.Decoder(model, MAX_SEQ, mtg.TYPE_F32)
    h0 = orc.prefill(rows)
    _same(serial.prefill(rows), h0, "serial prefill")
    _same(batch.prefill(rows), h0, "batch prefill")
    k_prefix, v_prefix = orc.kv_read(prefix)
    for count in (1, 2, 4, 8):
        tag = "mode %d prefix %d count %d" % (mode, prefix, count)
        for m in (serial, batch, orc):
            m.rewind(prefix)
        x = tail[:count]
        hs = np.concatenate([serial.append(x[i:i + 1]) for i in range(count)])
        hb = batch.append(x)
        ho = orc.run(x)
        _same(hb, hs, tag + ": batch vs row-by-row hidden")
        _same(hb, ho, tag + ": batch vs oracle hidden")
        ls, lb = serial.logits(hs), batch.logits(hb)
        _same(lb, ls, tag + ": logits of every row")
        _same(lb, orc.logits(ho), tag + ": logits vs oracle")
        assert np.array_equal(np.argmax(lb, axis=1), np.argmax(ls, axis=1))
        ks, vs = serial.kv_read(prefix + count)
        kb, vb = batch.kv_read(prefix + count)
        _same(kb, ks, tag + ": K")
        _same(vb, vs, tag + ": V")
        # invalid rewinds fail and leave the position where it was
        for bad in (-1, prefix + count + 1):
            with pytest.raises(mtg.MtgError):
                batch.rewind(bad)
            assert batch.past_len == prefix + count
        accepted = count // 2
        pos = prefix + accepted
        for m in (serial, batch, orc):
            m.rewind(pos)
        _poison_beyond(batch, pos)
        changed = orc.embed([(int(tail_ids[accepted]) + 1) % hp.vocab])
        assert not np.array_equal(changed[0], tail[accepted])
        a, b, o = serial.append(changed), batch.append(changed), orc.run(changed)
        assert np.isfinite(b).all(), tag + ": the changed decode read a poisoned position"
        _same(b, a, tag + ": changed decode hidden")
        _same(b, o, tag + ": changed decode vs oracle")
        _same(batch.logits(b), serial.logits(a), tag + ": changed decode logits")
        ks, vs = serial.kv_read(pos + 1)
        kb, vb = batch.kv_read(pos + 1)
        _same(kb, ks, tag + ": K after the changed decode")
        _same(vb, vs, tag + ": V after the changed decode")
        _same(kb[:, :, :prefix], k_prefix, tag + ": prefix K unchanged")
        _same(vb[:, :, :prefix], v_prefix, tag + ": prefix V unchanged")
    serial.close()
    batch.close()
    orc.close()
