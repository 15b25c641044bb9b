"""Speculative policy on the CPU: n-gram draft, greedy choice and the controller's
accept / rewind accounting, for both the library's host code (libmtg) and the
oracle, against the known answers of the reference's own tests
(tests/golden/policy_vectors.json) and against properties that define them."""
import json
import os

import numpy as np
import pytest

import mtg
import oracle_py

HERE = os.path.dirname(os.path.abspath(__file__))
VECTORS = json.load(open(os.path.join(HERE, "golden", "policy_vectors.json")))

DRAFTERS = {"libmtg": mtg.ngram_draft, "oracle": oracle_py.ngram_draft}
CHOOSERS = {"libmtg": mtg.greedy_choice, "oracle": oracle_py.greedy_choice}


def _history(case):
    if "history" in case:
        return case["history"]
    h = [2] * 101
    h[0] = 0
    if "entries 0 and 1" in case["history_rule"]:
        h[1] = 0
    return h


@pytest.mark.parametrize("impl", sorted(DRAFTERS))
@pytest.mark.parametrize("case", VECTORS["ngram_draft"], ids=lambda c: c["ref"])
def test_ngram_draft_known_answers(impl, case):
    assert DRAFTERS[impl](case["history"], case["maximum"]) == case["expected"]


@pytest.mark.parametrize("impl", sorted(CHOOSERS))
@pytest.mark.parametrize("case", VECTORS["greedy_choice"], ids=lambda c: c["ref"])
def test_greedy_choice_known_answers(impl, case):
    raw = np.array(case["raw"], np.float32)
    assert CHOOSERS[impl](raw, _history(case), case["penalty"]) == case["expected"]


def _draft_properties(h, maximum, got):
    """The proposal follows the latest earlier occurrence of the longest suffix
    (2..16 tokens) that has one, truncated to `maximum`."""
    size = len(h)
    if maximum <= 0 or size < 3:
        return got == []
    for n in range(min(16, size - 1), 1, -1):
        starts = [s for s in range(size - n) if h[s:s + n] == h[size - n:]]
        if starts:
            s = max(starts)
            return got == h[s + n:s + n + maximum]
    return got == []


@pytest.mark.parametrize("impl", sorted(DRAFTERS))
def test_ngram_draft_properties_on_random_histories(impl):
    rng = np.random.default_rng(11)
    for trial in range(400):
        size = int(rng.integers(0, 40))
        alphabet = int(rng.integers(2, 6))
        h = [int(x) for x in rng.integers(0, alphabet, size)]
        maximum = int(rng.integers(0, 9))
        got = DRAFTERS[impl](h, maximum)
        assert _draft_properties(h, maximum, got), (h, maximum, got)


@pytest.mark.parametrize("impl", sorted(CHOOSERS))
def test_greedy_choice_first_max_and_penalty(impl):
    rng = np.random.default_rng(12)
    for trial in range(200):
        n = int(rng.integers(1, 300))
        raw = rng.integers(-4, 5, n).astype(np.float32) * np.float32(0.5)  # many ties
        assert CHOOSERS[impl](raw, [], 1.0) == int(np.argmax(raw))  # numpy argmax = first max
        hist = [int(x) for x in rng.integers(-3, n + 3, int(rng.integers(0, 160)))]
        pen = float(rng.choice([1.1, 1.3, 1.5]))
        adj = raw.copy()
        for i in set(hist[-100:]):
            if 0 <= i < n:
                adj[i] = adj[i] / np.float32(pen) if adj[i] > 0 else adj[i] * np.float32(pen)
        assert CHOOSERS[impl](raw, hist, pen) == int(np.argmax(adj))


def _scripted(gold):
    """Target whose greedy output after the committed prefix p is gold[len(p)]."""
    def verify(tokens, hist, penalty, past):
        base = len(hist)
        ch = [gold[min(base + i + 1, len(gold) - 1)] for i in range(len(tokens))]
        m = 0
        while m + 1 < len(tokens) and tokens[m + 1] == ch[m]:
            m += 1
        return ch, m
    return verify


def _run(impl, gold, eos, max_draft, max_new=1000, prefix=0, draft=None):
    if impl == "libmtg":
        return mtg.speculative_run(_scripted(gold), gold[0], max_new, eos=eos, max_draft=max_draft,
                                   past=prefix, draft=draft)
    return oracle_py.run_controller(_scripted(gold), gold[0], max_new, eos, max_draft=max_draft,
                                    past=prefix, draft=draft)


@pytest.mark.parametrize("impl", ["libmtg", "oracle"])
@pytest.mark.parametrize("case", VECTORS["controller"], ids=lambda c: c["ref"])
def test_controller_counters_known_answers(impl, case):
    ids, st, past = _run(impl, case["gold"], case["eos"], case["max_draft"])
    st = st.as_dict()
    assert ids == case["gold"]
    for k, v in case.get("expected", {}).items():
        assert st[k] == v, (k, st)
    if "expected_input_tokens_above" in case:
        assert st["target_input_tokens"] > case["expected_input_tokens_above"]
    if "expected_calls_below" in case:
        assert st["target_calls"] < case["expected_calls_below"]
    if "expected_accepted_above" in case:
        assert st["accepted"] > case["expected_accepted_above"]
    assert st["stop_reason"] == 1
    # the terminating token is emitted but never evaluated
    # (cpu-lab/moss_speculative_gate.cpp:218: past_len == prefix + |ids| - stop)
    assert past == len(ids) - 1


def _audit_counts(tokens, eos, maximum):
    """Counters of an ideal controller replaying a complete greedy sequence, in
    the accounting of cpu-lab/moss_speculative_audit.py:17-53 (rewind after a
    rejected or terminal draft)."""
    cursor = calls = drafted = proposed = accepted = work = rewinds = 0
    while tokens[cursor] != eos:
        prop = oracle_py.ngram_draft(tokens[:cursor + 1], maximum)
        matched, terminal = 0, False
        for cand, tgt in zip(prop, tokens[cursor + 1:]):
            if cand != tgt:
                break
            matched += 1
            if tgt == eos:
                terminal = True
                break
        calls += 1
        drafted += bool(prop)
        proposed += len(prop)
        accepted += matched
        work += 1 + len(prop)
        rewinds += matched != len(prop) or terminal
        cursor += 1 + matched
        if terminal:
            break
    return dict(target_calls=calls, drafted_calls=drafted, proposed=proposed, accepted=accepted,
                target_input_tokens=work, rewinds=rewinds)


@pytest.mark.parametrize("impl", ["libmtg", "oracle"])
def test_controller_matches_audit_accounting_on_random_traces(impl):
    rng = np.random.default_rng(13)
    for trial in range(60):
        period = int(rng.integers(2, 9))
        motif = [int(x) for x in rng.integers(0, 6, period)]
        n = int(rng.integers(3, 60))
        gold = [motif[i % period] if rng.random() < 0.85 else int(rng.integers(0, 6)) for i in range(n)]
        gold.append(99)
        maximum = int(rng.integers(1, 9))
        ids, st, past = _run(impl, gold, 99, maximum)
        assert ids == gold
        want = _audit_counts(gold, 99, maximum)
        got = {k: v for k, v in st.as_dict().items() if k in want}
        assert got == want, (gold, maximum)
        assert past == len(gold) - 1


@pytest.mark.parametrize("impl", ["libmtg", "oracle"])
@pytest.mark.parametrize("limit", [1, 2, 5])
def test_controller_token_limits(impl, limit):
    """Token limits 1/2/5 (cpu-lab/moss_speculative_gate.cpp:176-179): exactly
    `limit` ids, the limit stops the loop, the last emitted id is not kept."""
    gold = [1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 9]
    ids, st, past = _run(impl, gold, 9, 4, max_new=limit, prefix=10)
    assert ids == gold[:limit]
    assert st.stop_reason == 2
    assert past == 10 + limit - 1


def test_controller_rejects_out_of_vocab_drafts():
    with pytest.raises(mtg.MtgError):
        mtg.speculative_run(_scripted([1, 2, 3, 9]), 1, 10, eos=9, max_draft=4, vocab=10,
                            draft=lambda ids, budget: [3, 12])


def test_controller_budget_respects_capacity():
    """budget = min(max_draft, max_new - emitted, remaining - 1)
    (src/cpu_speculative.cpp:104): a target with 3 free positions gets at most 2 drafts."""
    seen = []

    def verify(tokens, hist, penalty, past):
        seen.append(len(tokens))
        return [0] * len(tokens), 0
    mtg.speculative_run(verify, 5, 1, max_draft=8, past=7, max_seq=10,
                        draft=lambda ids, b: [1] * b)
    assert seen == []  # max_new 1: the seed is the only token, no call
    mtg.speculative_run(verify, 5, 6, max_draft=8, past=7, max_seq=10, max_steps=1,
                        draft=lambda ids, b: [1] * b)
    assert seen == [3]


def test_stream_drafter_aligns_to_absolute_position():
    """mtg_stream_draft: the n-gram proposal over prompt ++ ids, completed from the
    periodic stream at the absolute index of each proposed token."""
    prompt = [7, 8, 9]
    stream = list(range(100, 137))
    fn, user, keep = mtg.stream_drafter(prompt, stream)
    ids = mtg.i32([3, 4, 5])
    out = np.zeros(6, np.int32)
    n = mtg.lib().mtg_stream_draft(user, ids.ctypes.data_as(mtg.POINTER(mtg.c_int32)), 3, 6,
                                   out.ctypes.data_as(mtg.POINTER(mtg.c_int32)))
    assert n == 6
    assert out.tolist() == [stream[(6 + i) % 37] for i in range(6)]  # no n-gram match
    ids = mtg.i32([1, 2, 3, 1, 2])
    n = mtg.lib().mtg_stream_draft(user, ids.ctypes.data_as(mtg.POINTER(mtg.c_int32)), 5, 4,
                                   out.ctypes.data_as(mtg.POINTER(mtg.c_int32)))
    assert n == 4
    # n-gram part [3, 1, 2] (latest earlier occurrence of the suffix 1,2), then stream
    assert out[:4].tolist() == [3, 1, 2, stream[(8 + 3) % 37]]


@pytest.mark.parametrize("impl", ["libmtg", "oracle"])
def test_controller_stops_when_the_cache_is_full(impl):
    """A full KV cache ends the loop the way the reference's failed append does
    (src/cpu_speculative.cpp:113-114): the seed is emitted, no verify call is made,
    the status is OK and stop_reason says why (3)."""
    gold = [1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 1, 2, 9]
    calls = []

    def verify(tokens, hist, penalty, past):
        calls.append((len(tokens), past))
        return _scripted(gold)(tokens, hist, penalty, past)
    kw = dict(max_draft=4, past=6, max_seq=10)
    if impl == "libmtg":
        ids, st, past = mtg.speculative_run(verify, gold[0], 100, eos=9, **kw)
    else:
        ids, st, past = oracle_py.run_controller(verify, gold[0], 100, 9, **kw)
    # every call fits: past + T <= max_seq, and the last one leaves no free position
    assert all(p + t <= 10 for t, p in calls)
    assert past == 10
    assert st.stop_reason == 3
    # the seed of the step that found no room is emitted (and not kept)
    assert ids == gold[:len(ids)] and len(ids) == 10 - 6 + 1
    # a full cache from the start: only the seed, no verify call
    calls.clear()
    kw["past"] = 10
    if impl == "libmtg":
        ids, st, past = mtg.speculative_run(verify, gold[0], 100, eos=9, **kw)
    else:
        ids, st, past = oracle_py.run_controller(verify, gold[0], 100, 9, **kw)
    assert ids == [gold[0]] and calls == [] and st.stop_reason == 3 and past == 10
