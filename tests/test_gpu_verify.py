"""Verify-step parity on the GPU against the oracle (same weights, same KV state).

Every execution mode of the library (the Qwen3-0.6B dataflow step kernel,
per-op kernels from a graph, per-op kernels launched eagerly) must match the oracle within the contract (logits 1e-3 relative
/ 1e-4 absolute) and return identical greedy choices and acceptance; in fact they
match bit for bit (shared canonical order)."""
import numpy as np
import pytest

import mtg
import oracle_py

pytestmark = pytest.mark.gpu

EXECS = [mtg.EXEC_STEP_KERNEL, mtg.EXEC_GRAPH, mtg.EXEC_EAGER]
EXEC_NAMES = {mtg.EXEC_STEP_KERNEL: "step", mtg.EXEC_GRAPH: "graph", mtg.EXEC_EAGER: "eager"}


def _setup(n_layers, prefix, kv_type=mtg.TYPE_F32, vocab=4096, seed=0, max_seq=256, jitter=0.05,
           exec_mode=mtg.EXEC_STEP_KERNEL, wtype=mtg.TYPE_Q8_0):
    model = mtg.SynthModel(wtype, seed=seed, std=0.02, gain_jitter=jitter, n_layers=n_layers,
                           vocab=vocab)
    orc = oracle_py.Oracle(model, max_seq, kv_type)
    dec = mtg.Decoder(model, max_seq, kv_type)
    dec.set_exec(exec_mode)
    rng = np.random.default_rng(seed + 1)
    ids = rng.integers(0, vocab, prefix)
    orc.prefill(orc.embed(ids))
    k, v = orc.kv_read(prefix)
    dec.kv_write(k, v)
    return model, orc, dec, rng


def _close(got, ref, what):
    """Device and oracle use the same canonical float order, so results are
    bit-identical; the contract tolerance (1e-3 rel / 1e-4 abs) is reported
    in the message for context."""
    got = np.asarray(got)
    ref = np.asarray(ref)
    if np.array_equal(got.view(np.uint8), ref.view(np.uint8)):
        return
    g64, r64 = got.astype(np.float64), ref.astype(np.float64)
    err = np.abs(g64 - r64)
    within = bool((err <= 1e-4 + 1e-3 * np.abs(r64)).all())
    raise AssertionError("%s: not bit-identical: %d elements differ, max err %.3g at %s (within tolerance: %s)"
                         % (what, int((got != ref).sum()), err.max(),
                            np.unravel_index(err.argmax(), err.shape), within))


@pytest.mark.parametrize("exec_mode", EXECS, ids=lambda e: EXEC_NAMES[e])
@pytest.mark.parametrize("T", [1, 4, 8, 9, 16])
def test_verify_matches_oracle(exec_mode, T):
    print("verify parity: exec=%s 2 layers, prefix 40, T=%d" % (EXEC_NAMES[exec_mode], T), flush=True)
    model, orc, dec, rng = _setup(2, 40, exec_mode=exec_mode)
    tokens = rng.integers(0, model.hp.vocab, T)
    c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
    c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
    _close(h1, h0, "hidden")
    _close(l1, l0, "logits")
    assert np.array_equal(c1, c0)
    assert m1 == m0
    assert dec.past_len == orc.past_len == 40 + T
    k0, v0 = orc.kv_read(40 + T)
    k1, v1 = dec.kv_read(40 + T)
    _close(k1, k0, "K cache")
    _close(v1, v0, "V cache")


@pytest.mark.parametrize("exec_mode", EXECS, ids=lambda e: EXEC_NAMES[e])
def test_f16_kv_verify_matches_oracle(exec_mode):
    print("f16 KV parity: exec=%s" % EXEC_NAMES[exec_mode], flush=True)
    model, orc, dec, rng = _setup(2, 70, kv_type=mtg.TYPE_F16, exec_mode=exec_mode)
    for T in (8, 16):
        tokens = rng.integers(0, model.hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(l1, l0, "logits")
        assert np.array_equal(c1, c0) and m1 == m0


@pytest.mark.parametrize("exec_mode", EXECS, ids=lambda e: EXEC_NAMES[e])
def test_penalty_and_acceptance_match_oracle(exec_mode):
    """Drafts built from the oracle's own choices are accepted up to a planted
    mismatch; the repetition penalty (last 100 ids of history ++ row tokens)
    changes choices the same way on both sides."""
    model, orc, dec, rng = _setup(2, 33, exec_mode=exec_mode)
    hist = rng.integers(0, model.hp.vocab, 150).tolist()
    # oracle choices for a probe batch give drafts that should be accepted
    tokens = [int(rng.integers(0, model.hp.vocab))]
    for penalty in (1.0, 1.3):
        past = orc.past_len
        for i in range(7):
            probe = tokens + [0]
            c, _, _, _ = orc.verify(probe, history=hist, penalty=penalty)
            orc.rewind(past)
            tokens = tokens + [int(c[len(tokens) - 1])]
        bad = list(tokens)
        bad[5] = (bad[5] + 1) % model.hp.vocab
        for batch, want in ((tokens, 7), (bad, 4)):
            c0, m0, _, l0 = orc.verify(batch, history=hist, penalty=penalty, want_logits=True)
            c1, m1, _, l1 = dec.verify(batch, history=hist, penalty=penalty, want_logits=True)
            _close(l1, l0, "logits")
            assert np.array_equal(c1, c0)
            assert m1 == m0 == want
            orc.rewind(past)
            dec.rewind(past)
        tokens = tokens[:1]


def test_gpu_prefill_matches_oracle():
    """mtg_prefill (chunks of 16 rows through the step kernel) against the oracle's
    single-batch prefill: hidden rows and the whole KV cache."""
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=3, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    orc = oracle_py.Oracle(model, 128)
    dec = mtg.Decoder(model, 128)
    rng = np.random.default_rng(4)
    rows = orc.embed(rng.integers(0, 4096, 37))
    h0 = orc.prefill(rows)
    h1 = dec.prefill(rows)
    _close(h1, h0, "prefill hidden")
    k0, v0 = orc.kv_read(37)
    k1, v1 = dec.kv_read(37)
    _close(k1, k0, "K cache")
    _close(v1, v0, "V cache")


def test_step_kernel_matches_per_op_kernels():
    """The persistent step kernel and the per-op kernels agree on a 4-layer model
    over several chained steps with rewinds in between."""
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=5, std=0.02, gain_jitter=0.05, n_layers=4, vocab=8192)
    a = mtg.Decoder(model, 512)
    b = mtg.Decoder(model, 512)
    a.set_exec(mtg.EXEC_STEP_KERNEL)
    b.set_exec(mtg.EXEC_GRAPH)
    rng = np.random.default_rng(6)
    rows = a.embed(rng.integers(0, 8192, 100))
    a.prefill(rows, want_hidden=False)
    b.prefill(rows, want_hidden=False)
    for step in range(6):
        T = int(rng.integers(1, 17))
        tokens = rng.integers(0, 8192, T)
        ca, ma, _, la = a.verify(tokens, want_logits=True)
        cb, mb, _, lb = b.verify(tokens, want_logits=True)
        _close(la, lb, "logits step %d" % step)
        assert np.array_equal(ca, cb) and ma == mb
        keep = int(rng.integers(1, T + 1))
        a.rewind(a.past_len - T + keep)
        b.rewind(b.past_len - T + keep)


@pytest.mark.parametrize("penalty", [1.0, 1.25])
def test_generated_token_stream_matches_oracle(penalty):
    """The controller on the device decoder and on the oracle, fed the same
    drafter (n-gram over prompt ++ ids, completed from a periodic stream), emit
    the same ids with the same counters, step for step."""
    print("token stream parity: penalty %.2f" % penalty, flush=True)
    model, orc, dec, rng = _setup(2, 48, vocab=4096, max_seq=512, seed=7)
    prompt = rng.integers(0, 4096, 20).astype(np.int32)
    stream = rng.integers(0, 4096, 37).astype(np.int32)
    fn, user, _keep = mtg.stream_drafter(prompt, stream)
    first = int(rng.integers(0, 4096))
    ids0, st0 = orc.generate_from(first, 200, max_steps=24, penalty=penalty, max_draft=7, draft=fn,
                                  user=user)
    ids1, st1 = dec.generate_from(first, 200, max_steps=24, penalty=penalty, max_draft=7, draft=fn,
                                  user=user)
    assert ids1.tolist() == ids0.tolist()
    for k in ("target_calls", "drafted_calls", "proposed", "accepted", "target_input_tokens",
              "rewinds", "next_seed"):
        assert getattr(st1, k) == getattr(st0, k), k
    assert dec.past_len == orc.past_len


WTYPES = [mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K]
WT_NAMES = {mtg.TYPE_F16: "f16", mtg.TYPE_F32: "f32", mtg.TYPE_Q4_K: "q4_K"}
# (weight type, exec mode): the persistent kernel streams q8_0 tiles and f16 / f32
# rows (its 8-row steps; 16-row steps of f16 / f32 weights take the per-op kernels)
ROW_STEP = (mtg.TYPE_F16, mtg.TYPE_F32)
WT_CASES = [(w, e) for w in WTYPES
            for e in ([mtg.EXEC_STEP_KERNEL] if w in ROW_STEP else []) + [mtg.EXEC_GRAPH, mtg.EXEC_EAGER]]
WT_IDS = ["%s-%s" % (WT_NAMES[w], EXEC_NAMES[e]) for w, e in WT_CASES]


@pytest.mark.parametrize("wtype,exec_mode", WT_CASES, ids=WT_IDS)
def test_f16_f32_and_q4k_weights_verify_matches_oracle(wtype, exec_mode):
    """f16, f32 and q4_K weights (the converter's dtypes and the k-quant path): hidden
    rows, logits, choices, acceptance and the appended KV equal the oracle's, for
    T = 1, 8, 16 in a row, with an f16 KV cache."""
    print("weights %s parity: exec=%s" % (WT_NAMES[wtype], EXEC_NAMES[exec_mode]), flush=True)
    model, orc, dec, rng = _setup(2, 40, kv_type=mtg.TYPE_F16, exec_mode=exec_mode, wtype=wtype)
    for T in (1, 8, 16):
        tokens = rng.integers(0, model.hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(h1, h0, "hidden T=%d" % T)
        _close(l1, l0, "logits T=%d" % T)
        assert np.array_equal(c1, c0) and m1 == m0
    assert dec.step_fallbacks == 0  # every step-kernel step ran to its end there
    # the persistent kernel took the 1- and 8-row steps (f16 weights, step mode)
    assert dec.step_kernel_runs == (2 if exec_mode == mtg.EXEC_STEP_KERNEL else 0)
    k0, v0 = orc.kv_read(orc.past_len)
    k1, v1 = dec.kv_read(dec.past_len)
    _close(k1, k0, "K cache")
    _close(v1, v0, "V cache")


@pytest.mark.parametrize("wtype,exec_mode", WT_CASES, ids=WT_IDS)
def test_long_f16_context_matches_oracle(wtype, exec_mode):
    """A context of 8300 cached positions (130 chunks of 64 keys, more than the
    chunk attention's workgroups per kv head, so each walks several chunks with
    the next one's rows in flight): hidden rows and logits equal the oracle's for
    T = 16, 5 and 12 (query columns that fill two, one and one and a half tiles)."""
    print("long f16 context %s: exec=%s" % (WT_NAMES[wtype], EXEC_NAMES[exec_mode]), flush=True)
    model = mtg.SynthModel(wtype, seed=11, std=0.02, gain_jitter=0.05, n_layers=1, vocab=4096)
    hp = model.hp
    prefix, max_seq = 8300, 8400
    orc = oracle_py.Oracle(model, max_seq, mtg.TYPE_F16)
    dec = mtg.Decoder(model, max_seq, mtg.TYPE_F16)
    dec.set_exec(exec_mode)
    dec.set_step_max_keys(1 << 30)  # the persistent kernel at this context too
    rng = np.random.default_rng(12)
    shape = (1, hp.n_kv_heads, prefix, hp.head_dim)
    k = rng.normal(0.0, 1.0, shape).astype(np.float16)
    v = rng.normal(0.0, 0.5, shape).astype(np.float16)
    orc.kv_write(k, v)
    dec.kv_write(k, v)
    for T in (16, 5, 12):
        tokens = rng.integers(0, hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(h1, h0, "hidden T=%d" % T)
        _close(l1, l0, "logits T=%d" % T)
        assert np.array_equal(c1, c0) and m1 == m0
    assert dec.step_fallbacks == 0
    assert dec.step_kernel_runs == (1 if exec_mode == mtg.EXEC_STEP_KERNEL else 0)  # the 5-row step


# default key limits of the persistent kernel (None: no limit)
KEY_LIMITS = [(mtg.TYPE_F16, 5120), (mtg.TYPE_F32, 8192), (mtg.TYPE_Q8_0, None)]


@pytest.mark.parametrize("wtype,limit", KEY_LIMITS, ids=["f16", "f32", "q8_0"])
def test_step_kernel_key_limit(wtype, limit):
    """Path selection by KV length: with f16 weights an 8-row step up to 5,120 keys
    (past + rows), with f32 weights up to 8,192, runs on the persistent kernel and a
    longer one on the per-op graph; q8_0 weights have no limit by default;
    mtg_set_step_max_keys moves it. Every step equals the oracle."""
    print("step kernel key limit: weights %d" % wtype, flush=True)
    model = mtg.SynthModel(wtype, seed=21, std=0.02, gain_jitter=0.05, n_layers=1, vocab=4096)
    hp = model.hp
    edge = limit or 3584  # q8_0: the same steps, all on the persistent kernel
    prefix, max_seq = edge + 16, edge + 116
    orc = oracle_py.Oracle(model, max_seq, mtg.TYPE_F16)
    dec = mtg.Decoder(model, max_seq, mtg.TYPE_F16)
    assert dec.exec_mode == mtg.EXEC_STEP_KERNEL
    rng = np.random.default_rng(22)
    shape = (1, hp.n_kv_heads, prefix, hp.head_dim)
    k = rng.normal(0.0, 1.0, shape).astype(np.float16)
    v = rng.normal(0.0, 0.5, shape).astype(np.float16)
    orc.kv_write(k, v)
    dec.kv_write(k, v)

    def step(past, limit=None):
        if limit is not None:
            dec.set_step_max_keys(limit)
        orc.rewind(past)
        dec.rewind(past)
        before = dec.step_kernel_runs
        tokens = rng.integers(0, hp.vocab, 8)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(h1, h0, "hidden, past %d" % past)
        _close(l1, l0, "logits, past %d" % past)
        assert np.array_equal(c1, c0) and m1 == m0
        return dec.step_kernel_runs - before

    over = 0 if limit else 1  # (each step rewinds to an earlier position)
    assert step(edge - 7) == over              # edge + 1 keys
    assert step(edge - 7, 1 << 20) == 1        # a higher limit
    assert step(edge - 7, 0) == over           # the default again
    assert step(edge - 8) == 1                 # edge keys
    assert step(3000, 2000) == 0               # a lower limit
    assert dec.step_fallbacks == 0


# (cached prefix, T, KV type): more than 32 chunks of 64 keys per kv head, so each
# workgroup of the step kernel's attention walks 2 or 4 chunks of one head with the
# q rows staged once. The new rows lie in one chunk (2050 + 16), straddle two
# chunks on two workgroups (2040 + 16: chunks 31 | 32) or two chunks of one
# workgroup (4030 + 9: chunks 62, 63), or end a 97-chunk context (6200 + 4); a
# 96-chunk context (6130 + 8: three chunks per workgroup) and a 194-chunk one
# (12400 + 16: seven).
CHUNK_GROUPS = [(2050, 16, mtg.TYPE_F32), (2040, 16, mtg.TYPE_F16), (4030, 9, mtg.TYPE_F16),
                (6200, 4, mtg.TYPE_F32), (3000, 1, mtg.TYPE_F16), (6130, 8, mtg.TYPE_F16),
                (12400, 16, mtg.TYPE_F16)]


@pytest.mark.parametrize("case", CHUNK_GROUPS, ids=["%d+%d-%s" % (p, t, "f32" if k == mtg.TYPE_F32 else "f16")
                                                    for p, t, k in CHUNK_GROUPS])
def test_step_kernel_chunk_groups_match_oracle(case):
    prefix, T, kv = case
    print("step kernel, chunk groups: prefix %d, T=%d, kv %d" % case, flush=True)
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=13, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    hp = model.hp
    max_seq = prefix + 2 * T + 8
    orc = oracle_py.Oracle(model, max_seq, kv)
    dec = mtg.Decoder(model, max_seq, kv)
    dec.set_exec(mtg.EXEC_STEP_KERNEL)
    rng = np.random.default_rng(prefix + T)
    dt = np.float32 if kv == mtg.TYPE_F32 else np.float16
    shape = (hp.n_layers, hp.n_kv_heads, prefix, hp.head_dim)
    k = rng.normal(0.0, 1.0, shape).astype(dt)
    v = rng.normal(0.0, 0.5, shape).astype(dt)
    orc.kv_write(k, v)
    dec.kv_write(k, v)
    for step in range(2):
        tokens = rng.integers(0, hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(h1, h0, "hidden, step %d" % step)
        _close(l1, l0, "logits, step %d" % step)
        assert np.array_equal(c1, c0) and m1 == m0
    n = dec.past_len
    assert n == orc.past_len
    k0, v0 = orc.kv_read(n)
    k1, v1 = dec.kv_read(n)
    _close(k1[:, :, prefix:], k0[:, :, prefix:], "K cache (new rows)")
    _close(v1[:, :, prefix:], v0[:, :, prefix:], "V cache (new rows)")


@pytest.mark.parametrize("wtype", WTYPES, ids=lambda w: WT_NAMES[w])
def test_f16_and_q4k_weights_penalty_prefill_and_stream(wtype):
    """The same weight types through the GPU prefill, the repetition penalty and
    the whole controller loop: token stream and counters equal the oracle's."""
    print("weights %s: prefill, penalty, token stream" % WT_NAMES[wtype], flush=True)
    model = mtg.SynthModel(wtype, seed=9, std=0.02, gain_jitter=0.05, n_layers=2, vocab=4096)
    orc = oracle_py.Oracle(model, 512)
    dec = mtg.Decoder(model, 512)
    if wtype in ROW_STEP:
        assert dec.exec_mode == mtg.EXEC_STEP_KERNEL
    else:
        assert dec.exec_mode == mtg.EXEC_GRAPH
        with pytest.raises(Exception):
            dec.set_exec(mtg.EXEC_STEP_KERNEL)
    rng = np.random.default_rng(10)
    rows = orc.embed(rng.integers(0, 4096, 37))
    ids = rng.integers(0, 4096, 5)
    _close(dec.embed(ids), orc.embed(ids), "embed")
    _close(dec.prefill(rows), orc.prefill(rows), "prefill hidden")
    hist = rng.integers(0, 4096, 120).tolist()
    tokens = rng.integers(0, 4096, 8)
    c0, m0, _, l0 = orc.verify(tokens, history=hist, penalty=1.3, want_logits=True)
    c1, m1, _, l1 = dec.verify(tokens, history=hist, penalty=1.3, want_logits=True)
    _close(l1, l0, "logits with penalty")
    assert np.array_equal(c1, c0) and m1 == m0
    prompt = rng.integers(0, 4096, 20).astype(np.int32)
    stream = rng.integers(0, 4096, 37).astype(np.int32)
    fn, user, _keep = mtg.stream_drafter(prompt, stream)
    first = int(rng.integers(0, 4096))
    ids0, st0 = orc.generate_from(first, 200, max_steps=12, penalty=1.1, max_draft=7, draft=fn, user=user)
    ids1, st1 = dec.generate_from(first, 200, max_steps=12, penalty=1.1, max_draft=7, draft=fn, user=user)
    assert dec.step_fallbacks == 0
    assert ids1.tolist() == ids0.tolist()
    assert st1.accepted == st0.accepted and st1.proposed == st0.proposed


@pytest.mark.parametrize("wtype", [mtg.TYPE_F16, mtg.TYPE_F32], ids=["f16", "f32"])
def test_f16_and_f32_weights_refuse_other_hidden_sizes(wtype):
    """The f16 and f32 lm_head kernels take K = 1,024: a model of hidden 2,048 with
    those weights is refused with MTG_ERR_UNSUPPORTED (the q8_0 and q4_K paths take
    it)."""
    model = mtg.SynthModel(wtype, seed=1, std=0.02, n_layers=1, vocab=256, hidden=2048)
    with pytest.raises(mtg.MtgError) as exc:
        mtg.Decoder(model, 64, mtg.TYPE_F32)
    assert exc.value.code == mtg.ERR_UNSUPPORTED
    model.close()


def test_step_kernel_abort_reports_and_recovers():
    """Failure path of the persistent kernel, forced from the host: with its error
    word raised before the launch, every bounded wait gives up at its first poll.
    The step fails with MTG_ERR_DEVICE, past_len and the KV cache stay, and the next
    step matches the oracle bit for bit."""
    print("step kernel abort path", flush=True)
    model, orc, dec, rng = _setup(2, 40)
    tokens = rng.integers(0, model.hp.vocab, 8)
    k_before, v_before = dec.kv_read(40)
    dec.debug_abort_next_step()
    with pytest.raises(mtg.MtgError) as exc:
        dec.verify(tokens)
    assert exc.value.code == mtg.ERR_DEVICE
    assert dec.past_len == 40
    k_after, v_after = dec.kv_read(40)
    _close(k_after, k_before, "K cache after the aborted step")
    _close(v_after, v_before, "V cache after the aborted step")
    for T in (8, 3):
        tokens = rng.integers(0, model.hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        _close(h1, h0, "hidden after recovery")
        _close(l1, l0, "logits after recovery")
        assert np.array_equal(c1, c0) and m1 == m0


def test_step_kernel_wait_timeout_falls_back_to_per_op_kernels():
    """A wait that runs out (forced from the host with a 1-poll limit on the
    kernel's own bounded waits) abandons the launch; the same step then runs on the
    per-op kernels in the same call, so the caller sees a normal result, equal to
    the oracle's bit for bit, and the fallback counter advances."""
    print("step kernel wait-timeout fallback", flush=True)
    model, orc, dec, rng = _setup(2, 40)
    before = dec.step_fallbacks
    dec.debug_wait_limit(1)
    dec.launch_timing(True)
    try:
        for T in (8, 5):
            tokens = rng.integers(0, model.hp.vocab, T)
            c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
            c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
            _close(h1, h0, "hidden after the fallback")
            _close(l1, l0, "logits after the fallback")
            assert np.array_equal(c1, c0) and m1 == m0
            assert dec.past_len == orc.past_len
        # both steps are timed: each counts once, with the abandoned launch and
        # the per-op rerun inside its time
        ms, launches, past_sum, rows_sum = dec.launch_timing_read()
        assert launches == 2 and rows_sum == 13 and past_sum == 40 + 48 and ms > 0.0
    finally:
        dec.launch_timing(False)
        dec.debug_wait_limit(0)
    assert dec.step_fallbacks == before + 2
    tokens = rng.integers(0, model.hp.vocab, 8)
    c0, m0, _, l0 = orc.verify(tokens, want_logits=True)
    c1, m1, _, l1 = dec.verify(tokens, want_logits=True)
    _close(l1, l0, "logits with the default bound")
    assert np.array_equal(c1, c0) and m1 == m0


@pytest.mark.parametrize("kv_type", [mtg.TYPE_F32, mtg.TYPE_F16], ids=["f32kv", "f16kv"])
@pytest.mark.parametrize("exec_mode", EXECS, ids=lambda e: EXEC_NAMES[e])
@pytest.mark.parametrize("prefix", [60, 2100])
def test_nan_poisoned_discarded_kv_is_never_read(prefix, exec_mode, kv_type):
    """cpu-lab/moss_speculative_gate.cpp:216-229 poisons a decoder's whole discarded
    capacity after every commit. Here, before each step, every cache position from
    past_len on (all layers and heads, both sides) is set to NaN; then T rows are
    verified, and the rewind keeps part of them. Hidden rows, logits, choices and
    the appended KV must be finite and bit-identical to the oracle's. Prefix 60
    puts the new keys across a 64-key chunk boundary; prefix 2,100 runs the step
    kernel's chunk groups (more than 32 chunks per kv head)."""
    print("NaN-poisoned discarded KV: prefix %d exec %s kv %d" % (prefix, EXEC_NAMES[exec_mode], kv_type),
          flush=True)
    max_seq = prefix + 40
    model, orc, dec, rng = _setup(2, prefix, kv_type=kv_type, exec_mode=exec_mode, max_seq=max_seq)
    for step, (T, keep) in enumerate(((8, 3), (5, 5), (16, 1), (4, 2))):
        past = dec.past_len
        assert orc.past_len == past
        k, v = orc.kv_read(max_seq)
        k[:, :, past:] = np.nan
        v[:, :, past:] = np.nan
        orc.kv_write(k, v)
        dec.kv_write(k, v)
        orc.rewind(past)
        dec.rewind(past)
        tokens = rng.integers(0, model.hp.vocab, T)
        c0, m0, h0, l0 = orc.verify(tokens, want_hidden=True, want_logits=True)
        c1, m1, h1, l1 = dec.verify(tokens, want_hidden=True, want_logits=True)
        assert np.isfinite(h1).all() and np.isfinite(l1).all(), "step %d read a poisoned position" % step
        _close(h1, h0, "hidden, step %d" % step)
        _close(l1, l0, "logits, step %d" % step)
        assert np.array_equal(c1, c0) and m1 == m0
        k0, v0 = orc.kv_read(past + T)
        k1, v1 = dec.kv_read(past + T)
        _close(k1, k0, "K cache, step %d" % step)
        _close(v1, v0, "V cache, step %d" % step)
        orc.rewind(past + keep)
        dec.rewind(past + keep)
