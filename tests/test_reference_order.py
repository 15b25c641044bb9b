"""How far the canonical order (the device's, bit for bit) is from an independent
published order: ggml's generic scalar CPU kernels (the oracle's
ORDER_GGML_GENERIC: sequential block sums, double-accumulated dots, soft_max_ext
over the whole row with the causal mask, then the context at each query's valid
length; src/qwen3.cpp:157-189, src/cpu_context.cpp:13-32).

* One GEMM (the north star's "cross-block float accumulation"): the two orders
  agree within 1e-3 relative / 1e-4 absolute at every shape of the step.
* One and two layers: the whole step agrees within the same contract.
* Full depth (28 layers): the orders do NOT agree within the contract, and no two
  float orders can. Every GEMM input is re-quantized to q8_0 codes; a float
  difference of delta moves an activation code by one step d with probability
  ~delta/d, so the difference after re-quantization is ~sqrt(d * delta), which
  exceeds delta while delta < d: differences grow layer by layer to the size of
  one quantization step (~1 % of the row's magnitude) and stay there. The test
  asserts that bound and that the greedy choices agree wherever the top-2 margin
  exceeds twice the largest logit difference, and prints the measured distances.
"""
import os

import numpy as np
import pytest

import mtg
import numpy_ref
import oracle_py

THREADS = max(1, min(16, len(os.sched_getaffinity(0))))


def _within(got, ref):
    got, ref = np.asarray(got, np.float64), np.asarray(ref, np.float64)
    return np.abs(got - ref) <= 1e-4 + 1e-3 * np.abs(ref)


def test_generic_order_matches_independent_float64_model():
    """The generic order composes the same ops: against the float64 numpy Qwen3 it
    is as close as the canonical order (tests/test_oracle_model.py)."""
    m = mtg.SynthModel(mtg.TYPE_Q8_0, seed=20261010, std=0.02, gain_jitter=0.05, n_layers=2, vocab=2048)
    hp = m.hp
    ref = numpy_ref.NumpyQwen3(m, numpy_ref.layer_weights(m))
    orc = oracle_py.Oracle(m, 64)
    orc.set_order(orc.ORDER_GGML_GENERIC)
    rng = np.random.default_rng(2)
    out_norm = np.ctypeslib.as_array(
        (mtg.c_float * hp.hidden).from_address(m.desc.contents.output_norm)).astype(np.float64)
    for T in (5, 1, 8):
        x = orc.embed(rng.integers(0, hp.vocab, T))
        h = orc.run(x).astype(np.float64)
        h_ref = numpy_ref.rms(ref.step(x), out_norm, hp.rms_eps)
        err = np.abs(h - h_ref)
        assert np.sqrt((err ** 2).mean()) <= 2e-4 * np.sqrt((h_ref ** 2).mean())
    orc.close()
    m.close()


@pytest.mark.parametrize("wtype", [mtg.TYPE_Q8_0, mtg.TYPE_F16, mtg.TYPE_F32, mtg.TYPE_Q4_K])
def test_one_gemm_within_contract_at_every_step_shape(wtype):
    rng = np.random.default_rng(61)
    shapes = [(1024, 4096), (2048, 1024), (1024, 3072), (3072, 1024), (1024, 151936)]
    for k, n in shapes:
        if n == 151936 and wtype != mtg.TYPE_Q8_0:
            continue
        w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
        raw = np.empty(mtg.lib().mtg_row_bytes(wtype, k) * n, np.uint8)
        if wtype == mtg.TYPE_Q8_0:
            mtg.lib().mtg_quantize_q8_0_weight(mtg.ptr(w), w.size, mtg.ptr(raw))
        elif wtype == mtg.TYPE_F16:
            raw[:] = w.astype(np.float16).view(np.uint8).reshape(-1)
        elif wtype == mtg.TYPE_F32:
            raw[:] = w.view(np.uint8).reshape(-1)
        else:
            mtg.lib().mtg_quantize_q4_k(mtg.ptr(w), w.size, mtg.ptr(raw))
        x = rng.standard_normal((8, k)).astype(np.float32)
        canon = oracle_py.mul_mat(wtype, raw, k, n, x)
        generic = oracle_py.mul_mat_generic(wtype, raw, k, n, x)
        ok = _within(generic, canon)
        assert ok.all(), (wtype, k, n, np.abs(generic - canon).max())


def _pair(n_layers, vocab, prefix=64, seed=3):
    model = mtg.SynthModel(mtg.TYPE_Q8_0, seed=seed, std=0.02, gain_jitter=0.05, n_layers=n_layers,
                           vocab=vocab)
    orcs = []
    for order in (oracle_py.Oracle.ORDER_CANONICAL, oracle_py.Oracle.ORDER_GGML_GENERIC):
        o = oracle_py.Oracle(model, prefix + 64, mtg.TYPE_F32)
        o.set_order(order)
        orcs.append(o)
    rng = np.random.default_rng(5)
    orcs[0].prefill(orcs[0].embed(rng.integers(0, model.hp.vocab, prefix)))
    k, v = orcs[0].kv_read(prefix)
    orcs[1].kv_write(k, v)
    return model, orcs, rng


def test_one_and_two_layers_within_contract():
    oracle_py.lib().orc_set_threads(THREADS)
    for L in (1, 2):
        model, orcs, rng = _pair(L, 4096)
        tokens = rng.integers(0, model.hp.vocab, 8)
        (c0, m0, h0, l0), (c1, m1, h1, l1) = [o.verify(tokens, want_hidden=True, want_logits=True)
                                              for o in orcs]
        assert _within(h1, h0).all() and _within(l1, l0).all(), L
        assert np.array_equal(c0, c1) and m0 == m1
        for o in orcs:
            o.close()
        model.close()


def test_full_depth_difference_is_bounded_by_requantization():
    oracle_py.lib().orc_set_threads(THREADS)
    model, orcs, rng = _pair(28, 151936)
    rows = []
    for step in range(2):
        tokens = rng.integers(0, model.hp.vocab, 8)
        (c0, _, h0, l0), (c1, _, h1, l1) = [o.verify(tokens, want_hidden=True, want_logits=True)
                                            for o in orcs]
        h0, h1 = h0.astype(np.float64), h1.astype(np.float64)
        rel = np.sqrt(((h1 - h0) ** 2).mean() / (h0 ** 2).mean())
        d = np.abs(l1.astype(np.float64) - l0)
        top = np.sort(l0, axis=1)
        margin = top[:, -1] - top[:, -2]
        print("step %d: hidden rel RMS %.2e, logits max |diff| %.3g (max |logit| %.3g), "
              "%.1f %% within 1e-3/1e-4, choices equal %s, top-2 margins %s"
              % (step, rel, d.max(), np.abs(l0).max(), 100 * _within(l1, l0).mean(),
                 (c0 == c1).tolist(), np.round(margin, 4).tolist()))
        # the saturation level: one quantization step of a q8_0 block
        assert rel <= 2e-2
        assert d.max() <= 0.02 * np.abs(l0).max() + 0.05
        # a choice may differ only where the margin is within the difference
        safe = margin > 2 * d.max()
        assert np.array_equal(c0[safe], c1[safe])
        rows.append(safe.sum())
        for o in orcs:
            o.rewind(64)
    for o in orcs:
        o.close()
    model.close()
