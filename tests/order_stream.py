"""The K=8 q8_0 workload's greedy stream (1,600-row prompt, 256 steps, the 37-token
periodic draft stream) run by the oracle in its canonical order and in ggml's
generic scalar order from the same prefilled KV cache, on the CPU. Prints how many
committed ids differ, the first divergence and the top-2 logit margins there, and
the per-step logit distance on the steps before it.

    python3 tests/order_stream.py [--steps 256] [--threads N]

This is a measurement, not a test: pytest does not collect it (it takes minutes).
"""
import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path[:0] = [os.path.join(ROOT, "moss-transcribe.cpp_amd"), os.path.join(ROOT, "oracle")]

import mtg  # noqa: E402
import oracle_py  # noqa: E402
from workloads import WORKLOADS, build_prompt, prompt_rows  # noqa: E402


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--threads", type=int, default=len(os.sched_getaffinity(0)))
    args = ap.parse_args()
    oracle_py.lib().orc_set_threads(args.threads)
    cfg = WORKLOADS[2]
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0)
    n_prompt, K = prompt_rows(cfg), cfg["K"]
    max_seq = n_prompt + (args.steps + 4) * K
    can = oracle_py.Oracle(model, max_seq, cfg["kv"])
    rows, text, stream = build_prompt(model, can.embed, cfg)
    t0 = time.time()
    hid = can.prefill(rows)
    first = int(np.argmax(can.logits(hid[-1:])[0]))
    print("prefill %d rows in %.0f s" % (n_prompt, time.time() - t0), flush=True)
    gen = oracle_py.Oracle(model, max_seq, cfg["kv"])
    k, v = can.kv_read(n_prompt)
    gen.kv_write(k, v)
    del k, v
    gen.set_order(gen.ORDER_GGML_GENERIC)
    fn, user, _keep = mtg.stream_drafter(text, stream)
    out = {}
    for name, o in (("canonical", can), ("generic", gen)):
        t0 = time.time()
        ids, st = o.generate_from(first, 1 << 20, max_steps=args.steps, max_draft=K - 1, draft=fn, user=user)
        out[name] = (ids, st)
        print("%s order: %d steps, %d ids, %d accepted drafts, %.0f s"
              % (name, st.target_calls, len(ids), st.accepted, time.time() - t0), flush=True)
    a, b = out["canonical"][0], out["generic"][0]
    n = min(len(a), len(b))
    diff = np.nonzero(a[:n] != b[:n])[0]
    print("ids: canonical %d, generic %d; differing positions among the first %d: %d"
          % (len(a), len(b), n, len(diff)), flush=True)
    if len(diff) == 0 and len(a) == len(b):
        print("streams identical", flush=True)
        return
    j = int(diff[0]) if len(diff) else n
    print("first divergence at committed id %d: canonical %s, generic %s"
          % (j, a[j] if j < len(a) else None, b[j] if j < len(b) else None), flush=True)
    # Replay of the canonical stream in K-row windows from the prefilled state, on
    # both orders: the input at position n_prompt + i is committed id i (the first
    # seed is id 0), and the row of input i chooses id i + 1.
    for o in (can, gen):
        o.rewind(n_prompt)
    margins, dists, agree, rows = [], [], 0, 0
    pos = 0
    while pos + K <= j:
        tok = a[pos:pos + K]
        c0, _, _, l0 = can.verify(tok, history=a[:pos], want_logits=True)
        c1, _, _, l1 = gen.verify(tok, history=a[:pos], want_logits=True)
        top = np.sort(l0, axis=1)
        margins.extend((top[:, -1] - top[:, -2]).tolist())
        dists.append(np.abs(l0.astype(np.float64) - l1).max())
        agree += int((c0 == c1).sum())
        rows += K
        pos += K
    m = np.array(margins)
    print("before the divergence: %d rows replayed, choices equal in %d; top-2 margin min %.3g, p1 %.3g; "
          "max |dlogit| between the orders %.3g" % (rows, agree, m.min(), np.percentile(m, 1), max(dists)),
          flush=True)
    # the window holding the row that chose id j (its input is id j - 1)
    pos = K * ((j - 1) // K)
    tok = a[pos:pos + K]
    for o in (can, gen):
        o.rewind(n_prompt + pos)
    c0, _, _, l0 = can.verify(tok, history=a[:pos], want_logits=True)
    c1, _, _, l1 = gen.verify(tok, history=a[:pos], want_logits=True)
    r = j - 1 - pos
    s0, s1 = np.sort(l0[r]), np.sort(l1[r])
    print("at the divergence (row %d of the window at %d): canonical choice %d, top-2 margin %.3g; generic "
          "choice %d, top-2 margin %.3g; |dlogit| of the two top ids %.3g / %.3g; max |dlogit| over the "
          "window %.3g" % (r, pos, c0[r], s0[-1] - s0[-2], c1[r], s1[-1] - s1[-2],
                           abs(float(l0[r][c0[r]]) - float(l1[r][c0[r]])),
                           abs(float(l0[r][c1[r]]) - float(l1[r][c1[r]])),
                           np.abs(l0.astype(np.float64) - l1).max()), flush=True)
    assert c0[r] == a[j], "the replay reproduces the canonical stream"


if __name__ == "__main__":
    main()
