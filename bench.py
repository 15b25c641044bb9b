"""Speculative verify-step benchmark on one MI355X.

Workload (default): Qwen3-0.6B-shaped decoder, 28 layers, q8_0 weights (seed 0,
N(0, 0.02), norm gains 1), f32 KV prefilled to 1,600 positions (4 blocks of 375
audio rows N(0,1) scaled to the RMS of the token embeddings, then 100 random
text ids), greedy decoding with K = 8 verify rows per step (seed + 7 drafts)
from an n-gram drafter over prompt ++ committed ids, completed from a seeded
37-token periodic stream. A step = one verify pass (append K rows, tied lm_head
over all rows, on-device greedy choice and acceptance) plus the host controller.

Prints one JSON line (metric, value = accepted tokens/s, ms_per_step, roofline of
the dominant kernel, cpu_baseline = the oracle on the host cores).
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "moss-transcribe.cpp_amd"), os.path.join(ROOT, "oracle")]

import mtg  # noqa: E402

METRIC = "verify-step µs + accepted tok/s (q8_0, K=8, ctx 1.6k); % of HBM peak"
HBM_PEAK_GBS = 8000.0

# (weight type, kv type, audio blocks, text ids, K rows, decode steps)
CONFIGS = {
    1: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F32, blocks=0, text=512, K=4, steps=1),
    2: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F32, blocks=4, text=100, K=8, steps=256),
    3: dict(wtype=mtg.TYPE_Q8_0, kv=mtg.TYPE_F16, blocks=10, text=250, K=16, steps=128),
    4: dict(wtype=mtg.TYPE_F16, kv=mtg.TYPE_F16, blocks=20, text=500, K=8, steps=128),
    5: dict(wtype=mtg.TYPE_Q4_K, kv=mtg.TYPE_F16, blocks=43, text=259, K=16, steps=64),
}
AUDIO_ROWS = 375
STREAM_PERIOD = 37


def weight_bytes(hp, wtype):
    H, D, F = hp.hidden, hp.head_dim, hp.intermediate
    layer = (H * (hp.n_heads * D) * 2 + H * (hp.n_kv_heads * D) * 2 + 3 * H * F) * hp.n_layers
    params = layer + hp.vocab * H
    per = {mtg.TYPE_Q8_0: 34 / 32, mtg.TYPE_F16: 2.0, mtg.TYPE_Q4_K: 144 / 256}[wtype]
    return params * per


def kv_bytes_per_pos(hp, kv):
    return hp.n_layers * 2 * hp.n_kv_heads * hp.head_dim * (4 if kv == mtg.TYPE_F32 else 2)


def build_prompt(model, dec, cfg):
    """Fused prompt rows: audio blocks (N(0,1) scaled to the embedding RMS) + text ids."""
    hp = model.hp
    rng = np.random.default_rng(1)
    text = rng.integers(0, hp.vocab, cfg["text"]).astype(np.int32)
    sample = dec.embed(np.arange(0, hp.vocab, max(1, hp.vocab // 2048))[:2048])
    rms = float(np.sqrt((sample.astype(np.float64) ** 2).mean()))
    n_audio = cfg["blocks"] * AUDIO_ROWS
    audio = mtg.normal(1, 0, n_audio * hp.hidden).reshape(n_audio, hp.hidden) * np.float32(rms)
    rows = np.concatenate([audio, dec.embed(text)]) if n_audio else dec.embed(text)
    stream = np.random.default_rng(2).integers(0, hp.vocab, STREAM_PERIOD).astype(np.int32)
    return rows.astype(np.float32), text, stream


def cpu_baseline(model, dec, cfg, first_seed, prior, drafter, budget_s):
    """The oracle (CPU restatement of the reference path) on this host's cores,
    from the same KV state, on a bounded number of verify steps."""
    import oracle_py
    threads = len(os.sched_getaffinity(0))
    oracle_py.lib().orc_set_threads(threads)
    orc = oracle_py.Oracle(model, dec.max_seq, cfg["kv"])
    past = dec.past_len
    k, v = dec.kv_read(past)
    orc.kv_write(k, v)
    fn, user, _keep = drafter
    # one warm step, then steps until the budget is used
    t0 = time.perf_counter()
    ids, st = orc.generate_from(first_seed, 1 << 20, max_steps=1, penalty=1.0, max_draft=cfg["K"] - 1,
                                draft=fn, user=user, prior=prior)
    seed = st.next_seed
    prior = np.concatenate([prior, ids])
    steps = tokens = 0
    t_steps = 0.0
    while t_steps < budget_s or steps < 2:
        t1 = time.perf_counter()
        ids, st = orc.generate_from(seed, 1 << 20, max_steps=1, penalty=1.0,
                                    max_draft=cfg["K"] - 1, draft=fn, user=user, prior=prior)
        t_steps += time.perf_counter() - t1
        steps += 1
        tokens += len(ids)
        seed = st.next_seed
        prior = np.concatenate([prior, ids])
    orc.close()
    return {"value": tokens / t_steps, "unit": "tok/s", "cores": threads, "kind": "port",
            "ms_per_step": 1e3 * t_steps / steps,
            "sample": "%d verify steps (K=%d) of the same workload from the GPU's KV state, "
                      "oracle C++/OpenMP on %d host threads" % (steps, cfg["K"], threads)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--layers", type=int, default=28)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--exec", choices=["step", "graph", "eager"], default="step",
                    help="persistent step kernel, per-op kernels from a graph, or eager per-op")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box here has one MI355X, and the verify path "
              "shards only across independent streams (see DESIGN.md).", file=sys.stderr)
        sys.exit(2)
    cfg = CONFIGS[args.config]
    steps = args.steps if args.steps is not None else cfg["steps"]
    t_setup = time.perf_counter()
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0, n_layers=args.layers)
    hp = model.hp
    n_prompt = cfg["blocks"] * AUDIO_ROWS + cfg["text"]
    max_seq = n_prompt + (args.warmup + steps + 2) * cfg["K"] + 16
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    dec.set_exec({"step": mtg.EXEC_STEP_KERNEL, "graph": mtg.EXEC_GRAPH, "eager": mtg.EXEC_EAGER}[args.exec])
    rows, text, stream = build_prompt(model, dec, cfg)
    hid = dec.prefill(rows)
    first = int(np.argmax(dec.logits(hid[-1:])[0]))
    drafter = mtg.stream_drafter(text, stream)
    fn, user, _keep = drafter
    print("setup %.1fs: prompt %d rows, max_seq %d" % (time.perf_counter() - t_setup, n_prompt, max_seq),
          file=sys.stderr, flush=True)
    # warmup
    ids_w, st_w = dec.generate_from(first, 1 << 20, max_steps=args.warmup, max_draft=cfg["K"] - 1,
                                    draft=fn, user=user)
    ctx_start = dec.past_len
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipDeviceSynchronize()
    t0 = time.perf_counter()
    ids, st = dec.generate_from(st_w.next_seed, 1 << 20, max_steps=steps, max_draft=cfg["K"] - 1,
                                draft=fn, user=user, prior=ids_w)
    hip.hipDeviceSynchronize()
    elapsed = time.perf_counter() - t0
    n_steps = int(st.target_calls)
    tokens = len(ids)
    ms_step = 1e3 * elapsed / max(n_steps, 1)
    ctx_mean = ctx_start + (dec.past_len - ctx_start) / 2.0
    step_bytes = weight_bytes(hp, cfg["wtype"]) + (ctx_mean + 2 * cfg["K"]) * kv_bytes_per_pos(hp, cfg["kv"])
    out = {
        "metric": METRIC,
        "value": tokens / elapsed,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": n_steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q8_0 int8 dots, f32 accumulate" if cfg["wtype"] == mtg.TYPE_Q8_0 else "f16/q4_K",
        "data": "synthetic (seeded random weights and prompt rows)",
        "config": {"workload": "config %d: Qwen3-0.6B-shaped verify, %d layers, K=%d, prompt %d rows, "
                               "%s KV" % (args.config, hp.n_layers, cfg["K"], n_prompt,
                                          "f32" if cfg["kv"] == mtg.TYPE_F32 else "f16"),
                   "verify_rows": cfg["K"], "context_start": ctx_start, "context_end": dec.past_len,
                   "accepted_per_step": st.accepted / max(n_steps, 1),
                   "tokens": tokens, "exec": args.exec},
        "step_us": 1e3 * ms_step,
        "step_bytes": step_bytes,
        "step_hbm_fraction": step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS,
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(model, dec, cfg, st.next_seed,
                                           np.concatenate([ids_w, ids]), drafter, args.cpu_seconds)
    print(json.dumps(out))


if __name__ == "__main__":
    main()
