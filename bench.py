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

roofline: the step's device work (one persistent kernel per verify step) is timed
with HIP events on the library's stream over the timed region; achieved = the
algorithmic bytes of a step (q8_0 weights + KV read of past + T rows + KV write of
T rows) / the mean event time. traffic: HBM bytes per launch from rocprofv3
FETCH_SIZE + WRITE_SIZE (profiles/traffic.json), reported only when that file was
measured on the current kernel sources, else null.
"""
import hashlib
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
KERNEL = "k_step"  # the dominant kernel: the whole verify step
CSRC = os.path.join(ROOT, "moss-transcribe.cpp_amd", "csrc")
TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def source_hash():
    """Hash of the kernel and runtime sources, to tie a profile to a build."""
    h = hashlib.sha256()
    for name in sorted(os.listdir(CSRC)):
        if name.endswith((".hip", ".cpp", ".hpp")):
            h.update(name.encode())
            h.update(open(os.path.join(CSRC, name), "rb").read())
    return h.hexdigest()[:16]


def measured_traffic(config):
    """HBM bytes per step launch from the committed rocprofv3 counter summary,
    if it was measured on these sources and this workload."""
    try:
        t = json.load(open(TRAFFIC))
    except (OSError, ValueError):
        return None
    if t.get("source_hash") != source_hash() or t.get("config") != config:
        return None
    return t.get("traffic_bytes_per_launch")

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
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, copy a buffer of this size 5 times (device to device) "
                         "so that a counter profile of the same command can calibrate FETCH_SIZE "
                         "and WRITE_SIZE against a known byte count")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box here has one MI355X, and the verify path "
              "shards only across independent streams (one decoder per recording, one GPU each).", file=sys.stderr)
        sys.exit(2)
    cfg = CONFIGS[args.config]
    steps = args.steps if args.steps is not None else cfg["steps"]
    t_setup = time.perf_counter()
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0, n_layers=args.layers)
    hp = model.hp
    n_prompt = cfg["blocks"] * AUDIO_ROWS + cfg["text"]
    max_seq = n_prompt + (args.warmup + steps + 2) * cfg["K"] + 16
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    if args.exec == "step" and dec.exec_mode != mtg.EXEC_STEP_KERNEL:
        # the persistent kernel streams q8_0 only: f16 / q4_K weights run the
        # per-op kernels from a captured graph
        args.exec = "graph"
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
    dec.launch_timing(True)
    t0 = time.perf_counter()
    ids, st = dec.generate_from(st_w.next_seed, 1 << 20, max_steps=steps, max_draft=cfg["K"] - 1,
                                draft=fn, user=user, prior=ids_w)
    hip.hipDeviceSynchronize()
    elapsed = time.perf_counter() - t0
    dev_ms, launches, past_sum, rows_sum = dec.launch_timing_read()
    dec.launch_timing(False)
    n_steps = int(st.target_calls)
    tokens = len(ids)
    ms_step = 1e3 * elapsed / max(n_steps, 1)
    kvpos = kv_bytes_per_pos(hp, cfg["kv"])
    # algorithmic bytes of one launch: weights + KV read of past + T rows + KV write of T rows
    bytes_launch = weight_bytes(hp, cfg["wtype"]) + (past_sum + 2 * rows_sum) / max(launches, 1) * kvpos
    launch_s = dev_ms * 1e-3 / max(launches, 1)
    achieved = bytes_launch / launch_s / 1e9
    traffic = measured_traffic(args.config) if args.layers == 28 and args.exec == "step" else None
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
        "dtype": {mtg.TYPE_Q8_0: "q8_0 (int8 dots, f32 accumulate)", mtg.TYPE_F16: "f16",
                  mtg.TYPE_Q4_K: "q4_K"}[cfg["wtype"]],
        "data": "synthetic: seeded random weights, seeded audio-like prompt rows and draft stream",
        "config": {"workload": "Qwen3-0.6B-shaped verify step, %d layers, K=%d rows, %s weights, "
                               "%s KV, %d-row prompt (%d audio + %d text), %d greedy steps"
                               % (hp.n_layers, cfg["K"], {mtg.TYPE_Q8_0: "q8_0", mtg.TYPE_F16: "f16",
                                                          mtg.TYPE_Q4_K: "q4_K"}[cfg["wtype"]],
                                  "f32" if cfg["kv"] == mtg.TYPE_F32 else "f16", n_prompt,
                                  cfg["blocks"] * AUDIO_ROWS, cfg["text"], n_steps),
                   "verify_rows": cfg["K"], "context_start": ctx_start, "context_end": dec.past_len,
                   "accepted_per_step": st.accepted / max(n_steps, 1),
                   "tokens": tokens, "exec": args.exec},
        "verify_step_us": 1e3 * dev_ms / max(launches, 1),
        "host_step_us": 1e3 * ms_step,
        "step_bytes": bytes_launch,
        "roofline": {"bound": "hbm", "kernel": KERNEL if args.exec == "step" else "per-op kernels",
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic,
                     "launch_us": launch_s * 1e6, "launches": launches},
        "source_hash": source_hash(),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(model, dec, cfg, st.next_seed,
                                           np.concatenate([ids_w, ids]), drafter, args.cpu_seconds)
    if args.copy_probe_mib > 0:
        import torch
        n = args.copy_probe_mib << 18  # float32 elements
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_probe_bytes"] = n * 4
    print(json.dumps(out))


if __name__ == "__main__":
    main()
