"""Speculative verify-step benchmark on one MI355X.

Workload (default): Qwen3-0.6B-shaped decoder, 28 layers, q8_0 weights (seed 0,
N(0, 0.02), norm gains 1), f32 KV prefilled to 1,600 positions (4 blocks of 375
audio rows N(0,1) scaled to the RMS of the token embeddings, then 100 random
text ids), greedy decoding with K = 8 verify rows per step (seed + 7 drafts)
from an n-gram drafter over prompt ++ committed ids, completed from a seeded
37-token periodic stream. A step = one verify pass (append K rows, tied lm_head
over all rows, on-device greedy choice and acceptance) plus the host controller
(--loop device: the device loop instead, a controller kernel between the step
kernels that commits the accepted ids, applies the stop rules and drafts the next
step with the same stream drafter, the host looking at the state every 8 steps).

Prints one JSON line (metric, value = accepted tokens/s, ms_per_step, roofline of
the dominant kernel, cpu_baseline = the oracle on the host cores).

roofline: the step's device work (one persistent kernel per verify step) is timed
with HIP events on the library's stream over the timed region; achieved = the
algorithmic bytes of a step (q8_0 weights + KV read of past + T rows + KV write of
T rows) / the mean event time. traffic: HBM bytes per launch from rocprofv3
FETCH_SIZE + WRITE_SIZE (profiles/traffic.json), reported only when that file was
measured on the current kernel sources, else null.

cpu_baseline (reference protocol, cpu-lab/moss_causal_context_bench.cpp:184-222:
one discarded warmup pair, then 5 alternating measured pairs, median and range):
the KV cache is snapshotted at the start of the timed region; the oracle (the CPU
restatement of the reference path, C++/OpenMP, one thread per core of this
process's CPU share, pinned) and the GPU each verify the same batch (the first
K ids of the timed stream) from that state, alternating; their choices must be
equal. Then the oracle replays the GPU's timed steps from the snapshot, as many as
fit the --cpu-seconds budget; its ids must equal the GPU's prefix. value =
committed tokens / time of that replay. The CPU leg runs after the GPU
measurement, and a failure in it is reported inside cpu_baseline without losing
the GPU fields.
"""
import argparse
import hashlib
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path[:0] = [os.path.join(ROOT, "moss-transcribe.cpp_amd"), os.path.join(ROOT, "oracle")]

import mtg  # noqa: E402
from workloads import AUDIO_ROWS, WORKLOADS, WNAME, build_prompt, prompt_rows  # noqa: E402

METRIC = "verify-step µs + accepted tok/s (q8_0, K=8, ctx 1.6k); % of HBM peak"
HBM_PEAK_GBS = 8000.0
KERNEL = "k_step"  # the dominant kernel: the whole verify step
CSRC = os.path.join(ROOT, "moss-transcribe.cpp_amd", "csrc")
TRAFFIC = os.path.join(ROOT, "profiles", "traffic.json")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


# the sources the step kernel is built from (its launch included)
STEP_SOURCES = ("step_kernel.hip", "step_kernel.hpp", "device_common.hpp", "lm_f16.hpp", "kernels.hpp",
                "mtg_internal.hpp", "runtime.cpp", "runtime.hpp")


def source_hash():
    """Hash of the step kernel's sources, to tie a counter profile of it to a build."""
    h = hashlib.sha256()
    for name in STEP_SOURCES:
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


def weight_bytes(hp, wtype):
    H, D, F = hp.hidden, hp.head_dim, hp.intermediate
    layer = (H * (hp.n_heads * D) * 2 + H * (hp.n_kv_heads * D) * 2 + 3 * H * F) * hp.n_layers
    params = layer + hp.vocab * H
    per = {mtg.TYPE_Q8_0: 34 / 32, mtg.TYPE_F16: 2.0, mtg.TYPE_F32: 4.0, mtg.TYPE_Q4_K: 144 / 256}[wtype]
    return params * per


def kv_bytes_per_pos(hp, kv):
    return hp.n_layers * 2 * hp.n_kv_heads * hp.head_dim * (4 if kv == mtg.TYPE_F32 else 2)


def cpu_threads():
    """Threads for the CPU leg: one per core of this process's CPU share
    (OMP_NUM_THREADS when the environment sets it lower than the affinity mask)."""
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return n


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(model, dec, cfg, snap, budget_s):
    """The oracle beside the GPU from the KV state at the start of the timed run.
    snap: (k, v, ctx_start, first_seed, prior ids, GPU timed ids, GPU steps, drafter)."""
    k, v, ctx_start, seed0, prior, gpu_ids, gpu_steps, drafter = snap
    threads = cpu_threads()
    # the host as this process sees it, before the OpenMP runtime pins the threads
    host = {"cpu_model": cpu_model(), "nproc": os.cpu_count(), "affinity": len(os.sched_getaffinity(0)),
            "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}
    # pinning: read by the OpenMP runtime when the oracle library loads
    os.environ.setdefault("OMP_PROC_BIND", "close")
    os.environ.setdefault("OMP_PLACES", "cores")
    import oracle_py
    oracle_py.lib().orc_set_threads(threads)
    orc = oracle_py.Oracle(model, dec.max_seq, cfg["kv"])
    try:
        orc.kv_write(k, v)
        K = cfg["K"]
        tokens = np.asarray(gpu_ids[:K], np.int32)
        if len(tokens) < 1:
            raise RuntimeError("the timed run emitted no ids")
        hist = np.asarray(prior, np.int32)
        gpu_ms, cpu_ms = [], []
        for pair in range(6):  # pair 0 is the discarded warmup
            dec.rewind(ctx_start)
            t0 = time.perf_counter()
            c_gpu, m_gpu, _, _ = dec.verify(tokens, history=hist)
            t1 = time.perf_counter()
            orc.rewind(ctx_start)
            t2 = time.perf_counter()
            c_cpu, m_cpu, _, _ = orc.verify(tokens, history=hist)
            t3 = time.perf_counter()
            if not (np.array_equal(c_gpu, c_cpu) and m_gpu == m_cpu):
                raise RuntimeError("pair %d: GPU choices %s / %d differ from the oracle's %s / %d"
                                   % (pair, c_gpu.tolist(), m_gpu, c_cpu.tolist(), m_cpu))
            if pair:
                gpu_ms.append(1e3 * (t1 - t0))
                cpu_ms.append(1e3 * (t3 - t2))
        log("cpu leg: pairs done, CPU verify median %.1f ms" % statistics.median(cpu_ms))
        # replay of the GPU's timed steps, bounded by the time budget
        n_steps = int(max(2, min(gpu_steps, budget_s / (statistics.median(cpu_ms) * 1e-3))))
        orc.rewind(ctx_start)
        fn, user, _keep = drafter
        t0 = time.perf_counter()
        ids, st = orc.generate_from(seed0, 1 << 20, max_steps=n_steps, penalty=1.0, max_draft=K - 1,
                                    draft=fn, user=user, prior=prior)
        t_replay = time.perf_counter() - t0
        same = bool(np.array_equal(ids, np.asarray(gpu_ids[:len(ids)], np.int32)))
        if not same:
            raise RuntimeError("oracle replay of %d steps emitted ids that differ from the GPU's" % n_steps)
        log("cpu leg: replayed %d steps in %.1f s, ids identical to the GPU's" % (n_steps, t_replay))
        return {"value": len(ids) / t_replay, "unit": "tok/s", "cores": threads, "kind": "port",
                "sample": "first %d of the GPU's timed verify steps (K=%d, context %d+), replayed by the "
                          "oracle (C++/OpenMP restatement of the reference path) from the same KV "
                          "snapshot; %d ids, identical to the GPU's" % (n_steps, K, ctx_start, len(ids)),
                "ms_per_step": 1e3 * t_replay / n_steps,
                "pairs": {"protocol": "1 warmup + 5 alternating GPU/CPU pairs, same verify batch "
                                      "(T=%d at past %d), choices equal in every pair" % (len(tokens), ctx_start),
                          "cpu_verify_ms_median": statistics.median(cpu_ms),
                          "cpu_verify_ms_range": [min(cpu_ms), max(cpu_ms)],
                          "gpu_verify_ms_median": statistics.median(gpu_ms),
                          "gpu_verify_ms_range": [min(gpu_ms), max(gpu_ms)]},
                "host": dict(host, threads=threads, OMP_PROC_BIND=os.environ.get("OMP_PROC_BIND"),
                             OMP_PLACES=os.environ.get("OMP_PLACES")),
                "stream_identical": same}
    finally:
        orc.close()


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
    ap.add_argument("--loop", choices=["device", "host"], default="host",
                    help="the speculative controller on the device (a controller kernel between the step "
                         "kernels, the stream drafter run there) or on the host; per-op execution always "
                         "runs the host loop")
    ap.add_argument("--prefill-runs", type=int, default=0,
                    help="only prefill the workload's prompt this many times (block prefill) and print "
                         "its device time; for kernel traces of the prefill")
    ap.add_argument("--weights", choices=["q8_0", "f16", "f32", "q4_K"], default=None,
                    help="run the workload with another weight type than its own (e.g. f32, the "
                         "converter's default dtype); not a bench line of the workload")
    ap.add_argument("--copy-probe-mib", type=int, default=0,
                    help="after the run, copy a buffer of this size 5 times (device to device) "
                         "so that a counter profile of the same command can calibrate FETCH_SIZE "
                         "and WRITE_SIZE against a known byte count")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box here has one MI355X, and the verify path "
              "shards only across independent streams (one decoder per recording, one GPU each).",
              file=sys.stderr)
        sys.exit(2)
    cfg = dict(WORKLOADS[args.config])
    if args.weights is not None:
        cfg["wtype"] = {v: k for k, v in WNAME.items()}[args.weights]
    steps = args.steps if args.steps is not None else cfg["steps"]
    t_setup = time.perf_counter()
    model = mtg.SynthModel(cfg["wtype"], seed=0, std=0.02, gain_jitter=0.0, n_layers=args.layers)
    hp = model.hp
    n_prompt = prompt_rows(cfg)
    max_seq = n_prompt + (args.warmup + steps + 2) * cfg["K"] + 16
    dec = mtg.Decoder(model, max_seq, cfg["kv"])
    if args.exec == "step" and dec.exec_mode != mtg.EXEC_STEP_KERNEL:
        # the persistent kernel streams q8_0 only: f16 / q4_K weights run the
        # per-op kernels from a captured graph
        args.exec = "graph"
    dec.set_exec({"step": mtg.EXEC_STEP_KERNEL, "graph": mtg.EXEC_GRAPH, "eager": mtg.EXEC_EAGER}[args.exec])
    rows, text, stream = build_prompt(model, dec.embed, cfg)
    if args.prefill_runs > 0:
        times = []
        for _ in range(args.prefill_runs):
            dec.prefill(rows, want_hidden=False)
            times.append(dec.last_prefill_ms)
        print(json.dumps({"metric": "block prefill device ms", "value": min(times), "unit": "ms",
                          "runs_ms": times, "rows": int(rows.shape[0]), "config": args.config,
                          "weights": WNAME[cfg["wtype"]], "higher_is_better": False}), flush=True)
        return
    hid = dec.prefill(rows)
    first = int(np.argmax(dec.logits(hid[-1:])[0]))
    drafter = mtg.stream_drafter(text, stream)
    fn, user, _keep = drafter
    log("setup %.1fs: prompt %d rows, max_seq %d" % (time.perf_counter() - t_setup, n_prompt, max_seq))
    # warmup, on the same controller as the timed steps (its buffers and events are
    # made by the first call)
    loop = args.loop if args.exec == "step" else "host"
    if loop == "device":
        ids_w, st_w = dec.generate_device(first, 1 << 20, max_steps=args.warmup, max_draft=cfg["K"] - 1,
                                          stream=drafter)
    else:
        ids_w, st_w = dec.generate_from(first, 1 << 20, max_steps=args.warmup, max_draft=cfg["K"] - 1,
                                        draft=fn, user=user)
    ctx_start = dec.past_len
    # KV snapshot for the CPU leg (outside the timed region)
    snap_kv = dec.kv_read(ctx_start) if not args.no_cpu else None
    import ctypes
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipDeviceSynchronize()
    dec.launch_timing(True)
    fallbacks0 = dec.step_fallbacks
    runs0 = dec.step_kernel_runs
    t0 = time.perf_counter()
    if loop == "device":
        ids, st = dec.generate_device(st_w.next_seed, 1 << 20, max_steps=steps, max_draft=cfg["K"] - 1,
                                      prior=ids_w, stream=drafter)
    else:
        ids, st = dec.generate_from(st_w.next_seed, 1 << 20, max_steps=steps, max_draft=cfg["K"] - 1,
                                    draft=fn, user=user, prior=ids_w)
    hip.hipDeviceSynchronize()
    elapsed = time.perf_counter() - t0
    dev_ms, launches, past_sum, rows_sum = dec.launch_timing_read()
    dec.launch_timing(False)
    # steps whose persistent kernel gave up on a bounded wait and ran again on the
    # per-op kernels (their event time covers both launches)
    fallbacks = dec.step_fallbacks - fallbacks0
    # the path the timed steps took: in step mode, steps past the persistent
    # kernel's KV length limit (f16 weights) run on the per-op graph
    runs = dec.step_kernel_runs - runs0
    if args.exec != "step":
        path = args.exec
    elif runs + fallbacks >= launches:
        path = "step"
    elif runs + fallbacks == 0:
        path = "graph"
    else:
        path = "step+graph"
    if fallbacks:
        log("WARNING: %d of %d timed steps fell back to the per-op kernels" % (fallbacks, launches))
    n_steps = int(st.target_calls)
    tokens = len(ids)
    log("timed: %d steps, %d tokens in %.3f s (%.1f us per launch)"
        % (n_steps, tokens, elapsed, 1e3 * dev_ms / max(launches, 1)))
    ms_step = 1e3 * elapsed / max(n_steps, 1)
    kvpos = kv_bytes_per_pos(hp, cfg["kv"])
    # algorithmic bytes of one launch: weights + KV read of past + T rows + KV write of T rows
    bytes_launch = weight_bytes(hp, cfg["wtype"]) + (past_sum + 2 * rows_sum) / max(launches, 1) * kvpos
    launch_s = dev_ms * 1e-3 / max(launches, 1)
    achieved = bytes_launch / launch_s / 1e9
    traffic = (measured_traffic(args.config) if args.layers == 28 and args.exec == "step" and args.weights is None
               and runs > 0 else None)
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
        "dtype": {mtg.TYPE_Q8_0: "q8_0 (int8 dots, f32 accumulate)", mtg.TYPE_F16: "f16", mtg.TYPE_F32: "f32",
                  mtg.TYPE_Q4_K: "q4_K"}[cfg["wtype"]],
        "data": "synthetic: seeded random weights, seeded audio-like prompt rows and draft stream",
        "config": {"workload": "Qwen3-0.6B-shaped verify step, %d layers, K=%d rows, %s weights, "
                               "%s KV, %d-row prompt (%d audio + %d text), %d greedy steps"
                               % (hp.n_layers, cfg["K"], WNAME[cfg["wtype"]],
                                  "f32" if cfg["kv"] == mtg.TYPE_F32 else "f16", n_prompt,
                                  cfg["blocks"] * AUDIO_ROWS, cfg["text"], n_steps),
                   "verify_rows": cfg["K"], "context_start": ctx_start, "context_end": dec.past_len,
                   "accepted_per_step": st.accepted / max(n_steps, 1),
                   "tokens": tokens, "exec": args.exec, "path": path, "loop": loop},
        "verify_step_us": 1e3 * dev_ms / max(launches, 1),
        "host_step_us": 1e3 * ms_step,
        "step_bytes": bytes_launch,
        "roofline": {"bound": "hbm", "kernel": KERNEL if path == "step" else
                     ("per-op kernels" if path in ("graph", "eager") else KERNEL + " + per-op kernels"),
                     "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS,
                     "traffic": traffic,
                     "launch_us": launch_s * 1e6, "launches": launches,
                     "fallback_steps": fallbacks},
        "source_hash": source_hash(),
    }
    if fallbacks:
        out["roofline"]["flag"] = ("%d timed steps reran on the per-op kernels after a bounded wait ran "
                                   "out; their time includes both launches" % fallbacks)
    if not args.no_cpu:
        try:
            snap = (snap_kv[0], snap_kv[1], ctx_start, st_w.next_seed, ids_w, ids, n_steps, drafter)
            out["cpu_baseline"] = cpu_baseline(model, dec, cfg, snap, args.cpu_seconds)
        except Exception as e:  # the GPU fields stay; the failure is reported in place
            out["cpu_baseline"] = {"value": None, "unit": "tok/s", "error": "%s: %s" % (type(e).__name__, e)}
            log("cpu leg failed: %s" % e)
    if args.copy_probe_mib > 0:
        import torch
        n = args.copy_probe_mib << 18  # float32 elements
        src = torch.ones(n, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["copy_probe_bytes"] = n * 4
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
