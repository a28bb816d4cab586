"""Batch-64 FP32 decode throughput of a SmolLM2-135M-shaped model through the
MiniPrefix engine on one MI355X (HIP runner), with the paged-attention
roofline and the CPU baseline.

Workload (one step = one engine step in which all 64 requests decode one
token): 64 requests, prompt lengths uniform in [256, 2048], token ids uniform
in [0, 49152), chunked prefill of 256, greedy decode, page 16, physical pool
ceil(1.25 * sum ceil((p + 127) / 16)) pages, no prefix cache, EOS disabled.
Weights are synthetic N(0, 0.02) (RMSNorm weights 1.0), seeded.

Prefill runs first (untimed); `--warmup` pure-decode steps follow, then
exactly `--steps` timed steps between two device synchronisations. Each
forward call ends with a device synchronisation of its own (the runner
returns argmax results to the host), so host time over the steps is the
whole job's time.

roofline: the dominant kernel is paged attention (score, softmax and value
kernels of one layer = one launch), timed live with HIP events over the
timed steps: one layer per step (rotating through the layers), the events
carried by the kernel dispatches on the runner's stream, so the timing adds
nothing between kernels. Algorithmic bytes per launch =
sum over sequences of T*kv_width*4*2 (K and V of every attended token, read
once) + rows*hidden*4*2 (q in, context out). `traffic` is this run's
algorithmic bytes times the measured/algorithmic ratio recorded in
profiles/attention_b64_decode_traffic.json (two rocprofv3 --pmc passes,
FETCH_SIZE and WRITE_SIZE, calibrated with a copy of known size).

cpu_baseline: the oracle (a C restatement of the reference CPU path,
bit-identical to it) on one host core, decoding single tokens at contexts
drawn from the same prompt distribution, for about --cpu-seconds.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s (B=64, SmolLM2-135M-shape FP32); paged-attn HBM GB/s % peak"
HBM_PEAK_GBS = 8000.0
BATCH, PAGE, CHUNK, BUDGET, MAX_NEW = 64, 16, 256, 8192, 128
PROMPT_MIN, PROMPT_MAX = 256, 2048
TRAFFIC_FILE = ROOT / "profiles" / "attention_b64_decode_traffic.json"


def model_config() -> dict:
    return dict(layers=30, hidden=576, intermediate=1536, heads=9, kv_heads=3, vocabulary=49152, context=4096,
                eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)


def workload(seed: int):
    rng = np.random.default_rng(seed)
    lengths = rng.integers(PROMPT_MIN, PROMPT_MAX + 1, size=BATCH)
    prompts = [rng.integers(0, 49152, size=int(p), dtype=np.int64).astype(np.int32) for p in lengths]
    pages = sum(-(-(int(p) + MAX_NEW - 1) // PAGE) for p in lengths)
    return prompts, int(math.ceil(1.25 * pages))


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def gpu_leg(args):
    import torch

    from tinyinfer_amd.backend import TIME_ATTENTION, TIME_HEAD, TIME_PROJECTION, TIME_SAMPLED, kernel_times, set_timing
    from tinyinfer_amd.host import Engine, Runner, Weights

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (no HIP device visible)")
    cfg = model_config()
    prompts, max_blocks = workload(args.seed)
    t = time.perf_counter()
    weights = Weights.synthetic(cfg, seed=args.seed, stddev=0.02)
    runner = Runner(weights, context=cfg["context"], block_tokens=PAGE, max_blocks=max_blocks,
                    prefix_cache_blocks=0, kind=2 if args.arithmetic == "fast" else 0)
    device = runner.device()
    engine = Engine(runner, max_batch_size=BATCH, token_budget=BUDGET, prefill_chunk=CHUNK, context=cfg["context"])
    engine.set_batching(True)
    ids = [f"r{i}" for i in range(BATCH)]
    for rid, p in zip(ids, prompts):
        engine.submit(rid, p, max_new_tokens=MAX_NEW, eos_token_id=None)
    log(f"setup {time.perf_counter() - t:.1f}s: pool {max_blocks} pages, prompts sum {sum(map(len, prompts))}")

    generated = {rid: 0 for rid in ids}

    def step():
        engine.step()
        for ev in engine.poll_events():
            if ev.get("error"):
                raise RuntimeError(f"request {ev['id']} failed: {ev['error']}")
            if ev.get("token") is not None:
                generated[ev["id"]] += 1
        if engine.failed():
            raise RuntimeError("engine failed")
        return engine.last_step_stats()

    t = time.perf_counter()
    prefill_steps = 0
    while min(generated.values()) == 0:
        step()
        prefill_steps += 1
        if prefill_steps > 200:
            raise RuntimeError("prefill did not finish")
    log(f"prefill: {prefill_steps} steps, {time.perf_counter() - t:.1f}s")
    if max(generated.values()) + args.warmup + args.steps > MAX_NEW:
        raise SystemExit(f"--warmup + --steps must leave every request decoding: at most "
                         f"{MAX_NEW - max(generated.values())} steps remain")
    for _ in range(args.warmup):
        s = step()
        assert s["decode_tokens"] == BATCH and s["prefill_tokens"] == 0, s
    used = {rid: engine.runner.sequence(rid)[1] for rid in ids}
    # Attention is timed on one layer per step (rotating through the layers,
    # events carried by the kernel dispatches) so that timing costs the
    # measured throughput nothing; --all-kernels times every launch.
    set_timing(device, TIME_ATTENTION | (TIME_PROJECTION | TIME_HEAD if args.all_kernels else TIME_SAMPLED))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        s = step()
        assert s["decode_tokens"] == BATCH and s["prefill_tokens"] == 0, s
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    times = kernel_times(device)
    for rid in ids:
        assert engine.runner.sequence(rid)[1] == used[rid] + args.steps
    K = args.steps
    sum_t = sum(K * u + K * (K + 1) // 2 for u in used.values())  # attended tokens over the timed steps
    kv_width = cfg["kv_heads"] * (cfg["hidden"] // cfg["heads"])
    launches = times["attention_launches"]
    timed_layers = cfg["layers"] if args.all_kernels else 1  # per step
    assert launches == K * timed_layers, times
    att_bytes = timed_layers * (sum_t * kv_width * 4 * 2) + launches * BATCH * cfg["hidden"] * 4 * 2
    att_s = times["attention_ns"] * 1e-9
    achieved = att_bytes / att_s / 1e9
    mean_context = sum_t / (K * BATCH)
    result = dict(
        value=BATCH * K / elapsed, ms_per_step=elapsed / K * 1e3, prefill_steps=prefill_steps,
        mean_context=mean_context, attention_us_per_launch=att_s / launches * 1e6,
        attention_bytes_per_launch=att_bytes / launches, achieved=achieved, times=times)
    engine.shutdown()
    engine.close()
    return result


def cpu_leg(args):
    """Oracle decode tokens on one core (single requests, as the reference CPU
    runner serves them)."""
    from oracle import OracleModel

    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[0]})
    except (AttributeError, OSError):
        pass
    cfg = model_config()
    model = OracleModel(cfg, seed=args.seed, stddev=0.02)
    rng = np.random.default_rng(args.seed + 1)
    kv_width = cfg["kv_heads"] * (cfg["hidden"] // cfg["heads"])
    pages = -(-(PROMPT_MAX + MAX_NEW) // PAGE)
    floats = pages * cfg["layers"] * PAGE * kv_width
    keys = rng.standard_normal(floats, dtype=np.float32)
    values = rng.standard_normal(floats, dtype=np.float32)
    table = np.arange(pages, dtype=np.int32)
    tokens, contexts, spent = 0, [], 0.0
    while spent < args.cpu_seconds or tokens < 2:
        used = int(rng.integers(PROMPT_MIN, PROMPT_MAX + 1)) + MAX_NEW // 2
        token = int(rng.integers(0, cfg["vocabulary"]))
        t = time.perf_counter()
        model.append(keys, values, PAGE, table, used, [token])
        spent += time.perf_counter() - t
        tokens += 1
        contexts.append(used + 1)
    return dict(value=tokens / spent, unit="tok/s", cores=1, kind="port",
                sample=f"{tokens} single-request decode tokens of the same model at contexts "
                       f"{min(contexts)}..{max(contexts)} (mean {np.mean(contexts):.0f}; prompt U[256,2048] + 64), "
                       f"{spent:.1f}s on 1 host core (oracle: C restatement of the reference CPU runner, "
                       f"bit-identical to it)")


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--seed", type=int, default=20250)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--all-kernels", action="store_true", help="also time projections and the LM head")
    ap.add_argument("--arithmetic", choices=["fast", "exact"], default="fast")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (decode would shard by request, "
              "one engine per GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")
    g = gpu_leg(args)
    cpu = None if args.no_cpu_baseline else cpu_leg(args)
    # HBM bytes per attention launch: the counter-measured bytes / algorithmic
    # bytes ratio of the committed two-pass FETCH_SIZE/WRITE_SIZE record (same
    # workload and seed, fewer steps), applied to this run's algorithmic bytes.
    traffic, traffic_ratio = None, None
    if TRAFFIC_FILE.exists():
        rec = json.loads(TRAFFIC_FILE.read_text())
        if rec.get("seed") == args.seed and rec.get("traffic_ratio"):
            traffic_ratio = rec["traffic_ratio"]
            traffic = int(round(traffic_ratio * g["attention_bytes_per_launch"]))
    frac = g["achieved"] / HBM_PEAK_GBS
    line = {
        "metric": METRIC, "value": round(g["value"], 2), "unit": "tok/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(g["ms_per_step"], 4), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights, seeded uniform prompt ids",
        "config": {"workload": "B=64 batched greedy decode, SmolLM2-135M shape (30 layers, hidden 576, "
                               "9/3 heads, head_dim 64, SwiGLU 1536, vocab 49152, tied), prompts U[256,2048], "
                               "prefill chunk 256, page 16, pool 1.25x",
                   "batch": BATCH, "page_tokens": PAGE, "prefill_chunk": CHUNK, "token_budget": BUDGET,
                   "seed": args.seed, "mean_context": round(g["mean_context"], 1)},
        "roofline": {"bound": "hbm", "kernel": "paged attention (score+softmax+value kernels, one layer)",
                     "achieved": round(g["achieved"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(frac, 4), "traffic": traffic, "traffic_ratio": traffic_ratio,
                     "algorithmic_bytes_per_launch": int(g["attention_bytes_per_launch"]),
                     "us_per_launch": round(g["attention_us_per_launch"], 2)},
        "cpu_baseline": cpu,
        "kernel_times_ns": g["times"],
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
