"""Writes the golden fixtures of the measured configurations (configs 2-5,
tinyinfer_amd/workloads.py) from the reference's own MiniPrefix, compiled
from its sources into oracle/_ref/libmp_ref.so (make -C oracle ref). Run in
the container that holds the reference tree; the fixtures are committed and
the GPU tests read only them.

Per configuration, tests/golden/<config>.npz holds:
- tokens [R, S], margins [R, S], top [R, S]: for selected requests, the
  greedy token, its logit, and the gap to the best other logit at every
  decode step, from the reference CpuRunner (make_cpu_runner) driven like
  the Engine drives it (prefill, then one token per step; per-row results
  do not depend on chunking or batching in the reference arithmetic);
- sample_steps [K], samples [R, K, 512]: every 96th logit at K steps;
- table_hash [T], step_stats [T, 3]: after every engine step, a hash of every
  resident sequence's committed page table (sorted by id) and the step's
  (reused, prefill, decode) token counts, from the reference Engine and
  KVManager running the whole workload. Block ids depend on token counts,
  pool and cache settings, and on token values only through prefix-cache
  matches, which no generated token reaches in these workloads (config 4's
  suffixes differ at their first token); so the engine run uses a one-layer
  stand-in model of the same vocabulary, and its ids are valid for the
  30-layer model;
- cow [2]: copy-on-write pages and bytes of that run, scaled to the real
  model's bytes per token.
With --engine-only there are no token streams (R = 0): the page tables, token
counts and COW counts alone, for a workload whose reference CPU prefill takes
too long (config 5A's 16,384-token prompts).

Usage: python tests/golden/make_fixtures.py [config ...] [--jobs N] [--engine-only]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import multiprocessing as mp
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import ref_library  # noqa: E402
from tinyinfer_amd.host import Engine, Runner, Weights  # noqa: E402
from tinyinfer_amd.workloads import WORKLOADS, model_config  # noqa: E402

OUT = Path(__file__).resolve().parent
SAMPLE_STRIDE = 96
STAND_IN = dict(layers=1, hidden=8, intermediate=8, heads=2, kv_heads=1, eos=0, rms_epsilon=1e-5,
                rope_theta=100000.0, tied=1)


def rows_of(name: str, wl):
    """Requests whose token streams the fixture records."""
    if name == "config4":
        return list(range(1, len(wl.requests)))  # every follower
    if name == "config5a":
        # Each request's 16,384-token reference CPU prefill takes about 7
        # hours on one core: six of the eight, one per job.
        return list(range(6))
    return list(range(len(wl.requests)))  # every request


def decode_steps(name: str, wl, index: int) -> int:
    return wl.requests[index].max_new_tokens


def sample_steps(steps: int):
    return sorted({0, steps // 2, steps - 1})


def margin(logits: np.ndarray):
    best = int(np.argmax(logits))
    top = float(logits[best])
    rest = np.delete(logits, best)
    return best, top, top - float(np.max(rest))


def stream_job(args):
    """Greedy stream of workload request `index` on the reference CpuRunner."""
    name, indices = args
    wl = WORKLOADS[name]()
    ref = ref_library()
    cfg = model_config(wl.context)
    weights = Weights.synthetic(cfg, seed=wl.weight_seed, stddev=0.02, library=ref)
    shared = name == "config4"
    # Pages for one request at a time (plus the shared prefix): the CPU
    # runner allocates its whole pool up front.
    longest = max(len(wl.requests[i].prompt) + decode_steps(name, wl, i) for i in indices)
    blocks = -(-longest // 16) + (64 if shared else 0) + 8
    runner = Runner(weights, context=wl.context, block_tokens=16, max_blocks=blocks,
                    prefix_cache_blocks=64 if shared else 0, kind=0)
    results = {}
    if shared:  # the 1000-token prefix, prefilled once and published
        prefix = wl.requests[0].prompt
        runner.create("prefix")
        runner.append("prefix", prefix)
        runner.cache_prefix("prefix")
    for index in indices:
        req = wl.requests[index]
        steps = decode_steps(name, wl, index)
        t0 = time.time()
        runner.create(req.id)
        start = runner.reuse_prefix(req.id, req.prompt) if shared else 0
        chunk = 2048
        logits = None
        for at in range(start, len(req.prompt), chunk):
            logits = runner.append(req.id, req.prompt[at:at + chunk])
        tokens, tops, margins, samples = [], [], [], []
        marks = sample_steps(steps)
        for step in range(steps):
            token, top, gap = margin(logits)
            tokens.append(token)
            tops.append(top)
            margins.append(gap)
            if step in marks:
                samples.append(logits[::SAMPLE_STRIDE].copy())
            if step + 1 < steps:
                logits = runner.append(req.id, [token])
        runner.release(req.id)
        results[index] = (tokens, tops, margins, samples)
        print(f"{name} request {index} ({len(req.prompt)} prompt tokens): {steps} tokens in "
              f"{time.time() - t0:.1f}s, min margin {min(margins):.3e}", flush=True)
    return results


def table_digest(runner: Runner, ids) -> str:
    h = hashlib.sha1()
    for rid in sorted(ids):
        try:
            blocks, used = runner.sequence(rid)
        except LookupError:
            continue
        h.update(f"{rid}@{used}:{','.join(map(str, blocks))};".encode())
    return h.hexdigest()[:16]


def engine_trace(name: str):
    """Per-step page-table digests of the whole workload on the reference
    Engine + KVManager (oracle-KV runner, one-layer stand-in model)."""
    wl = WORKLOADS[name]()
    ref = ref_library()
    cfg = dict(STAND_IN, vocabulary=wl.config()["vocabulary"], context=wl.context)
    weights = Weights.synthetic(cfg, seed=1, stddev=0.02, library=ref)
    runner = Runner(weights, context=wl.context, kind=1, **wl.kv_args())
    engine = Engine(runner, **wl.engine_args())
    digests, stats = [], []
    live = set()
    phases = sorted({r.phase for r in wl.requests})
    for phase in phases:
        for r in wl.requests:
            if r.phase == phase:
                engine.submit(r.id, r.prompt, max_new_tokens=r.max_new_tokens, eos_token_id=None)
                live.add(r.id)
        while not engine.idle():
            engine.step()
            for e in engine.poll_events():
                if e.get("error"):
                    raise RuntimeError(f"{name}: {e}")
                if e.get("finish") is not None:
                    live.discard(e["id"])
            digests.append(table_digest(runner, live))
            s = engine.last_step_stats()
            stats.append((s["prefix_reused_tokens"], s["prefill_tokens"], s["decode_tokens"]))
    cost = runner.cost_stats()
    engine.shutdown()
    # The stand-in's copy bytes are per float of its KV width and layers; the
    # copied tokens are the same.
    stand_in_bytes_per_token = 2 * 4 * (cfg["kv_heads"] * cfg["hidden"] // cfg["heads"]) * cfg["layers"]
    model = wl.config()
    real_bytes_per_token = 2 * 4 * (model["kv_heads"] * model["hidden"] // model["heads"]) * model["layers"]
    cow_bytes = cost["cow_bytes"] // stand_in_bytes_per_token * real_bytes_per_token
    return digests, np.array(stats, dtype=np.int64), np.array([cost["cow_pages"], cow_bytes], dtype=np.int64)


def generate(name: str, jobs: int, engine_only: bool = False):
    wl = WORKLOADS[name]()
    rows = [] if engine_only else rows_of(name, wl)
    t0 = time.time()
    digests, stats, cow = engine_trace(name)
    print(f"{name}: engine trace of {len(digests)} steps in {time.time() - t0:.1f}s, cow {cow.tolist()}", flush=True)
    merged = {}
    groups = [rows[i::jobs] for i in range(jobs) if rows[i::jobs]]
    if groups:
        with mp.get_context("spawn").Pool(len(groups)) as pool:
            parts = pool.map(stream_job, [(name, g) for g in groups])
        for p in parts:
            merged.update(p)
    steps = decode_steps(name, wl, rows[0]) if rows else 0
    np.savez_compressed(
        OUT / f"{name}.npz",
        rows=np.array(rows, dtype=np.int32),
        tokens=np.array([merged[r][0] for r in rows], dtype=np.int32).reshape(len(rows), steps),
        top=np.array([merged[r][1] for r in rows], dtype=np.float32).reshape(len(rows), steps),
        margins=np.array([merged[r][2] for r in rows], dtype=np.float32).reshape(len(rows), steps),
        sample_steps=np.array(sample_steps(steps) if steps else [], dtype=np.int32),
        samples=np.array([merged[r][3] for r in rows], dtype=np.float32),
        sample_stride=np.int32(SAMPLE_STRIDE),
        table_hash=np.array(digests),
        step_stats=stats,
        cow=cow,
        meta=np.array(json.dumps({"workload": name, "description": wl.description,
                                  "reference": "miniprefix CpuRunner + Engine compiled from its sources",
                                  "decode_steps": steps,
                                  "token_streams": "none: engine trace only" if engine_only else "rows"})))
    print(f"{name}: wrote {OUT / (name + '.npz')} in {time.time() - t0:.1f}s", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("configs", nargs="*", default=["config2", "config3", "config4", "config5b", "config5a"])
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--engine-only", action="store_true",
                    help="page tables, token counts and COW counts of the reference Engine only, no token streams "
                         "(config5a's reference CPU prefill of a 16,384-token prompt takes many hours)")
    args = ap.parse_args()
    if ref_library() is None:
        raise SystemExit("oracle/_ref/libmp_ref.so is not built (make -C oracle ref, with the reference tree)")
    for name in args.configs:
        generate(name, args.jobs, args.engine_only)


if __name__ == "__main__":
    main()
