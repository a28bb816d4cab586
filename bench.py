"""FP32 decode throughput of a SmolLM2-135M-shaped model through the
MiniPrefix engine on one MI355X (HIP runner), with the roofline of the
paged attention and of the projections, and the reference CPU path timed on
the host beside it.

Workloads (tinyinfer_amd/workloads.py; one step = one engine step in which
every request decodes one token):
- config3 (default, the headline): 64 requests, prompts uniform in
  [256, 2048], chunked prefill of 256, 128 greedy tokens each, page 16, pool
  1.25x the reserved pages, no prefix cache, EOS disabled;
- config2: 1 request, 128-token prompt, 128 greedy tokens;
- config4: a 1000-token prefix published once, then 32 requests of prefix +
  64 unique tokens with the prefix cache on (copy-on-write of the shared
  8-token tail), 64 greedy tokens each;
- config5a: 8 requests with 16384-token prompts (chunk 512), 256 greedy
  tokens each;
- config5b: 256 requests with 1024-token prompts, 64 greedy tokens each.
Weights are synthetic N(0, 0.02) (RMSNorm weights 1.0), seeded. The runner
computes in the fast arithmetic by default (FP32 matrix cores, flash-decoding
attention; logits within 1e-3 of the reference, greedy tokens checked
against the reference's in the GPU tests); --arithmetic exact selects the
bit-exact one.

Prefill runs first (untimed); `--warmup` pure-decode steps follow, then
exactly `--steps` timed steps between two device synchronisations (`value`).
Each forward call ends with a device synchronisation of its own (the runner
returns argmax results to the host), so host time over the steps is the
whole job's time. The timed window sits early in the decode, where the
contexts are shorter than the decode's mean: `timed_window` states its mean
context against the whole decode's, and `whole_decode` is the rate over
every decode step but the roofline pass (each step timed on the host).

roofline: after the timed window, a pass of up to 30 decode steps has one
layer per step (rotating through the layers) with its attention and its four
projections timed with HIP events on the runner's stream (timing keeps
these steps on direct launches). Attention algorithmic bytes per launch =
sum over sequences of
T*kv_width*4*2 (K and V of every attended token, read once) +
rows*hidden*4*2 (q in, context out). Projection algorithmic bytes per layer
= the layer's weights (q|k|v, o, gate, up, down) + the activations they read
and write; FLOPs per layer = 2*rows*(weights/4); the projections' line
carries both the HBM fraction and the fraction of the FP32 matrix peak. The
one the metric names (attention; the projections at B=1) is `roofline`, the
other `roofline_other`. `traffic` is this run's algorithmic bytes times the
measured/algorithmic ratio of the committed counter record
(profiles/*_traffic.json, written by --summarise-counters from two
rocprofv3 --pmc passes, FETCH_SIZE and WRITE_SIZE, calibrated with the copy
of known size that --traffic-probe runs).

cpu_baseline: the reference CPU runner (the reference's own CpuRunner,
Engine and KVManager compiled from its sources into oracle/_ref) on one
pinned host core, in a process of its own started before the GPU is
touched and run beside the GPU leg on another core: the prefill of a prompt
as long as the workload's mean decode context (capped at 1,300 tokens; the
prefix of the workload's longest prompt, in the workload's prefill chunks),
then single-token decode steps for about --cpu-seconds; prefill and decode
rates are reported separately. Without oracle/_ref the oracle (a C
restatement of the reference CPU path, bit-identical to it) stands in,
labelled "port".
"""
from __future__ import annotations

import argparse
import csv
import gc
import json
import os
import platform
import subprocess
import sys
import time
from collections import defaultdict
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRICS = {
    "config3": "decode tok/s (B=64, SmolLM2-135M-shape FP32); paged-attn HBM GB/s % peak",
    "config2": "decode tok/s (B=1, SmolLM2-135M-shape FP32); projections HBM GB/s % peak",
    "config4": "decode tok/s (32 prefix-sharing requests with COW, SmolLM2-135M-shape FP32); paged-attn HBM GB/s % peak",
    "config5a": "decode tok/s (B=8, 16384-token prompts, SmolLM2-135M-shape FP32); paged-attn HBM GB/s % peak",
    "config5b": "decode tok/s (B=256, 1024-token contexts, SmolLM2-135M-shape FP32); paged-attn HBM GB/s % peak",
}
DEFAULT_STEPS = {"config3": (64, 8), "config2": (64, 8), "config4": (24, 6), "config5a": (96, 8), "config5b": (24, 6)}
ROOFLINE_STEPS = 30  # decode steps of the roofline pass (fewer if the decode ends first)
CPU_CONTEXT_CAP = 1300  # tokens of the CPU baseline's prefill
HBM_PEAK_GBS = 8000.0
FP32_MATRIX_PEAK_TFLOPS = 157.3
PROBE_BYTES = 128 << 20  # --traffic-probe: one copy of 128 MiB (read and written)


def log(msg: str):
    print(msg, file=sys.stderr, flush=True)


def traffic_file(workload: str) -> Path:
    return ROOT / "profiles" / f"decode_{workload}_traffic.json"


def layer_shape(cfg: dict):
    hd, inter = cfg["hidden"], cfg["intermediate"]
    kvw = cfg["kv_heads"] * (hd // cfg["heads"])
    qw = hd + 2 * kvw
    weights = hd * qw + hd * hd + 2 * hd * inter + inter * hd  # floats
    acts = 8 * hd + 2 * kvw + 2 * inter  # floats read or written per row
    return kvw, weights, acts


def gpu_leg(args, wl):
    import torch

    from tinyinfer_amd.backend import TIME_ATTENTION, TIME_HEAD, TIME_PROJECTION, TIME_SAMPLED, kernel_times, set_timing
    from tinyinfer_amd.host import Engine, Runner, Weights

    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU (no HIP device visible)")
    cfg = wl.config()
    t = time.perf_counter()
    weights = Weights.synthetic(cfg, seed=wl.weight_seed, stddev=0.02)
    runner = Runner(weights, context=cfg["context"], kind=2 if args.arithmetic == "fast" else 0, **wl.kv_args())
    device = runner.device()
    engine = Engine(runner, **wl.engine_args())
    engine.set_batching(True)
    log(f"setup {time.perf_counter() - t:.1f}s: {wl.name}, pool {wl.max_blocks} pages, "
        f"prompts sum {sum(len(r.prompt) for r in wl.requests)}")
    # Long-lived objects (torch, numpy, the workload) move out of the cyclic
    # garbage collector's reach: a full collection over them otherwise lands
    # in some timed windows as one ~35 ms pause inside poll_events (the event
    # dicts trigger it), 0.9 ms per step at B=256.
    gc.collect()
    gc.freeze()

    generated = defaultdict(int)
    finished = set()

    def step():
        engine.step()
        for ev in engine.poll_events():
            if ev.get("error"):
                raise RuntimeError(f"request {ev['id']} failed: {ev['error']}")
            if ev.get("token") is not None:
                generated[ev["id"]] += 1
            if ev.get("finish") is not None:
                finished.add(ev["id"])
        if engine.failed():
            raise RuntimeError("engine failed")
        return engine.last_step_stats()

    t = time.perf_counter()
    setup_steps = 0
    phases = sorted({r.phase for r in wl.requests})
    for ph in phases[:-1]:  # earlier phases run to completion (config4's published prefix)
        for r in wl.requests:
            if r.phase == ph:
                engine.submit(r.id, r.prompt, max_new_tokens=r.max_new_tokens, eos_token_id=None)
        while not engine.idle():
            step()
            setup_steps += 1
    active = [r for r in wl.requests if r.phase == phases[-1]]
    for r in active:
        engine.submit(r.id, r.prompt, max_new_tokens=r.max_new_tokens, eos_token_id=None)
    ids = [r.id for r in active]
    prefill_steps = 0
    while min(generated[i] for i in ids) == 0:
        step()
        prefill_steps += 1
        if prefill_steps > 400:
            raise RuntimeError("prefill did not finish")
    log(f"prefill: {setup_steps} + {prefill_steps} steps, {time.perf_counter() - t:.1f}s")
    remaining = min(r.max_new_tokens for r in active) - max(generated[i] for i in ids)
    if args.warmup + args.steps + 2 > remaining:
        raise SystemExit(f"--warmup + --steps must leave every request decoding for two more steps (the roofline "
                         f"pass and the first requests' last token): {remaining} decode steps remain")
    batch = len(ids)
    used0 = {rid: engine.runner.sequence(rid)[1] for rid in ids}  # committed tokens before the first decode step
    clean = []  # (decode step index, host seconds) of the steps outside the roofline pass

    def decode_step(index):
        t = time.perf_counter()
        s = step()
        clean.append((index, time.perf_counter() - t))
        assert s["decode_tokens"] == batch and s["prefill_tokens"] == 0, s

    for i in range(args.warmup):
        decode_step(i)
    if args.cost_timing:
        runner.set_cost_timing(True)
    costs0 = runner.cost_stats()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.warmup, args.warmup + args.steps):
        decode_step(i)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    costs = {k: v - costs0.get(k, 0) for k, v in runner.cost_stats().items()}  # the timed steps
    for rid in ids:
        assert engine.runner.sequence(rid)[1] == used0[rid] + args.warmup + args.steps
    # Roofline pass: one layer per step (rotating) has its attention and
    # projections timed; --all-kernels times every layer and the LM head.
    first_rof = args.warmup + args.steps
    # It ends before the decode step in which the first requests emit their
    # last token (their releases may split that step's batch).
    rof_steps = min(ROOFLINE_STEPS, remaining - 1 - first_rof)
    if rof_steps < 1:
        raise SystemExit(f"--warmup + --steps leave no decode step for the roofline pass ({remaining} remain)")
    classes = TIME_ATTENTION | TIME_PROJECTION | (TIME_HEAD if args.all_kernels else TIME_SAMPLED)
    set_timing(device, classes)
    for _ in range(rof_steps):
        s = step()
        assert s["decode_tokens"] == batch and s["prefill_tokens"] == 0, s
    times = kernel_times(device)
    set_timing(device, 0)
    if args.traffic_probe:
        # A copy of known size for the counter calibration (--summarise-counters).
        src = torch.ones(PROBE_BYTES // 4, dtype=torch.float32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(2):
            dst.copy_(src)
        torch.cuda.synchronize()
    # The rest of the decode, step by step, for the whole-decode rate.
    for i in range(first_rof + rof_steps, remaining):
        decode_step(i)
    engine.shutdown()
    engine.close()

    def attended(first, count):  # attended tokens of every sequence over decode steps first..first+count-1
        return sum(count * u + count * first + count * (count + 1) // 2 for u in used0.values())

    K, R = args.steps, rof_steps
    sum_t = attended(first_rof, R)  # the roofline pass
    kvw, layer_floats, act_floats = layer_shape(cfg)
    timed_layers = cfg["layers"] if args.all_kernels else 1  # per step
    att_launches = times["attention_launches"]
    assert att_launches == R * timed_layers, times
    att_bytes = timed_layers * (sum_t * kvw * 4 * 2) + att_launches * batch * cfg["hidden"] * 4 * 2
    att_s = times["attention_ns"] * 1e-9
    proj_layers = times["projection_launches"] // 4
    assert proj_layers == R * timed_layers, times
    proj_bytes_layer = 4 * (layer_floats + batch * act_floats)
    proj_flops_layer = 2 * batch * layer_floats
    proj_s = times["projection_ns"] * 1e-9
    whole_s = sum(t for _, t in clean)
    whole_ctx = sum(attended(i, 1) for i, _ in clean) / (len(clean) * batch)
    return dict(
        value=batch * K / elapsed, ms_per_step=elapsed / K * 1e3, batch=batch, prefill_steps=setup_steps + prefill_steps,
        mean_context=attended(args.warmup, K) / (K * batch), decode_steps=remaining, roofline_steps=R,
        roofline_context=sum_t / (R * batch), times=times, cow=costs,
        roofline_lengths=(min(used0.values()) + first_rof + 1, max(used0.values()) + first_rof + R),
        whole=dict(value=round(batch * len(clean) / whole_s, 2), steps=len(clean),
                   ms_per_step=round(whole_s / len(clean) * 1e3, 4), mean_context=round(whole_ctx, 1)),
        attention=dict(us=att_s / att_launches * 1e6, bytes=att_bytes / att_launches, gbs=att_bytes / att_s / 1e9),
        projections=dict(us=proj_s / proj_layers * 1e6, bytes=proj_bytes_layer, flops=proj_flops_layer,
                         gbs=proj_bytes_layer * proj_layers / proj_s / 1e9,
                         tflops=proj_flops_layer * proj_layers / proj_s / 1e12))


def host_info():
    model = platform.processor() or ""
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count()
    return dict(host_nproc=os.cpu_count(), host_cpus_available=avail, cpu_model=model)


def cpu_prompt(wl):
    """The CPU baseline's prompt: the prefix of the workload's longest prompt
    as long as the mean context of its decode steps, capped at
    CPU_CONTEXT_CAP tokens."""
    last = max(r.phase for r in wl.requests)
    active = [r for r in wl.requests if r.phase == last]
    mean_context = sum(len(r.prompt) + r.max_new_tokens / 2 for r in active) / len(active)
    longest = max(active, key=lambda r: len(r.prompt)).prompt
    n = min(int(round(mean_context)), CPU_CONTEXT_CAP, len(longest))
    return np.asarray(longest[:n], dtype=np.int32), mean_context


def cpu_leg(args, wl):
    """The reference CPU path on one pinned core: a prompt as long as the
    workload's mean decode context, prefilled in the workload's chunks, then
    single-token decode steps (the reference CPU runner serves one sequence
    per call, so this is its throughput)."""
    from oracle import ref_library

    info = host_info()
    try:
        os.sched_setaffinity(0, {sorted(os.sched_getaffinity(0))[-1]})
    except (AttributeError, OSError):
        pass
    cfg = wl.config()
    prompt, mean_context = cpu_prompt(wl)
    ref = ref_library()
    if ref is None:
        return oracle_cpu_leg(args, wl, cfg, prompt, info)
    from tinyinfer_amd.host import Engine, Runner, Weights

    w = Weights.synthetic(cfg, seed=wl.weight_seed, stddev=0.02, library=ref)
    pages = -(-(len(prompt) + 256) // 16)
    chunk = min(wl.prefill_chunk, len(prompt))
    runner = Runner(w, context=cfg["context"], kind=0, block_tokens=16, max_blocks=pages, prefix_cache_blocks=0)
    engine = Engine(runner, max_batch_size=1, token_budget=chunk, prefill_chunk=chunk, context=cfg["context"])
    engine.submit("cpu", prompt, max_new_tokens=256, eos_token_id=None)
    t = time.perf_counter()
    prefill_steps = -(-len(prompt) // chunk)
    for _ in range(prefill_steps):  # the prompt in the workload's chunks, and its first token
        engine.step()
    prefill_s = time.perf_counter() - t
    decoded, spent = 0, 0.0
    while spent < args.cpu_seconds or decoded < 2:
        t = time.perf_counter()
        engine.step()
        spent += time.perf_counter() - t
        decoded += 1
        if decoded >= 200:
            break
    events = engine.poll_events()
    assert not any(e.get("error") for e in events), events
    engine.shutdown()
    engine.close()
    return dict(value=round(decoded / spent, 3), unit="tok/s", cores=1, kind="reference",
                prefill_tok_s=round(len(prompt) / prefill_s, 2), prefill_s=round(prefill_s, 2),
                sample=f"reference CpuRunner + Engine (oracle/_ref, built from the reference sources), 1 pinned core, "
                       f"beside the GPU leg: prefill of a {len(prompt)}-token prompt of the same workload in "
                       f"{chunk}-token chunks ({prefill_s:.1f}s), then {decoded} single-token decode steps at contexts "
                       f"{len(prompt) + 1}..{len(prompt) + decoded} ({spent:.1f}s); the workload's decode averages "
                       f"{mean_context:.0f} tokens of context", **info)


def oracle_cpu_leg(args, wl, cfg, prompt, info):
    from oracle import OracleModel

    model = OracleModel(cfg, seed=wl.weight_seed, stddev=0.02)
    kvw = cfg["kv_heads"] * (cfg["hidden"] // cfg["heads"])
    pages = -(-(len(prompt) + 256) // 16)
    keys = np.zeros(pages * cfg["layers"] * 16 * kvw, dtype=np.float32)
    values = np.zeros_like(keys)
    table = np.arange(pages, dtype=np.int32)
    t = time.perf_counter()
    logits = model.append(keys, values, 16, table, 0, [int(x) for x in prompt])
    prefill_s = time.perf_counter() - t
    used, decoded, spent = len(prompt), 0, 0.0
    token = int(np.argmax(logits))
    while spent < args.cpu_seconds or decoded < 2:
        t = time.perf_counter()
        logits = model.append(keys, values, 16, table, used, [token])
        spent += time.perf_counter() - t
        used += 1
        decoded += 1
        token = int(np.argmax(logits))
    return dict(value=round(decoded / spent, 3), unit="tok/s", cores=1, kind="port",
                prefill_tok_s=round(len(prompt) / prefill_s, 2), prefill_s=round(prefill_s, 2),
                sample=f"oracle (C restatement of the reference CPU runner, bit-identical to it), 1 pinned core, beside "
                       f"the GPU leg: {len(prompt)}-token prefill ({prefill_s:.1f}s), {decoded} decode steps at contexts "
                       f"{len(prompt) + 1}..{len(prompt) + decoded} ({spent:.1f}s)", **info)


SHORT_ROW_TOKENS = 256  # decode rows of up to this many tokens take the one-work-group attention kernel
GEMV_SEQUENCES = 4  # decode steps of up to this many sequences run their projections as GEMV


def roofline(kind: str, g: dict, rec: dict | None):
    if kind == "attention":
        a = g["attention"]
        ratio = rec.get("attention_ratio") if rec else None
        shortest, longest = g["roofline_lengths"]
        kernels = ("the short-row kernel" if longest <= SHORT_ROW_TOKENS else
                   "split kernel + merge kernel" if shortest > SHORT_ROW_TOKENS else
                   "split kernel + merge kernel, short-row kernel")
        return {"bound": "hbm", "kernel": f"paged attention (one layer: {kernels})",
                "achieved": round(a["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(a["gbs"] / HBM_PEAK_GBS, 4),
                "traffic": int(round(ratio * a["bytes"])) if ratio else None, "traffic_ratio": ratio,
                "algorithmic_bytes_per_launch": int(a["bytes"]), "us_per_launch": round(a["us"], 2),
                "measured_over": f"{g['roofline_steps']} decode steps after the timed window (one layer per step), "
                                 f"mean context {g['roofline_context']:.1f}"}
    p = g["projections"]
    ratio = rec.get("projection_ratio") if rec else None
    gemv = g["batch"] <= GEMV_SEQUENCES
    # GEMV runs on the vector ALUs, whose FP32 peak equals the matrix cores' on this chip.
    flops = {"achieved": round(p["tflops"], 2), "peak": FP32_MATRIX_PEAK_TFLOPS, "unit": "TFLOP/s",
             "frac": round(p["tflops"] / FP32_MATRIX_PEAK_TFLOPS, 4), "flops_per_launch": int(p["flops"])}
    return {"bound": "hbm", "kernel": f"projections (one layer: q|k|v+RoPE, o, gate/up+SwiGLU, down"
                                      f"{'; FP32 GEMV' if gemv else '; FP32 matrix cores'})",
            "achieved": round(p["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(p["gbs"] / HBM_PEAK_GBS, 4),
            "traffic": int(round(ratio * p["bytes"])) if ratio else None, "traffic_ratio": ratio,
            "algorithmic_bytes_per_launch": int(p["bytes"]), "us_per_launch": round(p["us"], 2),
            ("fp32_vector" if gemv else "mfma"): flops}


def decode_dispatches(rows: list, steps: int, path: str) -> range:
    """Dispatch ids of the roofline pass of a rocprofv3 --pmc run of this
    script with --traffic-probe: the last `steps` engine steps before the
    probe's copy of PROBE_BYTES (each step ends with the LM head's argmax
    kernel). Counting by step, not by kernel name or grid, keeps out the
    prefill steps, which run the same instantiations for their one-token
    rows and short chunks, and the probe places the window at the contexts
    whose algorithmic bytes the bench line reports."""
    # (The runtime's copy kernel moves about 1 KiB per work-item: the probe's
    # 128 MiB is a grid of 131,072, a step's metadata upload one of 512.)
    probe = [int(r["Dispatch_Id"]) for r in rows
             if r["Kernel_Name"].startswith("__amd_rocclr_copyBuffer") and int(r["Grid_Size"]) * 1024 >= PROBE_BYTES // 2]
    if not probe:
        raise SystemExit(f"{path}: no probe copy found (run bench.py with --traffic-probe)")
    ends = sorted({int(r["Dispatch_Id"]) for r in rows
                   if "head_argmax_kernel" in r["Kernel_Name"] and int(r["Dispatch_Id"]) < min(probe)})
    if len(ends) < steps + 1:
        raise SystemExit(f"{path}: {len(ends) - 1} complete steps, {steps} asked for")
    return range(ends[-steps - 1] + 1, ends[-1] + 1)


def summarise_counters(fetch_csv: str, write_csv: str, bench_json: str, out: str):
    """Per-launch HBM bytes of the decode attention and projections from two
    rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE; KiB per dispatch) of
    `bench.py --traffic-probe`, each counter scaled by what it reads for the
    probe's copy of known size."""
    line = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
    fast = line["config"].get("arithmetic") == "fast"
    # The decode kernels (prefill runs other instantiations).
    att_kernels = (("fast_attention_kernel<", "fast_attention_merge_kernel", "fast_attention_short_kernel") if fast
                   else ("attn_scores_kernel<16, 64, true>", "attn_decode_kernel<"))
    # The matrix-core projections of B=64 (the residual one twice per layer),
    # or the GEMV ones of steps of up to four sequences (each once).
    proj_kernels = (("fast_gemm_kernel<4, true, false, 1, 1, 12>", "fast_gemm_kernel<1, false, false, 1, 1, 12>",
                     "fast_gemm_kernel<2, true, false, 2, 1, 6>", "gemv_rope_kernel", "gemv_residual_kernel",
                     "gemv_swiglu_kernel") if fast else ("gemm_column",))

    def read(path):
        rows = list(csv.DictReader(open(path)))
        window = decode_dispatches(rows, line["kernel_times_ns"]["attention_launches"], path)
        per = defaultdict(list)  # name -> KiB per decode launch
        probe = []
        for r in rows:
            name = r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
            kib = float(r["Counter_Value"])
            if name.startswith("__amd_rocclr_copyBuffer") and kib * 1024 > PROBE_BYTES / 4:
                probe.append(kib)
            elif int(r["Dispatch_Id"]) in window:
                per[name].append(kib)
        return per, probe

    result = {"workload": line["config"]["workload"], "seed": line["config"]["seed"],
              "arithmetic": line["config"].get("arithmetic"),
              "window": line["roofline" if "attention" in line["roofline"]["kernel"] else "roofline_other"]["measured_over"],
              "steps": line["steps"], "warmup": line["warmup"]}
    for counter, path in (("fetch", fetch_csv), ("write", write_csv)):
        per, probe = read(path)
        if not probe:
            raise SystemExit(f"{path}: no probe copy found (run bench.py with --traffic-probe)")
        factor = float(np.mean(probe)) * 1024 / PROBE_BYTES
        result[f"{counter}_factor"] = round(factor, 6)
        att = {k: float(np.mean(v)) * 1024 / factor for k, v in per.items() if any(a in k for a in att_kernels)}
        proj = {k: float(np.mean(v)) * 1024 / factor for k, v in per.items() if any(p in k for p in proj_kernels)}
        result[f"attention_{counter}_bytes"] = {k: int(v) for k, v in att.items()}
        result[f"projection_{counter}_bytes"] = {k: int(v) for k, v in proj.items()}
    att_total = sum(result["attention_fetch_bytes"].values()) + sum(result["attention_write_bytes"].values())
    # One layer runs the residual projection twice (o and down): its mean counts twice.
    proj_total = sum(v * (2 if "<1, false, false" in k else 1) for k, v in result["projection_fetch_bytes"].items())
    proj_total += sum(v * (2 if "<1, false, false" in k else 1) for k, v in result["projection_write_bytes"].items())
    att_alg = line["roofline" if "attention" in line["roofline"]["kernel"] else "roofline_other"]
    proj_alg = line["roofline" if "projections" in line["roofline"]["kernel"] else "roofline_other"]
    result["attention_bytes_per_launch"] = int(att_total)
    result["attention_algorithmic_bytes"] = att_alg["algorithmic_bytes_per_launch"]
    result["attention_ratio"] = round(att_total / att_alg["algorithmic_bytes_per_launch"], 4)
    result["projection_bytes_per_layer"] = int(proj_total)
    result["projection_algorithmic_bytes"] = proj_alg["algorithmic_bytes_per_launch"]
    result["projection_ratio"] = round(proj_total / proj_alg["algorithmic_bytes_per_launch"], 4)
    Path(out).write_text(json.dumps(result, indent=1) + "\n")
    print(json.dumps(result, indent=1))


def trace_window(trace_csv: str, steps: str):
    """The dispatches of a rocprofv3 --kernel-trace run of bench.py in time
    order over `steps` engine steps (a step ends with the LM head's argmax
    kernel): "N" for the last N steps, "N+F" for N steps from engine step F
    (0-based, prefill steps included). Returns (rows, N, F or None)."""
    first = None
    if "+" in steps:
        steps, first = steps.split("+")
        first = int(first)
    steps = int(steps)
    rows = sorted(csv.DictReader(open(trace_csv)), key=lambda r: int(r["Start_Timestamp"]))
    ends = [i for i, r in enumerate(rows) if "head_argmax_kernel" in r["Kernel_Name"]]
    if first is None:
        if len(ends) < steps + 1:
            raise SystemExit(f"{trace_csv}: {len(ends) - 1} complete steps, {steps} asked for")
        return rows[ends[-steps - 1] + 1:ends[-1] + 1], steps, None
    if first < 1 or len(ends) < first + steps:
        raise SystemExit(f"{trace_csv}: {len(ends)} steps, steps {first}..{first + steps - 1} asked for")
    return rows[ends[first - 1] + 1:ends[first + steps - 1] + 1], steps, first


def summarise_trace(trace_csv: str, steps: str, out: str, command: str):
    """Markdown table of a rocprofv3 --kernel-trace run of bench.py: every
    kernel of `steps` engine steps (a step ends with the LM head's argmax
    kernel: "N" for the last N steps, "N+F" for N steps from engine step F,
    prefill steps included in the count), its launches, average and minimum
    duration and time per step, then the kernels of one layer in launch
    order."""
    window, steps, first = trace_window(trace_csv, steps)
    if first is not None:
        steps_text = f"steps {first}..{first + steps - 1}"
    name = lambda r: r["Kernel_Name"].replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
    dur = lambda r: int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    span = int(window[-1]["End_Timestamp"]) - int(window[0]["Start_Timestamp"])
    busy = sum(dur(r) for r in window)
    per = defaultdict(list)
    for r in window:
        per[(name(r), r["Grid_Size_X"], r["Workgroup_Size_X"])].append(dur(r))
    title = f"last {steps} steps" if first is None else f"{steps} engine {steps_text} (0-based, prefill included)"
    lines = [f"# Kernel trace: {title}", "", f"Command: `{command}`", "",
             f"Trace: {steps} steps in {span / 1e6:.3f} ms on the GPU clock ({span / 1e3 / steps:.1f} us per step "
             f"under the profiler); kernels busy {busy / 1e6:.3f} ms ({busy / 1e3 / steps:.1f} us per step).", "",
             "| kernel | grid (threads) | work-group | launches | avg us | min us | us per step | % of busy |",
             "|---|---|---|---|---|---|---|---|"]
    for (k, grid, wg), v in sorted(per.items(), key=lambda kv: -sum(kv[1])):
        lines.append(f"| `{k}` | {grid} | {wg} | {len(v)} | {np.mean(v) / 1e3:.2f} | {min(v) / 1e3:.2f} | "
                     f"{sum(v) / 1e3 / steps:.2f} | {100 * sum(v) / busy:.1f} |")
    # One layer in launch order: the kernels from one launch of the layer's
    # first projection (q|k|v with RoPE: the GEMV kernel of small steps, the
    # kRope = 4 matrix kernel otherwise) to the next.
    names = [name(r) for r in window]
    starters = [n for n in names if "gemv_rope" in n or "fast_gemm_kernel<4," in n]
    starter = starters[0] if starters else next(n for n in names if "gemm" in n)
    order, layer, instances = defaultdict(list), [], 0
    for r in window:
        if name(r) == starter and layer:
            for i, (k, d) in enumerate(layer):
                order[(i, k)].append(d)
            instances += 1
            layer = []
        if name(r) == starter or layer:
            layer.append((name(r), dur(r)))
    lines += ["", f"One layer in launch order (averages over the {steps} steps' layers):", "",
              "| # | kernel | avg us |", "|---|---|---|"]
    total = 0.0
    for (i, k), v in sorted(order.items()):
        if len(v) * 2 >= instances:
            lines.append(f"| {i} | `{k}` | {np.mean(v) / 1e3:.2f} |")
            total += np.mean(v) / 1e3
    lines += [f"| | sum | {total:.2f} |", ""]
    Path(out).write_text("\n".join(lines))
    print("\n".join(lines))


def summarise_sq(counter_csv: str, trace_csv: str, trace_steps: str, out: str, command: str):
    """Markdown table of a rocprofv3 --pmc run of bench.py with the SQ
    counters SQ_WAVE_CYCLES SQ_BUSY_CYCLES SQ_ACTIVE_INST_VALU SQ_INSTS_VALU
    SQ_INSTS_MFMA SQ_VALU_MFMA_BUSY_CYCLES SQ_INSTS_VALU_MFMA_MOPS_F32
    SQ_WAIT_INST_ANY GRBM_GUI_ACTIVE, for the decode step's kernels. The
    matrix-core utilisation divides a launch's SQ_VALU_MFMA_BUSY_CYCLES
    (summed over SIMDs) by all 1,024 SIMDs over the kernel's average
    duration in a --kernel-trace run of the same workload (`trace_csv`; the
    counter run serialises dispatches, so its own cycle counts include the
    profiler's gaps) at the 2.4 GHz peak engine clock."""
    clean = lambda n: n.replace("(anonymous namespace)::", "").replace("void ", "").split("(")[0]
    decode = ("fast_attention_kernel<", "fast_attention_merge_kernel", "fast_gemm_kernel<4, true, false, 1, 1, 12>",
              "fast_gemm_kernel<1, false, false, 1, 1, 12>", "fast_gemm_kernel<2, true, false, 2, 1, 6>",
              "fast_head_kernel<576, 4>")
    pick = lambda n: next((k for k in decode if k in n), None)
    # The roofline pass's decode steps only (the run has --traffic-probe):
    # prefill steps run the same instantiations on other shapes.
    rows = list(csv.DictReader(open(counter_csv)))
    window = decode_dispatches(rows, ROOFLINE_STEPS, counter_csv)
    per, meta = defaultdict(dict), {}
    for r in rows:
        k = pick(clean(r["Kernel_Name"]))
        d = int(r["Dispatch_Id"])
        if k is None or d not in window:
            continue
        per[d][r["Counter_Name"]] = float(r["Counter_Value"])
        meta[d] = k
    # Durations: every launch of the trace's window.
    durations = defaultdict(list)
    for r in trace_window(trace_csv, trace_steps)[0]:
        k = pick(clean(r["Kernel_Name"]))
        if k:
            durations[k].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    agg, n = defaultdict(lambda: defaultdict(float)), defaultdict(int)
    for d, c in per.items():
        n[meta[d]] += 1
        for k, v in c.items():
            agg[meta[d]][k] += v
    simds, clock = 256 * 4, 2.4e9
    lines = ["# SQ counters of the decode kernels (fast arithmetic)", "", f"Counters: `{command}`", "",
             f"Durations: the --kernel-trace run of the same workload over the same steps, the roofline pass "
             f"(engine steps {trace_steps}: decode_config3_fast_kernels_roofline_pass.md). "
             "Matrix-core utilisation = SQ_VALU_MFMA_BUSY_CYCLES per launch / (1,024 SIMDs x average duration x "
             "2.4 GHz); VALU active and waiting = SQ_ACTIVE_INST_VALU and SQ_WAIT_INST_ANY over SQ_WAVE_CYCLES.", "",
             "| kernel | launches | avg us | MFMA instr per launch | MFMA busy cycles per launch | matrix-core "
             "utilisation % | VALU instr per launch | VALU active % of wave cycles | waiting % of wave cycles |",
             "|---|---|---|---|---|---|---|---|---|"]
    for k in decode:
        if k not in agg:
            continue
        a, c = agg[k], n[k]
        us = float(np.mean(durations[k])) / 1e3 if durations[k] else float("nan")
        busy = a.get("SQ_VALU_MFMA_BUSY_CYCLES", 0) / c
        wave = a.get("SQ_WAVE_CYCLES", 0) / c
        lines.append(f"| `{k}` | {c} | {us:.2f} | {a.get('SQ_INSTS_MFMA', 0) / c:.0f} | {busy:.0f} | "
                     f"{100 * busy / (simds * us * 1e-6 * clock):.1f} | {a.get('SQ_INSTS_VALU', 0) / c:.0f} | "
                     f"{100 * a.get('SQ_ACTIVE_INST_VALU', 0) / c / wave:.1f} | "
                     f"{100 * a.get('SQ_WAIT_INST_ANY', 0) / c / wave:.1f} |")
    Path(out).write_text("\n".join(lines) + "\n")
    print("\n".join(lines))


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(METRICS), default="config3")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--cpu-seconds", type=float, default=8.0, help="decode time of the CPU baseline")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-leg", action="store_true", help=argparse.SUPPRESS)  # the CPU baseline's own process
    ap.add_argument("--all-kernels", action="store_true", help="time every layer and the LM head")
    ap.add_argument("--arithmetic", choices=["fast", "exact"], default="fast")
    ap.add_argument("--traffic-probe", action="store_true", help="run a copy of known size after the timed steps")
    ap.add_argument("--cost-timing", action="store_true",
                    help="time the host prefix-cache lookups/publications and the COW copies of the timed steps")
    ap.add_argument("--summarise-counters", nargs=4, metavar=("FETCH_CSV", "WRITE_CSV", "BENCH_JSON", "OUT"))
    ap.add_argument("--summarise-sq", nargs=5, metavar=("COUNTER_CSV", "TRACE_CSV", "TRACE_STEPS", "OUT", "COMMAND"),
                    help="markdown summary of a rocprofv3 --pmc run of this script with the SQ counters")
    ap.add_argument("--summarise-trace", nargs=4, metavar=("TRACE_CSV", "STEPS", "OUT", "COMMAND"),
                    help="markdown summary of a rocprofv3 --kernel-trace run of this script (STEPS: N, the last N "
                         "engine steps, or N+F, N steps from engine step F)")
    args = ap.parse_args()
    if args.summarise_sq:
        summarise_sq(*args.summarise_sq)
        return
    if args.summarise_trace:
        summarise_trace(*args.summarise_trace)
        return
    if args.summarise_counters:
        summarise_counters(*args.summarise_counters)
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: this library has no multi-GPU path (decode would shard by request, "
              "one engine per GPU); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    from tinyinfer_amd import workloads

    wl = getattr(workloads, args.workload)()
    if args.cpu_leg:
        print(json.dumps(cpu_leg(args, wl)), flush=True)
        return
    steps, warmup = DEFAULT_STEPS[args.workload]
    args.steps = steps if args.steps is None else args.steps
    args.warmup = warmup if args.warmup is None else args.warmup
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")
    # The CPU baseline runs in a process of its own, started before this one
    # touches the GPU, on the last host core; this process keeps the others.
    child = None
    if not args.no_cpu_baseline:
        child = subprocess.Popen([sys.executable, str(Path(__file__).resolve()), "--cpu-leg", "--workload",
                                  args.workload, "--cpu-seconds", str(args.cpu_seconds)],
                                 stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True)
        try:
            cores = sorted(os.sched_getaffinity(0))
            if len(cores) > 1:
                os.sched_setaffinity(0, set(cores[:-1]))
        except (AttributeError, OSError):
            pass
    g = gpu_leg(args, wl)
    cpu = None
    if child is not None:
        out, err = child.communicate(timeout=900)
        if child.returncode != 0:
            raise SystemExit(f"CPU baseline failed ({child.returncode}): {err[-2000:]}")
        cpu = json.loads(out.strip().splitlines()[-1])
    rec = None
    tf = traffic_file(args.workload)
    if tf.exists():
        r = json.loads(tf.read_text())
        if r.get("seed") == wl.weight_seed and r.get("arithmetic") == args.arithmetic:
            rec = r
    # The kernel the metric names: paged attention, except at B=1 where the
    # projections' weight stream dominates the step.
    dominant = "projections" if args.workload == "config2" else "attention"
    other = "projections" if dominant == "attention" else "attention"
    line = {
        "metric": METRICS[args.workload], "value": round(g["value"], 2), "unit": "tok/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(g["ms_per_step"], 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights, seeded uniform prompt ids",
        "config": {"workload": f"{wl.name}: {wl.description}; SmolLM2-135M shape (30 layers, hidden 576, 9/3 heads, "
                               f"head_dim 64, SwiGLU 1536, vocab 49152, tied), page 16",
                   "batch": g["batch"], "page_tokens": 16, "prefill_chunk": wl.prefill_chunk,
                   "token_budget": wl.token_budget, "seed": wl.weight_seed, "arithmetic": args.arithmetic,
                   "mean_context": round(g["mean_context"], 1),
                   "timed_window": f"decode steps {args.warmup + 1}..{args.warmup + args.steps} of "
                                   f"{g['decode_steps']} after prefill ({g['prefill_steps']} prefill steps untimed); "
                                   f"mean context {g['mean_context']:.1f} against {g['whole']['mean_context']:.1f} "
                                   f"over the decode, so the window attends "
                                   f"{g['mean_context'] / g['whole']['mean_context']:.3f}x the decode's mean KV bytes "
                                   f"per step"},
        "whole_decode": {"value": g["whole"]["value"], "unit": "tok/s", "steps": g["whole"]["steps"],
                         "ms_per_step": g["whole"]["ms_per_step"], "mean_context": g["whole"]["mean_context"],
                         "note": f"every decode step but the {g['roofline_steps']} of the roofline pass, each timed "
                                 f"on the host"},
        "roofline": roofline(dominant, g, rec),
        "roofline_other": roofline(other, g, rec),
        "cpu_baseline": cpu,
        "kernel_times_ns": g["times"],
        "cow": g["cow"] if args.cost_timing else {k: g["cow"][k] for k in ("cow_pages", "cow_bytes") if k in g["cow"]},
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
