"""The HIP Engine against the reference Engine, step by step.

Three engines run the same submissions on the same synthetic weights:
- this repository's Engine over the HIP runner with batched steps (the
  path bench.py measures);
- the same with batching off (one ModelRunner::append per request, the
  reference's loop);
- the reference's own Engine and KVManager, compiled from its sources
  (oracle/_ref), over the C oracle forward (bit-identical to the reference
  CpuRunner).
After every step the events (request, token, finish reason, error) and every
live sequence's committed page table must be identical, and at the end the
copy-on-write counters. The prefix cache is on: requests publish and reuse
pages within one step and across steps, partial tails are shared and
copied, and decoding requests copy their republished tail every step
(miniprefix/src/engine/engine.cpp:98, prefix_cache.cpp:147-148).

Two more variants set an EOS token (the token the scenario emits most often
without one, which ends a request early, in a step where others go on),
with the prefix cache on and off: a request that may finish releases
its sequence only once its result is known, and the batched Engine keeps the
appends after it in the same device pass unless they take pages from the
pool or publish into the cache.

A CPU variant runs the reference Engine over the reference CpuRunner against
the oracle-KV runner (tokens and events only), which checks the scenario
itself without a GPU."""
import numpy as np
import pytest

from tinyinfer_amd.host import Engine, Runner, Weights, smollm_config

from .helpers import reference_library

SEED = 31


def scenario(vocabulary: int):
    """(step, id, prompt, max_new_tokens) submissions."""
    rng = np.random.default_rng(SEED)
    base = [int(t) for t in rng.integers(0, vocabulary, 80)]
    other = [int(t) for t in rng.integers(0, vocabulary, 40)]
    return [
        # seed decodes twice; the followers map its pages in the steps that publish them
        (0, "seed", base[:37], 2),
        (0, "follower", base[:37] + other[:6], 3),      # 37 cached tokens: 2 pages + a 5-token tail
        (0, "interior", base[:20] + other[6:10], 4),    # interior of the seed's second page
        (1, "late", base[:45], 5),                       # the seed's history after its decode
        (2, "fresh", other[10:40], 6),
        (3, "turn2", base[:37] + other[:6] + [7, 8], 3),
        (4, "aligned", base[:32], 2),                    # whole-page prompt: its last token is recomputed
    ]


def transcript(engine: Engine, runner: Runner | None, submits, steps: int = 40, eos: int | None = None):
    out, live = [], set()
    pending = sorted(submits, key=lambda s: s[0])
    for step in range(steps):
        while pending and pending[0][0] <= step:
            _, rid, prompt, n = pending.pop(0)
            engine.submit(rid, prompt, max_new_tokens=n, eos_token_id=eos)
            live.add(rid)
        engine.step()
        events = engine.poll_events()
        for e in events:
            if e.get("finish") is not None:
                live.discard(e["id"])
        tables = {}
        if runner is not None:
            for rid in sorted(live):
                try:
                    tables[rid] = runner.sequence(rid)
                except LookupError:
                    pass  # admitted but not resident yet
        out.append((step, engine.last_step_stats(), events, tables))
        if not pending and engine.idle():
            break
    assert engine.idle() and not engine.failed()
    return out


CONFIG = dict(smollm_config(layers=2, context=512))
KV = dict(block_tokens=16, max_blocks=96, prefix_cache_blocks=48)
ENGINE = dict(max_batch_size=4, token_budget=96, prefill_chunk=24, context=512)
# (prefix cache pages, EOS from the scenario's own tokens)
VARIANTS = {"cache": (48, False), "cache_eos": (48, True), "no_cache_eos": (0, True)}


def frequent_token(t) -> int:
    """The token the transcript's events carry most often (ties: smallest)."""
    counts = {}
    for _, _, events, _ in t:
        for e in events:
            if e.get("token") is not None:
                counts[e["token"]] = counts.get(e["token"], 0) + 1
    return min(counts, key=lambda k: (-counts[k], k))


def reference_run(kind: int, variant: str = "cache"):
    """The reference Engine's transcript and COW counters, and the EOS token
    the variant uses (None for none)."""
    ref = reference_library()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    cache, with_eos = VARIANTS[variant]
    eos = None
    if with_eos:
        base, _, _ = reference_run(kind, "cache")
        eos = frequent_token(base)
    w = Weights.synthetic(CONFIG, seed=SEED, stddev=0.02, library=ref)
    runner = Runner(w, context=512, kind=kind, **dict(KV, prefix_cache_blocks=cache))
    engine = Engine(runner, **ENGINE)
    t = transcript(engine, runner if kind == 1 else None, scenario(CONFIG["vocabulary"]), eos=eos)
    costs = runner.cost_stats()
    engine.shutdown()
    return t, costs, eos


def strip_tables(t):
    return [(s, st, ev) for s, st, ev, _ in t]


def test_scenario_on_reference_runners():
    """CPU: the reference Engine over the reference CpuRunner and over the
    oracle-KV runner emit the same events (the oracle forward is the
    reference's arithmetic)."""
    cpu, _, _ = reference_run(0)
    okv, costs, _ = reference_run(1)
    assert strip_tables(cpu) == strip_tables(okv)
    assert costs["cow_pages"] > 0  # the scenario exercises copy-on-write


@pytest.mark.gpu
@pytest.mark.parametrize("variant", sorted(VARIANTS))
@pytest.mark.parametrize("kind", [0, 2], ids=["exact", "fast"])
@pytest.mark.parametrize("batching", [True, False])
def test_hip_engine_matches_reference_engine(torch_cuda, batching, kind, variant):
    """Exact arithmetic (kind 0) and fast arithmetic (kind 2) alike: the same
    events, tokens and page tables as the reference engine at every step."""
    want, want_costs, eos = reference_run(1, variant)
    if eos is not None:
        # The EOS token ends some requests early: the variant tests what it says.
        assert any(e.get("finish") == "eos" for _, _, events, _ in want for e in events), eos
    w = Weights.synthetic(CONFIG, seed=SEED, stddev=0.02)
    runner = Runner(w, context=512, kind=kind, **dict(KV, prefix_cache_blocks=VARIANTS[variant][0]))
    engine = Engine(runner, **ENGINE)
    engine.set_batching(batching)
    got = transcript(engine, runner, scenario(CONFIG["vocabulary"]), eos=eos)
    costs = runner.cost_stats()
    engine.shutdown()
    for g, r in zip(got, want):
        assert g == r, f"step {r[0]} differs:\nHIP       {g}\nreference {r}"
    assert len(got) == len(want)
    assert costs["cow_pages"] == want_costs["cow_pages"] and costs["cow_bytes"] == want_costs["cow_bytes"]


def test_undelivered_events_stay_with_their_engine():
    """CPU: events that did not fit the caller's buffer wait in their own
    engine; polling another engine in between neither returns nor drops
    them (two engines in one process, the reference CpuRunner)."""
    import ctypes

    ref = reference_library()
    if ref is None:
        pytest.skip("oracle/_ref not built")
    cfg = dict(smollm_config(layers=1, context=128))
    engines = []
    for rid in ("a", "b"):
        w = Weights.synthetic(cfg, seed=SEED, stddev=0.02, library=ref)
        runner = Runner(w, context=128, block_tokens=16, max_blocks=16)
        engine = Engine(runner, max_batch_size=1, token_budget=32, prefill_chunk=32, context=128)
        engine.submit(rid, [1, 2, 3, 4], max_new_tokens=1, eos_token_id=None)
        engine.step()
        engines.append((engine, runner, w))
    a, b = engines[0][0], engines[1][0]
    needed = ctypes.c_size_t()
    tiny = ctypes.create_string_buffer(4)
    assert a.lib.mpx_engine_poll(a.handle, tiny, len(tiny), ctypes.byref(needed)) == 0
    assert needed.value >= len(tiny)  # a's events did not fit: still pending in a
    got_b = b.poll_events()
    assert [e["id"] for e in got_b] == ["b"] and got_b[0]["finish"] is not None
    got_a = a.poll_events()
    assert [e["id"] for e in got_a] == ["a"] and got_a[0]["token"] == got_b[0]["token"]
    assert a.poll_events() == [] and b.poll_events() == []
    for engine, _, _ in engines:
        engine.shutdown()
