"""Every measured configuration at full size on the GPU, against fixtures
written from the reference's own MiniPrefix (tests/golden/make_fixtures.py).

Each workload (tinyinfer_amd/workloads.py: configs 2, 3, 4, 5A, 5B) runs
through this repository's Engine with batched steps over the HIP runner in
the fast arithmetic, as bench.py runs it (configs 2 and 4 also in the exact
arithmetic). After every engine step the digest of every resident
sequence's committed page table and the step's token counts must equal the
reference Engine's; the copy-on-write counters must equal its counts at the
end; and the greedy tokens of the fixture's requests must equal the
reference CpuRunner's at every recorded step (config 5A: the first 16
decode steps of one request, the reference's 16,384-token CPU prefill being
the cost; a fixture written with make_fixtures.py --engine-only holds no
token streams, and then only the page tables and counts are checked). The
fixtures also hold each step's top-2 logit margin, which tells how close a
mismatch would have been to a tie."""
import hashlib
from pathlib import Path

import numpy as np
import pytest

from tinyinfer_amd.host import Engine, Runner, Weights
from tinyinfer_amd.workloads import WORKLOADS

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"


def digest(runner, ids):
    h = hashlib.sha1()
    for rid in sorted(ids):
        try:
            blocks, used = runner.sequence(rid)
        except LookupError:
            continue
        h.update(f"{rid}@{used}:{','.join(map(str, blocks))};".encode())
    return h.hexdigest()[:16]


def run_workload(name, kind):
    wl = WORKLOADS[name]()
    weights = Weights.synthetic(wl.config(), seed=wl.weight_seed, stddev=0.02)
    runner = Runner(weights, context=wl.context, kind=kind, **wl.kv_args())
    engine = Engine(runner, **wl.engine_args())
    engine.set_batching(True)
    tokens = {r.id: [] for r in wl.requests}
    digests, stats, live = [], [], set()
    for phase in sorted({r.phase for r in wl.requests}):
        for r in wl.requests:
            if r.phase == phase:
                engine.submit(r.id, r.prompt, max_new_tokens=r.max_new_tokens, eos_token_id=None)
                live.add(r.id)
        while not engine.idle():
            engine.step()
            for e in engine.poll_events():
                assert not e.get("error"), e
                if e.get("token") is not None:
                    tokens[e["id"]].append(e["token"])
                if e.get("finish") is not None:
                    live.discard(e["id"])
            digests.append(digest(runner, live))
            s = engine.last_step_stats()
            stats.append((s["prefix_reused_tokens"], s["prefill_tokens"], s["decode_tokens"]))
    assert not engine.failed()
    costs = runner.cost_stats()
    engine.shutdown()
    return wl, tokens, digests, np.array(stats), costs


CASES = [(name, 2) for name in ("config2", "config3", "config4", "config5b", "config5a")] + \
        [("config2", 0), ("config4", 0)]


@pytest.mark.parametrize("name,kind", CASES, ids=[f"{n}-{'fast' if k == 2 else 'exact'}" for n, k in CASES])
def test_workload_matches_reference(torch_cuda, name, kind):
    """kind 2: the fast arithmetic (bench.py's runner); kind 0: the exact one."""
    path = GOLDEN / f"{name}.npz"
    if name == "config5a" and not path.exists():
        # Its reference run (a 16,384-token prefill on the reference CPU
        # runner) takes hours; tests/golden/make_fixtures.py config5a.
        pytest.skip("config5a fixture not generated")
    assert path.exists(), f"missing fixture {path}"
    fx = np.load(path, allow_pickle=False)
    wl, tokens, digests, stats, costs = run_workload(name, kind)
    assert list(fx["table_hash"]) == digests, "page tables differ from the reference engine's"
    assert np.array_equal(fx["step_stats"], stats)
    assert [costs["cow_pages"], costs["cow_bytes"]] == fx["cow"].tolist()
    for row, want, margins in zip(fx["rows"], fx["tokens"], fx["margins"]):
        rid = wl.requests[int(row)].id
        got = np.array(tokens[rid][: len(want)])
        assert len(got) == len(want)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"{rid}: first differing step {bad[0]} (reference token {want[bad[0]]}, got "
                               f"{got[bad[0]]}, reference top-2 margin {margins[bad[0]]:.3e})")
