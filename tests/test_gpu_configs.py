"""Every measured configuration at full size on the GPU, against fixtures
written from the reference's own MiniPrefix (tests/golden/make_fixtures.py).

Each workload (tinyinfer_amd/workloads.py: configs 2, 3, 4, 5A, 5B) runs
through this repository's Engine with batched steps over the HIP runner in
the fast arithmetic, as bench.py runs it, and in the exact arithmetic. After every engine step the digest of every resident
sequence's committed page table and the step's token counts must equal the
reference Engine's; the copy-on-write counters must equal its counts at the
end; and the greedy tokens of the fixture's requests must equal the
reference CpuRunner's at every recorded step (config 5A: six of its eight
requests, the reference's 16,384-token CPU prefill of each being the cost;
a fixture written with make_fixtures.py --engine-only holds no
token streams, and then only the page tables and counts are checked). The
fixtures also hold each step's top-2 logit margin, which tells how close a
mismatch would have been to a tie.

Logits are checked at full depth too, through the runner's logit keeping
(the batched step otherwise downloads only the argmax): at every recorded
decode step the logit of the reference's greedy token, and at three steps
per request every 96th logit. The fast arithmetic must stay within 1e-3
relative of the reference, taken normwise per step (max |got - want| over
the step's compared logits / max |want|), the exact one must equal it bit
for bit."""
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


class LogitCheck:
    """Compares the kept logits of the fixture's requests with the
    reference's at the recorded steps: the greedy token's logit at every
    step, every sample_stride-th logit at the sample steps."""

    def __init__(self, wl, fx):
        self.row_of = {wl.requests[int(r)].id: i for i, r in enumerate(fx["rows"])}
        self.tokens, self.top, self.samples = fx["tokens"], fx["top"], fx["samples"]
        self.sample_steps = [int(k) for k in fx["sample_steps"]]
        self.stride = int(fx["sample_stride"])
        self.worst = 0.0  # max over steps of max|got - want| / max|want|
        self.differing = 0  # compared values whose bits differ
        self.compared = 0

    def __call__(self, rid, step, logits):
        i = self.row_of.get(rid)
        if i is None or step >= self.tokens.shape[1]:
            return
        want_top = self.top[i, step]
        got_top = logits[self.tokens[i, step]]
        self.worst = max(self.worst, abs(float(got_top) - float(want_top)) / abs(float(want_top)))
        self.differing += int(got_top.view(np.uint32) != want_top.view(np.uint32))
        self.compared += 1
        if step in self.sample_steps:
            want = self.samples[i, self.sample_steps.index(step)]
            got = logits[:: self.stride][: want.size]
            self.worst = max(self.worst, float(np.max(np.abs(got - want)) / np.max(np.abs(want))))
            self.differing += int(np.count_nonzero(got.view(np.uint32) != want.view(np.uint32)))
            self.compared += want.size


def run_workload(name, kind, check=None):
    wl = WORKLOADS[name]()
    weights = Weights.synthetic(wl.config(), seed=wl.weight_seed, stddev=0.02)
    runner = Runner(weights, context=wl.context, kind=kind, **wl.kv_args())
    if check is not None:
        runner.keep_logits(True)
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
                    if check is not None:
                        check(e["id"], len(tokens[e["id"]]), runner.kept_logits(e["id"]))
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


CASES = [(name, kind) for kind in (2, 0) for name in ("config2", "config3", "config4", "config5b", "config5a")]


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
    check = LogitCheck(WORKLOADS[name](), fx) if len(fx["rows"]) else None
    wl, tokens, digests, stats, costs = run_workload(name, kind, check)
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
    if check is not None:
        print(f"{name} {'fast' if kind == 2 else 'exact'}: {len(fx['rows'])} requests, {check.compared} logits "
              f"compared, max relative error {check.worst:.3e}, {check.differing} not bit-identical")
        assert check.compared > 0
        if kind == 0:
            assert check.differing == 0, f"exact logits differ from the reference ({check.worst:.3e})"
        else:
            assert check.worst <= 1e-3, f"fast logits off the reference: {check.worst:.3e}"
