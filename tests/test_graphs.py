"""Graph replay of fast-arithmetic decode steps (mp_hip_set_graphs) against
direct launches: the same steps on two contexts, one replaying captured
graphs and one launching every kernel, must give bit-identical logits and
tokens at every step.

The steps change what the captured launches read between replays: a row
crosses a 128-token split boundary (three more split items), a row grows
from 250 to more than 256 tokens (it leaves the short-row kernel for the
splits and the merge: the counts the kernels read on the device change
under the same graph), one sequence finishes early (fewer sequences: a new
shape, captured anew), and steps alternate between wanting logits and the
argmax only (another shape). A second test holds replayed steps to the
oracle."""
import numpy as np
import pytest

from oracle import Oracle, OracleModel
from tinyinfer_amd.backend import ARITHMETIC_FAST, HipBackend, graphs_captured, set_graphs

from .helpers import smollm_config, upload_model

pytestmark = pytest.mark.gpu


def test_graph_replay_matches_direct_launches(torch_cuda):
    cfg = smollm_config(layers=2, context=1024, vocabulary=4096)
    model = OracleModel(cfg, seed=83)
    o = Oracle()
    lengths = [100, 250, 300, 370, 700]
    prompts = [[int(t) for t in o.fill_tokens(n, 83, 9950 + i, cfg["vocabulary"])] for i, n in enumerate(lengths)]
    tables = [np.arange(64 * i, 64 * i + 64, dtype=np.int32) for i in range(len(lengths))]

    def run(graphs: bool):
        backend = HipBackend(cfg, block_tokens=16, max_blocks=64 * len(lengths), max_sequences=len(lengths),
                             arithmetic=ARITHMETIC_FAST)
        upload_model(backend, model)
        set_graphs(backend.handle, graphs)
        for i, t in enumerate(tables):
            backend.table_write(i, 0, t)
        am, _ = backend.forward([(i, 0, n) for i, n in enumerate(lengths)], [t for p in prompts for t in p])
        used = list(lengths)
        nxt = [int(a) for a in am]
        live = list(range(len(lengths)))
        outs = []
        for step in range(70):
            if step == 40:
                live = live[:-1]  # the 700-token row stops: four sequences from here on
            want = step % 3 != 2
            am, logits = backend.forward([(i, used[i], 1) for i in live], [nxt[i] for i in live], want_logits=want)
            outs.append((list(am), None if logits is None else logits.copy()))
            for j, i in enumerate(live):
                used[i] += 1
                nxt[i] = int(am[j])
        captured = graphs_captured(backend.handle)
        backend.close()
        return outs, captured

    direct, none = run(False)
    replayed, captured = run(True)
    assert none == 0
    assert captured >= 2, captured  # five sequences with logits, four with logits
    for step, ((am_d, lg_d), (am_g, lg_g)) in enumerate(zip(direct, replayed)):
        assert am_d == am_g, f"step {step}: tokens differ"
        if lg_d is not None:
            assert np.array_equal(lg_d.view(np.uint32), lg_g.view(np.uint32)), f"step {step}: logits differ"


def test_graph_replay_tracks_the_oracle(torch_cuda):
    """Twenty teacher-forced decode steps of three sequences with replay on
    (captured at the second step), each step's logits within 1e-3 relative
    of the oracle."""
    cfg = smollm_config(layers=2, context=512, vocabulary=4096)
    model = OracleModel(cfg, seed=89)
    o = Oracle()
    bt = 16
    lengths = [40, 200, 290]
    prompts = [[int(t) for t in o.fill_tokens(n, 89, 9980 + i, cfg["vocabulary"])] for i, n in enumerate(lengths)]
    tables = [np.arange(32 * i, 32 * i + 32, dtype=np.int32) for i in range(3)]
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=96, max_sequences=3, arithmetic=ARITHMETIC_FAST)
    upload_model(backend, model)
    for i, t in enumerate(tables):
        backend.table_write(i, 0, t)
    n = 96 * cfg["layers"] * bt * 192
    keys, values = np.zeros(n, np.float32), np.zeros(n, np.float32)
    want = [model.append(keys, values, bt, tables[i], 0, prompts[i]) for i in range(3)]
    backend.forward([(i, 0, lengths[i]) for i in range(3)], [t for p in prompts for t in p])
    used = list(lengths)
    for step in range(20):
        nxt = [int(np.argmax(w)) for w in want]
        _, got = backend.forward([(i, used[i], 1) for i in range(3)], nxt)
        want = [model.append(keys, values, bt, tables[i], used[i], [nxt[i]]) for i in range(3)]
        for i in range(3):
            err = float(np.max(np.abs(got[i] - want[i])) / np.max(np.abs(want[i])))
            assert err <= 1e-3, f"step {step} row {i}: relative error {err:.3e}"
            used[i] += 1
    assert graphs_captured(backend.handle) >= 1
    backend.close()
