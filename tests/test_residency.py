"""The residency and allocation contract of the reference's device runner,
restated on make_hip_runner and on the backend's workspace.

The reference asserts for every warm decode append of its CUDA runner
(miniprefix/tools/verify_real_model.py:76-81) that:
- kv_uploaded_bytes stays 0 (K/V live in HBM and never cross the bus);
- weight_uploaded_bytes and device_allocations do not change;
- token_uploaded_bytes grows by exactly 4 (the one token id);
- block_table_uploaded_bytes grows by 4 when the new token starts a page and
  by 0 otherwise.
Here the same holds for per-request appends in both arithmetics, over a
decode that crosses from the short-row attention to the split kernels (256
tokens) in the fast one, and per step for batched Engine steps: 4 bytes per
decoded row, 4 per page a step adds, no allocation once the first decode
step has run.

The workspace is grow-only (resources.cpp:13-45, checked by
cuda_resources_test.cpp:17-40): a forward with fewer or as many rows as
before allocates nothing and keeps its size; a larger one grows it once."""
import numpy as np
import pytest

from oracle import Oracle
from tinyinfer_amd.backend import ARITHMETIC_EXACT, ARITHMETIC_FAST, HipBackend
from tinyinfer_amd.host import Engine, Runner, Weights

from .helpers import smollm_config

pytestmark = pytest.mark.gpu

BT = 16


def contract(before, after, tokens, table_entries):
    assert after["kv_uploaded_bytes"] == 0
    assert after["weight_uploaded_bytes"] == before["weight_uploaded_bytes"]
    assert after["device_allocations"] == before["device_allocations"], "a warm decode allocated device memory"
    assert after["token_uploaded_bytes"] - before["token_uploaded_bytes"] == 4 * tokens
    assert after["block_table_uploaded_bytes"] - before["block_table_uploaded_bytes"] == 4 * table_entries


@pytest.mark.parametrize("kind", [0, 2], ids=["exact", "fast"])
def test_warm_decode_append_residency(torch_cuda, kind):
    """37-token prompt, one warm-up decode, then 300 decode appends (to 338
    tokens: pages start at positions 48, 64, ..., 336)."""
    cfg = smollm_config(layers=2, context=1024, vocabulary=4096)
    weights = Weights.synthetic(cfg, seed=71, stddev=0.02)
    runner = Runner(weights, context=1024, block_tokens=BT, max_blocks=64, kind=kind)
    o = Oracle()
    runner.create("r")
    growing = [int(t) for t in o.fill_tokens(37, 71, 9800, cfg["vocabulary"])]
    logits = runner.append("r", growing)
    token = int(np.argmax(logits))
    growing.append(token)
    logits = runner.append("r", [token])  # warm-up decode
    crossings = 0
    for _ in range(300):
        token = int(np.argmax(logits))
        growing.append(token)
        before = runner.stats()
        logits = runner.append("r", [token])
        after = runner.stats()
        new_page = (len(growing) - 1) % BT == 0
        crossings += new_page
        contract(before, after, 1, 1 if new_page else 0)
        assert after["logits_downloaded_bytes"] - before["logits_downloaded_bytes"] == 4 * cfg["vocabulary"]
    assert crossings == 19
    assert runner.sequence("r")[1] == len(growing)
    runner.close()


@pytest.mark.parametrize("kind", [0, 2], ids=["exact", "fast"])
def test_batched_step_residency(torch_cuda, kind):
    """Six requests (prompts of 20 to 300 tokens, 64 new tokens each)
    through batched Engine steps: after the first step that decodes every
    request, each step in which all six decode and none finishes uploads 4
    bytes per decoded row and 4 per page it adds to any table, and
    allocates nothing."""
    cfg = smollm_config(layers=2, context=1024, vocabulary=4096)
    weights = Weights.synthetic(cfg, seed=73, stddev=0.02)
    runner = Runner(weights, context=1024, block_tokens=BT, max_blocks=160, kind=kind)
    engine = Engine(runner, max_batch_size=8, token_budget=2048, prefill_chunk=256, context=1024)
    engine.set_batching(True)
    o = Oracle()
    lengths = [20, 47, 128, 130, 255, 300]
    ids = [f"q{i}" for i in range(len(lengths))]
    for i, (rid, n) in enumerate(zip(ids, lengths)):
        engine.submit(rid, [int(t) for t in o.fill_tokens(n, 73, 9900 + i, cfg["vocabulary"])], max_new_tokens=64,
                      eos_token_id=None)
    warm = False
    checked = 0
    while not engine.idle():
        live = [rid for rid in ids if _has(runner, rid)]
        pages_before = {rid: len(runner.sequence(rid)[0]) for rid in live}
        before = runner.stats()
        engine.step()
        after = runner.stats()
        events = engine.poll_events()
        assert not any(e.get("error") for e in events)
        s = engine.last_step_stats()
        decode_only = s["prefill_tokens"] == 0 and s["decode_tokens"] == len(live) > 0
        finished = any(e.get("finish") is not None for e in events)
        if decode_only and warm and len(live) == len(ids) and not finished:
            added = sum(len(runner.sequence(rid)[0]) - pages_before[rid] for rid in live)
            contract(before, after, s["decode_tokens"], added)
            checked += 1
        warm = warm or decode_only
    assert checked >= 50
    engine.shutdown()


def _has(runner, rid):
    try:
        runner.sequence(rid)
        return True
    except LookupError:
        return False


@pytest.mark.parametrize("arithmetic", [ARITHMETIC_EXACT, ARITHMETIC_FAST], ids=["exact", "fast"])
def test_workspace_grows_only(torch_cuda, arithmetic):
    """Forwards of 2, 1, 2, then 70 rows: the first allocates the workspace,
    the next two allocate nothing and keep its size, the 70-row one (a
    second row tile) grows it once, after which 2 rows allocate nothing."""
    cfg = smollm_config(layers=1, context=512, vocabulary=4096)
    backend = HipBackend(cfg, block_tokens=BT, max_blocks=32, max_sequences=4, arithmetic=arithmetic)
    o = Oracle()
    rng_weights = o.fill_normal(cfg["vocabulary"] * cfg["hidden"], 75, 1, 0.02)
    from tinyinfer_amd.backend import TENSOR_EMBEDDING, TENSOR_FINAL_NORM
    backend.upload(-1, TENSOR_EMBEDDING, rng_weights)
    backend.upload(-1, TENSOR_FINAL_NORM, np.ones(cfg["hidden"], np.float32))
    shapes = [(576,), (576, 576), (576, 192), (576, 192), (576, 576), (576,), (576, 1536), (576, 1536), (1536, 576)]
    for slot, shape in enumerate(shapes):
        data = np.ones(shape, np.float32) if len(shape) == 1 else o.fill_normal(int(np.prod(shape)), 75, 10 + slot, 0.02)
        backend.upload(0, slot, data.reshape(-1))
    backend.table_write(0, 0, np.arange(32, dtype=np.int32))
    tokens = [int(t) for t in o.fill_tokens(80, 75, 2, cfg["vocabulary"])]
    base = backend.stats()
    used = 0

    def forward(n):
        nonlocal used
        backend.forward([(0, used, n)], tokens[used:used + n], want_logits=False)
        used += n
        return backend.stats()

    s2 = forward(2)
    grown = s2["device_allocations"] - base["device_allocations"]
    assert grown > 0 and s2["device_workspace_bytes"] > 0
    for n in (1, 2):
        s = forward(n)
        assert s["device_allocations"] == s2["device_allocations"]
        assert s["device_workspace_bytes"] == s2["device_workspace_bytes"]
    s70 = forward(70)
    assert s70["device_allocations"] > s2["device_allocations"]
    assert s70["device_workspace_bytes"] > s2["device_workspace_bytes"]
    s = forward(2)
    assert s["device_allocations"] == s70["device_allocations"]
    assert s["device_workspace_bytes"] == s70["device_workspace_bytes"]
    assert s["weight_uploaded_bytes"] == base["weight_uploaded_bytes"] and s["kv_uploaded_bytes"] == 0
    backend.close()
