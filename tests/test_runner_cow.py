"""The reference's device-runner regression (miniprefix/tests/cow_test.cpp:
138-256) restated on the HIP runner (make_hip_runner).

The runner under test and an oracle runner get the same weights: the tiny
GQA model of cow_test.cpp:118-137 (0.15*sinf weights, embedding row 15 NaN).
The oracle is the reference's own CpuRunner compiled from its sources
(oracle/_ref), and logits must match it bit for bit (the reference asks for
|a-b| < 2e-5 and the same argmax, cow_test.cpp:138-141). Covered:
- fork, copy-on-write of shared tails of 3, 4 and 7 tokens, an append that
  fails on non-finite logits with rollback, and a retry after the source's
  release (device block-table repair) (:142-168);
- partial-page and interior prefix-cache hits, failed appends after a hit,
  and a cache-only tail that becomes exclusive when its lease is evicted
  (:170-202);
- the copy-on-write cost counters, exact bytes included (:203-229);
- publication snapshot churn with evictions and cache clears (:230-256).

The same test body runs on the CPU with the reference build's oracle-KV
runner (the reference KVManager with this repository's C oracle forward) as
the runner under test, which checks the restated assertions themselves."""
import numpy as np
import pytest

from tinyinfer_amd.host import Runner

from .helpers import reference_library, sin_weight_tensors, tiny_config, weights_with

REF = None


def ref():
    global REF
    if REF is None:
        REF = reference_library()
        if REF is None:
            pytest.skip("oracle/_ref not built")
    return REF


@pytest.fixture(params=[pytest.param("hip", marks=pytest.mark.gpu), "reference-oracle-kv"])
def kind(request, tmp_path):
    if request.param == "hip":
        request.getfixturevalue("torch_cuda")
    else:
        ref()
    return request.param


class Setup:
    def __init__(self, kind: str):
        self.cfg = tiny_config()
        tensors = sin_weight_tensors()
        self.kind = kind
        self.oracle_weights = weights_with(tensors, self.cfg, library=ref())
        self.weights = weights_with(tensors, self.cfg, library=None if kind == "hip" else ref())

    def runner(self, block_tokens, max_blocks, cache):
        if self.kind == "hip":
            return Runner(self.weights, context=16, block_tokens=block_tokens, max_blocks=max_blocks,
                          prefix_cache_blocks=cache)
        return Runner(self.weights, context=16, block_tokens=block_tokens, max_blocks=max_blocks,
                      prefix_cache_blocks=cache, kind=1)

    def oracle(self):
        return Runner(self.oracle_weights, context=16, block_tokens=4, max_blocks=8, prefix_cache_blocks=0, kind=0)


def same(got, want):
    assert np.all(np.isfinite(got))
    assert np.array_equal(np.asarray(got).view(np.uint32), np.asarray(want).view(np.uint32)), \
        f"max abs diff {np.max(np.abs(got - want))}"
    assert int(np.argmax(got)) == int(np.argmax(want))


def rejects(f):
    with pytest.raises(Exception):
        f()


def test_fork_cow_rollback_retry(kind):
    s = Setup(kind)
    r, oracle = s.runner(4, 4, 0), s.oracle()
    for length in (3, 4, 7):
        for fail in (False, True):
            assert r.reserve_request("a", 8) == "ready" and r.reserve_request("b", 8) == "ready"
            r.create("a")
            r.create("b")
            oracle.create("ref")
            history = list(range(1, length + 1))
            r.append("a", history)
            r.fork_sequence("a", "b")
            oracle.append("ref", history)
            before = r.stats()
            if fail:
                rejects(lambda: r.append("b", [15, 9] if length == 3 else [15]))
                after = r.stats()
                assert after["forward_tokens"] == before["forward_tokens"]
                assert after["kv_live_blocks"] == before["kv_live_blocks"]
                # The retry after the source's release must repair the device table.
                r.release("a")
            suffix = [9, 8] if length == 3 else [9]
            same(r.append("b", suffix), oracle.append("ref", suffix))
            if not fail:
                oracle.release("ref")
                oracle.create("ref")
                oracle.append("ref", history)
                same(r.append("a", [10]), oracle.append("ref", [10]))
                r.release("a")
            r.release("b")
            oracle.clear()
            st = r.stats()
            assert st["kv_live_blocks"] == 0 and st["block_table_device_bytes"] == 0
    r.clear()
    assert r.stats()["live_sequences"] == 0


def test_partial_cache_hits(kind):
    s = Setup(kind)
    r, oracle = s.runner(4, 8, 8), s.oracle()
    for length in (1, 3, 4, 7, 8):
        history = list(range(1, length + 1))
        r.create("source")
        r.append("source", history)
        r.cache_prefix("source")
        # A cached partial page and an interior prefix of a full page.
        for common in (1, length):
            prompt = history[:common] + [10]
            r.create("target")
            assert r.reuse_prefix("target", prompt) == common
            before = r.stats()
            rejects(lambda: r.append("target", [15]))
            after = r.stats()
            assert after["forward_tokens"] == before["forward_tokens"]
            assert after["kv_live_blocks"] == before["kv_live_blocks"]
            oracle.create("ref")
            same(r.append("target", [10]), oracle.append("ref", prompt))
            r.release("target")
            oracle.clear()
        r.create("identical")
        assert r.reuse_prefix("identical", history) == length - 1
        oracle.create("ref")
        same(r.append("identical", [history[-1]]), oracle.append("ref", history))
        r.clear()
        oracle.clear()
        st = r.stats()
        assert st["kv_live_blocks"] == 0 and st["block_table_device_bytes"] == 0
    # Every page reserved: a tail shared only with the cache becomes exclusive
    # when its lease is evicted, without a replacement page.
    r = s.runner(4, 1, 1)
    r.create("seed")
    r.append("seed", [1, 2, 3])
    r.cache_prefix("seed")
    r.release("seed")
    assert r.reserve_request("next", 4) == "ready"
    r.create("next")
    assert r.reuse_prefix("next", [1, 2, 3, 4]) == 3
    oracle.create("ref")
    same(r.append("next", [4]), oracle.append("ref", [1, 2, 3, 4]))
    st = r.stats()
    assert st["kv_live_blocks"] == 1 and st["kv_cached_blocks"] == 0
    r.release("next")
    assert r.stats()["kv_live_blocks"] == 0


def test_cost_counters(kind):
    s = Setup(kind)
    for timed in (False, True):
        r = s.runner(4, 8, 8)
        r.set_cost_timing(timed)
        r.set_cost_timing(timed)
        r.create("a")
        r.append("a", [1, 2, 3])
        r.cache_prefix("a")
        r.create("b")
        assert r.reuse_prefix("b", [1, 2, 3, 4]) == 3
        r.append("b", [4])
        c = r.cost_stats()
        assert c["lookup_calls"] == 1 and c["publish_calls"] == 1
        # 3 tokens x 4 floats x 2 layers, K and V: 192 bytes.
        assert c["cow_pages"] == 1 and c["cow_bytes"] == 192
        if kind == "hip":
            assert c["cow_timed_copies"] == int(timed)
        if not timed:
            assert c["lookup_ns"] == 0 and c["publish_ns"] == 0 and c["cow_copy_ns"] == 0
        r.create("failed")
        r.fork_sequence("a", "failed")
        rejects(lambda: r.append("failed", [15]))
        c = r.cost_stats()
        # Copied work counts even when the forward fails.
        assert c["cow_pages"] == 2 and c["cow_bytes"] == 384
        if kind == "hip":
            assert c["cow_timed_copies"] == (2 if timed else 0)
        r.clear()
        assert r.cost_stats()["cow_bytes"] == 384 and r.stats()["kv_live_blocks"] == 0
        r.set_cost_timing(False)
        stopped = r.cost_stats()
        r.create("next")
        r.append("next", [1, 2, 3])
        r.cache_prefix("next")
        r.create("copy")
        assert r.reuse_prefix("copy", [1, 2, 3, 4]) == 3
        r.append("copy", [4])
        final = r.cost_stats()
        assert final["cow_bytes"] == 576 and final["cow_pages"] == 3
        for key in ("lookup_ns", "publish_ns", "cow_copy_ns", "cow_timed_copies"):
            assert final[key] == stopped[key]
        r.clear()


def test_publication_snapshot_churn(kind):
    s = Setup(kind)
    r, oracle = s.runner(4, 16, 5), s.oracle()
    for round_ in range(6):
        history = [1 + round_ % 2, 2, 3, 4, 5]
        r.create("source")
        r.append("source", history)
        for token in (6, 7, 8, 9, 10):
            r.cache_prefix("source")
            r.cache_prefix("source")
            r.append("source", [token])
            history.append(token)
        r.cache_prefix("source")
        r.release("source")
        prompt = history + [11]
        r.create("target")
        assert r.reuse_prefix("target", prompt) == len(history)
        before = r.stats()
        rejects(lambda: r.append("target", [15]))
        after = r.stats()
        assert after["kv_live_blocks"] == before["kv_live_blocks"]
        assert after["forward_tokens"] == before["forward_tokens"]
        oracle.create("ref")
        same(r.append("target", [11]), oracle.append("ref", prompt))
        r.cache_prefix("target")
        r.release("target")
        oracle.clear()
        if round_ % 2:
            r.clear_prefix_cache()
            assert r.stats()["kv_live_blocks"] == 0
    assert r.stats()["prefix_evictions"] > 0
    r.clear()
    st = r.stats()
    assert st["live_sequences"] == 0 and st["kv_live_blocks"] == 0 and st["block_table_device_bytes"] == 0
