"""The CPU oracle, pinned before it is trusted:
- bit-identical to the reference CpuRunner compiled from its own sources
  (oracle/_ref, built where /root/reference exists);
- closed forms and double-precision brute force for attention, RMSNorm,
  RoPE and SwiGLU;
- the synthetic-weight generator equals the product's;
- the device expf algorithm, emulated here in double precision, equals the
  oracle's expf (the C library's) on edge cases and a dense sample."""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest

from oracle import Oracle, OracleModel, ref_library
from oracle.oracle import REF_LIBRARY
from tinyinfer_amd import host

from .helpers import smollm_config, tiny_config

# The reference build is loaded only by the tests that use it, so a run that
# selects none of them (the GPU suite) never maps it.
needs_ref = pytest.mark.skipif(not REF_LIBRARY.exists(), reason="oracle/_ref not built (reference tree absent)")


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- closed forms
def test_attention_closed_form_and_causal_bound():
    """Keys {-1000,-999,1000,999,1001} against an all-ones query (the pattern of
    the reference's tests/paged_attention_test.cpp:44-68), values t + d/10,
    and NaN poison beyond the causal length."""
    o = Oracle()
    dim, bt = 16, 2
    keys = np.full((6, 1, bt, dim), np.nan, dtype=np.float32)  # 6 pages, 1 layer
    values = np.full_like(keys, np.nan)
    table = np.array([4, 1, 3], dtype=np.int32)
    key_values = [-1000, -999, 1000, 999, 1001]
    for t, kv in enumerate(key_values):
        page, slot = table[t // bt], t % bt
        keys[page, 0, slot, :] = kv / 4.0  # q.k = 16*kv/4 = 4kv; scaled by 1/sqrt(16) -> kv
        values[page, 0, slot, :] = t + np.arange(dim) / 10
    q = np.ones(dim, dtype=np.float32)
    for length in range(1, 6):
        out = o.attention(q, keys.ravel(), values.ravel(), table, length - 1, 1, 0, 1, bt, 1, 1, dim)[0]
        m = max(key_values[:length])
        w = [math.exp(k - m) for k in key_values[:length]]
        expect = sum(wi * t for t, wi in enumerate(w)) / sum(w) + np.arange(dim) / 10
        assert np.all(np.isfinite(out))
        assert np.max(np.abs(out - expect)) < 2e-5


def test_attention_matches_double_brute_force():
    o = Oracle()
    rng = np.random.default_rng(3)
    heads, kvh, dim, bt, layers, pages = 6, 2, 8, 4, 2, 9
    keys = rng.standard_normal((pages, layers, bt, kvh * dim)).astype(np.float32)
    values = rng.standard_normal(keys.shape).astype(np.float32)
    table = rng.permutation(pages).astype(np.int32)
    start, rows, layer = 21, 3, 1
    q = rng.standard_normal((rows, heads, dim)).astype(np.float32)
    out = o.attention(q, keys.ravel(), values.ravel(), table, start, rows, layer, layers, bt, heads, kvh, dim)
    for r in range(rows):
        length = start + r + 1
        for h in range(heads):
            kh = h // (heads // kvh)
            k = np.array([keys[table[t // bt], layer, t % bt, kh * dim:(kh + 1) * dim] for t in range(length)],
                         dtype=np.float64)
            v = np.array([values[table[t // bt], layer, t % bt, kh * dim:(kh + 1) * dim] for t in range(length)],
                         dtype=np.float64)
            s = k @ q[r, h].astype(np.float64) / math.sqrt(dim)
            p = np.exp(s - s.max())
            p /= p.sum()
            assert np.max(np.abs(out[r, h * dim:(h + 1) * dim] - p @ v)) < 1e-5


def test_rms_rope_swiglu_closed_forms():
    o = Oracle()
    x = np.array([[3.0, 4.0], [1.0, -1.0]], dtype=np.float32)
    y = o.rms(x, np.array([2.0, 0.5], dtype=np.float32), 0.0)
    # rms: x / sqrt(mean(x^2)): [3,4]/sqrt(12.5); [1,-1]/1
    np.testing.assert_allclose(y, [[6 / math.sqrt(12.5), 2 / math.sqrt(12.5)], [2.0, -0.5]], rtol=1e-6)
    q = np.arange(8, dtype=np.float32).reshape(1, 8)
    assert np.array_equal(o.rope(q, 1, 8, 0, 10000.0), q)  # position 0 is the identity
    r = o.rope(q, 1, 8, 3, 10000.0)[0]
    for d in range(4):  # split-half pairs (d, d+4), angle 3/10000^(2d/8)
        a = 3 / 10000 ** (2 * d / 8)
        np.testing.assert_allclose([r[d], r[d + 4]], [q[0, d] * math.cos(a) - q[0, d + 4] * math.sin(a),
                                                      q[0, d + 4] * math.cos(a) + q[0, d] * math.sin(a)], rtol=2e-6)
    g = np.array([-3.0, 0.0, 2.5], dtype=np.float32)
    u = np.array([2.0, 5.0, -1.0], dtype=np.float32)
    np.testing.assert_allclose(o.swiglu(g, u), g / (1 + np.exp(-g.astype(np.float64))) * u, rtol=1e-6)


def test_linear_is_sequential_k_without_fma():
    """out = sum_k x_k w_k accumulated in k order with separate roundings:
    cancellation that an FMA or a reordered sum would resolve differently."""
    o = Oracle()
    x = np.array([[1.0, 1.0, 1.0]], dtype=np.float32)
    w = np.array([[1e8], [1.0], [-1e8]], dtype=np.float32)
    assert o.linear(x, w)[0, 0] == 0.0  # (1e8 + 1) rounds to 1e8 in float
    x = np.array([[1.0 + 2 ** -12, 1.0]], dtype=np.float32)
    w = np.array([[1.0 + 2 ** -12], [-1.0]], dtype=np.float32)
    prod = np.float32(np.float32(1 + 2 ** -12) * np.float32(1 + 2 ** -12))
    assert o.linear(x, w)[0, 0] == np.float32(prod - np.float32(1.0))


# ---------------------------------------------------------------- generator
def test_synthetic_generator_matches_product():
    cfg = tiny_config(vocabulary=64)
    model = OracleModel(cfg, seed=99, stddev=0.3)
    w = host.Weights.synthetic(cfg, seed=99, stddev=0.3)
    assert np.array_equal(bits(model.tensor(0, -1)).ravel(), bits(w.tensor("model.embed_tokens.weight")))
    assert np.array_equal(bits(model.tensor(1, 8)).ravel(), bits(w.tensor("model.layers.1.mlp.down_proj.weight")))
    assert np.array_equal(bits(model.tensor(0, -3)).ravel(), bits(w.tensor("lm_head.weight")))
    o = Oracle()
    z = o.fill_normal(200000, 5, 77)
    assert abs(z.mean()) < 0.01 and abs(z.std() - 1) < 0.01


# ---------------------------------------------------------------- vs reference
@needs_ref
@pytest.mark.parametrize("name", ["tiny", "smollm2"])
def test_oracle_bit_identical_to_reference_cpu_runner(name):
    cfg = tiny_config() if name == "tiny" else smollm_config(layers=2, context=256)
    stddev = 0.15 if name == "tiny" else 0.02
    weights = host.Weights.synthetic(cfg, seed=7, stddev=stddev, library=ref_library())
    bt, blocks = (4, 8) if name == "tiny" else (16, 32)
    cpu = host.Runner(weights, cfg["context"] if name == "tiny" else 256, bt, blocks, 0, kind=0)
    mirror = host.Runner(weights, cfg["context"] if name == "tiny" else 256, bt, blocks, 0, kind=1)
    rng = np.random.default_rng(1)
    chunks = ([[1, 2, 3], [4], [5, 6, 7, 8, 9], [10], [11, 12]] if name == "tiny"
              else [list(rng.integers(0, cfg["vocabulary"], n)) for n in (37, 1, 16, 1, 1)])
    for r in (cpu, mirror):
        r.create("a")
    for chunk in chunks:
        a, b = cpu.append("a", chunk), mirror.append("a", chunk)
        assert np.array_equal(bits(a), bits(b))
    # a fork and a copy-on-write of the shared partial tail
    for r in (cpu, mirror):
        r.create("b")
        r.fork_sequence("a", "b")
    for chunk in ([13], [14, 15]):
        assert np.array_equal(bits(cpu.append("b", chunk)), bits(mirror.append("b", chunk)))
    assert cpu.stats()["forward_tokens"] == mirror.stats()["forward_tokens"]


@needs_ref
def test_reference_engine_tokens_match_mirror_runner():
    """The reference Engine produces the same tokens whether its runner is the
    reference CpuRunner or the oracle-forward mirror used as the golden
    source for page tables."""
    cfg = tiny_config(vocabulary=16, context=32)
    weights = host.Weights.synthetic(cfg, seed=3, stddev=0.2, library=ref_library())
    outs = []
    for kind in (0, 1):
        engine = host.Engine(host.Runner(weights, 32, 4, 24, 4, kind=kind), 3, 8, 4, 32)
        for i, p in enumerate(([1, 2, 3, 4, 5, 6], [1, 2, 3, 9], [7, 7])):
            engine.submit(f"r{i}", p, max_new_tokens=5)
        events = []
        while not engine.idle():
            engine.step()
            events += engine.poll_events()
        outs.append([(e["id"], e["token"], e["finish"]) for e in events])
        engine.close()
    assert outs[0] == outs[1]


# ---------------------------------------------------------------- device expf
def _fma(a: float, b: float, c: float) -> float:
    """Exact fused multiply-add, rounded once to double (round-half-even)."""
    return float(Fraction(a) * Fraction(b) + Fraction(c))


_H = float.fromhex
_TABLE = [struct.unpack("<Q", struct.pack("<d", 2.0 ** (i / 32)))[0] - (i << 47) for i in range(32)]


def _device_expf(x: np.float32) -> np.float32:
    """The double-precision algorithm of tinyinfer_amd/csrc/backend/exact_math.h."""
    u = int(np.float32(x).view(np.uint32))
    abstop = (u >> 20) & 0x7FF
    if abstop >= 0x42B:
        if u == 0xFF800000:
            return np.float32(0.0)
        if abstop >= 0x7F8:
            return np.float32(x) + np.float32(x)
        if x > np.float32(_H("0x1.62e42ep6")):
            return np.float32(np.inf)
        if x < np.float32(-_H("0x1.9fe368p6")):
            return np.float32(0.0)
    inv_ln2_n, shift = _H("0x1.71547652b82fep+5"), _H("0x1.8p+52")
    xd = float(x)
    kd = _fma(inv_ln2_n, xd, shift)
    ki = struct.unpack("<Q", struct.pack("<d", kd))[0]
    kd -= shift
    r = _fma(inv_ln2_n, xd, -kd)
    t = (_TABLE[ki % 32] + (ki << 47)) & 0xFFFFFFFFFFFFFFFF
    s = struct.unpack("<d", struct.pack("<Q", t))[0]
    z = _fma(_H("0x1.c6af84b912394p-20"), r, _H("0x1.ebfce50fac4f3p-13"))
    y = _fma(_H("0x1.62e42ff0c52d6p-6"), r, 1.0)
    y = _fma(z, r * r, y)
    return np.float32(y * s)


def test_device_expf_algorithm_matches_c_library():
    """Edge cases, two inputs the C library rounds away from the correctly
    rounded value (a plain double exp would disagree there), and a sample."""
    o = Oracle()
    special = np.float32([0.0, -0.0, -1e-30, -87.9, -103.2, -103.97, 88.7, -50.5, _H("-0x1.f8cbb2p+5"),
                          _H("0x1.04845ep+5"), -np.inf, 89.0, -120.0])
    sample = np.random.default_rng(0).uniform(-104, 0, 3000).astype(np.float32)
    xs = np.concatenate([special, sample])
    got = np.array([_device_expf(x) for x in xs], dtype=np.float32)
    assert np.array_equal(bits(got), bits(o.expf(xs)))
