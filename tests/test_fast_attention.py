"""The fast arithmetic's decode attention kernels -- the split, short-row and
merge kernels that a fast-mode forward runs for its one-token rows, and that
bench.py times -- through their stand-alone entry point
(mp_hip_paged_attention_decode_fast), held to the attention bound of 1e-4
absolute against the oracle (which restates llama_runner.cpp:85-93) and
against a double-precision evaluation of the same softmax:
- config 1, the single paged-attention op: 9 query heads on 3 KV heads,
  T=503 (31 full pages + 7), a seeded permutation of a 256-page pool,
  Q/K/V ~ N(0,1), scale 1/sqrt(64);
- rows of 1 to 65 splits in one call (1 to 16,640 tokens: the short-row
  work-group up to 256 tokens, 128-token splits up to 4,096, 256-token
  splits beyond), over N(0,1) keys and over keys scaled by 6, whose softmax
  peaks at a few tokens and whose running maxima climb inside splits;
- the closed form of the reference's tests/paged_attention_test.cpp:40-68
  adapted to 64-dim heads and 16-token pages: keys that give scores
  {-1000, -999, 1000, 999, 1001}, values t + d/10, every length from 1 to 5,
  and every slot past the five tokens NaN; and the same five tokens after
  300 and 4,100 tokens of score 0 (values -1 - d/10), so that splits whose
  maxima differ by 1,000 are merged and a split's reference maximum jumps by
  1,000 within it.
The pools are in the device page order (layout.h), as the forward keeps
them."""
import math

import numpy as np
import pytest

from oracle import Oracle
from tinyinfer_amd.backend import paged_attention_decode_fast

from .helpers import device_key_order, device_value_order

pytestmark = pytest.mark.gpu

BT, DIM, HEADS, KV_HEADS = 16, 64, 9, 3
KVW = KV_HEADS * DIM


def run_fast(torch, q, keys, values, tables, lengths, layer, layers):
    """q [rows][heads*64]; keys/values plain [blocks][layers][16][kv_width];
    tables [rows][stride]."""
    blocks = keys.shape[0]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    dk = dev(device_key_order(keys.reshape(-1), blocks, layers, KV_HEADS))
    dv = dev(device_value_order(values.reshape(-1), blocks, layers, KV_HEADS))
    dq, dt = dev(q.astype(np.float32)), dev(tables.astype(np.int32))
    out = torch.full((len(lengths), HEADS * DIM), float("nan"), dtype=torch.float32, device="cuda")
    paged_attention_decode_fast(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), tables.shape[1],
                                lengths, layer, layers, HEADS, KV_HEADS, out.data_ptr(), None)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def double_attention(q, keys, values, table, length, layer):
    """Softmax attention of one row in double precision (the reference's
    definition: scores q.k/sqrt(64), maximum subtracted)."""
    t = np.arange(length)
    k = keys[table[t // BT], layer, t % BT].astype(np.float64).reshape(length, KV_HEADS, DIM)
    v = values[table[t // BT], layer, t % BT].astype(np.float64).reshape(length, KV_HEADS, DIM)
    out = np.empty(HEADS * DIM)
    for h in range(HEADS):
        kh = h // (HEADS // KV_HEADS)
        s = k[:, kh] @ q[h * DIM:(h + 1) * DIM].astype(np.float64) / 8.0
        p = np.exp(s - s.max())
        out[h * DIM:(h + 1) * DIM] = (p @ v[:, kh]) / p.sum()
    return out


def test_config1_fast_attention(torch_cuda):
    """Config 1 through the fast kernels (503 tokens: four 128-token splits
    and the merge), against the oracle and double precision."""
    o = Oracle()
    seed, pages, T = 2024, 256, 503
    keys = o.fill_normal(pages * BT * KVW, seed, 2001).reshape(pages, 1, BT, KVW)
    values = o.fill_normal(pages * BT * KVW, seed, 2002).reshape(pages, 1, BT, KVW)
    q = o.fill_normal(HEADS * DIM, seed, 2003)
    table = o.permutation(pages, seed, 2004)[:32].copy()
    want = o.attention(q, keys.ravel(), values.ravel(), table, T - 1, 1, 0, 1, BT, HEADS, KV_HEADS, DIM)[0]
    got = run_fast(torch_cuda, q[None], keys, values, table[None], [T], 0, 1)[0]
    err = float(np.max(np.abs(got - want)))
    exact = float(np.max(np.abs(got - double_attention(q, keys, values, table, T, 0))))
    print(f"config 1 fast attention: max |got - oracle| {err:.3e}, max |got - double| {exact:.3e}")
    assert err <= 1e-4 and exact <= 1e-4


@pytest.mark.parametrize("key_scale", [1.0, 6.0])
def test_fast_attention_rows_of_1_to_65_splits(torch_cuda, key_scale):
    """Thirteen rows in one call, each over its own pages of a two-layer
    pool (layer 1 attended): 1, 10, 17 and 33 tokens (short rows of one to
    three splits), 256 (eight 32-token splits in one work-group), 257 and 503
    (three and four 128-token splits), 1,901, 4,096 (32 splits), 4,097 (17
    of 256 tokens), 8,251 (33), 16,401 (65, the last of one token) and
    16,640 (65) tokens; the pages of the rows are a seeded permutation of
    the pool."""
    o = Oracle()
    seed, layers, layer = 61, 2, 1
    lengths = [1, 10, 17, 33, 256, 257, 503, 1901, 4096, 4097, 8251, 16401, 16640]
    pages = [-(-n // BT) for n in lengths]
    blocks = sum(pages) + 8
    perm = o.permutation(blocks, seed, 9700)
    stride = max(pages)
    tables = np.zeros((len(lengths), stride), dtype=np.int32)
    at = 0
    for r, p in enumerate(pages):
        tables[r, :p] = perm[at:at + p]
        at += p
    keys = o.fill_normal(blocks * layers * BT * KVW, seed, 9701, key_scale).reshape(blocks, layers, BT, KVW)
    values = o.fill_normal(blocks * layers * BT * KVW, seed, 9702).reshape(blocks, layers, BT, KVW)
    q = o.fill_normal(len(lengths) * HEADS * DIM, seed, 9703).reshape(len(lengths), HEADS * DIM)
    got = run_fast(torch_cuda, q, keys, values, tables, lengths, layer, layers)
    worst = worst_double = 0.0
    for r, n in enumerate(lengths):
        want = o.attention(q[r], keys.ravel(), values.ravel(), tables[r], n - 1, 1, layer, layers, BT, HEADS,
                           KV_HEADS, DIM)[0]
        err = float(np.max(np.abs(got[r] - want)))
        err_double = float(np.max(np.abs(got[r] - double_attention(q[r], keys, values, tables[r], n, layer))))
        worst, worst_double = max(worst, err), max(worst_double, err_double)
        assert err <= 1e-4, f"row of {n} tokens: max |got - oracle| {err:.3e}"
        assert err_double <= 1e-4, f"row of {n} tokens: max |got - double| {err_double:.3e}"
    print(f"key scale {key_scale}: max |got - oracle| {worst:.3e}, max |got - double| {worst_double:.3e}")


def test_fast_attention_closed_form_and_nan_tail(torch_cuda):
    """Query all ones, keys k/8 in every dim (score = k) for the five tokens
    k = -1000, -999, 1000, 999, 1001 with values t + d/10 (t = 0..4), every
    other slot of the pool NaN; rows of lengths 1..5 attend the first j of
    them directly (one short-row work-group), and after 300 and 4,100
    tokens of score 0 with values -1 - d/10 (three 128-token splits; 17
    splits of 256). The expected output follows in double precision from
    the scores alone: with j <= 2 the score-0 tokens outweigh the specials
    by e^999, so the output is -1 - d/10; with j >= 3 the specials outweigh
    them by e^1000."""
    specials = [-1000.0, -999.0, 1000.0, 999.0, 1001.0]
    bases = [0, 300, 4100]
    pages = [-(-(b + 5) // BT) for b in bases]
    blocks = sum(pages) + 4
    keys = np.full((blocks, 1, BT, KVW), np.nan, dtype=np.float32)
    values = np.full_like(keys, np.nan)
    stride = max(pages)
    base_tables = []
    at = 3  # pages 0-2 stay NaN and unreferenced
    for b, p in zip(bases, pages):
        table = np.arange(at + p - 1, at - 1, -1, dtype=np.int32)  # pages in descending order
        at += p
        for t in range(b + 5):
            page, slot = table[t // BT], t % BT
            if t < b:
                keys[page, 0, slot, :] = 0.0
                values[page, 0, slot, :] = np.tile(-1.0 - np.arange(DIM, dtype=np.float32) / 10, KV_HEADS)
            else:
                keys[page, 0, slot, :] = specials[t - b] / 8.0
                values[page, 0, slot, :] = np.tile((t - b) + np.arange(DIM, dtype=np.float32) / 10, KV_HEADS)
        padded = np.zeros(stride, dtype=np.int32)
        padded[:p] = table
        base_tables.append(padded)
    rows = [(b, j) for b in range(len(bases)) for j in range(1, 6)]
    tables = np.stack([base_tables[b] for b, _ in rows])
    lengths = [bases[b] + j for b, j in rows]
    q = np.ones((len(rows), HEADS * DIM), dtype=np.float32)
    got = run_fast(torch_cuda, q, keys, values, tables, lengths, 0, 1)
    d = np.arange(DIM) / 10
    for (b, j), out in zip(rows, got):
        if bases[b] and j <= 2:
            expect = -1.0 - d
        else:
            m = max(specials[:j])
            w = [math.exp(s - m) for s in specials[:j]]
            expect = sum(wi * t for t, wi in enumerate(w)) / sum(w) + d
        assert np.all(np.isfinite(out)), f"base {bases[b]}, length {j}: non-finite output"
        err = float(np.max(np.abs(out.reshape(HEADS, DIM) - expect[None])))
        assert err <= 1e-4, f"base {bases[b]}, {j} special tokens: max error {err:.3e}"


def test_fast_attention_rejects_other_shapes(torch_cuda):
    """Pages other than 16 tokens, heads other than 64 dims, more than 4
    query heads per KV head, or a row longer than its table are refused
    before any launch (the buffers are real and large enough either way)."""
    import ctypes
    from tinyinfer_amd.backend import lib
    torch = torch_cuda
    buf = torch.zeros(1 << 20, dtype=torch.float32, device="cuda")
    tab = torch.zeros(64, dtype=torch.int32, device="cuda")
    p, t = buf.data_ptr(), tab.data_ptr()
    for bt, heads, kvh, dim, length in ((8, 9, 3, 64, 5), (16, 9, 3, 32, 5), (16, 10, 2, 64, 5),
                                        (16, 9, 3, 64, 4 * 16 + 1)):
        n = np.array([length], dtype=np.int32)
        status = lib().mp_hip_paged_attention_decode_fast(p, p, p, t, 4, n.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                                          1, 0, 1, bt, heads, kvh, dim, p, None)
        assert status == -1, (bt, heads, kvh, dim, length)
        assert lib().mp_hip_last_error(None)
