"""mp_hip_paged_attention_decode_noalloc (the allocation-free variant)
against mp_hip_paged_attention_decode, the entry point it shares its kernel
with, and against the oracle.

Two calls in a row on rows long enough that their scores leave LDS for the
static device scratch (a KV head's 3 query heads x round_up(length, 16) >
kAttentionLdsScores = 10,240 floats), the second shorter than the first, so
it runs over what the first left there; then a row of 100 tokens, whose
scores stay in LDS although the entry point passes the scratch as well.
Outputs must be bit-identical to the allocating entry point's (and to the
oracle's: the kernel keeps the reference CPU path's order). A row beyond
the scratch is rejected before any launch."""
import math

import numpy as np
import pytest

from oracle import Oracle
from tinyinfer_amd.backend import BackendError, paged_attention_decode, paged_attention_decode_noalloc

pytestmark = pytest.mark.gpu

HEADS, KV_HEADS, DIM, BT, LAYERS, LAYER = 9, 3, 64, 16, 2, 1


def _inputs(o, seed, length):
    pages = math.ceil(length / BT) + 8
    kvw = KV_HEADS * DIM
    keys = o.fill_normal(pages * LAYERS * BT * kvw, seed, 1)
    values = o.fill_normal(pages * LAYERS * BT * kvw, seed, 2)
    q = o.fill_normal(HEADS * DIM, seed, 3)
    table = o.permutation(pages, seed, 4)[: math.ceil(length / BT)].copy()
    return q, keys, values, table


def test_noalloc_matches_allocating_entry_point(torch_cuda):
    torch = torch_cuda
    o = Oracle()
    held = None
    # 3 x round_up(length, 16) > 10240 for 6000 and 4000 (scores in the
    # scratch), not for 100 (scores in LDS).
    for seed, length in ((5, 6000), (6, 4000), (7, 100)):
        q, keys, values, table = _inputs(o, seed, length)
        dq, dk, dv, dt = (torch.from_numpy(a).cuda() for a in (q, keys, values, table))
        base = torch.empty(HEADS * DIM, dtype=torch.float32, device="cuda")
        got = torch.full((HEADS * DIM,), float("nan"), dtype=torch.float32, device="cuda")
        args = (dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), length, LAYER, LAYERS, BT, HEADS,
                KV_HEADS, DIM)
        paged_attention_decode(*args, base.data_ptr(), None)
        torch.cuda.synchronize()
        paged_attention_decode_noalloc(*args, got.data_ptr(), None)
        torch.cuda.synchronize()
        b, g = base.cpu().numpy(), got.cpu().numpy()
        assert np.all(np.isfinite(g))
        assert np.array_equal(g.view(np.uint32), b.view(np.uint32)), f"length {length}: differs from the allocating call"
        want = o.attention(q, keys, values, table, length - 1, 1, LAYER, LAYERS, BT, HEADS, KV_HEADS, DIM)[0]
        assert np.max(np.abs(g - want)) <= 1e-4
        assert np.array_equal(g.view(np.uint32), want.view(np.uint32))
        held = args
    # Beyond the scratch (9 x 30000 > 262144 floats): rejected before any launch.
    long_args = held[:4] + (30000,) + held[5:]
    out = torch.empty(HEADS * DIM, dtype=torch.float32, device="cuda")
    with pytest.raises(BackendError) as error:
        paged_attention_decode_noalloc(*long_args, out.data_ptr(), None)
    assert "exceeds" in str(error.value)
