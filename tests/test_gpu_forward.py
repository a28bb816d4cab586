"""HIP forward vs the CPU oracle on identical seeded inputs.

The oracle restates the reference CPU path (miniprefix/src/backend/cpu/
llama_runner.cpp:10-104) op for op; the HIP kernels keep its floating-point
order, so logits are compared bit for bit (the specified bar, max relative
error 1e-3, is asserted as well to report how far off a failure is)."""
import numpy as np
import pytest

from oracle import Oracle, OracleModel
from tinyinfer_amd.backend import HipBackend, paged_attention_decode

from .helpers import pool_elements, smollm_config, tiny_config, upload_model

pytestmark = pytest.mark.gpu


def _logits_match(got, want):
    assert np.all(np.isfinite(got))
    rel = np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-30))
    assert rel <= 1e-3, f"max relative error {rel}"
    mism = np.count_nonzero(got.view(np.uint32) != want.view(np.uint32))
    assert mism == 0, f"{mism} logits differ in bits (max rel {rel})"
    assert int(np.argmax(got)) == int(np.argmax(want))


def test_config1_paged_attention_decode(torch_cuda):
    """The single paged-attention op: T=503 (31 full pages + 7), 256-page
    pool, seeded permutation table, Q/K/V ~ N(0,1), scale 1/sqrt(64)."""
    torch = torch_cuda
    o = Oracle()
    seed, bt, pages, heads, kvh, dim, T = 2024, 16, 256, 9, 3, 64, 503
    kvw = kvh * dim
    keys = o.fill_normal(pages * bt * kvw, seed, 2001)
    values = o.fill_normal(pages * bt * kvw, seed, 2002)
    q = o.fill_normal(heads * dim, seed, 2003)
    table = o.permutation(pages, seed, 2004)[:32].copy()
    want = o.attention(q, keys, values, table, T - 1, 1, 0, 1, bt, heads, kvh, dim)[0]
    dev = lambda a: torch.from_numpy(a).cuda()
    dq, dk, dv, dt = dev(q), dev(keys), dev(values), dev(table)
    out = torch.empty(heads * dim, dtype=torch.float32, device="cuda")
    paged_attention_decode(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dt.data_ptr(), T, 0, 1, bt, heads, kvh,
                           dim, out.data_ptr(), None)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.max(np.abs(got - want)) <= 1e-4
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _run_sequence(model, backend, bt, chunks, table, slot=0):
    """Append `chunks` (lists of token ids) to one sequence on both sides."""
    c = model.config
    n = pool_elements(c, bt, backend.max_blocks)
    keys = np.zeros(n, dtype=np.float32)
    values = np.zeros(n, dtype=np.float32)
    used = 0
    backend.table_write(slot, 0, table)
    for chunk in chunks:
        want = model.append(keys, values, bt, table, used, chunk)
        am, got = backend.forward([(slot, used, len(chunk))], chunk)
        _logits_match(got[0], want)
        assert am[0] == int(np.argmax(want))
        used += len(chunk)
    return keys, values


def test_tiny_model_chunks(torch_cuda):
    cfg = tiny_config()
    model = OracleModel(cfg, seed=7, stddev=0.15)
    backend = HipBackend(cfg, block_tokens=4, max_blocks=8, max_sequences=4)
    upload_model(backend, model)
    table = np.array([5, 2, 7, 0, 3, 1, 6, 4], dtype=np.int32)
    _run_sequence(model, backend, 4, [[1, 2, 3], [4], [5, 6, 7, 8, 9], [10], [11]], table)


def test_smollm_shape_two_layers(torch_cuda):
    cfg = smollm_config(layers=2, context=256)
    model = OracleModel(cfg, seed=11)
    backend = HipBackend(cfg, block_tokens=16, max_blocks=32, max_sequences=4)
    upload_model(backend, model)
    o = Oracle()
    prompt = o.fill_tokens(37, 11, 3000, cfg["vocabulary"])
    table = o.permutation(32, 11, 3001)[:16].copy()
    chunks = [list(prompt[:16]), list(prompt[16:37])] + [[int(t)] for t in o.fill_tokens(5, 11, 3002, 49152)]
    _run_sequence(model, backend, 16, chunks, table)


def test_wide_shape_streamed_weight_paths(torch_cuda):
    """hidden 640 / intermediate 1600 / 5 query heads per KV head: the
    decode projections stream weight blocks through the register ring (gate
    and up over 640, down over 1600), RMSNorm runs as its own kernel (wider
    than the folded path takes), and decode attention takes the generic
    kernels with the separate RoPE/append kernel."""
    cfg = tiny_config(hidden=640, intermediate=1600, heads=10, kv_heads=2, vocabulary=512, context=128, tied=1)
    model = OracleModel(cfg, seed=17)
    backend = HipBackend(cfg, block_tokens=16, max_blocks=16, max_sequences=2)
    upload_model(backend, model)
    o = Oracle()
    prompt = o.fill_tokens(29, 17, 3100, cfg["vocabulary"])
    table = o.permutation(16, 17, 3101)[:8].copy()
    chunks = [list(prompt[:20]), list(prompt[20:29])] + [[int(t)] for t in o.fill_tokens(4, 17, 3102, 512)]
    _run_sequence(model, backend, 16, chunks, table)


def test_narrow_shape_short_weight_columns(torch_cuda):
    """hidden 128 / intermediate 192: the decode projections run on the
    one-row-tile kernels with columns of 2 and 3 64-k blocks. QKV takes the
    folded RMSNorm with LDS-held weights, gate/up the folded RMSNorm with the
    up-weight ring past its last block, and O and down the LDS-held weights
    well short of their capacity. Decode attention takes the fused kernels
    (head dim 64, two query heads per KV head)."""
    cfg = tiny_config(hidden=128, intermediate=192, heads=2, kv_heads=1, vocabulary=256, context=128, tied=0)
    model = OracleModel(cfg, seed=23)
    backend = HipBackend(cfg, block_tokens=16, max_blocks=16, max_sequences=2)
    upload_model(backend, model)
    o = Oracle()
    prompt = o.fill_tokens(37, 23, 3200, cfg["vocabulary"])
    table = o.permutation(16, 23, 3201)[:8].copy()
    chunks = [list(prompt[:24]), list(prompt[24:37])] + [[int(t)] for t in o.fill_tokens(5, 23, 3202, 256)]
    _run_sequence(model, backend, 16, chunks, table)


def test_batched_rows_match_single_sequences(torch_cuda):
    """Several sequences in one forward call == each appended alone."""
    cfg = smollm_config(layers=2, context=256)
    model = OracleModel(cfg, seed=5)
    bt, max_blocks = 16, 64
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=8)
    upload_model(backend, model)
    o = Oracle()
    perm = o.permutation(max_blocks, 5, 4000)
    n = pool_elements(cfg, bt, max_blocks)
    keys = np.zeros(n, dtype=np.float32)
    values = np.zeros(n, dtype=np.float32)
    lengths = [20, 3, 33, 16, 1, 7]
    tables = [perm[8 * i: 8 * i + 8].copy() for i in range(len(lengths))]
    used = [0] * len(lengths)
    for i, t in enumerate(tables):
        backend.table_write(i, 0, t)
    for step in range(3):
        chunks = [list(o.fill_tokens(lengths[i] if step == 0 else 1, 5, 5000 + 10 * step + i, 49152))
                  for i in range(len(lengths))]
        want = [model.append(keys, values, bt, tables[i], used[i], chunks[i]) for i in range(len(lengths))]
        steps = [(i, used[i], len(chunks[i])) for i in range(len(lengths))]
        am, got = backend.forward(steps, [t for ch in chunks for t in ch])
        for i in range(len(lengths)):
            _logits_match(got[i], want[i])
            assert am[i] == int(np.argmax(want[i]))
            used[i] += len(chunks[i])


def test_long_prefill_row_blocks(torch_cuda):
    """Prefill chunks of 256 rows (row blocks of several positions each,
    several 256-token score chunks) followed by decode rows."""
    cfg = smollm_config(layers=2, context=1024)
    model = OracleModel(cfg, seed=13)
    backend = HipBackend(cfg, block_tokens=16, max_blocks=64, max_sequences=4)
    upload_model(backend, model)
    o = Oracle()
    prompt = [int(t) for t in o.fill_tokens(700, 13, 6000, cfg["vocabulary"])]
    table = o.permutation(64, 13, 6001)[:48].copy()
    chunks = [prompt[:256], prompt[256:512], prompt[512:700], [17], [4242]]
    _run_sequence(model, backend, 16, chunks, table)


def test_batched_prefill_and_decode_rows(torch_cuda):
    """One forward call mixing two prefill chunks (ragged row blocks) with
    decode rows, as the engine's batched steps do."""
    cfg = smollm_config(layers=2, context=512)
    model = OracleModel(cfg, seed=21)
    bt, max_blocks = 16, 96
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=8)
    upload_model(backend, model)
    o = Oracle()
    perm = o.permutation(max_blocks, 21, 7000)
    n = pool_elements(cfg, bt, max_blocks)
    keys = np.zeros(n, dtype=np.float32)
    values = np.zeros(n, dtype=np.float32)
    tables = [perm[24 * i: 24 * i + 24].copy() for i in range(4)]
    for i, t in enumerate(tables):
        backend.table_write(i, 0, t)
    used = [0, 0, 0, 0]
    plan = [[290, 45, 1, 17], [1, 1, 300, 1], [3, 1, 1, 20]]
    for step, counts in enumerate(plan):
        chunks = [[int(t) for t in o.fill_tokens(counts[i], 21, 7100 + 10 * step + i, cfg["vocabulary"])]
                  for i in range(4)]
        want = [model.append(keys, values, bt, tables[i], used[i], chunks[i]) for i in range(4)]
        am, got = backend.forward([(i, used[i], counts[i]) for i in range(4)], [t for ch in chunks for t in ch])
        for i in range(4):
            _logits_match(got[i], want[i])
            assert am[i] == int(np.argmax(want[i]))
            used[i] += counts[i]


@pytest.mark.parametrize("shape", ["paged16_dim64", "paged16_dim64_beyond_fused", "tiny_generic"])
def test_long_context_softmax_windows(torch_cuda, shape):
    """Rows longer than one 2048-token softmax window: the denominators are
    summed over several staged windows and e_t is formed again per window
    (prefill row blocks with every head of a group in one task), then decode
    rows: on the 16-token page / dim-64 path (decode through the fused
    kernel up to 4096 tokens, through the two-kernel path beyond) and on the
    generic path."""
    if shape.startswith("paged16_dim64"):
        context = 2720 if shape == "paged16_dim64" else 4400
        cfg = dict(layers=1, hidden=192, intermediate=256, heads=3, kv_heads=1, vocabulary=512, context=context,
                   eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)
        bt = 16
        chunks = [1100, 1100, 500, 1, 1] if context == 2720 else [2048, 2048, 200, 1, 1]
    else:
        cfg = tiny_config(context=2600)
        bt, chunks = 4, [1000, 1100, 300, 1, 1]
    model = OracleModel(cfg, seed=31)
    pages = (cfg["context"] + bt - 1) // bt
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=pages + 8, max_sequences=2)
    upload_model(backend, model)
    o = Oracle()
    table = o.permutation(pages + 8, 31, 8000)[:pages].copy()
    tokens = [int(t) for t in o.fill_tokens(sum(chunks), 31, 8001, cfg["vocabulary"])]
    split, at = [], 0
    for n in chunks:
        split.append(tokens[at:at + n])
        at += n
    _run_sequence(model, backend, bt, split, table)


def test_queued_tail_copies(torch_cuda):
    """Copies-on-write are queued and run as one launch before the next
    forward: three copies of one shared tail page into fresh pages, and a
    chain (tail -> X, then X -> Y: the second reads a page the first
    writes, which flushes the queue first). Each fork then appends a token
    through its own table in one batched forward; logits equal the oracle's
    over pools where the same regions were copied on the CPU, bit for bit."""
    cfg = smollm_config(layers=2, context=128)
    model = OracleModel(cfg, seed=31)
    bt, max_blocks = 16, 32
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=8)
    upload_model(backend, model)
    o = Oracle()
    n = pool_elements(cfg, bt, max_blocks)
    keys = np.zeros(n, dtype=np.float32)
    values = np.zeros(n, dtype=np.float32)
    kvw = cfg["kv_heads"] * (cfg["hidden"] // cfg["heads"])
    page, layers = bt * kvw, cfg["layers"]
    block = page * layers
    source = np.array([3, 11, 20], dtype=np.int32)
    prompt = [int(t) for t in o.fill_tokens(37, 31, 8000, cfg["vocabulary"])]
    backend.table_write(0, 0, source)
    want = model.append(keys, values, bt, source, 0, prompt)
    _, got = backend.forward([(0, 0, len(prompt))], prompt)
    _logits_match(got[0], want)
    valid = len(prompt) % bt

    def cow(dst, src):
        backend.copy_tail(dst * block, src * block, page, valid * kvw, layers)
        for layer in range(layers):
            d, s = dst * block + layer * page, src * block + layer * page
            keys[d:d + valid * kvw] = keys[s:s + valid * kvw]
            values[d:d + valid * kvw] = values[s:s + valid * kvw]

    forks = {1: 5, 2: 6, 3: 7}  # table slot -> fresh tail page
    for slot, fresh in forks.items():
        cow(fresh, 20)
    cow(9, 20)
    cow(12, 9)  # reads the page the previous copy writes
    forks[4] = 12
    tables = {slot: np.array([3, 11, fresh], dtype=np.int32) for slot, fresh in forks.items()}
    for slot, t in tables.items():
        backend.table_write(slot, 0, t)
    tokens = [int(t) for t in o.fill_tokens(len(tables), 31, 8001, cfg["vocabulary"])]
    expect = [model.append(keys, values, bt, tables[slot], len(prompt), [tok])
              for slot, tok in zip(tables, tokens)]
    before = backend.stats()["cow_copies"]
    am, got = backend.forward([(slot, len(prompt), 1) for slot in tables], tokens)
    for i, w in enumerate(expect):
        _logits_match(got[i], w)
        assert am[i] == int(np.argmax(w))
    assert backend.stats()["cow_copies"] == before
    # A copy queued and flushed by sync alone.
    cow(13, 12)
    backend.sync()
    backend.table_write(5, 0, np.array([3, 11, 13], dtype=np.int32))
    tok = tokens[0]
    w = model.append(keys, values, bt, np.array([3, 11, 13], dtype=np.int32), len(prompt), [tok])
    _, got = backend.forward([(5, len(prompt), 1)], [tok])
    _logits_match(got[0], w)
