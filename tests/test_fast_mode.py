"""The fast arithmetic mode (MP_ARITHMETIC_FAST: projections and LM head on
FP32 matrix cores, decode attention split over the context) against the
oracle, which restates the reference CPU path.

The fast mode sums in its own order, so logits are compared within the
specified bound, max relative error 1e-3, taken over the whole logit vector
(max |got - want| / max |want|: an element-wise ratio is meaningless for
logits near zero), and the greedy token must equal the oracle's, which the
test also reports against the oracle's top-2 margin. Per-row results must
not depend on the batch: a row computed with others equals the row computed
alone, bit for bit."""
import numpy as np
import pytest

from oracle import Oracle, OracleModel
from tinyinfer_amd.backend import ARITHMETIC_FAST, HipBackend

from .helpers import pool_elements, smollm_config, upload_model, write_pools

pytestmark = pytest.mark.gpu


def rel_inf(got, want):
    return float(np.max(np.abs(got - want)) / np.max(np.abs(want)))


def margin(v):
    top = np.sort(v)[-2:]
    return float(top[1] - top[0])


NARROW = dict(layers=2, hidden=128, intermediate=192, heads=2, kv_heads=1, vocabulary=256, context=1024, eos=0,
              rms_epsilon=1e-5, rope_theta=10000.0, tied=0)


@pytest.mark.parametrize("shape", ["smollm", "narrow_untied"])
def test_fast_prefill_and_decode_track_the_oracle(torch_cuda, shape):
    """smollm: the SmolLM2 shape (tied head, 3 query heads per KV head);
    narrow_untied: hidden 128, 2 query heads on 1 KV head, an untied LM head
    (uploaded [hidden][vocab]), 192-wide SwiGLU."""
    cfg = smollm_config(layers=2, context=1024) if shape == "smollm" else dict(NARROW)
    model = OracleModel(cfg, seed=41)
    bt, max_blocks = 16, 192
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=8, arithmetic=ARITHMETIC_FAST)
    upload_model(backend, model)
    o = Oracle()
    perm = o.permutation(max_blocks, 41, 9000)
    n = pool_elements(cfg, bt, max_blocks)
    keys = np.zeros(n, dtype=np.float32)
    values = np.zeros(n, dtype=np.float32)
    lengths = [300, 17, 129, 600]
    tables = [perm[48 * i: 48 * i + 48].copy() for i in range(len(lengths))]
    for i, t in enumerate(tables):
        backend.table_write(i, 0, t)
    used = [0] * len(lengths)
    chunks = [[int(t) for t in o.fill_tokens(L, 41, 9100 + i, cfg["vocabulary"])] for i, L in enumerate(lengths)]
    worst = 0.0
    for step in range(24):
        want = [model.append(keys, values, bt, tables[i], used[i], chunks[i]) for i in range(len(lengths))]
        am, got = backend.forward([(i, used[i], len(chunks[i])) for i in range(len(lengths))],
                                  [t for ch in chunks for t in ch])
        for i in range(len(lengths)):
            assert np.all(np.isfinite(got[i]))
            err = rel_inf(got[i], want[i])
            worst = max(worst, err)
            assert err <= 1e-3, f"step {step} row {i}: relative error {err:.3e}"
            assert am[i] == int(np.argmax(got[i]))
            # A near-tie may go either way under another summation order.
            assert am[i] == int(np.argmax(want[i])) or margin(want[i]) < 1e-5, \
                f"step {step} row {i}: token differs (oracle top-2 margin {margin(want[i]):.3e})"
            used[i] += len(chunks[i])
        # Teacher-forced with the oracle's tokens: both sides extend the same history.
        chunks = [[int(np.argmax(w))] for w in want]
    print(f"max relative logit error {worst:.3e}")


def test_fast_rows_do_not_depend_on_the_batch(torch_cuda):
    """70 sequences (two row tiles) decoded together and in groups of 10
    give bit-identical logits on the matrix cores, and decoded in groups of
    4 and one by one bit-identical logits on the GEMV projections: no row's
    sums depend on the other rows of its step. (Decode steps of up to four
    sequences take the GEMV projections, larger ones the matrix cores, whose
    summation orders differ; both are held to the oracle elsewhere.)"""
    cfg = smollm_config(layers=1, context=512, vocabulary=4096)
    model = OracleModel(cfg, seed=43)
    bt, count = 16, 70
    o = Oracle()
    lengths = [int(x) for x in 5 + o.fill_tokens(count, 43, 9200, 120)]
    prompts = [[int(t) for t in o.fill_tokens(L, 43, 9300 + i, cfg["vocabulary"])] for i, L in enumerate(lengths)]
    results = {}
    def split(size):
        return [list(range(i, min(i + size, count))) for i in range(0, count, size)]

    for label, groups in (("together", [list(range(count))]), ("tens", split(10)), ("fours", split(4)),
                          ("ones", split(1))):
        backend = HipBackend(cfg, block_tokens=bt, max_blocks=count * 10, max_sequences=count,
                             arithmetic=ARITHMETIC_FAST)
        upload_model(backend, model)
        for i in range(count):
            backend.table_write(i, 0, np.arange(10 * i, 10 * i + 10, dtype=np.int32))
        out = {}
        for group in groups:
            used = {i: 0 for i in group}
            step_chunks = {i: prompts[i] for i in group}
            for step in range(3):
                am, got = backend.forward([(i, used[i], len(step_chunks[i])) for i in group],
                                          [t for i in group for t in step_chunks[i]])
                for k, i in enumerate(group):
                    out[(i, step)] = got[k].copy()
                    used[i] += len(step_chunks[i])
                    step_chunks[i] = [int(am[k])]
        results[label] = out
        backend.close()
    for key, v in results["together"].items():
        if key[1] == 0:
            continue  # prefill steps run the same kernels whatever the grouping; compared below too
        assert np.array_equal(v.view(np.uint32), results["tens"][key].view(np.uint32)), key
        assert np.array_equal(results["fours"][key].view(np.uint32), results["ones"][key].view(np.uint32)), key
    for key, v in results["together"].items():
        if key[1] == 0:
            assert np.array_equal(v.view(np.uint32), results["ones"][key].view(np.uint32)), key



def attention_probe_model(context: int, seed: int, layers: int = 1) -> OracleModel:
    """Layers whose logits follow the attention output: o_proj the
    identity, the MLP zero, an embedding 1e-3 the attention's scale and an
    untied N(0, 1) head, so a logit's relative error is about the attention
    output's (hidden 192: 3 query heads on 1 KV head of 64 dims). With two
    layers, the second layer's keys and values carry the first layer's
    attention output of every row."""
    o = Oracle()
    h, kv, inter, vocab = 192, 64, 64, 256
    cfg = dict(layers=layers, hidden=h, intermediate=inter, heads=3, kv_heads=1, vocabulary=vocab, context=context,
               eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=0)
    normal = lambda shape, std, stream: o.fill_normal(int(np.prod(shape)), seed, stream, std).reshape(shape)
    stack = [dict(input_norm=np.ones(h, np.float32), q=normal((h, h), 0.1, 1 + 10 * l),
                  k=normal((h, kv), 0.1, 2 + 10 * l), v=normal((h, kv), 0.1, 3 + 10 * l),
                  o=np.eye(h, dtype=np.float32), post_norm=np.ones(h, np.float32),
                  gate=np.zeros((h, inter), np.float32), up=np.zeros((h, inter), np.float32),
                  down=np.zeros((inter, h), np.float32)) for l in range(layers)]
    tensors = dict(layers=stack, embedding=normal((vocab, h), 1e-3, 4), final_norm=np.ones(h, np.float32),
                   lm_head=normal((h, vocab), 1.0, 5))
    return OracleModel(cfg, tensors=tensors)


@pytest.mark.parametrize("key_scale", [0.5, 6.0])
def test_fast_long_rows_merge_many_splits(torch_cuda, key_scale):
    """Decode rows whose contexts are cut into 1 to 129 splits (16,401 tokens:
    three rounds of the merge's loads; 8,251: two; 1,901; 257: the shortest
    row of 128-token splits, three of them; 256: the longest row combined in
    one work-group, 8 splits of 32 tokens; 131, 33, 17 tokens in 32- and
    16-token splits; 10: one split), over pools of
    seeded keys and values: key_scale 0.5 spreads the softmax over the whole
    context, 6.0 makes it peak at a few tokens and raises the running
    maxima inside splits. One decode step against the oracle on the same
    pools, logits within 1e-3 relative."""
    used = [16400, 8250, 1900, 256, 255, 130, 32, 16, 9]
    context = 16640
    model = attention_probe_model(context, seed=47)
    cfg = model.config
    bt = 16
    pages = [(u + 1 + bt - 1) // bt for u in used]
    max_blocks = sum(pages) + 24
    o = Oracle()
    perm = o.permutation(max_blocks, 47, 9400)
    tables, at = [], 0
    for p in pages:
        tables.append(perm[at:at + p].copy())
        at += p
    n = pool_elements(cfg, bt, max_blocks)
    keys = o.fill_normal(n, 47, 9401, key_scale)
    values = o.fill_normal(n, 47, 9402, 1.0)
    tokens = [int(t) for t in o.fill_tokens(len(used), 47, 9403, cfg["vocabulary"])]
    backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=len(used),
                         arithmetic=ARITHMETIC_FAST)
    upload_model(backend, model)
    for i, t in enumerate(tables):
        backend.table_write(i, 0, t)
    write_pools(backend, keys, values)
    am, got = backend.forward([(i, used[i], 1) for i in range(len(used))], tokens)
    worst = 0.0
    for i in range(len(used)):
        want = model.append(keys, values, bt, tables[i], used[i], [tokens[i]])
        assert np.all(np.isfinite(got[i]))
        err = rel_inf(got[i], want)
        worst = max(worst, err)
        assert err <= 1e-3, f"row {i} ({used[i] + 1} tokens): relative error {err:.3e}"
        assert am[i] == int(np.argmax(got[i]))
    backend.close()
    print(f"max relative logit error {worst:.3e}")


def test_fast_decode_rows_same_in_mixed_steps(torch_cuda):
    """A decoding row's logits are bit-identical whether its step only
    decodes or also prefills another sequence: one-token rows take the
    decode attention in both (rows of 33 to 200 tokens: one work-group;
    300 to 699 tokens: splits and merge), the prefilling rows the
    matrix-core prefill kernel, and with nine decoding sequences both steps
    run the matrix-core projections (steps of up to four decoding sequences
    run the GEMV projections instead, which sum in another order). In the
    mixed step every row is also checked against the oracle."""
    cfg = smollm_config(layers=2, context=1024, vocabulary=4096)
    model = OracleModel(cfg, seed=53)
    bt, o = 16, Oracle()
    lengths = [119, 699, 200, 450, 64, 80, 330, 520, 33, 300]  # the last one prefills in the mixed step
    dec = len(lengths) - 1
    prompts = [[int(t) for t in o.fill_tokens(L, 53, 9500 + i, cfg["vocabulary"])] for i, L in enumerate(lengths)]
    tables = [np.arange(60 * i, 60 * i + 60, dtype=np.int32) for i in range(len(lengths))]
    blocks = 60 * len(lengths)

    def run(mixed):
        backend = HipBackend(cfg, block_tokens=bt, max_blocks=blocks, max_sequences=len(lengths),
                             arithmetic=ARITHMETIC_FAST)
        upload_model(backend, model)
        for i, t in enumerate(tables):
            backend.table_write(i, 0, t)
        am, _ = backend.forward([(i, 0, lengths[i]) for i in range(dec)], [t for p in prompts[:dec] for t in p])
        nxt = [int(a) for a in am]
        steps = [(i, lengths[i], 1) for i in range(dec)] + ([(dec, 0, lengths[dec])] if mixed else [])
        _, got = backend.forward(steps, nxt + (prompts[dec] if mixed else []))
        backend.close()
        return nxt, got

    nxt, alone = run(False)
    nxt_mixed, mixed = run(True)
    assert nxt == nxt_mixed
    for i in range(dec):
        assert np.array_equal(alone[i].view(np.uint32), mixed[i].view(np.uint32)), f"row {i}"
    n = pool_elements(cfg, bt, blocks)
    keys, values = np.zeros(n, dtype=np.float32), np.zeros(n, dtype=np.float32)
    for i in range(dec):
        model.append(keys, values, bt, tables[i], 0, prompts[i])
    want = [model.append(keys, values, bt, tables[i], lengths[i], [nxt[i]]) for i in range(dec)]
    want.append(model.append(keys, values, bt, tables[dec], 0, prompts[dec]))
    for i in range(len(lengths)):
        assert rel_inf(mixed[i], want[i]) <= 1e-3, f"row {i}: relative error {rel_inf(mixed[i], want[i]):.3e}"


def test_fast_prefill_chunking_does_not_change_rows(torch_cuda):
    """A 300-token prompt prefilled in one chunk and in chunks of 100, 7 and
    193 tokens (blocks starting inside a page) gives bit-identical logits,
    and so does the decode step after it: a prefill row's attention walks
    its own keys page by page whatever block it sits in, and the
    projections sum in an order that does not depend on the row count."""
    cfg = smollm_config(layers=2, context=512, vocabulary=4096)
    model = OracleModel(cfg, seed=59)
    o = Oracle()
    prompt = [int(t) for t in o.fill_tokens(300, 59, 9600, cfg["vocabulary"])]

    def run(chunks):
        backend = HipBackend(cfg, block_tokens=16, max_blocks=40, max_sequences=1, arithmetic=ARITHMETIC_FAST)
        upload_model(backend, model)
        backend.table_write(0, 0, np.arange(8, 40, dtype=np.int32)[::-1].copy())  # 32 pages, scattered down
        used = 0
        for n in chunks:
            am, got = backend.forward([(0, used, n)], prompt[used:used + n])
            used += n
        am2, got2 = backend.forward([(0, used, 1)], [int(am[0])])
        backend.close()
        return got[0].copy(), got2[0].copy()

    one = run([300])
    three = run([100, 7, 193])
    for a, b in zip(one, three):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_fast_prefill_climbing_scores(torch_cuda):
    """Prefill rows whose scores climb by far more than the softmax's
    rescale margin of 16 across the pages a wavefront walks: 2,000 cached
    tokens of seeded keys whose scale grows from 0.25 to 12 with the
    position (scores from about +-0.3 to about +-20), then a prompt chunk of
    100 tokens on the two-layer attention probe. Each chunk's last-row
    logits are within 1e-3 relative of the oracle, and prefilling the 100
    tokens in one chunk or in chunks of 30, 7 and 63 gives bit-identical
    last-row logits."""
    used, n, bt = 2000, 100, 16
    model = attention_probe_model(4096, seed=67, layers=2)
    cfg = model.config
    o = Oracle()
    max_blocks = (used + n + bt - 1) // bt + 8
    table = o.permutation(max_blocks, 67, 9450)[: (used + n + bt - 1) // bt].copy()
    size = pool_elements(cfg, bt, max_blocks)
    keys = o.fill_normal(size, 67, 9451, 1.0).reshape(max_blocks, cfg["layers"], bt, 64)
    values = o.fill_normal(size, 67, 9452, 1.0)
    for t in range(used):  # the cached tokens' key scale grows with the position
        keys[table[t // bt], :, t % bt, :] *= np.float32(0.25 + 11.75 * (t / used) ** 2)
    keys = keys.reshape(-1)
    prompt = [int(t) for t in o.fill_tokens(n, 67, 9453, cfg["vocabulary"])]

    def run(chunks):
        backend = HipBackend(cfg, block_tokens=bt, max_blocks=max_blocks, max_sequences=1,
                             arithmetic=ARITHMETIC_FAST)
        upload_model(backend, model)
        backend.table_write(0, 0, table)
        write_pools(backend, keys, values)
        k, v = keys.copy(), values.copy()
        at, outs = used, []
        for c in chunks:
            am, got = backend.forward([(0, at, c)], prompt[at - used: at - used + c])
            want = model.append(k, v, bt, table, at, prompt[at - used: at - used + c])
            err = rel_inf(got[0], want)
            assert err <= 1e-3, f"chunk at {at} of {c} rows: relative error {err:.3e}"
            assert am[0] == int(np.argmax(got[0]))
            outs.append(got[0].copy())
            at += c
        backend.close()
        return outs

    one = run([n])
    three = run([30, 7, 63])
    assert np.array_equal(one[-1].view(np.uint32), three[-1].view(np.uint32))


def test_fast_small_batch_decode_gemv(torch_cuda):
    """Decode steps of up to four sequences take the GEMV projections
    (row-major weights, RMSNorm computed inside the projections): 90
    teacher-forced steps of one sequence from a 200-token prompt, crossing
    from the short-row attention to the splits at 256 tokens, each within
    1e-3 relative of the oracle with the oracle's greedy token; the same row
    decoded beside two others gives bit-identical logits (each row's sums
    are its own), and beside five others (matrix-core projections) it stays
    within 1e-3 of the oracle too."""
    cfg = smollm_config(layers=2, context=512, vocabulary=4096)
    model = OracleModel(cfg, seed=97)
    o = Oracle()
    bt = 16
    prompt = [int(t) for t in o.fill_tokens(200, 97, 9990, cfg["vocabulary"])]
    lengths = (90, 300, 40, 120, 230)
    others = [[int(t) for t in o.fill_tokens(n, 97, 9991 + i, cfg["vocabulary"])] for i, n in enumerate(lengths)]
    n = pool_elements(cfg, bt, 192)
    keys, values = np.zeros(n, np.float32), np.zeros(n, np.float32)
    table = np.arange(32, dtype=np.int32)
    want = model.append(keys, values, bt, table, 0, prompt)
    sizes = (1, 3, 6)  # GEMV alone and beside two others; matrix cores beside five
    backends = [HipBackend(cfg, block_tokens=bt, max_blocks=192, max_sequences=6, arithmetic=ARITHMETIC_FAST)
                for _ in sizes]
    for backend, size in zip(backends, sizes):
        upload_model(backend, model)
        for i in range(6):
            backend.table_write(i, 0, np.arange(32 * i, 32 * i + 32, dtype=np.int32))
        backend.forward([(0, 0, 200)] + [(i + 1, 0, lengths[i]) for i in range(size - 1)],
                        prompt + [t for p in others[:size - 1] for t in p])
    used = [200] + list(lengths)
    nxt = [0] * 6
    worst = 0.0
    for step in range(90):
        token = int(np.argmax(want))
        outs = []
        for backend, size in zip(backends, sizes):
            am, got = backend.forward([(i, used[i], 1) for i in range(size)], [token] + nxt[1:size])
            assert am[0] == int(np.argmax(got[0]))
            outs.append(got)
        nxt[1:] = [int(np.argmax(g)) for g in outs[2][1:]]
        want = model.append(keys, values, bt, table, used[0], [token])
        assert np.array_equal(outs[0][0].view(np.uint32), outs[1][0].view(np.uint32)), f"step {step}"
        for label, g in (("alone", outs[0][0]), ("beside five", outs[2][0])):
            err = rel_inf(g, want)
            worst = max(worst, err)
            assert err <= 1e-3, f"step {step} ({label}): relative error {err:.3e}"
            assert int(np.argmax(g)) == int(np.argmax(want)) or margin(want) < 1e-5, f"step {step} ({label})"
        used = [u + 1 for u in used]
    for backend in backends:
        backend.close()
    print(f"max relative logit error {worst:.3e}")
