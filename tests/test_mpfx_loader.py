"""MPFX0001 checkpoints (miniprefix/src/model/model.cpp:20-56; writer
miniprefix/tools/prepare_model.py:33-51): files written here in that
format load into identical tensors through this repository's loader and
through the reference's own loader (compiled from its sources, oracle/_ref),
and malformed files are refused by both with the same message. On the GPU,
a runner over the loaded file produces the logits of a runner over the
weights the file was written from."""
import struct

import numpy as np
import pytest

from tinyinfer_amd.host import Runner, Weights

from .helpers import reference_library, tiny_config


def tensor_names(c):
    names = ["model.embed_tokens.weight", "model.norm.weight"] + ([] if c["tied"] else ["lm_head.weight"])
    for l in range(c["layers"]):
        for s in ("input_layernorm", "self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                  "post_attention_layernorm", "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"):
            names.append(f"model.layers.{l}.{s}.weight")
    return names


def shape_of(c, name):
    h, i, v = c["hidden"], c["intermediate"], c["vocabulary"]
    kv = c["kv_heads"] * h // c["heads"]
    if name == "model.embed_tokens.weight":
        return (v, h)
    if name == "lm_head.weight":
        return (h, v)
    if name.endswith("norm.weight"):
        return (h,)
    for key, shape in (("q_proj", (h, h)), ("o_proj", (h, h)), ("k_proj", (h, kv)), ("v_proj", (h, kv)),
                       ("gate_proj", (h, i)), ("up_proj", (h, i)), ("down_proj", (i, h))):
        if key in name:
            return shape
    raise KeyError(name)


def write_mpfx(path, c, tensors, names=None, magic=b"MPFX0001", tied=None, trailing=b"", count=None):
    """The on-disk format of prepare_model.py:33-51 (little endian):
    magic, 8 int32 fields, eps and theta float32, uint32 tied, uint32 count,
    then name length, name, rank, int32 dims, uint64 bytes and FP32 data."""
    names = tensor_names(c) if names is None else names
    with open(path, "wb") as f:
        f.write(magic)
        f.write(struct.pack("<8i2fII", c["layers"], c["hidden"], c["intermediate"], c["heads"], c["kv_heads"],
                            c["vocabulary"], c["context"], c["eos"], c["rms_epsilon"], c["rope_theta"],
                            c["tied"] if tied is None else tied, len(names) if count is None else count))
        for name in names:
            shape = shape_of(c, name) if name in tensor_names(c) else np.shape(tensors[name])
            value = np.asarray(tensors[name], dtype="<f4").reshape(shape)
            encoded = name.encode()
            f.write(struct.pack("<I", len(encoded)) + encoded)
            f.write(struct.pack("<I", value.ndim) + struct.pack("<" + "i" * value.ndim, *value.shape))
            f.write(struct.pack("<Q", value.nbytes))
            f.write(value.tobytes())
        f.write(trailing)


def source_tensors(c, seed=5):
    w = Weights.synthetic(c, seed=seed, stddev=0.05)
    return {n: w.tensor(n) for n in tensor_names(c)}


def loaders():
    out = [("repo", None)]
    ref = reference_library()
    if ref is not None:
        out.append(("reference", ref))
    return out


@pytest.mark.parametrize("tied", [0, 1])
def test_round_trip_through_both_loaders(tmp_path, tied):
    c = tiny_config(tied=tied, vocabulary=40)
    tensors = source_tensors(c)
    path = tmp_path / "model.mpf"
    write_mpfx(path, c, tensors)
    for label, lib in loaders():
        w = Weights.load(str(path), library=lib)
        got = w.config()
        for k in ("layers", "hidden", "intermediate", "heads", "kv_heads", "vocabulary", "context", "eos", "tied"):
            assert got[k] == c[k], (label, k)
        for name, want in tensors.items():
            assert np.array_equal(w.tensor(name).view(np.uint32), np.asarray(want, np.float32).view(np.uint32)), \
                (label, name)


def malformed(c, tensors):
    names = tensor_names(c)
    bad_nan = dict(tensors)
    bad_nan[names[3]] = np.array(tensors[names[3]], np.float32)
    bad_nan[names[3]][0] = np.nan
    extra = dict(tensors)
    extra["model.layers.0.extra.weight"] = np.zeros(c["hidden"], np.float32)
    return {
        "magic": dict(magic=b"MPFX0002"),
        "tied flag": dict(tied=2),
        "count": dict(count=len(names) + 1),
        "unknown tensor": dict(names=names[:-1] + ["model.layers.0.extra.weight"], tensors=extra),
        "duplicate tensor": dict(names=names[:-1] + [names[0]]),
        "nonfinite": dict(tensors=bad_nan),
        "trailing data": dict(trailing=b"\0"),
    }


def test_malformed_files_are_refused_alike(tmp_path):
    c = tiny_config(vocabulary=40)
    tensors = source_tensors(c)
    cases = malformed(c, tensors)
    truncated = tmp_path / "truncated.mpf"
    write_mpfx(truncated, c, tensors)
    truncated.write_bytes(truncated.read_bytes()[:-7])
    paths = {"truncated": truncated}
    for label, kw in cases.items():
        p = tmp_path / (label.replace(" ", "_") + ".mpf")
        kw = dict(kw)
        write_mpfx(p, c, kw.pop("tensors", tensors), **kw)
        paths[label] = p
    # A tensor of the wrong shape: a k projection written as a q projection.
    wrong = tmp_path / "shape.mpf"
    names = tensor_names(c)
    swapped = dict(tensors)
    k_name = "model.layers.0.self_attn.k_proj.weight"
    with open(wrong, "wb") as f:
        f.write(b"MPFX0001")
        f.write(struct.pack("<8i2fII", c["layers"], c["hidden"], c["intermediate"], c["heads"], c["kv_heads"],
                            c["vocabulary"], c["context"], c["eos"], c["rms_epsilon"], c["rope_theta"], c["tied"],
                            len(names)))
        for name in names:
            shape = (c["hidden"], c["hidden"]) if name == k_name else shape_of(c, name)
            value = np.zeros(shape, "<f4") if name == k_name else np.asarray(swapped[name], "<f4").reshape(shape)
            f.write(struct.pack("<I", len(name)) + name.encode())
            f.write(struct.pack("<I", value.ndim) + struct.pack("<" + "i" * value.ndim, *value.shape))
            f.write(struct.pack("<Q", value.nbytes))
            f.write(value.tobytes())
    paths["shape"] = wrong
    messages = {}
    for label, lib in loaders():
        for case, p in paths.items():
            with pytest.raises(RuntimeError) as error:
                Weights.load(str(p), library=lib)
            messages.setdefault(case, {})[label] = str(error.value)
    for case, by_loader in messages.items():
        assert len(set(by_loader.values())) == 1, (case, by_loader)


@pytest.mark.gpu
def test_loaded_checkpoint_runs_on_the_device(torch_cuda, tmp_path):
    c = dict(tiny_config(vocabulary=40))
    tensors = source_tensors(c, seed=9)
    path = tmp_path / "model.mpf"
    write_mpfx(path, c, tensors)
    loaded = Runner(Weights.load(str(path)), context=32, block_tokens=4, max_blocks=16)
    direct_weights = Weights.synthetic(c, seed=9, stddev=0.05)
    direct = Runner(direct_weights, context=32, block_tokens=4, max_blocks=16)
    for r in (loaded, direct):
        r.create("s")
    for chunk in ([1, 2, 3, 4, 5], [6], [7, 8]):
        a, b = loaded.append("s", chunk), direct.append("s", chunk)
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
