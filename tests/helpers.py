"""Shared test helpers: upload oracle weights to the HIP backend, seeded pools."""
from __future__ import annotations

import numpy as np

from oracle import OracleModel
from tinyinfer_amd.backend import HipBackend, TENSOR_EMBEDDING, TENSOR_FINAL_NORM, TENSOR_LM_HEAD


def tiny_config(**overrides) -> dict:
    # The reference's device regression model (miniprefix/tests/cow_test.cpp:118-121).
    c = dict(layers=2, hidden=8, intermediate=12, heads=2, kv_heads=1, vocabulary=16, context=32, eos=0,
             rms_epsilon=1e-5, rope_theta=10000.0, tied=0)
    c.update(overrides)
    return c


def smollm_config(layers: int = 30, context: int = 2048, vocabulary: int = 49152) -> dict:
    return dict(layers=layers, hidden=576, intermediate=1536, heads=9, kv_heads=3, vocabulary=vocabulary,
                context=context, eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)


def upload_model(backend: HipBackend, model: OracleModel):
    c = model.config
    backend.upload(-1, TENSOR_EMBEDDING, model.tensor(0, -1))
    backend.upload(-1, TENSOR_FINAL_NORM, model.tensor(0, -2))
    if not c["tied"]:
        backend.upload(-1, TENSOR_LM_HEAD, model.tensor(0, -3))
    for layer in range(c["layers"]):
        for slot in range(9):
            backend.upload(layer, slot, model.tensor(layer, slot))
    assert backend.ready()


def pool_elements(config: dict, block_tokens: int, max_blocks: int) -> int:
    kv = config["kv_heads"] * (config["hidden"] // config["heads"])
    return max_blocks * config["layers"] * block_tokens * kv


def reference_library():
    """The reference's own MiniPrefix (Engine, KVManager, CpuRunner) compiled
    from its sources into oracle/_ref, or None if not built."""
    from oracle import ref_library
    return ref_library()


def sin_weight_tensors() -> dict:
    """The device regression model of the reference's cow_test.cpp:118-137:
    tiny_config() shape, every non-norm weight 0.15f*sinf(k) for k = 1, 2, ...
    in the order the reference adds them, norms 1, and embedding row 15 NaN
    (appending token 15 makes any runner produce non-finite logits)."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.sinf.restype = ctypes.c_float
    libm.sinf.argtypes = [ctypes.c_float]
    counter = [0]

    def fill(shape, norm=False):
        n = int(np.prod(shape))
        if norm:
            return np.ones(n, dtype=np.float32)
        out = np.empty(n, dtype=np.float32)
        for i in range(n):
            counter[0] += 1
            out[i] = np.float32(0.15) * np.float32(libm.sinf(float(counter[0])))
        return out

    t = {"model.embed_tokens.weight": fill((16, 8)), "lm_head.weight": fill((8, 16)),
         "model.norm.weight": fill((8,), True)}
    for layer in range(2):
        p = f"model.layers.{layer}."
        t[p + "input_layernorm.weight"] = fill((8,), True)
        t[p + "post_attention_layernorm.weight"] = fill((8,), True)
        for name, shape in (("self_attn.q_proj", (8, 8)), ("self_attn.k_proj", (8, 4)), ("self_attn.v_proj", (8, 4)),
                            ("self_attn.o_proj", (8, 8)), ("mlp.gate_proj", (8, 12)), ("mlp.up_proj", (8, 12)),
                            ("mlp.down_proj", (12, 8))):
            t[p + name + ".weight"] = fill(shape)
    t["model.embed_tokens.weight"][15 * 8:16 * 8] = np.nan
    return t


def weights_with(tensors: dict, config: dict, library=None):
    from tinyinfer_amd.host import Weights
    w = Weights.synthetic(config, seed=1, stddev=0.02, library=library)
    for name, data in tensors.items():
        w.set_tensor(name, data)
    return w


def device_key_order(pool: np.ndarray, blocks: int, layers: int, kv_heads: int) -> np.ndarray:
    """A K pool of 16-token pages and 64-dim heads from the reference order
    (block, layer, slot, kv head, d) to the device order: per (block,
    layer), kv head major, then [d/4][slot][4]."""
    p = pool.reshape(blocks, layers, 16, kv_heads, 16, 4)  # slot, head, d/4, d%4
    return np.ascontiguousarray(p.transpose(0, 1, 3, 4, 2, 5)).reshape(-1)


def device_value_order(pool: np.ndarray, blocks: int, layers: int, kv_heads: int) -> np.ndarray:
    """The V pool likewise: per (block, layer), kv head major, then
    [slot/4][d][4]."""
    p = pool.reshape(blocks, layers, 4, 4, kv_heads, 64)  # slot/4, slot%4, head, d
    return np.ascontiguousarray(p.transpose(0, 1, 4, 2, 5, 3)).reshape(-1)


def write_pools(backend: HipBackend, keys: np.ndarray, values: np.ndarray):
    """Host pools in the reference order into a context's device pools
    (16-token pages, 64-dim heads)."""
    import ctypes
    c = backend.config
    layers, kv_heads = c["layers"], c["kv_heads"]
    assert c["hidden"] // c["heads"] == 64 and backend.block_tokens == 16
    k_ptr, v_ptr, n = backend.kv_pools()
    page = layers * 16 * kv_heads * 64
    assert keys.size == n and values.size == n and n % page == 0
    hip = ctypes.CDLL("libamdhip64.so.7")  # the HIP runtime this process has loaded
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    backend.sync()
    for ptr, data in ((k_ptr, device_key_order(keys, n // page, layers, kv_heads)),
                      (v_ptr, device_value_order(values, n // page, layers, kv_heads))):
        data = np.ascontiguousarray(data, dtype=np.float32)
        assert data.size == n
        assert hip.hipMemcpy(ptr, data.ctypes.data, data.nbytes, 1) == 0  # host to device
