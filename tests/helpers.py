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
