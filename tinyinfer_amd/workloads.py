"""The synthetic workloads of the five measured configurations.

Every workload runs a SmolLM2-135M-shaped model (30 layers, hidden 576,
9 query / 3 KV heads, head_dim 64, SwiGLU 1536, vocab 49152, tied
embeddings, RMSNorm eps 1e-5, RoPE theta 100000) with synthetic FP32
weights N(0, 0.02) and RMSNorm weights 1.0 (SplitMix64/Box-Muller streams,
synthetic.h), prompt ids uniform in [0, 49152), greedy decoding, EOS off,
pages of 16 tokens. Seeds are fixed here, so a benchmark, the fixture
generator (tests/golden/make_fixtures.py) and the GPU parity tests build the
same requests.

Engine settings: the physical pool is 1.25x the pages the requests reserve
(KVManager::reserve_request reserves ceil((prompt + new - 1) / 16) pages,
kv_manager.cpp:46; engine.cpp:66), so every request is admitted at once.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

VOCAB = 49152
PAGE = 16


def model_config(context: int) -> dict:
    return dict(layers=30, hidden=576, intermediate=1536, heads=9, kv_heads=3, vocabulary=VOCAB, context=context,
                eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)


@dataclass
class Request:
    id: str
    prompt: np.ndarray  # int32
    max_new_tokens: int
    phase: int = 0  # submitted after every request of an earlier phase finished


@dataclass
class Workload:
    name: str
    description: str
    weight_seed: int
    context: int
    requests: list
    max_batch_size: int
    token_budget: int
    prefill_chunk: int
    max_blocks: int
    prefix_cache_blocks: int = 0
    decode_batch: int = 0  # requests decoding together in a steady step
    notes: dict = field(default_factory=dict)

    def config(self) -> dict:
        return model_config(self.context)

    def engine_args(self) -> dict:
        return dict(max_batch_size=self.max_batch_size, token_budget=self.token_budget,
                    prefill_chunk=self.prefill_chunk, context=self.context)

    def kv_args(self) -> dict:
        return dict(block_tokens=PAGE, max_blocks=self.max_blocks, prefix_cache_blocks=self.prefix_cache_blocks)


def reserved_pages(prompt_tokens: int, max_new_tokens: int) -> int:
    return -(-(prompt_tokens + max_new_tokens - 1) // PAGE)


def _ids(rng, n):
    return rng.integers(0, VOCAB, size=n, dtype=np.int64).astype(np.int32)


def config2() -> Workload:
    """1 request, 128-token prompt, 128 greedy tokens."""
    rng = np.random.default_rng(20252)
    req = Request("c2", _ids(rng, 128), 128)
    pages = reserved_pages(128, 128)
    return Workload("config2", "B=1: 128-token prompt, 128 greedy decode tokens", 20252, 512, [req], 1, 128, 128,
                    math.ceil(1.25 * pages), decode_batch=1)


def config3(seed: int = 20250) -> Workload:
    """64 requests, prompts U[256, 2048], chunk 256, 128 greedy tokens each."""
    rng = np.random.default_rng(seed)
    lengths = rng.integers(256, 2048 + 1, size=64)
    prompts = [rng.integers(0, VOCAB, size=int(p), dtype=np.int64).astype(np.int32) for p in lengths]
    reqs = [Request(f"r{i}", p, 128) for i, p in enumerate(prompts)]
    pages = sum(reserved_pages(len(p), 128) for p in prompts)
    return Workload("config3", "B=64: prompts U[256,2048], chunked prefill 256, 128 greedy decode steps", seed, 4096,
                    reqs, 64, 8192, 256, math.ceil(1.25 * pages), decode_batch=64)


def config4() -> Workload:
    """A 1000-token prefix prefilled once and published (62 full pages + 8
    tokens), then 32 requests of prefix + 64 unique tokens, 64 greedy tokens
    each: every request copies the shared 8-token tail on its first append,
    and, the cache holding every page, again after every publish of a
    partial tail (engine.cpp:98, prefix_cache.cpp:147-148)."""
    rng = np.random.default_rng(20254)
    prefix = _ids(rng, 1000)
    seed = Request("prefix", prefix, 1, phase=0)
    followers = [Request(f"f{i}", np.concatenate([prefix, _ids(rng, 64)]), 64, phase=1) for i in range(32)]
    firsts = {int(f.prompt[1000]) for f in followers}
    assert len(firsts) == 32, "unique suffixes must differ at their first token"
    pages = reserved_pages(1000, 1) + sum(reserved_pages(1064, 64) for _ in followers)
    blocks = math.ceil(1.25 * pages)
    return Workload("config4", "prefix reuse + COW: 32 x (1000 shared + 64 unique), 64 greedy decode steps", 20254,
                    2048, [seed] + followers, 32, 2048, 64, blocks, prefix_cache_blocks=blocks, decode_batch=32)


def config5a() -> Workload:
    """8 requests with 16384-token prompts, chunk 512, 256 greedy tokens."""
    rng = np.random.default_rng(20255)
    reqs = [Request(f"a{i}", _ids(rng, 16384), 256) for i in range(8)]
    pages = sum(reserved_pages(16384, 256) for _ in reqs)
    return Workload("config5a", "long context: 8 x 16384-token prompts, chunk 512, 256 greedy decode steps", 20255,
                    16640, reqs, 8, 4096, 512, math.ceil(1.25 * pages), decode_batch=8)


def config5b() -> Workload:
    """256 requests with 1024-token contexts, 64 greedy tokens."""
    rng = np.random.default_rng(20256)
    reqs = [Request(f"b{i}", _ids(rng, 1024), 64) for i in range(256)]
    pages = sum(reserved_pages(1024, 64) for _ in reqs)
    return Workload("config5b", "wide batch: 256 x 1024-token contexts, 64 greedy decode steps", 20256, 2048, reqs,
                    256, 16384, 512, math.ceil(1.25 * pages), decode_batch=256)


WORKLOADS = {"config2": config2, "config3": config3, "config4": config4, "config5a": config5a, "config5b": config5b}
