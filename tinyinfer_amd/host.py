"""Python view of the host runtime's C entry points (include/miniprefix_c.h):
Engine, ModelRunner and weights.

The same entry points are exported by this package's native library and,
for tests, by a build of the reference's own sources; `library` selects
which one a Weights/Runner/Engine talks to (default: this package's).
"""
from __future__ import annotations

import ctypes
import json

import numpy as np

from ._native import F32P, I32P, library as _product_library

vp = ctypes.c_void_p
U64P = ctypes.POINTER(ctypes.c_uint64)

MPX_OK, MPX_INVALID_ARGUMENT, MPX_RUNTIME_ERROR, MPX_KV_CAPACITY, MPX_LOGIC_ERROR, MPX_OTHER = 0, -1, -2, -5, -6, -7

RUNNER_STATS_FIELDS = (
    "live_sequences", "live_kv_bytes", "peak_kv_bytes", "forward_tokens", "device_weight_bytes",
    "weight_uploaded_bytes", "token_uploaded_bytes", "kv_uploaded_bytes", "logits_downloaded_bytes",
    "device_allocations", "device_workspace_bytes", "kv_block_tokens", "kv_total_blocks", "kv_live_blocks",
    "kv_peak_blocks", "kv_reserved_bytes", "block_table_uploaded_bytes", "block_table_device_bytes",
    "prefix_cache_capacity", "kv_cached_blocks", "kv_cache_only_blocks", "prefix_hits", "prefix_misses",
    "prefix_reused_tokens", "prefix_evictions")
COST_STATS_FIELDS = ("lookup_calls", "lookup_ns", "publish_calls", "publish_ns", "cow_pages", "cow_bytes",
                     "cow_copy_ns", "cow_timed_copies")
ADMISSION = ("ready", "wait", "impossible")


class KvCapacityError(RuntimeError):
    """miniprefix::KvCapacityError."""


class MpxLogicError(RuntimeError):
    """std::logic_error."""


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("layers", "hidden", "intermediate", "heads", "kv_heads", "vocabulary", "context", "eos")] + [
        ("rms_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float), ("tied", ctypes.c_int32)]


def smollm_config(layers: int = 30, context: int = 2048, vocabulary: int = 49152) -> dict:
    """SmolLM2-135M shape (hidden 576, 9/3 heads, SwiGLU 1536, tied head)."""
    return dict(layers=layers, hidden=576, intermediate=1536, heads=9, kv_heads=3, vocabulary=vocabulary,
                context=context, eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)


def bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    if getattr(lib, "_mpx_bound", False):
        return lib
    c = ctypes.c_char_p
    i32, u32, u64, sz = ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_size_t
    sig = {
        "mpx_last_error": ([], c),
        "mpx_weights_synthetic": ([ctypes.POINTER(Config), u64, ctypes.c_double], vp),
        "mpx_weights_load": ([c], vp),
        "mpx_weights_config": ([vp, ctypes.POINTER(Config)], ctypes.c_int),
        "mpx_weights_tensor": ([vp, c, ctypes.POINTER(F32P), ctypes.POINTER(sz)], ctypes.c_int),
        "mpx_weights_set": ([vp, c, F32P, sz], ctypes.c_int),
        "mpx_weights_free": ([vp], None),
        "mpx_runner_create": ([vp, i32, i32, i32, i32, i32], vp),
        "mpx_runner_free": ([vp], None),
        "mpx_runner_reserve": ([vp, c, sz, I32P], ctypes.c_int),
        "mpx_runner_release_reservation": ([vp, c], ctypes.c_int),
        "mpx_runner_create_sequence": ([vp, c], ctypes.c_int),
        "mpx_runner_fork": ([vp, c, c], ctypes.c_int),
        "mpx_runner_reuse_prefix": ([vp, c, I32P, i32, ctypes.POINTER(sz)], ctypes.c_int),
        "mpx_runner_cache_prefix": ([vp, c], ctypes.c_int),
        "mpx_runner_clear_prefix_cache": ([vp], ctypes.c_int),
        "mpx_runner_append": ([vp, c, I32P, i32, F32P], ctypes.c_int),
        "mpx_runner_release": ([vp, c], ctypes.c_int),
        "mpx_runner_clear": ([vp], ctypes.c_int),
        "mpx_runner_stats": ([vp, U64P], ctypes.c_int),
        "mpx_runner_cost_stats": ([vp, U64P], ctypes.c_int),
        "mpx_runner_set_cost_timing": ([vp, i32], ctypes.c_int),
        "mpx_runner_sequence": ([vp, c, I32P, i32, I32P, I32P], ctypes.c_int),
        "mpx_runner_device": ([vp], vp),
        "mpx_runner_keep_logits": ([vp, i32], ctypes.c_int),
        "mpx_runner_kept_logits": ([vp, c, F32P, sz, ctypes.POINTER(sz)], ctypes.c_int),
        "mpx_engine_create": ([vp, i32, i32, i32, i32], vp),
        "mpx_engine_free": ([vp], None),
        "mpx_engine_set_batching": ([vp, i32], ctypes.c_int),
        "mpx_engine_submit": ([vp, c, I32P, i32, u32, i32], ctypes.c_int),
        "mpx_engine_step": ([vp, I32P], ctypes.c_int),
        "mpx_engine_poll": ([vp, ctypes.c_char_p, sz, ctypes.POINTER(sz)], ctypes.c_int),
        "mpx_engine_cancel": ([vp, c], ctypes.c_int),
        "mpx_engine_shutdown": ([vp], ctypes.c_int),
        "mpx_engine_state": ([vp, I32P, I32P], ctypes.c_int),
        "mpx_engine_step_stats": ([vp, U64P], ctypes.c_int),
        "mpx_engine_runner": ([vp], vp),
    }
    for name, (args, res) in sig.items():
        f = getattr(lib, name)
        f.argtypes = args
        f.restype = res
    lib._mpx_bound = True
    return lib


def _check(lib, status: int):
    if status == MPX_OK:
        return
    message = (lib.mpx_last_error() or b"").decode()
    if status == MPX_KV_CAPACITY:
        raise KvCapacityError(message)
    if status == MPX_INVALID_ARGUMENT:
        raise ValueError(message)
    if status == MPX_LOGIC_ERROR:
        raise MpxLogicError(message)
    if status == MPX_OTHER:
        raise LookupError(message)
    raise RuntimeError(message)


def _b(s: str) -> bytes:
    return s.encode()


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


class Weights:
    """ModelWeights: synthetic (seeded) or loaded from an MPFX0001 file."""

    def __init__(self, handle, lib):
        self.lib, self.handle = lib, handle

    @classmethod
    def synthetic(cls, config: dict, seed: int = 1234, stddev: float = 0.02, library=None) -> "Weights":
        lib = bind(library or _product_library())
        cfg = Config(**{k: config[k] for k in (f for f, _ in Config._fields_)})
        h = lib.mpx_weights_synthetic(ctypes.byref(cfg), seed, stddev)
        if not h:
            _check(lib, MPX_INVALID_ARGUMENT)
        return cls(h, lib)

    @classmethod
    def load(cls, path: str, library=None) -> "Weights":
        lib = bind(library or _product_library())
        h = lib.mpx_weights_load(_b(path))
        if not h:
            _check(lib, MPX_RUNTIME_ERROR)
        return cls(h, lib)

    def config(self) -> dict:
        c = Config()
        _check(self.lib, self.lib.mpx_weights_config(self.handle, ctypes.byref(c)))
        return {n: getattr(c, n) for n, _ in Config._fields_}

    def tensor(self, name: str) -> np.ndarray:
        p, n = F32P(), ctypes.c_size_t()
        _check(self.lib, self.lib.mpx_weights_tensor(self.handle, _b(name), ctypes.byref(p), ctypes.byref(n)))
        return np.ctypeslib.as_array(p, shape=(n.value,)).copy()

    def set_tensor(self, name: str, data: np.ndarray):
        a = np.ascontiguousarray(data, dtype=np.float32).ravel()
        _check(self.lib, self.lib.mpx_weights_set(self.handle, _b(name), a.ctypes.data_as(F32P), a.size))

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mpx_weights_free(self.handle)
            self.handle = None

    __del__ = close


class Runner:
    """ModelRunner (model.h:35-58 of the reference)."""

    def __init__(self, weights: Weights, context: int, block_tokens: int = 16, max_blocks: int = 128,
                 prefix_cache_blocks: int = 0, kind: int = 0):
        self.lib = weights.lib
        self.weights = weights
        self.vocabulary = weights.config()["vocabulary"]
        self.handle = self.lib.mpx_runner_create(weights.handle, kind, context, block_tokens, max_blocks,
                                                 prefix_cache_blocks)
        if not self.handle:
            _check(self.lib, MPX_INVALID_ARGUMENT if "invalid" in (self.lib.mpx_last_error() or b"").decode()
                   else MPX_RUNTIME_ERROR)
        self.owned = True

    def close(self):
        if getattr(self, "handle", None) and self.owned:
            self.lib.mpx_runner_free(self.handle)
        self.handle = None

    __del__ = close

    def reserve_request(self, rid: str, tokens: int) -> str:
        a = ctypes.c_int32()
        _check(self.lib, self.lib.mpx_runner_reserve(self.handle, _b(rid), tokens, ctypes.byref(a)))
        return ADMISSION[a.value]

    def release_reservation(self, rid: str):
        _check(self.lib, self.lib.mpx_runner_release_reservation(self.handle, _b(rid)))

    def create(self, rid: str):
        _check(self.lib, self.lib.mpx_runner_create_sequence(self.handle, _b(rid)))

    def fork_sequence(self, source: str, target: str):
        _check(self.lib, self.lib.mpx_runner_fork(self.handle, _b(source), _b(target)))

    def reuse_prefix(self, rid: str, prompt) -> int:
        p = _i32(prompt)
        n = ctypes.c_size_t()
        _check(self.lib, self.lib.mpx_runner_reuse_prefix(self.handle, _b(rid), p.ctypes.data_as(I32P), p.size,
                                                          ctypes.byref(n)))
        return n.value

    def cache_prefix(self, rid: str):
        _check(self.lib, self.lib.mpx_runner_cache_prefix(self.handle, _b(rid)))

    def clear_prefix_cache(self):
        _check(self.lib, self.lib.mpx_runner_clear_prefix_cache(self.handle))

    def append(self, rid: str, tokens) -> np.ndarray:
        t = _i32(tokens)
        logits = np.empty(self.vocabulary, dtype=np.float32)
        _check(self.lib, self.lib.mpx_runner_append(self.handle, _b(rid), t.ctypes.data_as(I32P), t.size,
                                                    logits.ctypes.data_as(F32P)))
        return logits

    def release(self, rid: str):
        _check(self.lib, self.lib.mpx_runner_release(self.handle, _b(rid)))

    def clear(self):
        _check(self.lib, self.lib.mpx_runner_clear(self.handle))

    def stats(self) -> dict:
        out = (ctypes.c_uint64 * 25)()
        _check(self.lib, self.lib.mpx_runner_stats(self.handle, out))
        return dict(zip(RUNNER_STATS_FIELDS, list(out)))

    def cost_stats(self) -> dict:
        out = (ctypes.c_uint64 * 8)()
        _check(self.lib, self.lib.mpx_runner_cost_stats(self.handle, out))
        return dict(zip(COST_STATS_FIELDS, list(out)))

    def set_cost_timing(self, enabled: bool):
        _check(self.lib, self.lib.mpx_runner_set_cost_timing(self.handle, int(enabled)))

    def keep_logits(self, enabled: bool = True):
        """Keep every forward's last-row logits per sequence on the host (also
        in the batched Engine step, which otherwise downloads only the argmax)."""
        _check(self.lib, self.lib.mpx_runner_keep_logits(self.handle, int(enabled)))

    def kept_logits(self, rid: str) -> np.ndarray:
        """The last-row logits of sequence rid's latest forward (keep_logits)."""
        out = np.empty(self.vocabulary, dtype=np.float32)
        n = ctypes.c_size_t()
        _check(self.lib, self.lib.mpx_runner_kept_logits(self.handle, _b(rid), out.ctypes.data_as(F32P), out.size,
                                                         ctypes.byref(n)))
        assert n.value == out.size
        return out

    def device(self) -> int | None:
        """The runner's device context (mp_hip*), or None."""
        return self.lib.mpx_runner_device(self.handle)

    def sequence(self, rid: str) -> tuple[list[int], int]:
        """(page table, used tokens) of a committed sequence."""
        blocks = getattr(self, "_table_buffer", None)
        if blocks is None:
            blocks = self._table_buffer = np.empty(1 << 12, dtype=np.int32)
        n, used = ctypes.c_int32(), ctypes.c_int32()
        _check(self.lib, self.lib.mpx_runner_sequence(self.handle, _b(rid), blocks.ctypes.data_as(I32P), blocks.size,
                                                      ctypes.byref(n), ctypes.byref(used)))
        if n.value > blocks.size:  # grow and read again
            self._table_buffer = np.empty(n.value, dtype=np.int32)
            return self.sequence(rid)
        return blocks[: n.value].tolist(), used.value


class Engine:
    """Engine (engine.h:12-36 of the reference); owns its runner."""

    def __init__(self, runner: Runner, max_batch_size: int = 2, token_budget: int = 32, prefill_chunk: int = 16,
                 context: int = 512):
        self.lib = runner.lib
        h = self.lib.mpx_engine_create(runner.handle, max_batch_size, token_budget, prefill_chunk, context)
        if not h:
            _check(self.lib, MPX_INVALID_ARGUMENT)
        self.handle = h
        runner.owned = False  # the engine frees it; the handle stays a borrowed view
        self.runner = runner
        self._poll_buffer = ctypes.create_string_buffer(1 << 16)

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mpx_engine_free(self.handle)
            self.handle = None
            self.runner.handle = None

    __del__ = close

    def set_batching(self, enabled: bool):
        _check(self.lib, self.lib.mpx_engine_set_batching(self.handle, int(enabled)))

    def submit(self, rid: str, prompt, max_new_tokens: int = 32, eos_token_id: int | None = None):
        p = _i32(prompt)
        _check(self.lib, self.lib.mpx_engine_submit(self.handle, _b(rid), p.ctypes.data_as(I32P), p.size,
                                                    max_new_tokens, -1 if eos_token_id is None else eos_token_id))

    def step(self) -> bool:
        progressed = ctypes.c_int32()
        _check(self.lib, self.lib.mpx_engine_step(self.handle, ctypes.byref(progressed)))
        return bool(progressed.value)

    def poll_events(self) -> list[dict]:
        # One call into a reused buffer; the library keeps the events until
        # a call whose buffer holds them, so a short buffer is grown and the
        # call repeated.
        needed = ctypes.c_size_t()
        while True:
            buf = self._poll_buffer
            _check(self.lib, self.lib.mpx_engine_poll(self.handle, buf, len(buf), ctypes.byref(needed)))
            if needed.value < len(buf):
                return json.loads(buf.value)
            self._poll_buffer = ctypes.create_string_buffer(2 * (needed.value + 1))

    def cancel(self, rid: str):
        _check(self.lib, self.lib.mpx_engine_cancel(self.handle, _b(rid)))

    def shutdown(self):
        _check(self.lib, self.lib.mpx_engine_shutdown(self.handle))

    def state(self) -> tuple[bool, bool]:
        idle, failed = ctypes.c_int32(), ctypes.c_int32()
        _check(self.lib, self.lib.mpx_engine_state(self.handle, ctypes.byref(idle), ctypes.byref(failed)))
        return bool(idle.value), bool(failed.value)

    def idle(self) -> bool:
        return self.state()[0]

    def failed(self) -> bool:
        return self.state()[1]

    def last_step_stats(self) -> dict:
        out = (ctypes.c_uint64 * 3)()
        _check(self.lib, self.lib.mpx_engine_step_stats(self.handle, out))
        return dict(zip(("prefix_reused_tokens", "prefill_tokens", "decode_tokens"), list(out)))
