"""Python view of the device backend C ABI (include/mp_hip.h)."""
from __future__ import annotations

import ctypes

import numpy as np

from ._native import F32P, I32P, library

MP_OK, MP_INVALID_ARGUMENT, MP_DEVICE_ERROR, MP_OUT_OF_MEMORY, MP_NONFINITE = 0, -1, -2, -3, -4
TENSOR_EMBEDDING, TENSOR_FINAL_NORM, TENSOR_LM_HEAD = 100, 101, 102
ARITHMETIC_EXACT, ARITHMETIC_FAST = 0, 1


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("layers", "hidden", "intermediate", "heads", "kv_heads", "vocabulary", "context")] + [
        ("rms_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float), ("tied", ctypes.c_int32),
        ("arithmetic", ctypes.c_int32)]


class KvDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("block_tokens", "max_blocks", "max_sequences", "max_sequence_blocks")]


class TailRegion(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in ("destination", "source", "pitch", "width", "rows")]


class SeqStep(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("table_slot", "used", "count")]


class Counters(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "device_weight_bytes", "weight_uploaded_bytes", "token_uploaded_bytes", "kv_uploaded_bytes",
        "logits_downloaded_bytes", "device_allocations", "device_workspace_bytes", "block_table_uploaded_bytes",
        "block_table_device_bytes", "kv_pool_bytes", "forward_calls", "forward_rows", "cow_copies", "cow_bytes")]


class KernelTimes(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "attention_ns", "attention_launches", "projection_ns", "projection_launches", "head_ns", "head_launches")]


TIME_ATTENTION, TIME_PROJECTION, TIME_HEAD, TIME_SAMPLED = 1, 2, 4, 8


class BackendError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


def _bind(lib):
    if getattr(lib, "_mp_bound", False):
        return lib
    vp = ctypes.c_void_p
    lib.mp_hip_create.argtypes = [ctypes.POINTER(ModelDesc), ctypes.POINTER(KvDesc), ctypes.POINTER(vp)]
    lib.mp_hip_destroy.argtypes = [vp]
    lib.mp_hip_last_error.argtypes = [vp]
    lib.mp_hip_last_error.restype = ctypes.c_char_p
    lib.mp_hip_upload_tensor.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, F32P, ctypes.c_size_t]
    lib.mp_hip_ready.argtypes = [vp, I32P]
    lib.mp_hip_table_write.argtypes = [vp, ctypes.c_int32, ctypes.c_int32, I32P, ctypes.c_int32]
    lib.mp_hip_copy_tail.argtypes = [vp, ctypes.POINTER(TailRegion)]
    lib.mp_hip_forward.argtypes = [vp, ctypes.POINTER(SeqStep), ctypes.c_int32, I32P, F32P, I32P, I32P]
    lib.mp_hip_copy_tail_timed.argtypes = [vp, ctypes.POINTER(TailRegion), ctypes.POINTER(ctypes.c_uint64)]
    lib.mp_hip_paged_attention_decode.argtypes = [vp, vp, vp, vp] + [ctypes.c_int32] * 7 + [vp, vp]
    lib.mp_hip_paged_attention_decode_noalloc.argtypes = [vp, vp, vp, vp] + [ctypes.c_int32] * 7 + [vp, vp]
    lib.mp_hip_paged_attention_decode_fast.argtypes = [vp, vp, vp, vp, ctypes.c_int32, I32P] + \
        [ctypes.c_int32] * 7 + [vp, vp]
    lib.mp_hip_sync.argtypes = [vp]
    lib.mp_hip_stats.argtypes = [vp, ctypes.POINTER(Counters)]
    lib.mp_hip_kv_pools.argtypes = [vp, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t)]
    lib.mp_hip_stream.argtypes = [vp]
    lib.mp_hip_stream.restype = vp
    lib.mp_hip_set_timing.argtypes = [vp, ctypes.c_uint32]
    lib.mp_hip_kernel_times.argtypes = [vp, ctypes.POINTER(KernelTimes)]
    lib.mp_hip_set_graphs.argtypes = [vp, ctypes.c_int32]
    lib.mp_hip_graphs_captured.argtypes = [vp, I32P]
    lib._mp_bound = True
    return lib


def lib():
    return _bind(library())


class HipBackend:
    """One device context: resident weights, paged K/V pools, block tables."""

    def __init__(self, config: dict, block_tokens: int, max_blocks: int, max_sequences: int = 64,
                 max_sequence_blocks: int | None = None, arithmetic: int = ARITHMETIC_EXACT):
        self.lib = lib()
        self.config = dict(config)
        m = ModelDesc(**{k: config[k] for k in ("layers", "hidden", "intermediate", "heads", "kv_heads",
                                                "vocabulary", "context", "rms_epsilon", "rope_theta", "tied")},
                      arithmetic=arithmetic)
        if max_sequence_blocks is None:
            max_sequence_blocks = -(-config["context"] // block_tokens)
        k = KvDesc(block_tokens, max_blocks, max_sequences, max_sequence_blocks)
        handle = ctypes.c_void_p()
        status = self.lib.mp_hip_create(ctypes.byref(m), ctypes.byref(k), ctypes.byref(handle))
        if status:
            raise BackendError(status, f"mp_hip_create failed ({status})")
        self.handle = handle
        self.block_tokens = block_tokens
        self.max_blocks = max_blocks

    def close(self):
        if getattr(self, "handle", None):
            self.lib.mp_hip_destroy(self.handle)
            self.handle = None

    __del__ = close

    def _check(self, status: int):
        if status:
            raise BackendError(status, self.lib.mp_hip_last_error(self.handle).decode())

    def upload(self, layer: int, slot: int, data: np.ndarray):
        a = np.ascontiguousarray(data, dtype=np.float32)
        self._check(self.lib.mp_hip_upload_tensor(self.handle, layer, slot, a.ctypes.data_as(F32P), a.size))

    def ready(self) -> bool:
        r = ctypes.c_int32()
        self._check(self.lib.mp_hip_ready(self.handle, ctypes.byref(r)))
        return bool(r.value)

    def table_write(self, slot: int, first: int, blocks):
        b = np.ascontiguousarray(blocks, dtype=np.int32)
        self._check(self.lib.mp_hip_table_write(self.handle, slot, first, b.ctypes.data_as(I32P), b.size))

    def copy_tail(self, destination: int, source: int, pitch: int, width: int, rows: int):
        r = TailRegion(destination, source, pitch, width, rows)
        self._check(self.lib.mp_hip_copy_tail(self.handle, ctypes.byref(r)))

    def forward(self, steps, tokens, want_logits: bool = True):
        """steps: [(table_slot, used, count)], tokens: concatenated ids.
        Returns (argmax[nseq], logits[nseq, vocab] or None)."""
        n = len(steps)
        arr = (SeqStep * n)(*[SeqStep(*s) for s in steps])
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        am = np.empty(n, dtype=np.int32)
        logits = np.empty((n, self.config["vocabulary"]), dtype=np.float32) if want_logits else None
        status = self.lib.mp_hip_forward(self.handle, arr, n, t.ctypes.data_as(I32P),
                                         logits.ctypes.data_as(F32P) if want_logits else None,
                                         am.ctypes.data_as(I32P), None)
        if status == MP_NONFINITE:
            raise FloatingPointError(self.lib.mp_hip_last_error(self.handle).decode())
        self._check(status)
        return am, logits

    def sync(self):
        self._check(self.lib.mp_hip_sync(self.handle))

    def stats(self) -> dict:
        c = Counters()
        self._check(self.lib.mp_hip_stats(self.handle, ctypes.byref(c)))
        return {n: getattr(c, n) for n, _ in Counters._fields_}

    def kv_pools(self):
        k, v, n = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_size_t()
        self._check(self.lib.mp_hip_kv_pools(self.handle, ctypes.byref(k), ctypes.byref(v), ctypes.byref(n)))
        return k.value, v.value, n.value

    def stream(self) -> int:
        return self.lib.mp_hip_stream(self.handle)


def set_timing(handle: int, classes: int):
    """Enables HIP-event timing of forward launches of a device context."""
    status = lib().mp_hip_set_timing(handle, classes)
    if status:
        raise BackendError(status, lib().mp_hip_last_error(handle).decode())


def set_graphs(handle: int, enabled: bool):
    """Graph replay of decode steps on a device context (mp_hip*)."""
    status = lib().mp_hip_set_graphs(handle, int(enabled))
    if status:
        raise BackendError(status, "mp_hip_set_graphs failed")


def graphs_captured(handle: int) -> int:
    n = np.zeros(1, dtype=np.int32)
    status = lib().mp_hip_graphs_captured(handle, n.ctypes.data_as(I32P))
    if status:
        raise BackendError(status, "mp_hip_graphs_captured failed")
    return int(n[0])


def kernel_times(handle: int) -> dict:
    t = KernelTimes()
    status = lib().mp_hip_kernel_times(handle, ctypes.byref(t))
    if status:
        raise BackendError(status, "mp_hip_kernel_times failed")
    return {n: getattr(t, n) for n, _ in KernelTimes._fields_}


def paged_attention_decode(q, keys, values, table, length: int, layer: int, layers: int, block_tokens: int,
                           heads: int, kv_heads: int, dim: int, out, stream: int | None = None):
    """Stand-alone decode attention over device buffers (raw device pointers)."""
    status = lib().mp_hip_paged_attention_decode(q, keys, values, table, length, layer, layers, block_tokens,
                                                 heads, kv_heads, dim, out, stream)
    if status:
        message = (lib().mp_hip_last_error(None) or b"").decode()
        raise BackendError(status, f"mp_hip_paged_attention_decode failed ({status}): {message}")


def paged_attention_decode_noalloc(q, keys, values, table, length: int, layer: int, layers: int,
                                   block_tokens: int, heads: int, kv_heads: int, dim: int, out,
                                   stream: int | None = None):
    """The same attention with no allocation (the library's static device
    scratch holds a long row's scores)."""
    status = lib().mp_hip_paged_attention_decode_noalloc(q, keys, values, table, length, layer, layers,
                                                         block_tokens, heads, kv_heads, dim, out, stream)
    if status:
        message = (lib().mp_hip_last_error(None) or b"").decode()
        raise BackendError(status, f"mp_hip_paged_attention_decode_noalloc failed ({status}): {message}")


def paged_attention_decode_fast(q, keys, values, tables, table_stride: int, lengths, layer: int, layers: int,
                                heads: int, kv_heads: int, out, stream: int | None = None):
    """The fast arithmetic's decode attention of len(lengths) rows over
    device buffers (raw device pointers; pools in the device page order,
    row r's table at tables + r * table_stride). Synchronous."""
    n = np.ascontiguousarray(lengths, dtype=np.int32)
    status = lib().mp_hip_paged_attention_decode_fast(q, keys, values, tables, table_stride, n.ctypes.data_as(I32P),
                                                      n.size, layer, layers, 16, heads, kv_heads, 64, out, stream)
    if status:
        message = (lib().mp_hip_last_error(None) or b"").decode()
        raise BackendError(status, f"mp_hip_paged_attention_decode_fast failed ({status}): {message}")
