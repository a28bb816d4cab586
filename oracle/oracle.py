"""ctypes access to the C oracle (oracle/libmp_oracle.so).

TEST INFRASTRUCTURE ONLY: a CPU restatement of the reference CPU path
(miniprefix/src/backend/cpu/llama_runner.cpp:10-104) used to check the HIP
backend. Build with `make -C oracle`.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "libmp_oracle.so"
REF_LIBRARY = HERE / "_ref" / "libmp_ref.so"

F32P = ctypes.POINTER(ctypes.c_float)
I32P = ctypes.POINTER(ctypes.c_int32)


class Config(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in
                ("layers", "hidden", "intermediate", "heads", "kv_heads", "vocabulary", "context", "eos")] + [
        ("rms_epsilon", ctypes.c_float), ("rope_theta", ctypes.c_float), ("tied", ctypes.c_int)]


def _f(a: np.ndarray):
    return a.ctypes.data_as(F32P)


def _i(a: np.ndarray):
    return a.ctypes.data_as(I32P)


_lib = None


def load(build: bool = True) -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIBRARY.exists() and build:
        subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
    lib = ctypes.CDLL(str(LIBRARY))
    u64, i32, c_double = ctypes.c_uint64, ctypes.c_int32, ctypes.c_double
    lib.mpo_fill_normal.argtypes = [F32P, ctypes.c_size_t, u64, u64, c_double]
    lib.mpo_fill_tokens.argtypes = [I32P, ctypes.c_size_t, u64, u64, i32]
    lib.mpo_permutation.argtypes = [I32P, i32, u64, u64]
    lib.mpo_model_synthetic.argtypes = [ctypes.POINTER(Config), u64, c_double]
    lib.mpo_model_synthetic.restype = ctypes.c_void_p
    lib.mpo_model_from_tensors.argtypes = [ctypes.POINTER(Config), F32P, F32P, ctypes.POINTER(F32P), F32P]
    lib.mpo_model_from_tensors.restype = ctypes.c_void_p
    lib.mpo_model_free.argtypes = [ctypes.c_void_p]
    lib.mpo_model_tensor.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
    lib.mpo_model_tensor.restype = F32P
    lib.mpo_append.argtypes = [ctypes.c_void_p, F32P, F32P, ctypes.c_int, I32P, ctypes.c_int, ctypes.c_int,
                               I32P, ctypes.c_int, F32P]
    lib.mpo_append.restype = ctypes.c_int
    lib.mpo_rms.argtypes = [F32P, F32P, F32P, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    lib.mpo_linear.argtypes = [F32P, F32P, F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.mpo_linear_transposed.argtypes = [F32P, F32P, F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.mpo_rope.argtypes = [F32P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    lib.mpo_rope_table.argtypes = [F32P, F32P, ctypes.c_int, ctypes.c_int, ctypes.c_float]
    lib.mpo_swiglu.argtypes = [F32P, F32P, ctypes.c_size_t]
    lib.mpo_add.argtypes = [F32P, F32P, ctypes.c_size_t]
    lib.mpo_expf.argtypes = [ctypes.c_float]
    lib.mpo_expf.restype = ctypes.c_float
    lib.mpo_attention.argtypes = [F32P, F32P, F32P, I32P] + [ctypes.c_int] * 8 + [F32P]
    _lib = lib
    return lib


def ref_library():
    """The reference's own CPU path compiled from /root/reference, if built."""
    return ctypes.CDLL(str(REF_LIBRARY)) if REF_LIBRARY.exists() else None


def smollm_config(layers: int = 30, context: int = 2048, vocabulary: int = 49152) -> dict:
    return dict(layers=layers, hidden=576, intermediate=1536, heads=9, kv_heads=3, vocabulary=vocabulary,
                context=context, eos=0, rms_epsilon=1e-5, rope_theta=100000.0, tied=1)


SLOTS = ("input_norm", "q", "k", "v", "o", "post_norm", "gate", "up", "down")


class OracleModel:
    """A synthetic (or caller-supplied) model held by the C oracle."""

    def __init__(self, config: dict, seed: int | None = 1234, stddev: float = 0.02, tensors: dict | None = None):
        self.lib = load()
        self.config = dict(config)
        self.cfg = Config(**{k: self.config[k] for k in
                             ("layers", "hidden", "intermediate", "heads", "kv_heads", "vocabulary", "context",
                              "eos", "rms_epsilon", "rope_theta", "tied")})
        if tensors is None:
            self.handle = self.lib.mpo_model_synthetic(ctypes.byref(self.cfg), seed, stddev)
        else:
            layers = self.config["layers"]
            keep = [np.ascontiguousarray(tensors["layers"][l][s], dtype=np.float32)
                    for l in range(layers) for s in SLOTS]
            arr = (F32P * len(keep))(*[_f(a) for a in keep])
            emb = np.ascontiguousarray(tensors["embedding"], dtype=np.float32)
            norm = np.ascontiguousarray(tensors["final_norm"], dtype=np.float32)
            head = tensors.get("lm_head")
            head = None if head is None else np.ascontiguousarray(head, dtype=np.float32)
            self.handle = self.lib.mpo_model_from_tensors(ctypes.byref(self.cfg), _f(emb), _f(norm), arr,
                                                          _f(head) if head is not None else None)
        if not self.handle:
            raise ValueError("invalid oracle model configuration")

    def __del__(self):
        if getattr(self, "handle", None):
            self.lib.mpo_model_free(self.handle)
            self.handle = None

    @property
    def kv_width(self) -> int:
        c = self.config
        return c["kv_heads"] * (c["hidden"] // c["heads"])

    def shape(self, layer: int, slot: int) -> tuple:
        c = self.config
        h, kv, i = c["hidden"], self.kv_width, c["intermediate"]
        if slot == -1:
            return (c["vocabulary"], h)
        if slot == -2:
            return (h,)
        if slot == -3:
            return (h, c["vocabulary"])
        return [(h,), (h, h), (h, kv), (h, kv), (h, h), (h,), (h, i), (h, i), (i, h)][slot]

    def tensor(self, layer: int, slot: int) -> np.ndarray:
        """Copy of a weight tensor (slot -1 embedding, -2 final norm, -3 untied head)."""
        p = self.lib.mpo_model_tensor(self.handle, layer, slot)
        if not p:
            raise KeyError((layer, slot))
        shape = self.shape(layer, slot)
        return np.ctypeslib.as_array(p, shape=(int(np.prod(shape)),)).reshape(shape).copy()

    def append(self, keys: np.ndarray, values: np.ndarray, block_tokens: int, blocks, used: int,
               tokens) -> np.ndarray:
        blocks = np.ascontiguousarray(blocks, dtype=np.int32)
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.empty(self.config["vocabulary"], dtype=np.float32)
        status = self.lib.mpo_append(self.handle, _f(keys), _f(values), block_tokens, _i(blocks), len(blocks),
                                     used, _i(tokens), len(tokens), _f(logits))
        if status == -1:
            raise ValueError("invalid oracle append")
        if status == -2:
            raise FloatingPointError("nonfinite logits")
        return logits


class Oracle:
    """Thin namespace for the single-op entry points."""

    def __init__(self):
        self.lib = load()

    def fill_normal(self, count: int, seed: int, stream: int, stddev: float = 1.0) -> np.ndarray:
        out = np.empty(count, dtype=np.float32)
        self.lib.mpo_fill_normal(_f(out), count, seed, stream, stddev)
        return out

    def fill_tokens(self, count: int, seed: int, stream: int, vocabulary: int) -> np.ndarray:
        out = np.empty(count, dtype=np.int32)
        self.lib.mpo_fill_tokens(_i(out), count, seed, stream, vocabulary)
        return out

    def permutation(self, count: int, seed: int, stream: int) -> np.ndarray:
        out = np.empty(count, dtype=np.int32)
        self.lib.mpo_permutation(_i(out), count, seed, stream)
        return out

    def rms(self, x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        self.lib.mpo_rms(_f(x), _f(np.ascontiguousarray(w, dtype=np.float32)), _f(out), x.shape[0], x.shape[1], eps)
        return out

    def linear(self, x: np.ndarray, w: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = np.ascontiguousarray(w, dtype=np.float32)
        out = np.empty((x.shape[0], w.shape[1]), dtype=np.float32)
        self.lib.mpo_linear(_f(x), _f(w), _f(out), x.shape[0], x.shape[1], w.shape[1])
        return out

    def rope(self, x: np.ndarray, heads: int, dim: int, start: int, theta: float) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32).copy()
        self.lib.mpo_rope(_f(x), x.shape[0], heads, dim, start, theta)
        return x

    def swiglu(self, gate: np.ndarray, up: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(gate, dtype=np.float32).copy()
        self.lib.mpo_swiglu(_f(g), _f(np.ascontiguousarray(up, dtype=np.float32)), g.size)
        return g

    def expf(self, x: np.ndarray) -> np.ndarray:
        return np.array([self.lib.mpo_expf(float(v)) for v in np.asarray(x, dtype=np.float32)], dtype=np.float32)

    def attention(self, q, keys, values, blocks, start: int, rows: int, layer: int, layers: int,
                  block_tokens: int, heads: int, kv_heads: int, dim: int) -> np.ndarray:
        q = np.ascontiguousarray(q, dtype=np.float32)
        out = np.empty((rows, heads * dim), dtype=np.float32)
        blocks = np.ascontiguousarray(blocks, dtype=np.int32)
        self.lib.mpo_attention(_f(q), _f(keys), _f(values), _i(blocks), start, rows, layer, layers, block_tokens,
                               heads, kv_heads, dim, _f(out))
        return out
