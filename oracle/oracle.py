"""TEST INFRASTRUCTURE ONLY: ctypes wrapper of the CPU oracle
(oracle/qwen_oracle.cpp, a restatement of the reference's Rust CPU forward
pass). Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker. The product never imports it."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "lib" / "libqwen_oracle.so"
REF_BRIDGE = HERE / "_ref" / "libqwen_rocm_test.so"

REFERENCE, VECTOR = 0, 2

_TRACE = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                          ctypes.c_int64)
_F = ctypes.POINTER(ctypes.c_float)
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            raise RuntimeError(f"oracle library missing: {LIB} (run __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB))
        L.qo_error.restype = ctypes.c_char_p
        L.qo_model_create.restype = ctypes.c_void_p
        L.qo_model_create.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.qo_model_free.argtypes = [ctypes.c_void_p]
        L.qo_model_set_lm_head.argtypes = [ctypes.c_void_p, _F]
        L.qo_state_create.restype = ctypes.c_void_p
        L.qo_state_create.argtypes = [ctypes.c_void_p]
        L.qo_state_clone.restype = ctypes.c_void_p
        L.qo_state_clone.argtypes = [ctypes.c_void_p]
        L.qo_state_free.argtypes = [ctypes.c_void_p]
        L.qo_state_position.restype = ctypes.c_int64
        L.qo_state_position.argtypes = [ctypes.c_void_p]
        L.qo_state_size.restype = ctypes.c_int64
        L.qo_state_size.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.qo_state_read.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _F]
        L.qo_step.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int, _F, _F, _TRACE,
                              ctypes.c_void_p]
        L.qo_select_greedy.restype = ctypes.c_int64
        L.qo_select_greedy.argtypes = [_F, ctypes.c_int64]
        L.qo_quantize_int8_rows.argtypes = [_F, ctypes.c_int64, ctypes.c_int64, _F, ctypes.c_void_p]
        L.qo_project.argtypes = [_F, ctypes.c_int64, ctypes.c_int64, _F, ctypes.c_int, _F]
        L.qo_rms_norm.argtypes = [_F, ctypes.c_int64, _F, ctypes.c_float, ctypes.c_int, _F]
        L.qo_softmax.argtypes = [_F, ctypes.c_int64, _F]
        L.qo_silu.argtypes = [_F, ctypes.c_int64, _F]
        L.qo_delta_rule.argtypes = [_F, _F, _F, ctypes.c_int64, ctypes.c_int64, ctypes.c_float, ctypes.c_float, _F,
                                    _F]
        L.qo_rotate.argtypes = [_F, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_float]
        L.qo_attend.argtypes = [_F, _F, _F, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, _F]
        L.qo_set_threads.argtypes = [ctypes.c_int]
        L.qo_state_load.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p]
        L.qo_model_set_edit.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        _lib = L
    return _lib


def fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def check(status: int):
    if status != 0:
        raise RuntimeError(lib().qo_error().decode())


def set_threads(n: int):
    check(lib().qo_set_threads(int(n)))


def threads() -> int:
    return lib().qo_threads()


class Oracle:
    """The reference CPU model (Model::step, src/model.rs:335-382) on a tensor set."""

    def __init__(self, weights):
        self.weights = weights  # keeps the arrays alive
        self.config = weights.config
        self._cfg = weights.config  # ctypes struct, passed by reference
        self.ptr = lib().qo_model_create(ctypes.byref(self._cfg), ctypes.cast(weights.table, ctypes.c_void_p))
        if not self.ptr:
            raise RuntimeError(lib().qo_error().decode())

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().qo_model_free(self.ptr)
            self.ptr = None

    def set_lm_head(self, w: np.ndarray):
        """Project the vocabulary with `w` [vocab, hidden] instead of the embedding."""
        self._lm_head = np.ascontiguousarray(w, dtype=np.float32)
        lib().qo_model_set_lm_head(self.ptr, fp(self._lm_head))

    def set_edit(self, edits):
        """The edit manifest every following step applies (the reference's
        EditManifest, src/edit.rs): a list of dicts with layer, columns,
        direction (hidden floats or None) and coefficient; [] removes it."""
        n = len(edits)
        layers = np.array([e["layer"] for e in edits] or [0], np.int32)
        offsets = np.cumsum([0] + [len(e["columns"]) for e in edits]).astype(np.int64)
        columns = np.array([j for e in edits for j in e["columns"]] or [0], np.int64)
        dirs = [None if e.get("direction") is None else np.ascontiguousarray(e["direction"], dtype=np.float32)
                for e in edits]
        self._edit_dirs = dirs
        table = (ctypes.c_void_p * max(n, 1))(*[d.ctypes.data if d is not None else None for d in dirs])
        coef = np.array([e["coefficient"] for e in edits] or [0], np.float32)
        check(lib().qo_model_set_edit(self.ptr, n, layers.ctypes.data, offsets.ctypes.data, columns.ctypes.data,
                                      table, coef.ctypes.data))

    def new_state(self) -> "State":
        return State(self, lib().qo_state_create(self.ptr))


class State:
    def __init__(self, oracle: Oracle, ptr):
        self.oracle = oracle
        self.ptr = ptr

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().qo_state_free(self.ptr)
            self.ptr = None

    def clone(self) -> "State":
        return State(self.oracle, lib().qo_state_clone(self.ptr))

    @property
    def position(self) -> int:
        return lib().qo_state_position(self.ptr)

    def step(self, token: int, backend: int = VECTOR, trace: bool = False):
        """Returns logits (and, with trace, a list of (layer, name, values))."""
        c = self.oracle.config
        logits = np.empty(c.vocab_size, dtype=np.float32)
        records = []
        if trace:
            def cb(_user, layer, name, values, n):
                records.append((layer, name.decode(), np.ctypeslib.as_array(values, shape=(n,)).copy()))
            fn = _TRACE(cb)
        else:
            fn = _TRACE()
        check(lib().qo_step(self.oracle.ptr, self.ptr, int(token), backend, fp(logits), None, fn, None))
        return (logits, records) if trace else logits

    def load(self, position: int, read):
        """Replace the whole state with `position` tokens' worth; read(layer,
        which) returns each part as part() lays it out."""
        c = self.oracle.config
        keep = []
        table = (ctypes.c_void_p * (4 * c.num_layers))()
        for layer in range(c.num_layers):
            for which in range(4):
                v = np.ascontiguousarray(read(layer, which), dtype=np.float32)
                keep.append(v)
                table[4 * layer + which] = v.ctypes.data if v.size else None
        check(lib().qo_state_load(self.oracle.ptr, self.ptr, int(position), table))

    def part(self, layer: int, which: int) -> np.ndarray:
        """which: 0 conv history, 1 recurrent state, 2 keys, 3 values."""
        n = lib().qo_state_size(self.oracle.ptr, self.ptr, layer, which)
        out = np.empty(max(n, 0), dtype=np.float32)
        if n > 0:
            check(lib().qo_state_read(self.oracle.ptr, self.ptr, layer, which, fp(out)))
        return out


def select_greedy(logits: np.ndarray) -> int:
    v = lib().qo_select_greedy(fp(np.ascontiguousarray(logits, dtype=np.float32)), logits.size)
    if v < 0:
        raise RuntimeError(lib().qo_error().decode())
    return int(v)


def quantize_int8_rows(w: np.ndarray, rows: int, cols: int):
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    scales = np.empty(rows, dtype=np.float32)
    q = np.empty(rows * cols, dtype=np.int8)
    lib().qo_quantize_int8_rows(fp(w), rows, cols, fp(scales), q.ctypes.data_as(ctypes.c_void_p))
    return scales, q


def dequantize_int8_rows(scales: np.ndarray, q: np.ndarray, rows: int, cols: int) -> np.ndarray:
    """The values the int8 path multiplies by, as fp32: scale * q. (The device
    path computes scale * sum(q x); the CPU comparison point is the dequantised
    matrix, as BASELINE config 5 states.)"""
    return (q.reshape(rows, cols).astype(np.float32) * scales[:, None]).astype(np.float32).reshape(-1)


def project(w, rows, cols, x, backend=VECTOR):
    out = np.empty(rows, dtype=np.float32)
    check(lib().qo_project(fp(w), rows, cols, fp(x), backend, fp(out)))
    return out


def rms_norm(x, w, eps, zero_centered):
    out = np.empty_like(x)
    check(lib().qo_rms_norm(fp(x), x.size, fp(w), eps, int(zero_centered), fp(out)))
    return out


def softmax(x):
    out = np.empty_like(x)
    check(lib().qo_softmax(fp(x), x.size, fp(out)))
    return out


def silu(x):
    out = np.empty_like(x)
    check(lib().qo_silu(fp(x), x.size, fp(out)))
    return out


def delta_rule(q, k, v, g, beta, state):
    out = np.empty(v.size, dtype=np.float32)
    check(lib().qo_delta_rule(fp(q), fp(k), fp(v), q.size, v.size, g, beta, fp(state), fp(out)))
    return out


def rotate(x, position, dim, theta):
    check(lib().qo_rotate(fp(x), x.size, position, dim, theta))
    return x


def attend(query, keys, values, heads, kv_heads, d):
    """attend (reference src/attention.rs:63-130): query [heads * d], keys and
    values [positions, kv_heads * d]; returns the context [heads * d]."""
    q = np.ascontiguousarray(query, dtype=np.float32).reshape(-1)
    k = np.ascontiguousarray(keys, dtype=np.float32).reshape(-1)
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
    positions = k.size // (kv_heads * d)
    out = np.empty(heads * d, dtype=np.float32)
    check(lib().qo_attend(fp(q), fp(k), fp(v), positions, heads, kv_heads, d, fp(out)))
    return out
