"""Direct ctypes access to a qr_* bridge (include/qwen_bridge.h), for op-level
tests and kernel benchmarks: allocate, write, run an op or a projection, read.
Mirrors the reference's private `Api` helper (src/device.rs:249-532)."""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .engine import BRIDGE, EngineError, require_current

_F = ctypes.POINTER(ctypes.c_float)


class Params(ctypes.Structure):
    _fields_ = [("p", ctypes.c_void_p * 8), ("n", ctypes.c_int32 * 8), ("f", ctypes.c_float * 4)]


class Projection(ctypes.Structure):
    _fields_ = [("y", ctypes.c_void_p), ("a", ctypes.c_void_p), ("rows", ctypes.c_int32)]


class AddNormPost(ctypes.Structure):
    _fields_ = [("sum", ctypes.c_void_p), ("u", ctypes.c_void_p), ("v", ctypes.c_void_p), ("weight", ctypes.c_void_p),
                ("norm", ctypes.c_void_p), ("eps", ctypes.c_float), ("offset", ctypes.c_float)]


class Delta(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("convolved", "projected", "conv_w", "conv_state", "query", "key", "core",
                                               "recurrent", "a", "b", "gates", "gated", "norm_w", "z")] + \
               [(n, ctypes.c_int32) for n in ("key_heads", "value_heads", "key_dim", "value_dim", "kernel", "tokens",
                                              "channels")] + [("eps", ctypes.c_float)]


OPS = dict(RMS_NORM=1, ADD=2, SILU_PRODUCT=3, CONV_SILU=4, DELTA_QK=5, DELTA_GATES=6, DELTA_RULE=7,
           ATTENTION_QUERY=8, ATTENTION_KV=9, ATTENTION_READ=10, EMBED_BF16=11, ADD_RMS_NORM=12, RMS_NORM_GATE=13,
           DELTA_RULE_GATED=14, ATTENTION_QUERY_KV=15, ARGMAX=16, EMBED_BF16_PICKED=17)


class Buffer:
    def __init__(self, bridge: "Bridge", n: int):
        self.bridge = bridge
        self.n = n
        p = ctypes.c_void_p()
        bridge._check(bridge.L.qr_alloc(bridge.ctx, ctypes.byref(p), ctypes.c_size_t(n)))
        self.ptr = p.value

    def __del__(self):
        if getattr(self, "ptr", None) and self.bridge.ctx:
            self.bridge.L.qr_free(self.bridge.ctx, ctypes.c_void_p(self.ptr))
            self.ptr = None

    def write(self, values):
        v = np.ascontiguousarray(values).view(np.uint32) if np.asarray(values).dtype.itemsize == 4 else None
        if v is None:
            raise TypeError("32-bit words only")
        assert v.size <= self.n
        self.bridge._check(self.bridge.L.qr_write(self.bridge.ctx, ctypes.c_void_p(self.ptr),
                                                  v.ctypes.data_as(ctypes.c_void_p), ctypes.c_size_t(v.size)))
        return self

    def read(self, n: int | None = None) -> np.ndarray:
        n = self.n if n is None else n
        out = np.empty(n, dtype=np.float32)
        self.bridge._check(self.bridge.L.qr_read(self.bridge.ctx, out.ctypes.data_as(ctypes.c_void_p),
                                                 ctypes.c_void_p(self.ptr), ctypes.c_size_t(n)))
        return out

    def at(self, offset: int) -> int:
        assert 0 <= offset < self.n
        return self.ptr + 4 * offset


class Bridge:
    """One bridge context. kind: 1 for the MI355X bridge, 0 for a CPU bridge."""

    def __init__(self, path: str | Path = BRIDGE, kind: int = 1):
        if not Path(path).exists():
            raise EngineError(f"bridge library missing: {path}")
        if Path(path).resolve() == BRIDGE.resolve():
            require_current(BRIDGE)
        self.L = L = ctypes.CDLL(str(path))
        L.qr_error.restype = ctypes.c_char_p
        L.qr_error.argtypes = [ctypes.c_void_p]
        L.qr_info.restype = ctypes.c_char_p
        L.qr_info.argtypes = [ctypes.c_void_p]
        for name in ("qr_alloc", "qr_write", "qr_read", "qr_copy", "qr_run", "qr_gemv", "qr_gemm", "qr_sync",
                     "qr_gemm_i8", "qr_gemv_bf16", "qr_gemm_bf16", "qr_destroy", "qr_free", "qr_set_option"):
            if hasattr(L, name):
                getattr(L, name).restype = ctypes.c_int
        L.qr_free.restype = None
        L.qr_destroy.restype = None
        if L.qr_abi() != 3 or L.qr_kind() != kind:
            raise EngineError("bridge ABI/kind mismatch")
        ctx = ctypes.c_void_p()
        st = L.qr_create(ctypes.byref(ctx))
        if st != 0 or not ctx.value:
            raise EngineError(f"qr_create failed: {st}")
        self.ctx = ctx

    def close(self):
        if getattr(self, "ctx", None):
            self.L.qr_destroy(self.ctx)
            self.ctx = None

    def _check(self, status: int):
        if status != 0:
            raise EngineError(self.L.qr_error(self.ctx).decode() + f" (status={status})")

    @property
    def info(self) -> str:
        return self.L.qr_info(self.ctx).decode()

    def has(self, name: str) -> bool:
        try:
            getattr(self.L, name)
            return True
        except AttributeError:
            return False

    def alloc(self, n: int) -> Buffer:
        return Buffer(self, n)

    def upload(self, values) -> Buffer:
        v = np.ascontiguousarray(values)
        return Buffer(self, v.size).write(v)

    def sync(self):
        self._check(self.L.qr_sync(self.ctx))

    def copy(self, dst: Buffer, src: Buffer, n: int):
        """qr_copy: n floats device to device, on the context stream."""
        self._check(self.L.qr_copy(self.ctx, ctypes.c_void_p(dst.ptr), ctypes.c_void_p(src.ptr), ctypes.c_size_t(n)))

    def embed_rows(self, dst: Buffer, table: Buffer, table_rows: int, width: int, ids, bf16: bool = False):
        """qr_embed_rows: dst[r] = row ids[r] of the (fp32 or packed BF16) table."""
        v = np.ascontiguousarray(ids, dtype=np.int32)
        self._check(self.L.qr_embed_rows(self.ctx, ctypes.c_void_p(dst.ptr), ctypes.c_void_p(table.ptr), table_rows,
                                         width, int(bf16), v.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
                                         int(v.size)))

    def run(self, op, count: int, p=(), n=(), f=()):
        a = Params()
        for i, v in enumerate(p):
            a.p[i] = v.ptr if isinstance(v, Buffer) else v
        for i, v in enumerate(n):
            a.n[i] = int(v)
        for i, v in enumerate(f):
            a.f[i] = float(v)
        code = OPS[op] if isinstance(op, str) else op
        self._check(self.L.qr_run(self.ctx, code, int(count), ctypes.byref(a)))

    def gemm(self, y: Buffer, a: Buffer, x: Buffer, rows: int, cols: int, batch: int, kind: str = "f32"):
        fn = {"f32": self.L.qr_gemm, "bf16": self.L.qr_gemm_bf16, "i8": self.L.qr_gemm_i8}[kind]
        self._check(fn(self.ctx, ctypes.c_void_p(y.ptr), ctypes.c_void_p(a.ptr), ctypes.c_void_p(x.ptr), rows, cols,
                       batch))

    def prepare(self, a: Buffer, rows: int, cols: int, kind: str = "f32"):
        """qr_gemm_f32_prepare (qr_gemm_bf16_prepare / qr_gemm_i8_prepare for kind
        "bf16" / "i8"): keep a's planes for the prefill projections."""
        fn = {"f32": self.L.qr_gemm_f32_prepare, "bf16": self.L.qr_gemm_bf16_prepare,
              "i8": self.L.qr_gemm_i8_prepare}[kind]
        self._check(fn(self.ctx, ctypes.c_void_p(a.ptr), rows, cols))

    def release(self, a: Buffer):
        self._check(self.L.qr_gemm_f32_release(self.ctx, ctypes.c_void_p(a.ptr)))

    def gemv(self, y: Buffer, a: Buffer, x: Buffer, rows: int, cols: int, kind: str = "f32"):
        fn = {"f32": self.L.qr_gemv, "bf16": self.L.qr_gemv_bf16}[kind]
        self._check(fn(self.ctx, ctypes.c_void_p(y.ptr), ctypes.c_void_p(a.ptr), ctypes.c_void_p(x.ptr), rows, cols))

    def group(self, items, x: Buffer, cols: int, batch: int, kind: str = "f32"):
        arr = (Projection * len(items))()
        for i, (y, a, rows) in enumerate(items):
            arr[i].y, arr[i].a, arr[i].rows = y.ptr, a.ptr, rows
        fn = getattr(self.L, f"qr_gemm_{kind}_group")
        self._check(fn(self.ctx, len(items), arr, ctypes.c_void_p(x.ptr), cols, batch))

    def glu(self, product, gate_y, up_y, gate, up, x, rows, cols, batch, kind="f32"):
        fn = getattr(self.L, f"qr_gemm_{kind}_glu")
        self._check(fn(self.ctx, *(ctypes.c_void_p(b.ptr) for b in (product, gate_y, up_y, gate, up, x)), rows, cols,
                       batch))

    def add_norm(self, y, a, x, rows, cols, sum_, u, v, weight, norm, eps, offset, kind="f32"):
        post = AddNormPost(sum_.ptr, u.ptr, v.ptr, weight.ptr, norm.ptr, eps, offset)
        fn = getattr(self.L, f"qr_gemm_{kind}_add_norm")
        self._check(fn(self.ctx, ctypes.c_void_p(y.ptr), ctypes.c_void_p(a.ptr), ctypes.c_void_p(x.ptr), rows, cols,
                       ctypes.byref(post)))

    def delta_mixer(self, **kw):
        d = Delta()
        for k, v in kw.items():
            setattr(d, k, v.ptr if isinstance(v, Buffer) else v)
        self._check(self.L.qr_delta_mixer(self.ctx, ctypes.byref(d)))


def pack_bf16(values: np.ndarray) -> np.ndarray:
    """BF16 words as the reference's upload_bf16 packs them (src/device.rs:535-549)."""
    bits = (np.ascontiguousarray(values, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint32)
    if bits.size % 2:
        bits = np.append(bits, np.uint32(0))
    return (bits[0::2] | (bits[1::2] << 16)).astype(np.uint32)


def pack_int8(scales: np.ndarray, q: np.ndarray) -> np.ndarray:
    """[scales | int8 values, 4 per word] as upload_int8 (src/device.rs:550-561)."""
    qb = np.ascontiguousarray(q, dtype=np.int8).view(np.uint8)
    pad = (-qb.size) % 4
    if pad:
        qb = np.append(qb, np.zeros(pad, dtype=np.uint8))
    return np.concatenate([np.ascontiguousarray(scales, dtype=np.float32).view(np.uint32), qb.view(np.uint32)])
