"""Real-checkpoint loading: a model directory (config.json + one safetensors
file, the layout the reference loads, src/weights.rs:330-548) into a Weights
tensor set, through the engine library's streaming safetensors reader
(include/qwen_engine.h qe_safetensors_*: SHA-256 over every byte, header
checks, BF16 kept as bits and widened exactly to fp32 here).

A BF16 checkpoint gives fp32 tensors that are BF16-exact, so a model loaded
with fmt=BF16_EXACT uploads every matrix as BF16 (half the bytes of fp32),
as the reference's default BF16 weight format does."""
from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

from .engine import EngineError, lib
from .model import Weights, config_from_text_config, tensor_specs

CHECKPOINT = "model.safetensors-00001-of-00001.safetensors"
F32, BF16 = 0, 1


def _bind():
    L = lib()
    if getattr(L, "_st_bound", False):
        return L
    L.qe_safetensors_read.restype = ctypes.c_void_p
    L.qe_safetensors_read.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_void_p, ctypes.c_int64]
    L.qe_safetensors_error.restype = ctypes.c_char_p
    L.qe_safetensors_free.argtypes = [ctypes.c_void_p]
    L.qe_safetensors_sha256.restype = ctypes.c_char_p
    L.qe_safetensors_sha256.argtypes = [ctypes.c_void_p]
    L.qe_safetensors_count.restype = ctypes.c_int64
    L.qe_safetensors_count.argtypes = [ctypes.c_void_p]
    L.qe_safetensors_info.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p),
                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int),
                                      ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int64)]
    L.qe_safetensors_f32.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_float),
                                     ctypes.c_int64]
    L.qe_safetensors_bf16.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_uint16),
                                      ctypes.c_int64]
    L._st_bound = True
    return L


class Safetensors:
    """One verified safetensors file (read_checkpoint_kept, reference
    src/weights.rs:364-466): `tensors` maps each name to (dtype, shape, kept)."""

    def __init__(self, path, sha256: str | None = None, ignored=()):
        L = _bind()
        names = [str(n).encode() for n in ignored]
        arr = (ctypes.c_char_p * max(len(names), 1))(*names)
        self.ptr = L.qe_safetensors_read(str(path).encode(), sha256.encode() if sha256 else None,
                                         ctypes.cast(arr, ctypes.c_void_p), len(names))
        if not self.ptr:
            raise EngineError(L.qe_safetensors_error().decode())
        self.sha256 = L.qe_safetensors_sha256(self.ptr).decode()
        self.tensors = {}
        for i in range(L.qe_safetensors_count(self.ptr)):
            name, dtype, kept, ndim = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
            shape = (ctypes.c_int64 * 8)()
            if L.qe_safetensors_info(self.ptr, i, ctypes.byref(name), ctypes.byref(dtype), ctypes.byref(kept),
                                     ctypes.byref(ndim), shape) != 0:
                raise EngineError(L.qe_safetensors_error().decode())
            self.tensors[name.value.decode()] = (dtype.value, tuple(shape[:ndim.value]), bool(kept.value))

    def close(self):
        if getattr(self, "ptr", None):
            _bind().qe_safetensors_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.close()

    def f32(self, name: str) -> np.ndarray:
        """The tensor as fp32 (BF16 widened exactly), flattened."""
        if name not in self.tensors or not self.tensors[name][2]:
            raise EngineError(f"missing tensor: {name}")
        n = int(np.prod(self.tensors[name][1])) if self.tensors[name][1] else 1
        out = np.empty(n, np.float32)
        if _bind().qe_safetensors_f32(self.ptr, name.encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                      n) != 0:
            raise EngineError(_bind().qe_safetensors_error().decode())
        return out

    def bf16_bits(self, name: str) -> np.ndarray:
        n = int(np.prod(self.tensors[name][1]))
        out = np.empty(n, np.uint16)
        if _bind().qe_safetensors_bf16(self.ptr, name.encode(), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)),
                                       n) != 0:
            raise EngineError(_bind().qe_safetensors_error().decode())
        return out


def load_config(model_dir) -> "QwConfig":  # noqa: F821
    """load_config (reference src/weights.rs:330-350): config.json's
    text_config, with the reference's model-type and flag checks."""
    v = json.loads((Path(model_dir) / "config.json").read_text())
    if v.get("model_type") != "qwen3_5":
        raise EngineError("unsupported model type")
    tc = v["text_config"]
    if tc.get("attention_bias") is not False or tc.get("hidden_act") != "silu" or tc.get("attn_output_gate") is not True:
        raise EngineError("unsupported attention/activation flags")
    return config_from_text_config(tc)


def load_model(model_dir, sha256: str | None = None, filename: str = CHECKPOINT):
    """load_model (reference src/weights.rs:526-539, model_from_tensors
    187-337): every language-model tensor by name (conv1d [channels, 1, k]
    read as [channels, k]; the tied lm_head is the embedding); the other
    tensors (vision tower, MTP head) are read, hashed and returned as
    `unused`. Returns (Weights, unused names, the file's SHA-256)."""
    c = load_config(model_dir)
    st = Safetensors(Path(model_dir) / filename, sha256)
    try:
        tensors = {}
        used = set()
        for spec in tensor_specs(c):
            if spec.name not in st.tensors:
                raise EngineError(f"missing tensor: {spec.name}")
            shape = st.tensors[spec.name][1]
            want = int(np.prod(spec.shape))
            if int(np.prod(shape)) != want:
                raise EngineError(f"tensor shape mismatch: {spec.name} {shape} vs {spec.shape}")
            tensors[spec.index] = np.ascontiguousarray(st.f32(spec.name))
            used.add(spec.name)
        unused = sorted(n for n in st.tensors if n not in used)
        return Weights(c, tensors), unused, st.sha256
    finally:
        st.close()
