"""Model configs and tensor sets for the Qwen3.5 hybrid, mirrored from
include/qwen_model.h (the C struct and the tensor slot order).

The configs are the reference's `TextConfig` resolved as
`model_from_tensors` resolves it (reference src/weights.rs:27-95,187-337).
Named configs:
  * ``fixture``  - the tiny model of tests/golden/hybrid.json (the reference's
    tests/fixtures/hybrid.json, official PyTorch vectors);
  * ``tiny``     - the 4-layer "demo hybrid"-shaped synthetic model (width 64);
  * ``qwen08b``  - the Qwen3.5-0.8B shape (reference spec/upstream/config.json).
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass

import numpy as np

QW_MAX_LAYERS = 256
QW_SLOTS_BASE = 2
QW_SLOTS_LAYER = 15

# slot indices (include/qwen_model.h)
INPUT_NORM, POST_NORM, GATE, UP, DOWN = 0, 1, 2, 3, 4
Q, K, V, O, Q_NORM, K_NORM = 5, 6, 7, 8, 9, 10
QKV, Z, A, B, CONV, DT, A_LOG, DELTA_NORM, OUT = 5, 6, 7, 8, 9, 10, 11, 12, 13


class QwConfig(ctypes.Structure):
    _fields_ = [
        ("hidden_size", ctypes.c_int32),
        ("intermediate_size", ctypes.c_int32),
        ("num_layers", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("num_heads", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("rotary_dim", ctypes.c_int32),
        ("key_heads", ctypes.c_int32),
        ("value_heads", ctypes.c_int32),
        ("key_dim", ctypes.c_int32),
        ("value_dim", ctypes.c_int32),
        ("conv_kernel", ctypes.c_int32),
        ("max_positions", ctypes.c_int32),
        ("rms_norm_eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("attention", ctypes.c_uint8 * QW_MAX_LAYERS),
    ]

    @property
    def layer_types(self):
        return ["full_attention" if self.attention[i] else "linear_attention" for i in range(self.num_layers)]

    @property
    def channels(self):
        return 2 * self.key_heads * self.key_dim + self.value_heads * self.value_dim

    def describe(self):
        return {f: getattr(self, f) for f, _ in self._fields_ if f != "attention"} | {"layer_types": self.layer_types}


def make_config(*, hidden, intermediate, vocab, layer_types, heads, kv_heads, head_dim, rotary_dim,
                key_heads, value_heads, key_dim, value_dim, conv_kernel, max_positions, eps, theta):
    c = QwConfig()
    c.hidden_size, c.intermediate_size, c.vocab_size = hidden, intermediate, vocab
    c.num_layers = len(layer_types)
    c.num_heads, c.num_kv_heads, c.head_dim, c.rotary_dim = heads, kv_heads, head_dim, rotary_dim
    c.key_heads, c.value_heads, c.key_dim, c.value_dim = key_heads, value_heads, key_dim, value_dim
    c.conv_kernel, c.max_positions = conv_kernel, max_positions
    c.rms_norm_eps, c.rope_theta = eps, theta
    for i, t in enumerate(layer_types):
        assert t in ("full_attention", "linear_attention"), t
        c.attention[i] = 1 if t == "full_attention" else 0
    return c


def config_from_text_config(tc: dict) -> QwConfig:
    """TextConfig JSON (reference src/weights.rs:27-45) to QwConfig, with the
    rotary width resolved as head_dim * partial_rotary_factor (weights.rs:281)."""
    rope = tc["rope_parameters"]
    d = tc["head_dim"]
    rotary = int(np.float32(d) * np.float32(rope["partial_rotary_factor"]))
    return make_config(
        hidden=tc["hidden_size"], intermediate=tc["intermediate_size"], vocab=tc["vocab_size"],
        layer_types=tc["layer_types"], heads=tc["num_attention_heads"], kv_heads=tc["num_key_value_heads"],
        head_dim=d, rotary_dim=rotary, key_heads=tc["linear_num_key_heads"],
        value_heads=tc["linear_num_value_heads"], key_dim=tc["linear_key_head_dim"],
        value_dim=tc["linear_value_head_dim"], conv_kernel=tc["linear_conv_kernel_dim"],
        max_positions=tc["max_position_embeddings"], eps=tc["rms_norm_eps"], theta=float(rope["rope_theta"]))


def config_tiny() -> QwConfig:
    """demo-hybrid structure [L,L,L,F], width 64, FFN 256,
    vocab 512, attention 4Q/1KV d=16 rot 8, DeltaNet 4 heads dk=dv=16, conv 4.
    theta 1e4 (the demo hybrid fixture's value)."""
    return make_config(hidden=64, intermediate=256, vocab=512,
                       layer_types=["linear_attention"] * 3 + ["full_attention"], heads=4, kv_heads=1,
                       head_dim=16, rotary_dim=8, key_heads=4, value_heads=4, key_dim=16, value_dim=16,
                       conv_kernel=4, max_positions=4096, eps=1e-6, theta=1e4)


def config_qwen08b(max_positions: int = 262144) -> QwConfig:
    """Qwen3.5-0.8B text shape (reference spec/upstream/config.json:14-68)."""
    return make_config(hidden=1024, intermediate=3584, vocab=248320,
                       layer_types=(["linear_attention"] * 3 + ["full_attention"]) * 6, heads=8, kv_heads=2,
                       head_dim=256, rotary_dim=64, key_heads=16, value_heads=16, key_dim=128, value_dim=128,
                       conv_kernel=4, max_positions=max_positions, eps=1e-6, theta=1e7)


@dataclass
class TensorSpec:
    index: int
    name: str
    shape: tuple
    kind: str  # "matrix", "norm_zero" (Qwen zero-centred gain), "norm_direct", "vector"


def tensor_specs(c: QwConfig) -> list[TensorSpec]:
    """Every tensor with its slot index, checkpoint name and shape, in slot order."""
    H, I, vocab = c.hidden_size, c.intermediate_size, c.vocab_size
    specs = [TensorSpec(0, "model.language_model.embed_tokens.weight", (vocab, H), "matrix"),
             TensorSpec(1, "model.language_model.norm.weight", (H,), "norm_zero")]
    for layer in range(c.num_layers):
        base = QW_SLOTS_BASE + layer * QW_SLOTS_LAYER
        p = f"model.language_model.layers.{layer}."
        specs += [TensorSpec(base + INPUT_NORM, p + "input_layernorm.weight", (H,), "norm_zero"),
                  TensorSpec(base + POST_NORM, p + "post_attention_layernorm.weight", (H,), "norm_zero"),
                  TensorSpec(base + GATE, p + "mlp.gate_proj.weight", (I, H), "matrix"),
                  TensorSpec(base + UP, p + "mlp.up_proj.weight", (I, H), "matrix"),
                  TensorSpec(base + DOWN, p + "mlp.down_proj.weight", (H, I), "matrix")]
        if c.attention[layer]:
            d = c.head_dim
            q, kv = c.num_heads * d, c.num_kv_heads * d
            a = p + "self_attn."
            specs += [TensorSpec(base + Q, a + "q_proj.weight", (2 * q, H), "matrix"),
                      TensorSpec(base + K, a + "k_proj.weight", (kv, H), "matrix"),
                      TensorSpec(base + V, a + "v_proj.weight", (kv, H), "matrix"),
                      TensorSpec(base + O, a + "o_proj.weight", (H, q), "matrix"),
                      TensorSpec(base + Q_NORM, a + "q_norm.weight", (d,), "norm_zero"),
                      TensorSpec(base + K_NORM, a + "k_norm.weight", (d,), "norm_zero")]
        else:
            vd, vh = c.value_heads * c.value_dim, c.value_heads
            a = p + "linear_attn."
            specs += [TensorSpec(base + QKV, a + "in_proj_qkv.weight", (c.channels, H), "matrix"),
                      TensorSpec(base + Z, a + "in_proj_z.weight", (vd, H), "matrix"),
                      TensorSpec(base + A, a + "in_proj_a.weight", (vh, H), "matrix"),
                      TensorSpec(base + B, a + "in_proj_b.weight", (vh, H), "matrix"),
                      TensorSpec(base + CONV, a + "conv1d.weight", (c.channels, c.conv_kernel), "vector"),
                      TensorSpec(base + DT, a + "dt_bias", (vh,), "vector"),
                      TensorSpec(base + A_LOG, a + "A_log", (vh,), "vector"),
                      TensorSpec(base + DELTA_NORM, a + "norm.weight", (c.value_dim,), "norm_direct"),
                      TensorSpec(base + OUT, a + "out_proj.weight", (H, vd), "matrix")]
    return specs


def n_slots(c: QwConfig) -> int:
    return QW_SLOTS_BASE + c.num_layers * QW_SLOTS_LAYER


class Weights:
    """A full tensor set in slot order, plus the pointer table the C APIs take."""

    def __init__(self, config: QwConfig, tensors: dict[int, np.ndarray]):
        self.config = config
        self.tensors = tensors
        for s in tensor_specs(config):
            t = tensors[s.index]
            assert t.dtype == np.float32 and t.flags.c_contiguous and t.size == int(np.prod(s.shape)), s.name
        self._table = (ctypes.POINTER(ctypes.c_float) * n_slots(config))()
        for i, t in tensors.items():
            self._table[i] = t.ctypes.data_as(ctypes.POINTER(ctypes.c_float))

    @property
    def table(self):
        return self._table

    def matrix_bytes(self) -> int:
        return sum(4 * int(np.prod(s.shape)) for s in tensor_specs(self.config) if s.kind == "matrix")


def fixture_config_and_weights(fixture: dict) -> tuple[QwConfig, Weights]:
    """The reference's Model::from_fixture (src/model.rs:100-104): config and
    tensors from hybrid.json; conv1d [channels, 1, k] is read as [channels, k]."""
    c = config_from_text_config(fixture["config"])
    tensors = {}
    for s in tensor_specs(c):
        t = fixture["tensors"][s.name]
        a = np.asarray(t["values"], dtype=np.float32).reshape(-1)
        assert a.size == int(np.prod(s.shape)), s.name
        tensors[s.index] = np.ascontiguousarray(a)
    return c, Weights(c, tensors)


def synthetic_weights(c: QwConfig, seed: int = 0, std: float = 0.02, fill=None) -> Weights:
    """BASELINE's random init: every matrix, the conv kernel, dt_bias and A_log
    from N(0, std); zero-centred RMSNorm weights 0 (gain 1); the DeltaNet
    (direct) norm weight 1. ``fill(array, seed, stream, std)`` draws the normals
    (the engine library's counter-based generator, so the values do not depend
    on the thread count); the stream of each tensor is its slot index."""
    if fill is None:
        from .engine import synth_normal as fill
    tensors = {}
    for s in tensor_specs(c):
        a = np.empty(int(np.prod(s.shape)), dtype=np.float32)
        if s.kind == "norm_zero":
            a[:] = 0.0
        elif s.kind == "norm_direct":
            a[:] = 1.0
        else:
            fill(a, seed, s.index, std)
        tensors[s.index] = a
    return Weights(c, tensors)


def bf16_weights(w: Weights) -> Weights:
    """The tensors rounded to BF16 (nearest, ties to even), kept as fp32: a
    BF16-exact model whose matrices the engine uploads as packed BF16 under
    fmt=BF16_EXACT (the reference's deployed precision, src/device.rs:535-549)."""
    out = {}
    for i, t in w.tensors.items():
        u = np.ascontiguousarray(t, dtype=np.float32).view(np.uint32)
        out[i] = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32).view(np.float32)
    return Weights(w.config, out)


def load_fixture(path) -> dict:
    with open(path) as f:
        return json.load(f)
