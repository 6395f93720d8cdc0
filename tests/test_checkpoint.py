"""The checkpoint reader (engine library qe_safetensors_*, Python
qwen_mi355x.checkpoint): the reference's streaming reader test
(src/weights.rs:553-598) restated on a file written here, the SHA-256
against Python's hashlib, the header checks, and a model directory written
from the fixture model in BF16 loaded back and run through the engine bit for
bit against the oracle on the same (BF16-rounded) weights."""
import hashlib
import json
import struct

import numpy as np
import pytest

from conftest import GOLDEN
from qwen_mi355x import checkpoint as C
from qwen_mi355x import engine as E
from qwen_mi355x import model as M
from test_engine_cpu import OPS_BRIDGE

import oracle as O


def safetensors_bytes(tensors, pad=True):
    """tensors: list of (name, dtype, shape, raw bytes) in data order."""
    header, offset = {}, 0
    for name, dtype, shape, raw in tensors:
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(raw)]}
        offset += len(raw)
    text = json.dumps(header).encode()
    if pad:
        text += b" " * (-len(text) % 8)
    return struct.pack("<Q", len(text)) + text + b"".join(raw for *_, raw in tensors)


def test_streaming_reader(tmp_path):
    """streaming_checkpoint_reader (reference src/weights.rs:553-598): BF16 kept
    as bits, F32 decoded, an ignored tensor hashed and not kept, a wrong hash
    or a truncated file refused."""
    bf16 = struct.pack("<4H", 0x3F80, 0xC000, 0x0000, 0x4040)
    f32 = struct.pack("<2f", 1.5, -2.0)
    data = safetensors_bytes([("a", "BF16", (2, 2), bf16), ("b", "F32", (2,), f32), ("vision", "BF16", (2,), b"\x07" * 4)])
    path = tmp_path / "m.safetensors"
    path.write_bytes(data)
    sha = hashlib.sha256(data).hexdigest()
    st = C.Safetensors(path, sha, ignored=["vision"])
    assert st.sha256 == sha
    assert list(st.bf16_bits("a")) == [0x3F80, 0xC000, 0x0000, 0x4040]
    assert list(st.f32("a")) == [1.0, -2.0, 0.0, 3.0]
    assert st.tensors["a"] == (C.BF16, (2, 2), True)
    assert list(st.f32("b")) == [1.5, -2.0]
    assert st.tensors["vision"][2] is False
    with pytest.raises(E.EngineError, match="missing"):
        st.f32("vision")
    with pytest.raises(E.EngineError, match="SHA-256"):
        C.Safetensors(path, "0" * 64)
    path.write_bytes(data[:-1])
    with pytest.raises(E.EngineError):
        C.Safetensors(path, sha)


@pytest.mark.parametrize("case,match", [
    ("gap", "offsets"), ("size", "offsets"), ("tail", "data length"), ("nan", "NaN"), ("header", "header"),
    ("dtype", "unsupported dtype")])
def test_reader_refuses_bad_files(tmp_path, case, match):
    """The header checks of the safetensors format (and the reference's
    finiteness check): contiguous offsets, size = shape x dtype size, data
    ending at the end of the file, finite values, a JSON header."""
    f32 = struct.pack("<2f", 1.5, -2.0)
    if case == "gap":
        header = json.dumps({"b": {"dtype": "F32", "shape": [2], "data_offsets": [4, 12]}}).encode()
        data = struct.pack("<Q", len(header)) + header + b"\0" * 4 + f32
    elif case == "size":
        data = safetensors_bytes([("b", "F32", (3,), f32)])
    elif case == "tail":
        data = safetensors_bytes([("b", "F32", (2,), f32)]) + b"\0"
    elif case == "nan":
        data = safetensors_bytes([("b", "F32", (2,), struct.pack("<2f", 1.0, float("nan")))])
    elif case == "header":
        text = b'{"b": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]'
        data = struct.pack("<Q", len(text)) + text + f32
    else:
        data = safetensors_bytes([("b", "F16", (2,), f32[:4])])
    path = tmp_path / "bad.safetensors"
    path.write_bytes(data)
    with pytest.raises(E.EngineError, match=match):
        C.Safetensors(path)


def test_sha256_against_hashlib(tmp_path):
    """The reader's SHA-256 (FIPS 180-4, implemented in the engine library)
    against Python's hashlib on files whose lengths cross the 64-byte block and
    56-byte padding boundaries."""
    rng = np.random.default_rng(0)
    for n in (1, 13, 14, 15, 16, 100, 1000, 70000):
        raw = rng.standard_normal(n).astype(np.float32).tobytes()
        data = safetensors_bytes([("t", "F32", (n,), raw)], pad=bool(n % 2))
        path = tmp_path / f"t{n}.safetensors"
        path.write_bytes(data)
        assert C.Safetensors(path).sha256 == hashlib.sha256(data).hexdigest()


def bf16_round(a):
    """Round-to-nearest-even float32 -> BF16, returned widened to float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def write_model_dir(tmp_path, fixture, vision=True):
    """The fixture model as a model directory: config.json (the fixture's
    text_config with the reference's flags) and a BF16 safetensors checkpoint
    with the language tensors under their checkpoint names (conv1d as
    [channels, 1, k]) plus a vision tensor the loader must skip."""
    c, w = M.fixture_config_and_weights(fixture)
    tc = dict(fixture["config"], attention_bias=False, hidden_act="silu", attn_output_gate=True)
    (tmp_path / "config.json").write_text(json.dumps({"model_type": "qwen3_5", "text_config": tc}))
    entries = []
    for spec in M.tensor_specs(c):
        bits = (bf16_round(w.tensors[spec.index]).view(np.uint32) >> 16).astype("<u2")
        shape = (spec.shape[0], 1, spec.shape[1]) if spec.name.endswith("conv1d.weight") else spec.shape
        entries.append((spec.name, "BF16", shape, bits.tobytes()))
    if vision:
        entries.append(("model.visual.patch_embed.weight", "BF16", (4,), b"\x01\x02" * 4))
    data = safetensors_bytes(entries)
    (tmp_path / C.CHECKPOINT).write_bytes(data)
    return c, w, hashlib.sha256(data).hexdigest()


def test_model_directory_round_trip(tmp_path):
    """load_model on a BF16 checkpoint of the fixture model: every tensor the
    BF16 rounding of the original, the vision tensor reported unused, the hash
    pinned; the loaded weights through the engine (BF16 format: every matrix
    BF16-exact) equal the oracle on the same weights bit for bit."""
    fixture = M.load_fixture(GOLDEN / "hybrid.json")
    c, w, sha = write_model_dir(tmp_path, fixture)
    loaded, unused, got_sha = C.load_model(tmp_path, sha)
    assert got_sha == sha and unused == ["model.visual.patch_embed.weight"]
    for spec in M.tensor_specs(c):
        assert np.array_equal(loaded.tensors[spec.index], bf16_round(w.tensors[spec.index])), spec.name
    m = E.Model(loaded, bridge=OPS_BRIDGE, kind=E.KIND_CPU_TEST, fmt=E.BF16_EXACT)
    assert m.weight_summary()[0] == m.weight_summary()[1]  # every matrix uploaded as BF16
    run = m.new_run(len(fixture["ids"]))
    s = O.Oracle(loaded).new_state()
    for tok in fixture["ids"]:
        assert np.array_equal(run.step(tok), s.step(tok, O.REFERENCE))
    with pytest.raises(E.EngineError, match="SHA-256"):
        C.load_model(tmp_path, "f" * 64)
