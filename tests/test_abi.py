"""The C-ABI libraries load on the CPU and export every symbol their headers
declare (no compute call: there is no GPU here)."""
import ctypes
import re
from pathlib import Path

import pytest

from conftest import ROOT
from qwen_mi355x import engine as E


def declared(header: str, prefix: str):
    text = (ROOT / "include" / header).read_text()
    return sorted(set(re.findall(r"\b(" + prefix + r"[a-z0-9_]+)\s*\(", text)))


def test_bridge_exports_every_declared_symbol():
    names = declared("qwen_bridge.h", "qr_")
    assert len(names) == 48
    assert sorted(E.BRIDGE_SYMBOLS) == names
    lib = ctypes.CDLL(str(E.BRIDGE))  # loading does not touch the GPU
    for n in names:
        assert hasattr(lib, n), n
    assert lib.qr_abi() == 3 and lib.qr_kind() == 1
    assert lib.qr_max_op() == 15 and lib.qr_snapshots() == 1 and lib.qr_argmax() == 2


def test_engine_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(E.ENGINE))
    names = declared("qwen_engine.h", "qe_") + declared("qwen_engine.h", "qw_")
    assert len(names) > 30
    for n in names:
        assert hasattr(lib, n), n


def test_bridge_kind_mismatch_is_refused():
    """The engine refuses a CPU bridge as a device and the HIP bridge as a CPU
    bridge (reference src/device.rs:322-350, tests.rs:61-66)."""
    from qwen_mi355x import model as M
    from conftest import GOLDEN
    c, w = M.fixture_config_and_weights(M.load_fixture(GOLDEN / "hybrid.json"))
    cpu = ROOT / "oracle" / "lib" / "libqwen_ops_bridge.so"
    with pytest.raises(E.EngineError, match="kind mismatch"):
        E.Model(w, bridge=cpu, kind=E.KIND_ROCM)
    with pytest.raises(E.EngineError, match="kind mismatch"):
        E.Model(w, bridge=E.BRIDGE, kind=E.KIND_CPU_TEST)
    with pytest.raises(E.EngineError):
        E.Model(w, bridge=ROOT / "no" / "such.so", kind=E.KIND_ROCM)
