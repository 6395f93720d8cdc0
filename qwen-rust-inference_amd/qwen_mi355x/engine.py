"""ctypes bindings of the host engine (include/qwen_engine.h) and the device
bridge (include/qwen_bridge.h).

The engine mirrors the reference's `DeviceModel` / `DeviceRun`
(reference src/device.rs:866-2566): load a model through a qr_* bridge,
open runs, step / step_greedy / prefill / verify / verify_rollback / accept,
inspect and restore state. The MI355X bridge is lib/libqwen_mi355x.so; the
engine refuses any other bridge kind unless a test asks for the CPU kind.
Nothing here falls back to a CPU path: without the built libraries every
call raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import numpy as np

from .model import QwConfig, Weights

PKG = Path(__file__).resolve().parent.parent
LIB_DIR = PKG / "lib"
BRIDGE = LIB_DIR / "libqwen_mi355x.so"
ENGINE = LIB_DIR / "libqwen_engine.so"

KIND_CPU_TEST, KIND_ROCM = 0, 1
F32, BF16_EXACT, INT8 = 0, 1, 2
NO_F32_FUSIONS, NO_FUSIONS, NO_DELTA_MIXER, NO_FUSED_OPS, NO_ARGMAX, NO_SNAPSHOTS = 1, 2, 4, 8, 16, 32
NO_DECODE_STEP = 64
NO_EMBED_ROWS = 128
NO_PREPARED_GEMM = 256
NO_PLAIN_DECODE_LAUNCH = 512  # one-launch decode steps launched cooperatively
NO_DECODE_ROWS = 1024  # verify rows one launch each instead of qr_decode_rows
NO_DECODE_CAPTURE = 2048  # captured steps on the op sequence instead of qr_decode_step_capture
DECODE_RESIDENCY_TEST = 4096  # every plain one-launch step reads as non-resident: cooperative from the second on

# Every entry point of include/qwen_bridge.h.
BRIDGE_SYMBOLS = [
    "qr_abi", "qr_kind", "qr_create", "qr_alloc", "qr_free", "qr_write", "qr_read", "qr_copy", "qr_run", "qr_gemv",
    "qr_gemv_bf16", "qr_gemm", "qr_gemm_bf16", "qr_sync", "qr_error", "qr_info", "qr_destroy", "qr_max_op",
    "qr_snapshots", "qr_argmax", "qr_set_option", "qr_gemm_i8", "qr_gemm_bf16_group", "qr_gemm_i8_group",
    "qr_gemm_bf16_glu", "qr_gemm_i8_glu", "qr_gemm_bf16_add_norm", "qr_gemm_i8_add_norm", "qr_delta_mixer",
    "qr_gemm_f32_group", "qr_gemm_f32_glu", "qr_gemm_f32_add_norm", "qr_profile", "qr_profile_read",
    "qr_decode_plan", "qr_decode_step", "qr_decode_steps", "qr_decode_step_row", "qr_decode_plan_free",
    "qr_embed_rows", "qr_argmax_fixed", "qr_gemm_f32_prepare", "qr_gemm_f32_release", "qr_decode_rows",
    "qr_decode_step_capture", "qr_decode_accept", "qr_gemm_bf16_prepare", "qr_gemm_i8_prepare",
]

_F = ctypes.POINTER(ctypes.c_float)
_U32 = ctypes.POINTER(ctypes.c_uint32)
RECORD_FN = ctypes.CFUNCTYPE(None, ctypes.c_void_p, ctypes.c_int, ctypes.c_char_p, _F, ctypes.c_int64)
ABSORB_FN = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, _U32, ctypes.c_int64)
DRAFT_FN = ctypes.CFUNCTYPE(ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64, _U32)


class QeDraft(ctypes.Structure):
    _fields_ = [("user", ctypes.c_void_p), ("absorb", ABSORB_FN), ("draft", DRAFT_FN)]


class QeEdit(ctypes.Structure):
    _fields_ = [("layer", ctypes.c_int32), ("tensor_name", ctypes.c_char_p), ("columns", ctypes.POINTER(ctypes.c_int64)),
                ("n_columns", ctypes.c_int64), ("direction", ctypes.POINTER(ctypes.c_float)),
                ("coefficient", ctypes.c_float)]


class SpecStats(ctypes.Structure):
    """SpeculativeStats (reference src/device/speculative.rs:30-46)."""
    _fields_ = [("passes", ctypes.c_int64), ("offered", ctypes.c_int64 * 8), ("accepted", ctypes.c_int64 * 8),
                ("prefill_s", ctypes.c_double), ("draft_s", ctypes.c_double), ("verify_s", ctypes.c_double)]

    def as_dict(self, depth: int) -> dict:
        return {"passes": self.passes, "offered": list(self.offered[:depth]), "accepted": list(self.accepted[:depth]),
                "prefill_s": self.prefill_s, "draft_s": self.draft_s, "verify_s": self.verify_s}
_lib = None


class EngineError(RuntimeError):
    pass


STAMP = LIB_DIR / "sources.sha256"


def source_digest() -> str:
    """SHA-256 over every source the two libraries are built from (kernels,
    bridge, engine, headers, Makefile), in a fixed order."""
    import hashlib
    h = hashlib.sha256()
    files = sorted((PKG / "csrc").glob("*")) + sorted((PKG / "engine").glob("*")) + \
        sorted((PKG.parent / "include").glob("*.h")) + [PKG / "Makefile"]
    for f in files:
        if f.is_file():
            h.update(f.name.encode() + b"\0" + f.read_bytes() + b"\0")
    return h.hexdigest()


def write_stamp():
    STAMP.write_text(source_digest() + "\n")


def is_current() -> bool:
    """True when both libraries exist and were built from the sources as they are."""
    return BRIDGE.exists() and ENGINE.exists() and STAMP.exists() and \
        STAMP.read_text().strip() == source_digest()


def require_current(path: Path):
    if not path.exists():
        raise EngineError(f"library missing: {path} (run __graft_entry__.build())")
    if not is_current():
        raise EngineError(f"{path.name} was not built from the current sources (run __graft_entry__.build())")


def lib():
    global _lib
    if _lib is None:
        require_current(ENGINE)
        L = ctypes.CDLL(str(ENGINE))
        L.qe_last_error.restype = ctypes.c_char_p
        L.qe_model_load.restype = ctypes.c_void_p
        L.qe_model_load.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int]
        L.qe_model_free.argtypes = [ctypes.c_void_p]
        L.qe_model_info.restype = ctypes.c_char_p
        L.qe_model_info.argtypes = [ctypes.c_void_p]
        L.qe_model_weight_summary.argtypes = [ctypes.c_void_p] + [ctypes.POINTER(ctypes.c_int64)] * 3
        L.qe_model_set_run_budget.argtypes = [ctypes.c_void_p, ctypes.c_uint64]
        L.qe_model_sync.argtypes = [ctypes.c_void_p]
        L.qe_model_profile.argtypes = [ctypes.c_void_p, ctypes.c_int]
        L.qe_model_profile_read.restype = ctypes.c_long
        L.qe_model_profile_read.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]
        L.qe_model_run_bytes.restype = ctypes.c_uint64
        L.qe_model_run_bytes.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64]
        L.qe_run_new.restype = ctypes.c_void_p
        L.qe_run_new.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64]
        L.qe_run_free.argtypes = [ctypes.c_void_p]
        L.qe_run_reset.argtypes = [ctypes.c_void_p]
        L.qe_run_position.restype = ctypes.c_int64
        L.qe_run_position.argtypes = [ctypes.c_void_p]
        L.qe_run_decode_plan.argtypes = [ctypes.c_void_p]
        L.qe_step.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _F, RECORD_FN, ctypes.c_void_p]
        L.qe_step_greedy.argtypes = [ctypes.c_void_p, ctypes.c_uint32, _U32]
        L.qe_prefill.argtypes = [ctypes.c_void_p, _U32, ctypes.c_int64, _F, ctypes.POINTER(ctypes.c_int)]
        L.qe_verify.argtypes = [ctypes.c_void_p, _U32, ctypes.c_int64, _F]
        L.qe_verify_rollback.argtypes = [ctypes.c_void_p, _U32, ctypes.c_int64, _F]
        L.qe_verify_rollback_greedy.argtypes = [ctypes.c_void_p, _U32, ctypes.c_int64, _U32]
        L.qe_accept.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.qe_unread_logits.argtypes = [ctypes.c_void_p, _F]
        L.qe_state_size.restype = ctypes.c_int64
        L.qe_state_size.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.qe_state_read.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _F]
        L.qe_state_write.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _F, ctypes.c_int64]
        L.qe_state_set_position.argtypes = [ctypes.c_void_p, ctypes.c_int64]
        L.qe_checkpoint.restype = ctypes.c_void_p
        L.qe_checkpoint.argtypes = [ctypes.c_void_p]
        L.qe_initial_checkpoint.restype = ctypes.c_void_p
        L.qe_initial_checkpoint.argtypes = [ctypes.c_void_p]
        L.qe_restore.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.qe_checkpoint_free.argtypes = [ctypes.c_void_p]
        L.qe_checkpoint_position.restype = ctypes.c_int64
        L.qe_checkpoint_position.argtypes = [ctypes.c_void_p]
        L.qe_decode_greedy.argtypes = [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_int64, _U32,
                                       ctypes.POINTER(ctypes.c_double)]
        L.qe_quantize_int8_rows.argtypes = [_F, ctypes.c_int64, ctypes.c_int64, _F, ctypes.c_void_p]
        L.qe_speculative_generate.argtypes = [ctypes.c_void_p, ctypes.POINTER(QeDraft), _U32, ctypes.c_int64,
                                              ctypes.c_int64, ctypes.c_int64, _U32, ctypes.c_int64, _U32,
                                              ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(SpecStats)]
        L.qe_run_set_edit.argtypes = [ctypes.c_void_p, ctypes.POINTER(QeEdit), ctypes.c_int64, ctypes.c_void_p]
        L.qe_draft_ngram_new.restype = ctypes.POINTER(QeDraft)
        L.qe_draft_ngram_new.argtypes = [ctypes.c_int64]
        L.qe_draft_ngram_free.argtypes = [ctypes.POINTER(QeDraft)]
        L.qw_synth_normal.argtypes = [_F, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                      ctypes.c_int]
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _up(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_U32)


def _check(status: int):
    if status != 0:
        raise EngineError(lib().qe_last_error().decode())


def synth_normal(a: np.ndarray, seed: int, stream: int, std: float, threads: int = 0):
    """Fill a float32 array with the engine's counter-based N(0, std) values."""
    lib().qw_synth_normal(_fp(a), a.size, seed, stream, std, threads)


def quantize_int8_rows(w: np.ndarray, rows: int, cols: int):
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    scales = np.empty(rows, dtype=np.float32)
    q = np.empty(rows * cols, dtype=np.int8)
    lib().qe_quantize_int8_rows(_fp(w), rows, cols, _fp(scales), q.ctypes.data_as(ctypes.c_void_p))
    return scales, q


class Model:
    """DeviceModel: weights uploaded through a bridge."""

    def __init__(self, weights: Weights, bridge: str | Path = BRIDGE, kind: int = KIND_ROCM, fmt: int = F32,
                 disable: int = 0):
        if not Path(bridge).exists():
            raise EngineError(f"bridge library missing: {bridge} (run __graft_entry__.build())")
        self.weights = weights
        self.config: QwConfig = weights.config
        self._cfg = weights.config
        self.ptr = lib().qe_model_load(str(bridge).encode(), kind, ctypes.byref(self._cfg),
                                       ctypes.cast(weights.table, ctypes.c_void_p), fmt, disable)
        if not self.ptr:
            raise EngineError(lib().qe_last_error().decode())

    def close(self):
        if getattr(self, "ptr", None):
            lib().qe_model_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.close()

    @property
    def info(self) -> str:
        return lib().qe_model_info(self.ptr).decode()

    def weight_summary(self):
        a, b, c = ctypes.c_int64(), ctypes.c_int64(), ctypes.c_int64()
        lib().qe_model_weight_summary(self.ptr, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
        return a.value, b.value, c.value

    def sync(self):
        _check(lib().qe_model_sync(self.ptr))

    def profile(self, on: bool):
        """Switch the bridge's event-pair profiler on (clears totals) or off."""
        _check(lib().qe_model_profile(self.ptr, int(on)))

    def profile_read(self) -> dict:
        """{label: (calls, total_ms)} since profile(True)."""
        n = lib().qe_model_profile_read(self.ptr, None, 0)
        if n < 0:
            raise EngineError(lib().qe_last_error().decode())
        buf = ctypes.create_string_buffer(n + 1)
        lib().qe_model_profile_read(self.ptr, buf, n + 1)
        out = {}
        for line in buf.value.decode().splitlines():
            calls, ms, label = line.split("\t", 2)
            out[label] = (int(calls), float(ms))
        return out

    def set_run_budget(self, nbytes: int):
        lib().qe_model_set_run_budget(self.ptr, int(nbytes))

    def run_bytes(self, capacity: int, chunk: int) -> int:
        return lib().qe_model_run_bytes(self.ptr, capacity, chunk)

    def new_run(self, capacity: int, chunk: int = 128, snapshots: int = 0) -> "Run":
        ptr = lib().qe_run_new(self.ptr, capacity, chunk, snapshots)
        if not ptr:
            raise EngineError(lib().qe_last_error().decode())
        return Run(self, ptr)


class Checkpoint:
    def __init__(self, ptr):
        self.ptr = ptr

    @property
    def position(self):
        return lib().qe_checkpoint_position(self.ptr)

    def __del__(self):
        if getattr(self, "ptr", None):
            lib().qe_checkpoint_free(self.ptr)
            self.ptr = None


class Run:
    """DeviceRun: per-run state and scratch on the device."""

    def __init__(self, model: Model, ptr):
        self.model = model
        self.ptr = ptr
        self.vocab = model.config.vocab_size

    def close(self):
        if getattr(self, "ptr", None):
            lib().qe_run_free(self.ptr)
            self.ptr = None

    def __del__(self):
        self.close()

    @property
    def position(self) -> int:
        return lib().qe_run_position(self.ptr)

    @property
    def decode_plan(self) -> bool:
        """True when uncaptured one-token steps run the bridge's one-launch decode."""
        return bool(lib().qe_run_decode_plan(self.ptr))

    def reset(self):
        _check(lib().qe_run_reset(self.ptr))

    def step(self, token: int, capture: bool = False):
        logits = np.empty(self.vocab, dtype=np.float32)
        records = []
        if capture:
            def cb(_u, layer, name, values, n):
                records.append((layer, name.decode(), np.ctypeslib.as_array(values, shape=(n,)).copy()))
            fn = RECORD_FN(cb)
        else:
            fn = RECORD_FN()
        _check(lib().qe_step(self.ptr, int(token), _fp(logits), fn, None))
        return (logits, records) if capture else logits

    def step_greedy(self, token: int) -> int:
        out = ctypes.c_uint32()
        _check(lib().qe_step_greedy(self.ptr, int(token), ctypes.byref(out)))
        return out.value

    def prefill(self, ids) -> np.ndarray | None:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32)
        has = ctypes.c_int(0)
        _check(lib().qe_prefill(self.ptr, _up(ids), ids.size, _fp(logits), ctypes.byref(has)))
        return logits if has.value else None

    def verify(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty((ids.size, self.vocab), dtype=np.float32)
        _check(lib().qe_verify(self.ptr, _up(ids), ids.size, _fp(out)))
        return out

    def verify_rollback(self, ids) -> np.ndarray:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty((ids.size, self.vocab), dtype=np.float32)
        _check(lib().qe_verify_rollback(self.ptr, _up(ids), ids.size, _fp(out)))
        return out

    def verify_rollback_greedy(self, ids) -> list[int]:
        ids = np.ascontiguousarray(ids, dtype=np.uint32)
        out = np.empty(ids.size, dtype=np.uint32)
        _check(lib().qe_verify_rollback_greedy(self.ptr, _up(ids), ids.size, _up(out)))
        return [int(v) for v in out]

    def accept(self, rows: int):
        _check(lib().qe_accept(self.ptr, rows))

    def unread_logits(self):
        out = np.empty(self.vocab, dtype=np.float32)
        s = lib().qe_unread_logits(self.ptr, _fp(out))
        if s < 0:
            raise EngineError(lib().qe_last_error().decode())
        return out if s == 1 else None

    def state(self, layer: int, which: int) -> np.ndarray:
        n = lib().qe_state_size(self.ptr, layer, which)
        if n < 0:
            raise EngineError(lib().qe_last_error().decode())
        out = np.empty(n, dtype=np.float32)
        if n:
            _check(lib().qe_state_read(self.ptr, layer, which, _fp(out)))
        return out

    def write_state(self, layer: int, which: int, values: np.ndarray):
        values = np.ascontiguousarray(values, dtype=np.float32)
        _check(lib().qe_state_write(self.ptr, layer, which, _fp(values), values.size))

    def set_position(self, position: int):
        _check(lib().qe_state_set_position(self.ptr, position))

    def inspect_state(self) -> dict:
        """inspect_state (reference src/device.rs:2380-2424): every state part
        at the current position, {(layer, which): values}."""
        n = lib().qe_state_size(self.ptr, 0, 0)
        if n < 0:
            raise EngineError(lib().qe_last_error().decode())
        out = {}
        layer = 0
        while lib().qe_state_size(self.ptr, layer, 0) >= 0:
            for which in range(4):
                out[(layer, which)] = self.state(layer, which)
            layer += 1
        return out

    def load_state(self, position: int, read):
        """load_state (reference src/device.rs:2493-2516): a complete host
        state of `position` tokens (read(layer, which) returns each part as
        state() lays it out: keys / values `position` rows) into this run."""
        self.set_position(position)
        layer = 0
        while lib().qe_state_size(self.ptr, layer, 0) >= 0:
            for which in range(4):
                want = self.state_size(layer, which)
                v = np.ascontiguousarray(read(layer, which), dtype=np.float32).reshape(-1)
                if v.size != want:
                    raise EngineError(f"state part {layer}/{which}: {v.size} values, the run holds {want}")
                if want:
                    self.write_state(layer, which, v)
            layer += 1

    def state_size(self, layer: int, which: int) -> int:
        n = lib().qe_state_size(self.ptr, layer, which)
        if n < 0:
            raise EngineError(lib().qe_last_error().decode())
        return int(n)

    def checkpoint(self) -> Checkpoint:
        p = lib().qe_checkpoint(self.ptr)
        if not p:
            raise EngineError(lib().qe_last_error().decode())
        return Checkpoint(p)

    def initial_checkpoint(self) -> Checkpoint:
        return Checkpoint(lib().qe_initial_checkpoint(self.ptr))

    def restore(self, c: Checkpoint):
        _check(lib().qe_restore(self.ptr, c.ptr))

    def set_edit(self, edits, weights=None):
        """set_edit (reference src/device.rs:1401-1438): a list of dicts with
        layer, columns, direction (hidden floats or None), coefficient and
        optionally tensor_name; [] removes the edit. `weights`: the tensor set
        the model was loaded from (default: the model's own)."""
        weights = weights or self.model.weights
        arr = (QeEdit * max(len(edits), 1))()
        keep = []
        for i, e in enumerate(edits):
            cols = np.ascontiguousarray(e["columns"], dtype=np.int64)
            name = e.get("tensor_name", f"model.language_model.layers.{e['layer']}.mlp.down_proj.weight").encode()
            d = None if e.get("direction") is None else np.ascontiguousarray(e["direction"], dtype=np.float32)
            keep += [cols, name, d]
            arr[i] = QeEdit(e["layer"], name, cols.ctypes.data_as(ctypes.POINTER(ctypes.c_int64)), cols.size,
                            None if d is None else d.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), e["coefficient"])
        _check(lib().qe_run_set_edit(self.ptr, arr, len(edits), ctypes.cast(weights.table, ctypes.c_void_p)))
        self._edit_keep = keep

    def speculative_generate(self, prompt, max_new: int, depth: int, draft="ngram", eos=()):
        """generate (reference src/device/speculative.rs:53-160) on this fresh
        run (snapshots >= depth). draft: "ngram" (the engine's prompt-lookup
        draft) or an object with absorb(tokens) and draft(k) -> list of ids.
        Returns (tokens, stats dict)."""
        prompt = np.ascontiguousarray(prompt, dtype=np.uint32)
        eos_a = np.ascontiguousarray(list(eos) or [0], dtype=np.uint32)
        out = np.empty(max(max_new, 1), dtype=np.uint32)
        n = ctypes.c_int64()
        st = SpecStats()
        owned = None
        if draft == "ngram":
            owned = lib().qe_draft_ngram_new(3)
            dp = owned
        else:
            def absorb(_u, toks, k):
                try:
                    draft.absorb([int(toks[i]) for i in range(k)])
                    return 0
                except Exception:  # noqa: BLE001 - reported to the engine as a failed draft
                    return -1

            def make(_u, k, outp):
                try:
                    ids = list(draft.draft(int(k)))[:k]
                    for i, v in enumerate(ids):
                        outp[i] = int(v)
                    return len(ids)
                except Exception:  # noqa: BLE001
                    return -1
            keep = (ABSORB_FN(absorb), DRAFT_FN(make))
            d = QeDraft(None, keep[0], keep[1])
            dp = ctypes.pointer(d)
        try:
            _check(lib().qe_speculative_generate(self.ptr, dp, _up(prompt), prompt.size, max_new, depth, _up(eos_a),
                                                 len(eos), _up(out), ctypes.byref(n), ctypes.byref(st)))
        finally:
            if owned is not None:
                lib().qe_draft_ngram_free(owned)
        return [int(v) for v in out[:n.value]], st.as_dict(depth)

    def decode_greedy(self, first: int, n_new: int):
        """n_new greedy tokens starting with `first` (n_new - 1 forwards);
        returns (ids, seconds of the forwards)."""
        ids = np.empty(n_new, dtype=np.uint32)
        secs = ctypes.c_double()
        _check(lib().qe_decode_greedy(self.ptr, int(first), n_new, _up(ids), ctypes.byref(secs)))
        return [int(v) for v in ids], secs.value
