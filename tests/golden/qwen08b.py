"""Golden vectors of the CPU oracle at the full BASELINE workloads of the
Qwen3.5-0.8B-shaped model, and the helpers the GPU tests use to read them.

The oracle (a restatement of the reference's Rust `Backend::Vector` path) is
far too slow to run inside a GPU test at these sizes (about 0.2 s per token on
8 threads, so 2644 tokens take ~9 minutes and 8192 tokens ~28), so it is run
once here and a sample of its outputs is committed:

  * at every point of the reference's `long_checkpoints(n)` (prefill lengths
    1, 2^k-1, 2^k, 2^k+1, n; reference src/device/cli.rs:368-380): a fixed
    sample of the logits, the top-16 (index, value) pairs and the top-2 margin,
    and a fixed sample of every state part (conv history, recurrent state,
    keys, values) of every layer; at the last point a larger state sample;
  * for the greedy decode after the prompt: every chosen id, and at every
    step the same logits summary.

The sampled indices are a pure function of (workload, point, layer, part), so
the tests draw the same ones (`sample`). Workloads:

  c2  454-token prompt (ids seed 4) + 128 greedy tokens, fp32
  c3  2644-token prompt (ids seed 2), checkpoints only, fp32
  c4  8192-token prompt (ids seed 5) + 64 greedy tokens, fp32
  c5  int8 per-row weights: the oracle on the dequantised weights, 454-token
      prompt (ids seed 4), then the 4 draft tokens (seed 6) as sequential steps
      (what each verify row must equal) and 16 greedy tokens
  c2l the c2 prompt and greedy tokens with every layer's output (the hidden
      state after each block, the reference's per-layer `validate_device`
      record, src/device/cli.rs:229-366) sampled at every checkpoint and at
      greedy steps 1, 2, 4, ..., 64, 127 (only those: the rest is c2's)
  c3l 10,240-token prompt (ids seed 2), checkpoints and layer outputs

Weights: `synthetic_weights(config_qwen08b(), seed=0)` (the engine library's
counter-based normal generator, thread-count independent).

Usage (CPU, this container or the GPU box's host):
    python tests/golden/qwen08b.py c2 [c3 c4 c5]
writes tests/golden/qwen08b_<name>.npz.
"""
from __future__ import annotations

import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent

VOCAB = 248320
WORKLOADS = {
    "c2": dict(prompt=454, seed=4, greedy=128, int8=False),
    "c3": dict(prompt=2644, seed=2, greedy=0, int8=False),
    "c4": dict(prompt=8192, seed=5, greedy=64, int8=False),
    "c5": dict(prompt=454, seed=4, greedy=16, int8=True, draft_seed=6, draft=4),
    "c2l": dict(prompt=454, seed=4, greedy=128, int8=False, layers=True, layers_only=True),
    "c3l": dict(prompt=10240, seed=2, greedy=0, int8=False, layers=True),
}
LOGIT_SAMPLES = 1024
TOP = 16
STATE_SAMPLES = 64
FINAL_STATE_SAMPLES = 1024
LAYER_SAMPLES = 256
LAYER_PART = 7  # sample key of a layer output, beside the state parts 0-3
GREEDY_LAYER_STEPS = (1, 2, 4, 8, 16, 32, 64, 127)
WORKLOAD_ID = {"c2": 2, "c3": 3, "c4": 4, "c5": 5, "c2l": 2, "c3l": 3}


def prompt_ids(name: str) -> list[int]:
    w = WORKLOADS[name]
    return [int(v) for v in np.random.default_rng(w["seed"]).integers(0, VOCAB, w["prompt"])]


def draft_ids(name: str) -> list[int]:
    w = WORKLOADS[name]
    return [int(v) for v in np.random.default_rng(w["draft_seed"]).integers(0, VOCAB, w["draft"])]


def long_checkpoints(n: int) -> list[int]:
    """Reference src/device/cli.rs:368-380: 1, then k-1, k, k+1 for k = 32,
    64, ... <= n, then n (sorted, unique, within 1..n)."""
    points = [1]
    k = 32
    while k <= n:
        points += [k - 1, k, k + 1]
        k *= 2
    points.append(n)
    return sorted({p for p in points if 1 <= p <= n})


def sample(name: str, key: tuple, n: int, k: int) -> np.ndarray:
    """k indices in [0, n) (with repeats), a pure function of the key."""
    rng = np.random.default_rng([WORKLOAD_ID[name], *[int(v) for v in key]])
    return rng.integers(0, n, k)


def logits_summary(name: str, key: tuple, logits: np.ndarray) -> dict:
    order = np.lexsort((np.arange(logits.size), -logits.astype(np.float64)))[:TOP]
    idx = sample(name, (*key, 1 << 20), logits.size, LOGIT_SAMPLES)
    return dict(top_idx=order.astype(np.int32), top_val=logits[order].astype(np.float32),
                sampled=logits[idx].astype(np.float32))


def state_parts(num_layers: int):
    for layer in range(num_layers):
        for which in range(4):
            yield layer, which


def state_summary(name: str, point: int, read, num_layers: int, k: int) -> np.ndarray:
    """Concatenated samples of every non-empty state part; read(layer, which)."""
    out = []
    for layer, which in state_parts(num_layers):
        v = read(layer, which)
        if v.size:
            out.append(v[sample(name, (point, layer, which, k), v.size, k)])
    return np.concatenate(out).astype(np.float32)


def layer_summary(name: str, point: int, records, hidden: int) -> np.ndarray:
    """[layers, LAYER_SAMPLES]: each layer's output ("layer" in the oracle's
    trace, "output" in the engine's capture) at the sampled indices."""
    out = [v[sample(name, (point, layer, LAYER_PART, LAYER_SAMPLES), hidden, LAYER_SAMPLES)]
           for layer, v in records]
    return np.stack(out).astype(np.float32)


def oracle_layers(records) -> list:
    return [(layer, v) for layer, nm, v in records if nm == "layer"]


def load(name: str) -> dict:
    with np.load(HERE / f"qwen08b_{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def _oracle(name: str, threads: int):
    for p in (ROOT / "qwen-rust-inference_amd", ROOT / "oracle", ROOT / "tests"):
        if str(p) not in sys.path:
            sys.path.insert(0, str(p))
    import oracle as O
    from qwen_mi355x import model as M

    O.set_threads(threads)
    c = M.config_qwen08b()
    w = M.synthetic_weights(c, seed=0)
    if WORKLOADS[name]["int8"]:
        from test_engine_cpu import dequantised
        return O, c, dequantised(c, w)
    return O, c, O.Oracle(w)


def make(name: str, threads: int = 8) -> Path:
    O, c, o = _oracle(name, threads)
    spec = WORKLOADS[name]
    ids = prompt_ids(name)
    points = long_checkpoints(len(ids))
    s = o.new_state()
    rec = {"points": np.array(points, np.int32), "prompt": np.array(ids, np.int32)}
    t0 = time.time()
    logits = None
    layers = spec.get("layers", False)
    for p, tok in enumerate(ids, start=1):
        if layers and p in points:
            logits, records = s.step(tok, O.VECTOR, trace=True)
            rec[f"p{p}_layers"] = layer_summary(name, p, oracle_layers(records), c.hidden_size)
        else:
            logits = s.step(tok, O.VECTOR)
        if p in points:
            summ = logits_summary(name, (p,), logits)
            for k, v in summ.items():
                rec[f"p{p}_{k}"] = v
            rec[f"p{p}_pick"] = np.int32(O.select_greedy(logits))
            k = FINAL_STATE_SAMPLES if p == len(ids) else STATE_SAMPLES
            rec[f"p{p}_state"] = state_summary(name, p, s.part, c.num_layers, k)
            print(f"{name}: checkpoint {p}/{len(ids)} ({time.time() - t0:.0f} s)", flush=True)
    if spec.get("draft"):
        branch = s.clone()
        rows = []
        for r, tok in enumerate(draft_ids(name)):
            row = branch.step(tok, O.VECTOR)
            summ = logits_summary(name, (1_000_000 + r,), row)
            for k, v in summ.items():
                rec[f"d{r}_{k}"] = v
            rows.append(O.select_greedy(row))
        rec["draft"] = np.array(draft_ids(name), np.int32)
        rec["draft_picks"] = np.array(rows, np.int32)
    greedy = []
    for i in range(spec["greedy"]):
        if i and layers and i in GREEDY_LAYER_STEPS:
            logits, records = s.step(greedy[-1], O.VECTOR, trace=True)
            rec[f"g{i}_layers"] = layer_summary(name, 2_000_000 + i, oracle_layers(records), c.hidden_size)
        elif i:
            logits = s.step(greedy[-1], O.VECTOR)
        summ = logits_summary(name, (2_000_000 + i,), logits)
        for k, v in summ.items():
            rec[f"g{i}_{k}"] = v
        greedy.append(O.select_greedy(logits))
    if greedy:
        rec["greedy"] = np.array(greedy, np.int32)
        rec["greedy_state"] = state_summary(name, 3_000_000, s.part, c.num_layers, FINAL_STATE_SAMPLES)
        print(f"{name}: {len(greedy)} greedy tokens ({time.time() - t0:.0f} s)", flush=True)
    if spec.get("layers_only"):  # the rest is c2's fixture
        keep = ("points", "prompt", "greedy")
        rec = {k: v for k, v in rec.items() if k in keep or k.endswith("_layers")}
    out = HERE / f"qwen08b_{name}.npz"
    np.savez_compressed(out, **rec)
    return out


if __name__ == "__main__":
    for arg in sys.argv[1:]:
        print("wrote", make(arg), flush=True)
