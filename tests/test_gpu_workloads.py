"""The full BASELINE workloads of the Qwen3.5-0.8B-shaped model on the MI355X,
against the CPU oracle's golden vectors (tests/golden/qwen08b.py made them:
the oracle restates the reference's Rust Backend::Vector path and is run once
on the CPU, since 2644 tokens take it ~9 minutes and 8192 tokens ~28).

At every point of the reference's long-context check (`long_checkpoints`,
src/device/cli.rs:368-507: prefill lengths 1, 2^k-1, 2^k, 2^k+1, N, each
segment prefilled in one call) the run's logits and every state part are
compared on the fixture's sampled indices within the fp32 bound (int8: the
oracle on the dequantised weights at 1e-2), and the top-1 token must match
unless the oracle's top-2 margin is inside the bound. Greedy decode after the
prompt must pick the oracle's tokens (same near-tie rule, which ends the id
comparison); the logits of every decode step are compared teacher-forced.

  C2  454-token prompt + 128 greedy tokens (the bench workload); every
      layer's output (the hidden state after each block) at every checkpoint
      and at greedy steps 1, 2, 4, ..., 64, 127 (the reference's per-layer
      validate_device, src/device/cli.rs:229-366)
  C3  2644-token prefill: one chunk, the checkpoint walk, 128-token chunks
      (the reference's PREFILL_CHUNK); 10,240 tokens in one chunk against
      the same prompt in 128-token chunks
  C4  8192-token prefill (checkpoint walk) + 64 greedy tokens, one-launch
      decode against the op sequence
  C5  int8 per-row weights: 454-token prompt, the 4-row verify with
      snapshots, 16 greedy tokens
"""
import sys

import numpy as np
import pytest

from conftest import GOLDEN
from parity import FP32_RTOL, INT8_RTOL, parity
from qwen_mi355x import engine as E
from qwen_mi355x import model as M

sys.path.insert(0, str(GOLDEN))
import qwen08b as G  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def weights():
    print("synthesising 0.8B weights", flush=True)
    c = M.config_qwen08b(max_positions=16384)
    return c, M.synthetic_weights(c, seed=0)


@pytest.fixture(scope="module")
def fast(weights):
    c, w = weights
    m = E.Model(w)
    m.set_run_budget(64 << 30)
    return m


def nonempty_parts(run, c):
    return [(l, k) for (l, k) in G.state_parts(c.num_layers) if run.state(l, k).size]


def check_logits(name, key, logits, rec, prefix, rtol, where):
    """Sampled logits within the bound; returns (oracle top-2 margin, bound at the top)."""
    idx = G.sample(name, (*key, 1 << 20), logits.size, rec[prefix + "sampled"].size)
    parity(logits[idx], rec[prefix + "sampled"], rtol=rtol, where=where)
    top = rec[prefix + "top_val"].astype(np.float64)
    parity(logits[rec[prefix + "top_idx"]], top, rtol=rtol, where=where + " top-16")
    floor = float(np.sqrt(np.mean(rec[prefix + "sampled"].astype(np.float64) ** 2)))
    margin = float(top[0] - top[1])
    return margin, rtol * (abs(top[0]) + floor)


def check_pick(got, want, margin, bound, where):
    """The greedy token must equal the oracle's unless the oracle's top-2
    margin is within twice the logits bound (a near-tie that fp32 summation
    order may legitimately flip). Returns True when they are equal."""
    if got == want:
        return True
    assert margin <= 2 * bound, f"{where}: picked {got}, oracle {want} with top-2 margin {margin:.3e} > 2 x {bound:.3e}"
    print(f"{where}: near-tie (margin {margin:.2e} <= 2 x bound {bound:.2e}): picked {got}, oracle {want}", flush=True)
    return False


# The DeltaNet recurrent state (part 1) after thousands of tokens: the rule's
# residual d = beta (v - S^T k) cancels, which amplifies fp32 ordering noise
# there. Measured on the 8192-token prompt of C4: two correct fp32 GPU
# evaluations (one prefill chunk against 128-token chunks) differ by up to
# 1.15e-4 in the recurrent state of layers 17-21, while every conv, key and
# value part agrees to 4.1e-5 and the logits to 3.4e-5; each of the two is
# within 1.2e-4 of the oracle there. Past 4096 tokens the recurrent state is
# held to twice the fp32 bound, every other part and the logits to the bound.
LONG_RECURRENT_RTOL = 2 * FP32_RTOL


def check_state(name, point, run, c, rec, key, rtol, where, recurrent_rtol=None):
    parts = nonempty_parts(run, c)
    flat = rec[key]
    k = flat.size // len(parts)
    assert k * len(parts) == flat.size
    for n, (layer, which) in enumerate(parts):
        v = run.state(layer, which)
        got = v[G.sample(name, (point, layer, which, k), v.size, k)]
        r = recurrent_rtol if (recurrent_rtol is not None and which == 1) else rtol
        parity(got, flat[n * k:(n + 1) * k], rtol=r, where=f"{where} state {layer}/{which}")


def walk_checkpoints(name, run, c, rec, rtol=FP32_RTOL):
    """validate_long (reference src/device/cli.rs:391-507) on the fixture's
    points: each segment in one prefill call, logits + top-1 + every state."""
    ids = [int(v) for v in rec["prompt"]]
    done = 0
    margins = []
    logits = None
    for p in [int(v) for v in rec["points"]]:
        logits = run.prefill(ids[done:p])
        done = p
        assert run.position == p
        margin, bound = check_logits(name, (p,), logits, rec, f"p{p}_", rtol, f"{name} checkpoint {p}")
        check_pick(int(np.argmax(logits)), int(rec[f"p{p}_pick"]), margin, bound, f"{name} checkpoint {p}")
        check_state(name, p, run, c, rec, f"p{p}_state", rtol, f"{name} checkpoint {p}",
                    recurrent_rtol=LONG_RECURRENT_RTOL if p > 4096 and rtol == FP32_RTOL else None)
        margins.append(margin)
        print(f"{name}: checkpoint {p} ok (top-2 margin {margin:.3e})", flush=True)
    return logits


def greedy_against_fixture(name, run, rec, rtol=FP32_RTOL):
    """decode_greedy from the prompt's last logits: identical ids up to the
    first near-tie; then every step teacher-forced on the oracle's tokens
    (from a checkpoint of the run), its logits against the fixture."""
    want = [int(v) for v in rec["greedy"]]
    cp = run.checkpoint()
    got, _ = run.decode_greedy(want[0], len(want))
    margins = []
    for i in range(len(want)):
        top = rec[f"g{i}_top_val"].astype(np.float64)
        margins.append(float(top[0] - top[1]))
    same = 0
    for i in range(1, len(want)):
        floor = float(np.sqrt(np.mean(rec[f"g{i}_sampled"].astype(np.float64) ** 2)))
        bound = rtol * (abs(float(rec[f"g{i}_top_val"][0])) + floor)
        if not check_pick(got[i], want[i], margins[i], bound, f"{name} greedy step {i}"):
            break
        same = i
    print(f"{name}: {same + 1}/{len(want)} greedy ids identical; smallest oracle top-2 margin "
          f"{min(margins):.3e} (step {int(np.argmin(margins))})", flush=True)
    run.restore(cp)
    for i in range(1, len(want)):
        logits = run.step(want[i - 1])
        check_logits(name, (2_000_000 + i,), logits, rec, f"g{i}_", rtol, f"{name} teacher-forced step {i}")
    return got


def test_c2_prompt_checkpoints_and_greedy(weights, fast):
    """the 454-token prompt (checkpoint walk) and 128 greedy tokens."""
    c, _ = weights
    rec = G.load("c2")
    run = fast.new_run(454 + 136, chunk=454)
    assert run.decode_plan
    walk_checkpoints("c2", run, c, rec)
    greedy_against_fixture("c2", run, rec)
    check_state("c2", 3_000_000, run, c, rec, "greedy_state", FP32_RTOL, "c2 after greedy")


def check_layers(name, key, records, want, c, rtol, where):
    """The captured "output" record of every layer (the engine's capture of
    forward_body) against the fixture's samples of the oracle's "layer"."""
    outs = {layer: v for layer, nm, v in records if nm == "output"}
    assert sorted(outs) == list(range(c.num_layers)), sorted(outs)
    for layer in range(c.num_layers):
        idx = G.sample(name, (key, layer, G.LAYER_PART, G.LAYER_SAMPLES), c.hidden_size, G.LAYER_SAMPLES)
        parity(outs[layer][idx], want[layer], rtol=rtol, where=f"{where} layer {layer} output")


def test_c2_layer_outputs(weights, fast):
    """Config 2's prompt: at every checkpoint p the tokens before p in one
    prefill chunk and token p as a captured step (the engine's op path records
    every layer's output), each layer's hidden state and the logits against
    the oracle; then the greedy tokens, with steps 1, 2, 4, ..., 64 and 127
    captured, the others on the one-launch decode."""
    c, _ = weights
    rec, full = G.load("c2l"), G.load("c2")
    ids = [int(v) for v in rec["prompt"]]
    run = fast.new_run(454 + 136, chunk=454)
    assert run.decode_plan
    done = 0
    for p in [int(v) for v in rec["points"]]:
        if p - 1 > done:
            run.prefill(ids[done:p - 1])
        logits, records = run.step(ids[p - 1], capture=True)
        done = p
        check_layers("c2", p, records, rec[f"p{p}_layers"], c, FP32_RTOL, f"c2 checkpoint {p}")
        check_logits("c2", (p,), logits, full, f"p{p}_", FP32_RTOL, f"c2 checkpoint {p} (captured)")
        print(f"c2: checkpoint {p}: {c.num_layers} layer outputs ok", flush=True)
    greedy = [int(v) for v in rec["greedy"]]
    for i in range(1, len(greedy)):
        if i in G.GREEDY_LAYER_STEPS:
            logits, records = run.step(greedy[i - 1], capture=True)
            check_layers("c2", 2_000_000 + i, records, rec[f"g{i}_layers"], c, FP32_RTOL, f"c2 greedy step {i}")
        else:
            logits = run.step(greedy[i - 1])
        check_logits("c2", (2_000_000 + i,), logits, full, f"g{i}_", FP32_RTOL, f"c2 greedy step {i}")
    print(f"c2: layer outputs at {len(rec['points'])} checkpoints and {len(G.GREEDY_LAYER_STEPS)} greedy steps ok",
          flush=True)


def test_c3_prefill_2644_one_chunk(weights, fast):
    """2644 tokens in one prefill chunk (the bench's call):
    last-row logits, pick and 1024 samples of every state part."""
    c, _ = weights
    rec = G.load("c3")
    run = fast.new_run(2644, chunk=2644)
    logits = run.prefill([int(v) for v in rec["prompt"]])
    margin, bound = check_logits("c3", (2644,), logits, rec, "p2644_", FP32_RTOL, "c3 one chunk")
    check_pick(int(np.argmax(logits)), int(rec["p2644_pick"]), margin, bound, "c3 one chunk")
    check_state("c3", 2644, run, c, rec, "p2644_state", FP32_RTOL, "c3 one chunk")


def test_c3_prefill_2644_checkpoints(weights, fast):
    c, _ = weights
    walk_checkpoints("c3", fast.new_run(2644, chunk=2644), c, G.load("c3"))


def test_c3_prefill_2644_reference_chunks(weights, fast):
    """The same prompt in 128-token chunks (the reference engine's
    PREFILL_CHUNK, src/device.rs): what an unmodified engine would send."""
    c, _ = weights
    rec = G.load("c3")
    run = fast.new_run(2644, chunk=128)
    logits = run.prefill([int(v) for v in rec["prompt"]])
    check_logits("c3", (2644,), logits, rec, "p2644_", FP32_RTOL, "c3 chunk 128")
    check_state("c3", 2644, run, c, rec, "p2644_state", FP32_RTOL, "c3 chunk 128")


def test_c3_prefill_10240_one_chunk_vs_chunks(weights, fast):
    """10,240 tokens (seed 2) in one chunk against 128-token chunks: last-row
    logits and every state part, whole. Both sides are GPU results, each
    within the fp32 bound of the exact value (the one-chunk prefill is held
    to it against the oracle at 2644 and 8192 tokens), so their difference is
    held to twice the bound."""
    c, _ = weights
    ids = [int(v) for v in np.random.default_rng(2).integers(0, c.vocab_size, 10240)]
    a, b = fast.new_run(10240, chunk=10240), fast.new_run(10240, chunk=128)
    la, lb = a.prefill(ids), b.prefill(ids)
    worst = [parity(la, lb, rtol=2 * FP32_RTOL, where="10240 logits")]
    for layer, which in nonempty_parts(a, c):
        worst.append(parity(a.state(layer, which), b.state(layer, which), rtol=2 * FP32_RTOL,
                            where=f"10240 state {layer}/{which}"))
    print(f"10240 one chunk vs 128-token chunks: largest relative difference {max(worst):.3e}", flush=True)


def test_c3_prefill_10240_one_chunk_against_oracle(weights, fast):
    """BASELINE config 3's second size against the oracle (fixture c3l): the
    10,240-token prompt in one prefill chunk (the bench's call), last-row
    logits, pick and 1024 samples of every state part; then the same prompt
    as one chunk of 10,239 tokens and token 10,240 as a captured one-launch
    step: its logits and every layer's output against the oracle's trace."""
    c, _ = weights
    rec = G.load("c3l")
    ids = [int(v) for v in rec["prompt"]]
    n = len(ids)
    run = fast.new_run(n, chunk=n)
    logits = run.prefill(ids)
    margin, bound = check_logits("c3l", (n,), logits, rec, f"p{n}_", FP32_RTOL, "c3 10240 one chunk")
    check_pick(int(np.argmax(logits)), int(rec[f"p{n}_pick"]), margin, bound, "c3 10240 one chunk")
    check_state("c3l", n, run, c, rec, f"p{n}_state", FP32_RTOL, "c3 10240 one chunk",
                recurrent_rtol=LONG_RECURRENT_RTOL)
    run.close()
    run = fast.new_run(n, chunk=n - 1)
    assert run.decode_plan
    run.prefill(ids[:n - 1])
    logits, records = run.step(ids[n - 1], capture=True)
    check_layers("c3l", n, records, rec[f"p{n}_layers"], c, FP32_RTOL, "c3 10240 captured step")
    check_logits("c3l", (n,), logits, rec, f"p{n}_", FP32_RTOL, "c3 10240 captured step")
    print("c3: 10240 one chunk and captured last step against the oracle ok", flush=True)


def test_c3_prefill_10240_checkpoints(weights, fast):
    """validate_long on the 10,240-token prompt: every checkpoint (1 .. 8193,
    10,240) as one prefill call from the previous one, logits, pick and every
    state part against the oracle; at the checkpoints up to 8193 the captured
    step's layer outputs too (a second run: the tokens before the point in
    one chunk, the point's token captured)."""
    c, _ = weights
    rec = G.load("c3l")
    walk_checkpoints("c3l", fast.new_run(10240, chunk=10240), c, rec)
    ids = [int(v) for v in rec["prompt"]]
    run = fast.new_run(10240, chunk=10240)
    done = 0
    for p in [int(v) for v in rec["points"]]:
        if f"p{p}_layers" not in rec:
            continue
        if p - 1 > done:
            run.prefill(ids[done:p - 1])
        _, records = run.step(ids[p - 1], capture=True)
        done = p
        check_layers("c3l", p, records, rec[f"p{p}_layers"], c, FP32_RTOL, f"c3 checkpoint {p}")
    print("c3: 10240 checkpoint walk and layer outputs ok", flush=True)


def test_c4_prefill_8192_one_chunk(weights, fast):
    """The whole 8192-token prompt in one prefill chunk against the oracle:
    last-row logits, pick and 1024 samples of every state part."""
    c, _ = weights
    rec = G.load("c4")
    run = fast.new_run(8192, chunk=8192)
    logits = run.prefill([int(v) for v in rec["prompt"]])
    margin, bound = check_logits("c4", (8192,), logits, rec, "p8192_", FP32_RTOL, "c4 one chunk")
    check_pick(int(np.argmax(logits)), int(rec["p8192_pick"]), margin, bound, "c4 one chunk")
    check_state("c4", 8192, run, c, rec, "p8192_state", FP32_RTOL, "c4 one chunk", recurrent_rtol=LONG_RECURRENT_RTOL)


def test_c4_prefill_8192_checkpoints_and_greedy(weights, fast):
    """a real 8192-token prefill (checkpoint walk) then 64
    greedy tokens on the one-launch decode."""
    c, _ = weights
    rec = G.load("c4")
    run = fast.new_run(8192 + 72, chunk=8192)
    assert run.decode_plan
    walk_checkpoints("c4", run, c, rec)
    greedy_against_fixture("c4", run, rec)
    check_state("c4", 3_000_000, run, c, rec, "greedy_state", FP32_RTOL, "c4 after greedy",
                recurrent_rtol=LONG_RECURRENT_RTOL)


def test_c4_one_launch_vs_op_sequence_at_8192(weights, fast):
    """After the real 8192-token prefill, the oracle's 64 tokens on the
    one-launch decode and on the op sequence: logits of every step and every
    state part at the end within the fp32 bound."""
    c, w = weights
    rec = G.load("c4")
    ids = [int(v) for v in rec["prompt"]]
    ops = E.Model(w, disable=E.NO_DECODE_STEP)
    ops.set_run_budget(64 << 30)
    a, b = fast.new_run(8192 + 72, chunk=8192), ops.new_run(8192 + 72, chunk=8192)
    assert a.decode_plan and not b.decode_plan
    a.prefill(ids)
    b.prefill(ids)
    for i, t in enumerate([int(v) for v in rec["greedy"]]):
        parity(a.step(t), b.step(t), where=f"8192 + {i}: one-launch vs op sequence")
    for layer, which in nonempty_parts(a, c):
        parity(a.state(layer, which), b.state(layer, which), where=f"8192 + 64 state {layer}/{which}")
    ops.close()


def test_c5_int8_prompt_verify_and_greedy(weights):
    """int8 per-row weights against the oracle on the
    dequantised weights at 1e-2: the 454-token prompt (checkpoint walk), the
    4-row verify with snapshots (each row against the oracle's sequential
    step), then 16 greedy tokens."""
    c, w = weights
    rec = G.load("c5")
    m8 = E.Model(w, fmt=E.INT8)
    run = m8.new_run(454 + 24, chunk=454, snapshots=3)
    assert run.decode_plan
    walk_checkpoints("c5", run, c, rec, rtol=INT8_RTOL)
    cp = run.checkpoint()
    draft = [int(v) for v in rec["draft"]]
    rows = run.verify_rollback(draft)
    for r in range(len(draft)):
        check_logits("c5", (1_000_000 + r,), rows[r], rec, f"d{r}_", INT8_RTOL, f"c5 verify row {r}")
    run.accept(len(draft))
    run.restore(cp)
    greedy_against_fixture("c5", run, rec, rtol=INT8_RTOL)
    m8.close()


@pytest.mark.parametrize("rows,cols", [(6144, 1024), (3584, 1024), (1024, 3584), (1024, 2048), (16, 1024)])
@pytest.mark.parametrize("batch", [2644, 10240])
def test_gemm_f32_prefill_full_size(rows, cols, batch):
    """The prefill GEMM at config 3's token counts (the MFMA kernel with its
    K-split for N = 1024, and the skinny kernel for the 16-row a/b
    projections), a sample of 64 token rows against fp64 with the fp32
    dot-product bound."""
    from parity import dot_bound
    from qwen_mi355x.bridge import Bridge
    print(f"gemm f32 {rows}x{cols} batch {batch}", flush=True)
    gpu = Bridge()
    rng = np.random.default_rng(rows + cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    y = gpu.alloc(batch * rows)
    gpu.gemm(y, gpu.upload(w), gpu.upload(x), rows, cols, batch)
    got = y.read().reshape(batch, rows)
    pick = np.unique(np.concatenate([[0, batch - 1], rng.integers(0, batch, 62)]))
    W = w.reshape(rows, cols).astype(np.float64)
    X = x.reshape(batch, cols)[pick]
    want = X.astype(np.float64) @ W.T
    bound = dot_bound(W, X.T).T
    assert np.all(np.abs(got[pick] - want) <= bound), np.max(np.abs(got[pick] - want) - bound)
    gpu.close()
