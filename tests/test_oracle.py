"""Pins the CPU oracle (oracle/qwen_oracle.cpp) before anything is checked
against it: the reference's golden vectors (tests/golden, copied data files of
the reference's tests/fixtures and examples), its hand known-answer tests, and
closed forms / brute force where those leave gaps."""
import json
import math

import numpy as np
import pytest

from conftest import GOLDEN
from qwen_mi355x import model as M

import oracle as O


def close(a, b, atol, rtol):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    assert a.shape == b.shape
    err = np.abs(a - b)
    bad = ~(np.isfinite(a) & (err <= atol + rtol * np.abs(b)))
    assert not bad.any(), f"first divergence at {np.argmax(bad)}: {a[bad][:4]} vs {b[bad][:4]}, max err {err.max()}"
    return err.max() if err.size else 0.0


@pytest.fixture(scope="module")
def fixture():
    return M.load_fixture(GOLDEN / "hybrid.json")


@pytest.fixture(scope="module")
def fixture_model(fixture):
    c, w = M.fixture_config_and_weights(fixture)
    return O.Oracle(w)


@pytest.mark.parametrize("backend", [O.REFERENCE, O.VECTOR])
def test_hybrid_fixture_every_layer_and_state(fixture, fixture_model, backend):
    """Official PyTorch vectors (reference tests/hybrid.rs:2-70,
    tests/components.rs:43-92) at the reference's 2e-5 / 2e-4."""
    s = fixture_model.new_state()
    c = fixture_model.config
    for p, tok in enumerate(fixture["ids"]):
        logits, rec = s.step(tok, backend, trace=True)
        layers = [v for (_, n, v) in rec if n == "layer"]
        assert len(layers) == c.num_layers
        for layer, h in enumerate(layers):
            close(h, fixture["layers"][p][layer], 2e-5, 2e-4)
        close(logits, fixture["logits"][p], 2e-5, 2e-4)
        # per-op records of the official run
        ops = fixture["operations"][p]
        names = {"input_norm": "input_norm", "mixer": "mixer", "after_mixer": "after_mixer",
                 "post_norm": "post_norm", "ffn_product": "ffn.product", "ffn": "ffn.output"}
        for key, want in ops.items():
            layer, name = key.split(".", 1)
            got = [v for (l, n, v) in rec if l == int(layer) and n == names[name]]
            assert got, key
            close(got[0], want, 2e-5, 2e-4)
        for layer, st in fixture["states"][p].items():
            close(s.part(int(layer), 0), np.asarray(st["conv"]).reshape(-1), 2e-5, 2e-4)
            close(s.part(int(layer), 1), np.asarray(st["recurrent"]).reshape(-1), 2e-5, 2e-4)


def test_hybrid_fixture_chunked_prefill_logits(fixture, fixture_model):
    """Token-by-token logits equal the upstream chunked prefill's `full_logits`
    (reference tests/hybrid.rs:71-107)."""
    s = fixture_model.new_state()
    for p, tok in enumerate(fixture["ids"]):
        close(s.step(tok, O.REFERENCE), fixture["full_logits"][p], 2e-5, 2e-4)


def test_split_prefill_reproduces_state(fixture, fixture_model):
    """Any split of the prompt gives the same state (reference tests/hybrid.rs:23-38)."""
    ids = fixture["ids"]
    whole = fixture_model.new_state()
    for t in ids:
        whole.step(t, O.REFERENCE)
    for split in range(len(ids) + 1):
        s = fixture_model.new_state()
        for t in ids[:split]:
            s.step(t, O.REFERENCE)
        t2 = s.clone()
        for t in ids[split:]:
            t2.step(t, O.REFERENCE)
        for layer in range(fixture_model.config.num_layers):
            for which in range(4):
                assert np.array_equal(t2.part(layer, which), whole.part(layer, which))


def test_lesson_trace_reference_outputs(fixture_model):
    """Every op record of the reference's own Backend::Reference lesson run
    (examples/lesson-trace.ndjson, IDs [1, 4, 2]) at the lesson test's
    2e-6 / 2e-5 (reference tests/lesson.rs:100-145); nearly all are equal bits."""
    rows = [json.loads(line) for line in open(GOLDEN / "lesson-trace.ndjson")]
    s = fixture_model.new_state()
    recs = {}
    for p, tok in enumerate([1, 4, 2]):
        _, rec = s.step(tok, O.REFERENCE, trace=True)
        for (layer, name, v) in rec:
            recs[(p, layer, name)] = v
    same = total = checked = 0
    for r in rows:
        key = (r["token_position"], r["layer"], r["operation"])
        if r["operation"].startswith("lesson."):
            continue  # the lesson's own zero-unit edit records (FFN intervention, out of scope)
        assert key in recs, key
        a = recs[key]
        b = np.asarray(r["values"], dtype=np.float32)
        assert a.shape == b.shape, key
        close(a, b, 2e-6, 2e-5)
        same += int(np.sum(a.view(np.uint32) == b.view(np.uint32)))
        total += a.size
        checked += 1
    assert checked == 324
    assert same / total > 0.999


def test_lesson_answers_greedy(fixture_model):
    saved = json.load(open(GOLDEN / "lesson-answers.json"))
    s = fixture_model.new_state()
    for p, tok in enumerate([1, 4, 2]):
        logits = s.step(tok, O.REFERENCE)
        assert O.select_greedy(logits) == saved["steps"][p]["greedy_next"]
        top = sorted(range(logits.size), key=lambda i: (-logits[i], i))[:5]
        assert [t[0] for t in saved["steps"][p]["top5"]] == top


def test_phase1_official_vectors():
    """phase1.json: FFN, both RMSNorm scales, softmax (reference tests/fixtures.rs:33-85)."""
    d = json.load(open(GOLDEN / "phase1.json"))["data"]
    f = lambda k: np.asarray(d[k], dtype=np.float32)
    x = f("x")
    gate = O.project(f("gate_weights"), 16, 8, x, O.REFERENCE)
    up = O.project(f("up_weights"), 16, 8, x, O.REFERENCE)
    close(gate, d["gate"], 2e-6, 2e-5)
    close(up, d["up"], 2e-6, 2e-5)
    act = O.silu(gate)
    close(act, d["activated_gate"], 2e-6, 2e-5)
    product = (act * up).astype(np.float32)
    close(product, d["product"], 2e-6, 2e-5)
    out = O.project(f("down_weights"), 8, 16, product, O.REFERENCE)
    close(out, d["output"], 2e-6, 2e-5)
    edited = product.copy()
    edited[3] = 0
    close(O.project(f("down_weights"), 8, 16, edited, O.REFERENCE), d["edited_output"], 2e-6, 2e-5)
    close(O.rms_norm(x, f("norm_weight"), 1e-6, True), d["norm"], 2e-6, 2e-5)
    close(O.rms_norm(x, f("norm_weight"), 1e-6, False), d["direct_norm"], 2e-6, 2e-5)
    close(O.softmax(x), d["softmax"], 2e-6, 2e-5)
    close((x + out).astype(np.float32), d["residual"], 2e-6, 2e-5)


def test_hand_known_answers():
    """Reference tests/phase1.rs:24-44 and tests/components.rs:93-171."""
    for backend in (O.REFERENCE, O.VECTOR):
        assert list(O.project(np.array([1, 2, 3, 4], np.float32), 2, 2, np.array([1, 2], np.float32), backend)) == [5, 11]
        # the device tests' non-square KAT (src/device/tests.rs:61-95)
        w = np.array([1, 2, 3, 4, 5, 6], np.float32)
        assert list(O.project(w, 2, 3, np.array([2, -1, 3], np.float32), backend)) == [9, 21]
        odd = np.array([1, -2, 0.5, 4, 8, -0.25, 3, 6, 1.5], np.float32)
        assert list(O.project(odd, 3, 3, np.array([2, -1, 3], np.float32), backend)) == [5.5, -0.75, 4.5]
    assert list(O.softmax(np.array([1000, 1000], np.float32))) == [0.5, 0.5]
    close(O.silu(np.array([-1000, 0, 1, 1000], np.float32)), [0, 0, 0.7310586, 1000], 2e-6, 2e-5)
    close(O.rms_norm(np.array([3, 4], np.float32), np.ones(2, np.float32), 1e-6, False), [0.8485281, 1.1313709], 2e-6,
          2e-5)
    close(O.rms_norm(np.array([3, 4], np.float32), np.zeros(2, np.float32), 1e-6, True), [0.8485281, 1.1313709], 2e-6,
          2e-5)
    s = np.zeros(4, np.float32)
    q = np.array([1, 0], np.float32)
    assert list(O.delta_rule(q, q, np.array([2, 3], np.float32), 0.0, 1.0, s)) == [2, 3]
    assert list(s) == [2, 3, 0, 0]
    assert list(O.delta_rule(q, q, np.array([8, 9], np.float32), 0.0, 0.0, s)) == [2, 3]
    assert list(O.delta_rule(q, q, np.array([8, 9], np.float32), -1000.0, 0.0, s)) == [0, 0]
    with pytest.raises(RuntimeError):
        O.delta_rule(np.ones(1, np.float32), np.ones(1, np.float32), np.ones(1, np.float32), 1.0, 0.5,
                     np.zeros(1, np.float32))
    with pytest.raises(RuntimeError):
        O.delta_rule(np.ones(1, np.float32), np.ones(1, np.float32), np.ones(1, np.float32), 0.0, 1.1,
                     np.zeros(1, np.float32))
    s6 = np.zeros(6, np.float32)
    assert list(O.delta_rule(q, q, np.array([2, 3, 4], np.float32), 0.0, 1.0, s6)) == [2, 3, 4]
    assert list(s6) == [2, 3, 4, 0, 0, 0]
    x = np.array([1, 2, 7, 8], np.float32)
    O.rotate(x, 1, 2, 10000.0)
    close(x, [math.cos(1) - 2 * math.sin(1), 2 * math.cos(1) + math.sin(1), 7, 8], 2e-6, 2e-5)


def test_projection_brute_force_and_orders():
    """Both summation orders against an fp64 dot product on odd shapes (a
    dropped tail or transposed operand fails this)."""
    rng = np.random.default_rng(7)
    for rows, cols in [(1, 1), (7, 13), (5, 8), (3, 17), (64, 100)]:
        w = rng.standard_normal(rows * cols).astype(np.float32)
        x = rng.standard_normal(cols).astype(np.float32)
        exact = w.reshape(rows, cols).astype(np.float64) @ x.astype(np.float64)
        for backend in (O.REFERENCE, O.VECTOR):
            close(O.project(w, rows, cols, x, backend), exact, 1e-5, 1e-5)
    # Reference order is a plain left fold: compare bits with a float32 fold
    w = rng.standard_normal(3 * 29).astype(np.float32)
    x = rng.standard_normal(29).astype(np.float32)
    fold = []
    for r in range(3):
        acc = np.float32(0)
        for j in range(29):
            acc = np.float32(acc + np.float32(w[r * 29 + j] * x[j]))
        fold.append(acc)
    assert np.array_equal(O.project(w, 3, 29, x, O.REFERENCE), np.array(fold, np.float32))


def test_attention_hand_examples():
    """attend (reference tests/components.rs:117-150): one head reading
    exp(0):exp(ln 3) = 1:3 of the values 2 and 6 gives 5; with 4 query heads
    over 2 KV heads, heads 0-1 read KV head 0 and heads 2-3 KV head 1
    (contiguous groups; a modulo mapping gives [3, 12, 3, 12])."""
    one = O.attend(np.array([1], np.float32), np.array([[0], [math.log(3)]], np.float32),
                   np.array([[2], [6]], np.float32), 1, 1, 1)
    close(one, [5], 1e-6, 1e-6)
    gqa = O.attend(np.ones(4, np.float32), np.zeros((2, 2), np.float32), np.array([[2, 10], [4, 14]], np.float32),
                   4, 2, 1)
    close(gqa, [3, 3, 12, 12], 1e-6, 1e-6)
    # 8 query heads over 2 KV heads at head_dim 4 against a float64 dense
    # softmax, every head with its own query: the group of head h is h // 4
    rng = np.random.default_rng(17)
    q = rng.standard_normal(8 * 4).astype(np.float32)
    k = rng.standard_normal((6, 2 * 4)).astype(np.float32)
    v = rng.standard_normal((6, 2 * 4)).astype(np.float32)
    got = O.attend(q, k, v, 8, 2, 4)
    for h in range(8):
        g = h // 4
        s = k[:, g * 4:(g + 1) * 4].astype(np.float64) @ q[h * 4:(h + 1) * 4].astype(np.float64) / 2.0
        p = np.exp(s - s.max())
        p /= p.sum()
        close(got[h * 4:(h + 1) * 4], p @ v[:, g * 4:(g + 1) * 4].astype(np.float64), 1e-5, 1e-5)
    # the rotate-half RoPE at position 0 is the identity
    x = np.arange(8, dtype=np.float32)
    assert np.array_equal(O.rotate(x.copy(), 0, 8, 1e7), x)


@pytest.mark.parametrize("position,dim,length,theta", [(1, 64, 256, 1e7), (453, 64, 256, 1e7), (8190, 64, 256, 1e7),
                                                       (7, 8, 16, 1e4), (3, 16, 20, 1e6)])
def test_rope_closed_form(position, dim, length, theta):
    """rotate (reference src/attention.rs:41-57) against the RoFormer /
    upstream definition in float64: inv_freq_i = theta^(-2i/dim) for
    i < dim/2, angle = position * inv_freq_i, and the rotate-half pairing of
    x[i] with x[i + dim/2]; dims past `dim` pass through. A frequency
    exponent of i/dim, an adjacent-pair rotation or a wrong sign fails."""
    rng = np.random.default_rng(position + dim)
    x = rng.standard_normal(length).astype(np.float32)
    got = O.rotate(x.copy(), position, dim, theta)
    half = dim // 2
    i = np.arange(half, dtype=np.float64)
    angle = position * theta ** (-2.0 * i / dim)
    a, b = x[:half].astype(np.float64), x[half:dim].astype(np.float64)
    want = x.astype(np.float64).copy()
    want[:half] = a * np.cos(angle) - b * np.sin(angle)
    want[half:dim] = b * np.cos(angle) + a * np.sin(angle)
    # float32 angles: |error| <= a few ulp of the angle (position up to 8190)
    tol = 4 * np.spacing(np.float32(max(position, 1))) * (np.abs(a) + np.abs(b)).max() + 1e-6
    assert np.max(np.abs(got - want)) <= tol, np.max(np.abs(got - want))
    assert np.array_equal(got[dim:], x[dim:])


def test_int8_quantizer_invariants():
    """quantize_int8_rows (reference src/device.rs:220-239; invariants of
    src/device/tests.rs:1320-1347): |w - s q| <= s / 2, q in [-127, 127],
    zero rows have scale 0, ties round to even."""
    rng = np.random.default_rng(3)
    rows, cols = 9, 33
    w = rng.standard_normal(rows * cols).astype(np.float32)
    w[2 * cols:3 * cols] = 0
    w[5 * cols + 4] = 40.0
    s, q = O.quantize_int8_rows(w, rows, cols)
    wq = q.reshape(rows, cols).astype(np.float32) * s[:, None]
    assert s[2] == 0 and not q.reshape(rows, cols)[2].any()
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    assert np.all(np.abs(w.reshape(rows, cols) - wq) <= s[:, None] / 2 * (1 + 1e-6))
    assert q.reshape(rows, cols)[5, 4] == 127
    # ties to even: a row whose scale is exactly 1 (max 127)
    t = np.array([127.0, 0.5, 1.5, 2.5, -0.5, -1.5], np.float32)
    s1, q1 = O.quantize_int8_rows(t, 1, 6)
    assert s1[0] == 1.0 and list(q1) == [127, 0, 2, 2, 0, -2]


def test_vector_backend_matches_reference_backend(fixture):
    c, w = M.fixture_config_and_weights(fixture)
    o = O.Oracle(w)
    a, b = o.new_state(), o.new_state()
    for tok in fixture["ids"]:
        close(a.step(tok, O.VECTOR), b.step(tok, O.REFERENCE), 2e-6, 2e-5)


def test_greedy_selection_rules():
    """select (reference src/generate.rs:30-41): first index of the max; non-finite is an error."""
    assert O.select_greedy(np.array([1, 3, 3, 2], np.float32)) == 1
    assert O.select_greedy(np.array([-1], np.float32)) == 0
    with pytest.raises(RuntimeError):
        O.select_greedy(np.array([1, np.nan], np.float32))


def test_state_load_round_trip(fixture_model):
    """A state loaded part by part (the CPU side of the reference's
    load_state / inspect_state interchange, src/device.rs:2380-2537)
    continues exactly like the state it was read from."""
    s = fixture_model.new_state()
    for tok in [1, 4, 2, 8, 3, 5, 7]:
        s.step(tok, O.REFERENCE)
    t = fixture_model.new_state()
    t.load(s.position, s.part)
    assert t.position == s.position
    for tok in [6, 2]:
        assert np.array_equal(t.step(tok, O.REFERENCE), s.step(tok, O.REFERENCE))
    with pytest.raises(RuntimeError):
        t.load(3, lambda layer, which: np.zeros(0, np.float32))


def test_edit_overlay_closed_form(fixture):
    """EditManifest::apply (reference src/edit.rs:59-110) against what it
    stands for: disabling unit j with coefficient 1 is the model whose down
    column j is zero; removing direction d from columns J with coefficient a
    is the model whose down columns w_j (j in J) are w_j - a d (d.w_j)/(d.d)
    (reference comment src/edit.rs:88-91). The edited oracle matches both
    weight-edited oracles, on every prompt position."""
    c, w = M.fixture_config_and_weights(fixture)
    H, I = c.hidden_size, c.intermediate_size
    d = np.zeros(H, np.float32)
    d[0], d[H - 1] = 1.0, -0.5
    edits = [dict(layer=1, columns=[3], direction=None, coefficient=1.0),
             dict(layer=2, columns=[0, 5], direction=d, coefficient=0.7)]
    o = O.Oracle(w)
    o.set_edit(edits)
    t = dict(w.tensors)
    down1 = t[M.QW_SLOTS_BASE + 1 * M.QW_SLOTS_LAYER + M.DOWN].reshape(H, I).copy()
    down1[:, 3] = 0
    down2 = t[M.QW_SLOTS_BASE + 2 * M.QW_SLOTS_LAYER + M.DOWN].reshape(H, I).astype(np.float64)
    dd = d.astype(np.float64)
    for j in (0, 5):
        down2[:, j] -= 0.7 * dd * (dd @ down2[:, j]) / (dd @ dd)
    t[M.QW_SLOTS_BASE + 1 * M.QW_SLOTS_LAYER + M.DOWN] = np.ascontiguousarray(down1.reshape(-1))
    t[M.QW_SLOTS_BASE + 2 * M.QW_SLOTS_LAYER + M.DOWN] = np.ascontiguousarray(down2.astype(np.float32).reshape(-1))
    ref = O.Oracle(M.Weights(c, t))
    a, b = o.new_state(), ref.new_state()
    for tok in fixture["ids"]:
        close(a.step(tok, O.REFERENCE), b.step(tok, O.REFERENCE), 1e-6, 1e-5)
