"""The whole decode/prefill path on the MI355X bridge, driven by the host
engine exactly as the reference's engine drives its bridge, against the CPU
oracle on the same seeded weights: identical greedy IDs, per-layer records
and logits within the fp32 parity bound (int8: against the oracle on the
dequantised weights)."""
import numpy as np
import pytest

from conftest import GOLDEN
from parity import INT8_RTOL, bf16_weights, parity
from qwen_mi355x import engine as E
from qwen_mi355x import model as M
from test_engine_cpu import dequantised

import oracle as O

pytestmark = pytest.mark.gpu

NAMES = {"input_norm": "input_norm", "mixed": "mixer", "after_mixer": "after_mixer", "post_norm": "post_norm",
         "ffn_product": "ffn.product", "ffn": "ffn.output", "output": "layer"}


@pytest.fixture(scope="module")
def fixture():
    return M.load_fixture(GOLDEN / "hybrid.json")


@pytest.fixture(scope="module")
def tiny():
    c = M.config_tiny()
    return c, M.synthetic_weights(c, seed=0)


def tiny_prompt():
    return [int(v) for v in np.random.default_rng(1).integers(0, 512, 16)]


def oracle_greedy(o, prompt, n_new, backend=O.VECTOR):
    s = o.new_state()
    for t in prompt:
        logits = s.step(t, backend)
    ids, all_logits = [O.select_greedy(logits)], [logits]
    for _ in range(n_new - 1):
        logits = s.step(ids[-1], backend)
        all_logits.append(logits)
        ids.append(O.select_greedy(logits))
    return ids, all_logits, s


@pytest.mark.parametrize("fmt", [E.F32, E.BF16_EXACT])
def test_fixture_every_record(fixture, fmt):
    print(f"fixture format {fmt}", flush=True)
    c, w = M.fixture_config_and_weights(fixture)
    run = E.Model(w, fmt=fmt).new_run(len(fixture["ids"]))
    s = O.Oracle(w).new_state()
    for tok in fixture["ids"]:
        logits, rec = run.step(tok, capture=True)
        want, orec = s.step(tok, O.REFERENCE, trace=True)
        omap = {(l, n): v for (l, n, v) in orec}
        for (layer, name, v) in rec:
            if name in NAMES:
                parity(v, omap[(layer, NAMES[name])], where=f"{layer}.{name}")
        parity(logits, want, where="logits")
        assert O.select_greedy(logits) == O.select_greedy(want)
    for layer in range(c.num_layers):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"state {layer}/{which}")


def test_tiny_config1_greedy_bit_exact(tiny):
    """16-token prompt, 32 greedy tokens, identical IDs."""
    c, w = tiny
    ids = tiny_prompt()
    want, want_logits, s = oracle_greedy(O.Oracle(w), ids, 32)
    m = E.Model(w)
    for chunk in (1, 5, 16):
        run = m.new_run(64, chunk=chunk)
        logits = run.prefill(ids)
        parity(logits, want_logits[0], where=f"prefill chunk {chunk}")
        got, _ = run.decode_greedy(O.select_greedy(logits), 32)
        assert got == want, chunk
    # logits of every decode step (step, not step_greedy)
    run = m.new_run(64)
    run.prefill(ids)
    for i in range(31):
        parity(run.step(want[i]), want_logits[i + 1], where=f"decode {i}")
    for layer in range(c.num_layers):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"state {layer}/{which}")


def test_tiny_teacher_forced_walk(tiny):
    """Config 1 fed 48 random ids after its prompt (its greedy continuation is
    a fixed point for every prompt, so greedy ids alone discriminate little):
    every step's logits within the fp32 bound of the oracle's and the same
    pick (near-tie rule: none of the walk's steps is within twice the bound)."""
    c, w = tiny
    ids = tiny_prompt()
    walk = [int(v) for v in np.random.default_rng(101).integers(0, c.vocab_size, 48)]
    s = O.Oracle(w).new_state()
    for t in ids:
        s.step(t, O.VECTOR)
    run = E.Model(w).new_run(96, chunk=16)
    run.prefill(ids)
    for i, t in enumerate(walk):
        want = s.step(t, O.VECTOR)
        got = run.step(t)
        parity(got, want, where=f"walk step {i}")
        top = np.sort(want)[-2:]
        if top[1] - top[0] > 2e-4 * (abs(top[1]) + float(np.sqrt(np.mean(want * want)))):
            assert O.select_greedy(got) == O.select_greedy(want), i


def test_tiny_fused_and_unfused_paths_agree(tiny):
    """Every optional symbol switched off gives the same results (the
    reference's fallbacks, src/device.rs:368-441)."""
    c, w = tiny
    ids = tiny_prompt()
    base_model = E.Model(w)
    want = base_model.new_run(32).prefill(ids)
    for disable in (E.NO_F32_FUSIONS, E.NO_DELTA_MIXER, E.NO_FUSED_OPS, E.NO_ARGMAX, E.NO_EMBED_ROWS, 255):
        run = E.Model(w, disable=disable).new_run(32)
        parity(run.prefill(ids), want, where=f"disable {disable}")
        base = base_model.new_run(32)
        base.prefill(ids)
        got = [run.step_greedy(7)]
        ref = [base.step_greedy(7)]
        for _ in range(3):
            got.append(run.step_greedy(got[-1]))
            ref.append(base.step_greedy(ref[-1]))
        assert got == ref, disable


def verify_rows_equal_steps(c, m, prompt, draft, cap, chunk):
    """verify_rollback(draft) then accept(k), for k = 1..len(draft), leaves the
    run bit for bit where k sequential decode steps leave it, and every verify
    row's logits equal the decode step of its position bit for bit
    (reference src/device.rs:1514-1531, 1626-1662; native/rocm/bridge.cpp:197-215:
    the contract that makes speculative output equal greedy output);
    verify_rollback_greedy picks what step_greedy picks."""
    n = len(draft)
    b = m.new_run(cap, chunk=chunk)
    b.prefill(prompt)
    steps = [b.step(t) for t in draft]
    for k in range(1, n + 1):
        a = m.new_run(cap, chunk=chunk, snapshots=n - 1)
        a.prefill(prompt)
        rows = a.verify_rollback(draft)
        for r in range(n):
            assert np.array_equal(rows[r], steps[r]), f"verify row {r} differs from the decode step"
        a.accept(k)
        ref = m.new_run(cap, chunk=chunk)
        ref.prefill(prompt)
        for t in draft[:k]:
            ref.step(t)
        assert a.position == ref.position == len(prompt) + k
        for layer in range(c.num_layers):
            for which in range(4):
                assert np.array_equal(a.state(layer, which), ref.state(layer, which)), (k, layer, which)
        assert np.array_equal(a.step(9), ref.step(9)), f"the step after accept({k})"
    g = m.new_run(cap, chunk=chunk, snapshots=n - 1)
    g.prefill(prompt)
    picks = g.verify_rollback_greedy(draft)
    s = m.new_run(cap, chunk=chunk)
    s.prefill(prompt)
    assert picks == [s.step_greedy(t) for t in draft]


def test_tiny_verify_rollback(tiny):
    """The tiny model (op sequence: the bridge declines the one-launch plan for
    this geometry)."""
    c, w = tiny
    m = E.Model(w)
    assert not m.new_run(64).decode_plan
    verify_rows_equal_steps(c, m, tiny_prompt(), [5, 17, 300, 42], 64, 16)


def test_tiny_int8_against_dequantised_oracle(tiny):
    """BASELINE config 5 on the tiny model: int8 per-row weights against the
    CPU path on the dequantised weights at 1e-2; the 4-row verify too."""
    c, w = tiny
    ids = tiny_prompt()
    run = E.Model(w, fmt=E.INT8).new_run(64, snapshots=3)
    st = dequantised(c, w).new_state()
    for t in ids:
        want = st.step(t, O.VECTOR)
    parity(run.prefill(ids), want, rtol=INT8_RTOL, where="int8 prefill")
    draft = [3, 77, 500, 12]
    rows = run.verify_rollback(draft)
    for r, t in enumerate(draft):
        parity(rows[r], st.step(t, O.VECTOR), rtol=INT8_RTOL, where=f"int8 verify row {r}")


@pytest.mark.parametrize("chunk", [300, 130])
def test_mid_prefill_against_oracle(chunk):
    """Prefill chunks long enough for every prefill kernel: the chunked
    DeltaRule (dk = dv = 128, one key head feeding two value heads, ragged
    last chunk), the token-parallel conv, the MFMA and few-row GEMMs, prefill
    attention and the one-call embedding. 300 prompt tokens in one chunk, or
    as 130 + 130 + 40; logits of the last row, every state, then greedy
    decode, against the token-by-token oracle."""
    c = M.make_config(hidden=256, intermediate=512, vocab=1024,
                      layer_types=["linear_attention"] * 3 + ["full_attention"], heads=2, kv_heads=1, head_dim=64,
                      rotary_dim=16, key_heads=1, value_heads=2, key_dim=128, value_dim=128, conv_kernel=4,
                      max_positions=1024, eps=1e-6, theta=1e6)
    w = M.synthetic_weights(c, seed=5)
    prompt = [int(v) for v in np.random.default_rng(11).integers(0, c.vocab_size, 300)]
    print(f"oracle on the mid config, chunk {chunk}", flush=True)
    want, want_logits, s = oracle_greedy(O.Oracle(w), prompt, 8)
    run = E.Model(w).new_run(320, chunk=chunk)
    logits = run.prefill(prompt)
    parity(logits, want_logits[0], where="prefill logits")
    got, _ = run.decode_greedy(O.select_greedy(logits), 8)
    assert got == want
    for layer in range(c.num_layers):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"state {layer}/{which}")


@pytest.fixture(scope="module")
def qwen08b():
    print("synthesising 0.8B weights", flush=True)
    c = M.config_qwen08b(max_positions=16384)
    return c, M.synthetic_weights(c, seed=0)


@pytest.fixture(scope="module")
def qwen08b_models(qwen08b):
    """The 0.8B model twice on the device: with the bridge's one-launch decode
    step, and on the op sequence (the step's fallback and its reference)."""
    c, w = qwen08b
    print("loading 0.8B twice (one-launch decode / op sequence)", flush=True)
    return E.Model(w), E.Model(w, disable=E.NO_DECODE_STEP)


def test_qwen08b_short_greedy(qwen08b):
    """The 0.8B-shaped model (BASELINE config 2 shape) on a short prompt:
    identical greedy IDs and logits within the fp32 bound."""
    c, w = qwen08b
    prompt = [int(v) for v in np.random.default_rng(3).integers(0, c.vocab_size, 12)]
    print("oracle on 0.8B", flush=True)
    want, want_logits, s = oracle_greedy(O.Oracle(w), prompt, 6)
    print("gpu on 0.8B", flush=True)
    m = E.Model(w)
    print(m.info, flush=True)
    run = m.new_run(64, chunk=8)
    assert run.decode_plan, "0.8B fp32 steps should take the one-launch decode"
    logits = run.prefill(prompt)
    parity(logits, want_logits[0], where="0.8B prefill logits")
    got, _ = run.decode_greedy(O.select_greedy(logits), 6)
    assert got == want
    for layer in (0, 3):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"0.8B state {layer}/{which}")


@pytest.mark.parametrize("fmt", [E.F32, E.BF16_EXACT])
def test_qwen08b_capture_on_the_one_launch_step(qwen08b, qwen08b_models, fmt):
    """A captured step keeps the one-launch kernel (qr_decode_step_capture):
    every per-layer record of the 0.8B shape (input norm, mixer output,
    residual, post norm, FFN product, FFN output, layer output) and the final
    norm against the oracle's trace of the same step and against the op
    sequence's capture, within the fp32 bound, in the op sequence's order; the
    logits equal the uncaptured step's bit for bit (the records are extra
    stores of the same kernel)."""
    c, w0 = qwen08b
    w = w0 if fmt == E.F32 else bf16_weights(c, w0)
    fast = qwen08b_models[0] if fmt == E.F32 else E.Model(w, fmt=fmt)
    ops = E.Model(w, fmt=fmt, disable=E.NO_DECODE_STEP)
    prompt = [int(v) for v in np.random.default_rng(21).integers(0, c.vocab_size, 5)]
    s = O.Oracle(w).new_state()
    for t in prompt:
        s.step(t, O.VECTOR)
    run, ref, plain = (m.new_run(32, chunk=8) for m in (fast, ops, fast))
    assert run.decode_plan
    for r in (run, ref, plain):
        r.prefill(prompt)
    for i, tok in enumerate((7, 123456)):
        print(f"captured one-launch step {i}, format {fmt}", flush=True)
        fast.profile(True)
        logits, rec = run.step(tok, capture=True)
        stats = fast.profile_read()
        fast.profile(False)
        assert "decode_step_capture" in stats, stats
        want, orec = s.step(tok, O.VECTOR, trace=True)
        _, rrec = ref.step(tok, capture=True)
        assert [(l, n) for (l, n, _) in rec] == [(l, n) for (l, n, _) in rrec]
        omap = {(l, n): v for (l, n, v) in orec}
        names = dict(NAMES, normalized="final_norm", logits="logits")
        for (layer, name, v), (_, _, rv) in zip(rec, rrec):
            parity(v, omap[(layer, names[name])], where=f"step {i} {layer}.{name} vs oracle")
            parity(v, rv, where=f"step {i} {layer}.{name} vs op sequence")
        assert np.array_equal(logits, plain.step(tok))
        parity(logits, want, where=f"step {i} logits")
    ops.close()
    if fmt != E.F32:
        fast.close()


def test_qwen08b_bf16_one_launch(qwen08b):
    """The 0.8B-shaped model with BF16-exact weights (every matrix, the
    embedding and the tied LM head uploaded as BF16, the reference's deployed
    format) on the one-launch decode: identical greedy IDs and every step's
    logits within the fp32 bound against the oracle on the same weights, the
    op sequence's BF16 kernels within the bound, and verify rows (one
    multi-row launch) equal to decode steps bit for bit."""
    c, w0 = qwen08b
    w = bf16_weights(c, w0)
    prompt = [int(v) for v in np.random.default_rng(3).integers(0, c.vocab_size, 12)]
    print("oracle on the BF16-exact 0.8B", flush=True)
    want, want_logits, s = oracle_greedy(O.Oracle(w), prompt, 6)
    m = E.Model(w, fmt=E.BF16_EXACT)
    nb, nm, _ = m.weight_summary()
    assert nb == nm, "every matrix uploads as BF16"
    run = m.new_run(64, chunk=8)
    assert run.decode_plan, "all-BF16 steps should take the one-launch decode"
    logits = run.prefill(prompt)
    parity(logits, want_logits[0], where="BF16 0.8B prefill logits")
    tok = O.select_greedy(logits)
    ops = E.Model(w, fmt=E.BF16_EXACT, disable=E.NO_DECODE_STEP)
    ref = ops.new_run(64, chunk=8)
    ref.prefill(prompt)
    for i in range(5):
        print(f"BF16 one-launch step {i}", flush=True)
        got = run.step(tok)
        parity(got, want_logits[i + 1], where=f"BF16 0.8B step {i}")
        parity(got, ref.step(tok), where=f"BF16 0.8B step {i} against the op sequence")
        assert O.select_greedy(got) == want[i + 1]
        tok = want[i + 1]
    for layer in (0, 3):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"BF16 0.8B state {layer}/{which}")
    ops.close()
    draft = [int(v) for v in np.random.default_rng(13).integers(0, c.vocab_size, 4)]
    print("BF16 verify rows vs decode steps", flush=True)
    verify_rows_equal_steps(c, m, prompt, draft, 64, 8)
    m.close()


def test_qwen08b_bf16_prepared_prefill(qwen08b):
    """BF16-exact 0.8B prefill of a 96-token prompt as one chunk: every block
    projection over its prepared BF16 plane (qr_gemm_bf16_prepare: three part
    products on the plane kernels, the fused GLU, the BF16 a / b on the MFMA
    a / b kernel), the chunked DeltaRule with a ragged second chunk and
    prefill attention, against the oracle on the same weights fed token by
    token: the last row's logits and every state part of a DeltaNet and an
    attention layer within the fp32 bound, the greedy pick equal; the op
    sequence without prepared planes within the bound of it."""
    c, w0 = qwen08b
    w = bf16_weights(c, w0)
    prompt = [int(v) for v in np.random.default_rng(23).integers(0, c.vocab_size, 96)]
    print("oracle on the BF16-exact 0.8B, 96 tokens", flush=True)
    want, want_logits, s = oracle_greedy(O.Oracle(w), prompt, 1)
    m = E.Model(w, fmt=E.BF16_EXACT)
    run = m.new_run(128, chunk=96)
    logits = run.prefill(prompt)
    parity(logits, want_logits[0], where="BF16 0.8B prepared prefill logits")
    assert O.select_greedy(logits) == want[0]
    for layer in (0, 3):
        for which in range(4):
            parity(run.state(layer, which), s.part(layer, which), where=f"BF16 prepared prefill state {layer}/{which}")
    m.close()
    plain = E.Model(w, fmt=E.BF16_EXACT, disable=E.NO_PREPARED_GEMM)
    r2 = plain.new_run(128, chunk=96)
    parity(r2.prefill(prompt), logits, where="BF16 prefill without planes")
    plain.close()


@pytest.mark.parametrize("vocab", [1000, 3001])
@pytest.mark.parametrize("fmt", [E.F32, E.BF16_EXACT, E.INT8])
def test_one_launch_small_vocabulary(vocab, fmt):
    """The one-launch decode on the 0.8B geometry with 4 layers and a small
    vocabulary: 1000 rows all go to the lm_head chunk pool (no block range),
    3001 leave 2048 rows in the block ranges and a ragged last chunk. Every
    step's logits against the oracle (fp32 bound, also for BF16 matrices on
    BF16-exact weights; int8 against the oracle on the dequantised weights),
    identical greedy IDs."""
    c = M.make_config(hidden=1024, intermediate=3584, vocab=vocab,
                      layer_types=["linear_attention"] * 3 + ["full_attention"], heads=8, kv_heads=2, head_dim=256,
                      rotary_dim=64, key_heads=16, value_heads=16, key_dim=128, value_dim=128, conv_kernel=4,
                      max_positions=256, eps=1e-6, theta=1e7)
    w = M.synthetic_weights(c, seed=3)
    if fmt == E.BF16_EXACT:
        w = bf16_weights(c, w)
    prompt = [int(v) for v in np.random.default_rng(9).integers(0, vocab, 6)]
    m = E.Model(w, fmt=fmt)
    if fmt == E.BF16_EXACT:
        assert m.weight_summary()[0] == m.weight_summary()[1], "every matrix uploads as BF16"
    run = m.new_run(32, chunk=8)
    assert run.decode_plan
    st = (dequantised(c, w) if fmt == E.INT8 else O.Oracle(w)).new_state()
    for t in prompt:
        want = st.step(t, O.VECTOR)
    rtol = {"rtol": INT8_RTOL} if fmt == E.INT8 else {}
    parity(run.prefill(prompt), want, where=f"vocab {vocab} prefill", **rtol)
    tok = O.select_greedy(want)
    for i in range(5):
        print(f"vocab {vocab} fmt {fmt} one-launch step {i}", flush=True)
        got = run.step(tok)
        want = st.step(tok, O.VECTOR)
        parity(got, want, where=f"vocab {vocab} step {i}", **rtol)
        if fmt != E.INT8:
            assert O.select_greedy(got) == O.select_greedy(want)
        tok = O.select_greedy(want)


def test_qwen08b_decode_step_logits_against_oracle(qwen08b, qwen08b_models):
    """Each one-launch step's full logits against the oracle (fp32 bound)."""
    c, w = qwen08b
    fast, _ = qwen08b_models
    prompt = [int(v) for v in np.random.default_rng(5).integers(0, c.vocab_size, 5)]
    s = O.Oracle(w).new_state()
    run = fast.new_run(32, chunk=8)
    assert run.decode_plan
    for i, t in enumerate(prompt):
        print(f"one-launch step {i}", flush=True)
        got = run.step(t)
        parity(got, s.step(t, O.VECTOR), where=f"one-launch step {i}")


def _random_states(c, run, position, seed):
    """Seeded conv / recurrent states and K/V rows 0..position-1 on `run`."""
    rng = np.random.default_rng(seed)
    run.set_position(position)
    parts = []
    for layer in range(c.num_layers):
        for which in range(4):
            n = run.state(layer, which).size
            if n:
                scale = 0.05 if which == 1 else 1.0
                parts.append((layer, which, (rng.standard_normal(n) * scale).astype(np.float32)))
    return parts


@pytest.mark.parametrize("position", [0, 1, 453, 8190, 8191, 8192, 10239])
def test_qwen08b_one_launch_matches_op_sequence(qwen08b, qwen08b_models, position):
    """The one-launch step against the op sequence on the same seeded state,
    three tokens from `position`: logits within the fp32 bound, identical
    greedy picks, and every state part after the steps. The positions cross
    the attention span changes (8 positions per split up to 8192, longer
    spans after)."""
    c, w = qwen08b
    fast, ops = qwen08b_models
    cap = position + 8
    a, b = fast.new_run(cap, chunk=8), ops.new_run(cap, chunk=8)
    assert a.decode_plan and not b.decode_plan
    parts = _random_states(c, a, position, seed=position)
    b.set_position(position)
    for (layer, which, v) in parts:
        a.write_state(layer, which, v)
        b.write_state(layer, which, v)
    tokens = [int(v) for v in np.random.default_rng(position + 1).integers(0, c.vocab_size, 3)]
    for i, t in enumerate(tokens):
        print(f"position {position + i}: one-launch vs op sequence", flush=True)
        got, want = a.step(t), b.step(t)
        parity(got, want, where=f"logits at {position + i}")
        assert O.select_greedy(got) == O.select_greedy(want)
    for layer in range(c.num_layers):
        for which in range(4):
            parity(a.state(layer, which), b.state(layer, which), where=f"state {layer}/{which} at {position}")


def test_qwen08b_one_launch_greedy_matches_op_sequence(qwen08b_models):
    """BASELINE config 2's decode shape (a 454-token prompt) for 24 greedy
    tokens: the one-launch path and the op sequence pick identical IDs."""
    fast, ops = qwen08b_models
    prompt = [int(v) for v in np.random.default_rng(4).integers(0, 248320, 454)]
    got = []
    for m in (fast, ops):
        print(f"prefill 454 + 24 greedy, plan={m is fast}", flush=True)
        run = m.new_run(512, chunk=512)
        logits = run.prefill(prompt)
        ids, _ = run.decode_greedy(O.select_greedy(logits), 24)
        got.append(ids)
    assert got[0] == got[1]


def _bf16_embedding(w):
    """The weights with the embedding table rounded (truncated) to BF16, so the
    int8 upload keeps the lookup rows BF16 as the reference's does for a
    BF16 checkpoint (src/device.rs:978-1042)."""
    t = dict(w.tensors)
    t[0] = (t[0].view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32)
    return M.Weights(w.config, t)


@pytest.fixture(scope="module")
def qwen08b_int8_models(qwen08b):
    """The 0.8B model with int8 matrices (BASELINE config 5's format) and a
    BF16 embedding: one-launch decode step and op sequence."""
    c, w = qwen08b
    wb = _bf16_embedding(w)
    print("loading 0.8B int8 twice (one-launch decode / op sequence)", flush=True)
    return E.Model(wb, fmt=E.INT8), E.Model(wb, fmt=E.INT8, disable=E.NO_DECODE_STEP)


@pytest.mark.parametrize("position", [0, 453, 8191])
def test_qwen08b_int8_one_launch_matches_op_sequence(qwen08b, qwen08b_int8_models, position):
    """int8 weights: the one-launch step against the op sequence on the same
    seeded state. Both read the same int8 rows and scales and differ only in
    fp32 summation order, so the fp32 bound applies (tighter than config 5's
    1e-2); greedy picks identical."""
    c, _ = qwen08b
    fast, ops = qwen08b_int8_models
    cap = position + 8
    a, b = fast.new_run(cap, chunk=8), ops.new_run(cap, chunk=8)
    assert a.decode_plan and not b.decode_plan
    parts = _random_states(c, a, position, seed=position + 7)
    b.set_position(position)
    for (layer, which, v) in parts:
        a.write_state(layer, which, v)
        b.write_state(layer, which, v)
    tokens = [int(v) for v in np.random.default_rng(position + 2).integers(0, c.vocab_size, 3)]
    for i, t in enumerate(tokens):
        print(f"int8 position {position + i}: one-launch vs op sequence", flush=True)
        got, want = a.step(t), b.step(t)
        parity(got, want, where=f"int8 logits at {position + i}")
        assert O.select_greedy(got) == O.select_greedy(want)
    for layer in range(c.num_layers):
        for which in range(4):
            parity(a.state(layer, which), b.state(layer, which), where=f"int8 state {layer}/{which} at {position}")


def test_qwen08b_int8_one_launch_greedy_matches_op_sequence(qwen08b_int8_models):
    """Config 5's decode shape (a 454-token prompt, int8 weights) for 24
    greedy tokens: identical IDs on the one-launch path and the op sequence."""
    fast, ops = qwen08b_int8_models
    prompt = [int(v) for v in np.random.default_rng(4).integers(0, 248320, 454)]
    got = []
    for m in (fast, ops):
        print(f"int8 prefill 454 + 24 greedy, plan={m is fast}", flush=True)
        run = m.new_run(512, chunk=512)
        logits = run.prefill(prompt)
        ids, _ = run.decode_greedy(O.select_greedy(logits), 24)
        got.append(ids)
    assert got[0] == got[1]


def test_qwen08b_int8_one_launch_against_dequantised_oracle(qwen08b):
    """Config 5's bar on the one-launch path: int8 steps (fp32 embedding rows)
    against the CPU path on the dequantised weights at 1e-2."""
    c, w = qwen08b
    run = E.Model(w, fmt=E.INT8).new_run(16, chunk=8)
    assert run.decode_plan
    st = dequantised(c, w).new_state()
    for i, t in enumerate([int(v) for v in np.random.default_rng(6).integers(0, c.vocab_size, 4)]):
        print(f"int8 one-launch step {i} against the dequantised oracle", flush=True)
        parity(run.step(t), st.step(t, O.VECTOR), rtol=INT8_RTOL, where=f"int8 one-launch step {i}")


def test_qwen08b_chained_greedy_equals_stepwise(qwen08b_models):
    """decode_greedy queues its one-launch steps back to back, each kernel
    reading the previous step's argmax on the device (qr_decode_steps): the
    same IDs and bitwise the same states as one step_greedy call per token."""
    fast, _ = qwen08b_models
    prompt = [int(v) for v in np.random.default_rng(8).integers(0, 248320, 40)]
    runs = [fast.new_run(96, chunk=64) for _ in range(2)]
    first = [O.select_greedy(r.prefill(prompt)) for r in runs]
    assert first[0] == first[1]
    chained, _ = runs[0].decode_greedy(first[0], 17)
    stepped = [first[1]]
    for _ in range(16):
        stepped.append(runs[1].step_greedy(stepped[-1]))
    assert chained == stepped
    assert runs[0].position == runs[1].position == 40 + 16
    for layer in (0, 3, 23):
        for which in range(4):
            assert np.array_equal(runs[0].state(layer, which), runs[1].state(layer, which)), (layer, which)


def test_qwen08b_cooperative_launch_equals_plain(qwen08b, qwen08b_models):
    """The one-launch step as a cooperative launch (qr_set_option
    "decode_cooperative") and as the default plain launch: the same kernel on
    the same inputs, so bitwise the same logits, IDs and states."""
    c, w = qwen08b
    plain, _ = qwen08b_models
    coop = E.Model(w, disable=E.NO_PLAIN_DECODE_LAUNCH)
    prompt = [int(v) for v in np.random.default_rng(12).integers(0, c.vocab_size, 30)]
    runs = [m.new_run(64, chunk=32) for m in (plain, coop)]
    assert all(r.decode_plan for r in runs)
    first = [O.select_greedy(r.prefill(prompt)) for r in runs]
    assert first[0] == first[1]
    logits = [r.step(first[0]) for r in runs]
    assert np.array_equal(logits[0], logits[1])
    ids = [r.decode_greedy(O.select_greedy(logits[0]), 9)[0] for r in runs]
    assert ids[0] == ids[1]
    for layer in (0, 3, 23):
        for which in range(4):
            assert np.array_equal(runs[0].state(layer, which), runs[1].state(layer, which)), (layer, which)
    for r in runs:
        r.close()
    coop.close()


def test_qwen08b_residency_check_switches_to_cooperative(qwen08b, qwen08b_models):
    """The plain launch's residency check: a step whose blocks did not all
    start together (forced here from the host: qr_set_option
    "decode_residency_test" makes every start spread count) sets the plan's
    flag, and its next steps launch cooperatively, where the runtime
    guarantees residency. The switch changes no result: logits, IDs and states
    equal the plain plan's bit for bit."""
    c, w = qwen08b
    plain, _ = qwen08b_models
    test = E.Model(w, disable=E.DECODE_RESIDENCY_TEST)
    prompt = [int(v) for v in np.random.default_rng(17).integers(0, c.vocab_size, 20)]
    runs = [m.new_run(64, chunk=32) for m in (plain, test)]
    assert all(r.decode_plan for r in runs)
    first = [O.select_greedy(r.prefill(prompt)) for r in runs]
    assert first[0] == first[1]
    test.profile(True)
    logits = [r.step(first[0]) for r in runs]
    after = [r.step(7) for r in runs]
    stats = test.profile_read()
    test.profile(False)
    assert stats.get("decode_step", (0, 0))[0] == 1, stats
    assert stats.get("decode_step cooperative", (0, 0))[0] == 1, stats
    assert np.array_equal(logits[0], logits[1]) and np.array_equal(after[0], after[1])
    ids = [r.decode_greedy(O.select_greedy(after[0]), 6)[0] for r in runs]
    assert ids[0] == ids[1]
    for layer in (0, 3, 23):
        for which in range(4):
            assert np.array_equal(runs[0].state(layer, which), runs[1].state(layer, which)), (layer, which)
    for r in runs:
        r.close()
    test.close()


@pytest.mark.parametrize("fmt", [E.F32, E.INT8])
def test_qwen08b_verify_rows_equal_decode_steps(qwen08b, qwen08b_models, fmt):
    """Verify rows on the one-launch path: each row is a launch of the decode
    step at its position (snapshots written by the kernel), so rows, picks
    and the accepted state equal sequential decode bit for bit; for a random
    draft and for the model's own greedy continuation (fully accepted)."""
    c, w = qwen08b
    m = qwen08b_models[0] if fmt == E.F32 else E.Model(w, fmt=E.INT8)
    prompt = [int(v) for v in np.random.default_rng(12).integers(0, c.vocab_size, 200)]
    r = m.new_run(256, chunk=256, snapshots=3)
    assert r.decode_plan
    first = O.select_greedy(r.prefill(prompt))
    own, _ = r.decode_greedy(first, 4)
    for draft in ([int(v) for v in np.random.default_rng(13).integers(0, c.vocab_size, 4)], own):
        print(f"verify rows vs decode steps, format {fmt}, draft {draft}", flush=True)
        verify_rows_equal_steps(c, m, prompt, draft, 256, 256)
    if fmt != E.F32:
        m.close()


@pytest.mark.parametrize("fmt", [E.F32, E.INT8])
@pytest.mark.parametrize("prompt_len,n", [(200, 2), (200, 3), (200, 6), (2046, 4), (2046, 6)])
def test_qwen08b_verify_rows_multi(qwen08b, qwen08b_models, fmt, prompt_len, n):
    """Verify passes through qr_decode_rows (up to four rows per launch, the
    weights read once: 2 and 3 rows, 6 = a 4-row and a 2-row launch), rows
    straddling position 2048 (where a one-row step's attention splits grow
    from 8 to 16 positions, so consecutive rows are split differently): every
    row, accepted state and pick equals sequential decode steps bit for bit,
    and the rows equal the per-row launches (QE_NO_DECODE_ROWS)."""
    c, w = qwen08b
    m = qwen08b_models[0] if fmt == E.F32 else E.Model(w, fmt=E.INT8)
    prompt = [int(v) for v in np.random.default_rng(prompt_len + n).integers(0, c.vocab_size, prompt_len)]
    draft = [int(v) for v in np.random.default_rng(n).integers(0, c.vocab_size, n)]
    cap, chunk = prompt_len + 16, 256
    print(f"multi-row verify: format {fmt}, prompt {prompt_len}, {n} rows", flush=True)
    verify_rows_equal_steps(c, m, prompt, draft, cap, chunk)
    per_row = E.Model(w, fmt=fmt, disable=E.NO_DECODE_ROWS)
    a, b = m.new_run(cap, chunk=chunk, snapshots=n - 1), per_row.new_run(cap, chunk=chunk, snapshots=n - 1)
    assert a.decode_plan and b.decode_plan
    a.prefill(prompt)
    b.prefill(prompt)
    for ra, rb in zip(a.verify_rollback(draft), b.verify_rollback(draft)):
        assert np.array_equal(ra, rb)
    per_row.close()
    if fmt != E.F32:
        m.close()


@pytest.mark.parametrize("depth", [1, 2, 3])
def test_qwen08b_speculative_equals_greedy(qwen08b, qwen08b_models, depth):
    """generate (reference src/device/speculative.rs:53-160) on the 0.8B model
    with the one-launch decode: the output equals plain greedy decoding for
    drafts that are all right, partly wrong, and the prompt-lookup draft."""
    from test_engine_cpu import Replay
    c, _ = qwen08b
    fast, _ = qwen08b_models
    prompt = [int(v) for v in np.random.default_rng(14).integers(0, c.vocab_size, 100)]
    plain = fast.new_run(160, chunk=128)
    want, _ = plain.decode_greedy(O.select_greedy(plain.prefill(prompt)), 40)
    for draft in (Replay(len(prompt), want, vocab=c.vocab_size),
                  Replay(len(prompt), want, wrong=range(2, 40, 5), vocab=c.vocab_size), "ngram"):
        run = fast.new_run(160, chunk=128, snapshots=depth)
        assert run.decode_plan
        got, st = run.speculative_generate(prompt, 40, depth, draft=draft)
        print(f"depth {depth}, draft {getattr(draft, 'wrong', draft)!s:.20}: {st}", flush=True)
        assert got == want
        if isinstance(draft, Replay) and not draft.wrong:
            assert st["accepted"] == st["offered"]


def test_qwen08b_state_interchange_with_oracle(qwen08b, qwen08b_models):
    """CPU <-> GPU state interchange (the reference's inspect_state /
    load_state, src/device.rs:2380-2516): the oracle's state after a prompt,
    loaded into a one-launch run, continues with the oracle's greedy tokens
    and logits; a GPU run's state loaded into the oracle continues with the
    GPU's logits."""
    c, w = qwen08b
    fast, _ = qwen08b_models
    o = O.Oracle(w)
    prompt = [int(v) for v in np.random.default_rng(15).integers(0, c.vocab_size, 20)]
    want, want_logits, s = oracle_greedy(o, prompt, 5)
    cpu_state = o.new_state()
    for t in prompt:
        cpu_state.step(t, O.VECTOR)
    run = fast.new_run(64, chunk=32)
    assert run.decode_plan
    run.load_state(len(prompt), cpu_state.part)
    assert run.position == len(prompt)
    for i in range(4):
        parity(run.step(want[i]), want_logits[i + 1], where=f"after load_state, step {i}")
    for layer, which in [(0, 0), (0, 1), (3, 2), (3, 3), (23, 2)]:
        parity(run.state(layer, which), s.part(layer, which), where=f"state {layer}/{which}")
    g = fast.new_run(64, chunk=32)
    g.load_state(len(prompt), cpu_state.part)
    got, _ = g.decode_greedy(want[0], 5)
    assert got == want
    # GPU -> CPU
    gpu = fast.new_run(64, chunk=32)
    gpu.prefill(prompt + want[:4])
    back = o.new_state()
    back.load(gpu.position, lambda layer, which: gpu.state(layer, which))
    for t in [11, 22222]:
        parity(gpu.step(t), back.step(t, O.VECTOR), where="after loading the GPU state into the oracle")


def test_qwen08b_checkpoint_restore_across_verify(qwen08b, qwen08b_models):
    """checkpoint / restore (reference src/device.rs:2425-2490) around a
    verify_rollback + accept on the one-launch path: restoring the earlier
    checkpoint brings back its DeltaNet states bit for bit and the same
    continuation; a checkpoint after accept restores the accepted state."""
    c, _ = qwen08b
    fast, _ = qwen08b_models
    prompt = [int(v) for v in np.random.default_rng(16).integers(0, c.vocab_size, 40)]
    run = fast.new_run(96, chunk=64, snapshots=3)
    run.prefill(prompt)
    before = run.inspect_state()
    cp = run.checkpoint()
    run.verify_rollback([7, 8, 9, 10])
    run.accept(2)
    after = run.inspect_state()
    cp2 = run.checkpoint()
    a = run.step(123)
    run.restore(cp)
    assert run.position == 40
    now = run.inspect_state()
    for key, v in before.items():
        assert np.array_equal(now[key], v), key
    ref = fast.new_run(96, chunk=64)
    ref.prefill(prompt)
    assert np.array_equal(run.step(7), ref.step(7))
    # the accepted rows again (the same K/V rows at 40, 41), then back to cp2
    run.step(8)
    run.restore(cp2)
    assert run.position == 42
    now = run.inspect_state()
    for key, v in after.items():
        assert np.array_equal(now[key], v), key
    assert np.array_equal(run.step(123), a)


def test_edit_overlay_against_oracle(fixture):
    """The edit overlay (reference src/device.rs:2198-2250) on the HIP bridge:
    the fixture model with the reference test's manifest against the oracle's
    edited run (intervened product, FFN output, logits), in decode and chunked
    prefill; removing it restores the plain run."""
    from test_engine_cpu import fixture_edits
    c, w = M.fixture_config_and_weights(fixture)
    ids = fixture["ids"]
    edits = fixture_edits(c.hidden_size)
    o = O.Oracle(w)
    o.set_edit(edits)
    s = o.new_state()
    m = E.Model(w)
    run = m.new_run(len(ids))
    run.set_edit(edits)
    want = None
    for tok in ids:
        logits, rec = run.step(tok, capture=True)
        want, orec = s.step(tok, O.REFERENCE, trace=True)
        omap = {(l, n): v for (l, n, v) in orec}
        got = {(l, n): v for (l, n, v) in rec}
        for layer in (1, 2):
            parity(got[(layer, "ffn_intervened_product")], omap[(layer, "ffn.intervened_product")], where="product")
            parity(got[(layer, "ffn")], omap[(layer, "ffn.output")], where="ffn")
        parity(logits, want, where="edited logits")
    run = m.new_run(len(ids), chunk=3)
    run.set_edit(edits)
    parity(run.prefill(ids), want, where="edited prefill")
    run.reset()
    run.set_edit([])
    plain = O.Oracle(w).new_state()
    for tok in ids:
        last = plain.step(tok, O.REFERENCE)
    parity(run.prefill(ids), last, where="edit removed")


def test_qwen08b_edit_takes_the_op_sequence(qwen08b, qwen08b_models):
    """With an edit the 0.8B run leaves the one-launch decode (the overlay
    needs the product on the host) and matches the oracle's edited run."""
    c, w = qwen08b
    fast, _ = qwen08b_models
    d = np.zeros(c.hidden_size, np.float32)
    d[:8] = 1.0
    edits = [dict(layer=4, columns=[7, 1000], direction=None, coefficient=1.0),
             dict(layer=21, columns=[3, 3000], direction=d, coefficient=0.5)]
    o = O.Oracle(w)
    o.set_edit(edits)
    s = o.new_state()
    run = fast.new_run(16, chunk=8)
    run.set_edit(edits)
    for i, t in enumerate([5, 77, 12345, 200000]):
        parity(run.step(t), s.step(t, O.VECTOR), where=f"0.8B edited step {i}")
    # greedy decoding with the edit stays on the op sequence too
    want = [O.select_greedy(s.step(9, O.VECTOR))]
    for _ in range(2):
        want.append(O.select_greedy(s.step(want[-1], O.VECTOR)))
    got, _ = run.decode_greedy(9, 4)
    assert got[1:] == want
    run.set_edit([])
    s2 = O.Oracle(w).new_state()
    r2 = fast.new_run(16, chunk=8)
    for t in [5, 77]:
        parity(r2.step(t), s2.step(t, O.VECTOR), where="0.8B after removal")


def test_qwen08b_chained_greedy_bounds(qwen08b_models):
    """Chained greedy decoding refuses to run past the run's capacity or from an
    out-of-range token (checked on the host, before any launch), and leaves the
    run usable."""
    fast, _ = qwen08b_models
    run = fast.new_run(12, chunk=8)
    run.prefill([1, 2, 3, 4])
    with pytest.raises(E.EngineError):
        run.decode_greedy(5, 10)  # 9 steps from position 4 > capacity 12
    with pytest.raises(E.EngineError):
        run.decode_greedy(248320, 3)  # token id == vocab
    assert run.position == 4
    ids, _ = run.decode_greedy(5, 4)
    assert len(ids) == 4 and run.position == 7
