"""The host engine (the restatement of the reference's DeviceModel/DeviceRun)
on CPU bridges: the oracle's op bridge and, when it was built, the
reference's own CPU test bridge (oracle/_ref). Both compute every op with the
reference's scalar bodies in the Reference summation order, so the engine's
call sequence must reproduce the oracle's Backend::Reference results bit for
bit."""
import numpy as np
import pytest

from conftest import GOLDEN, ROOT
from parity import INT8_RTOL, parity
from qwen_mi355x import engine as E
from qwen_mi355x import model as M

import oracle as O

OPS_BRIDGE = ROOT / "oracle" / "lib" / "libqwen_ops_bridge.so"
REF_BRIDGE = ROOT / "oracle" / "_ref" / "libqwen_rocm_test.so"
BRIDGES = [pytest.param(OPS_BRIDGE, id="ops_bridge"),
           pytest.param(REF_BRIDGE, id="reference_cpu_bridge",
                        marks=pytest.mark.skipif(not REF_BRIDGE.exists(), reason="reference tree not built here"))]


@pytest.fixture(scope="module")
def fixture():
    return M.load_fixture(GOLDEN / "hybrid.json")


@pytest.fixture(scope="module")
def tiny():
    c = M.config_tiny()
    return c, M.synthetic_weights(c, seed=0)


def tiny_prompt():
    return [int(v) for v in np.random.default_rng(1).integers(0, 512, 16)]


@pytest.mark.parametrize("bridge", BRIDGES)
@pytest.mark.parametrize("fmt", [E.F32, E.BF16_EXACT])
def test_fixture_records_bitwise(fixture, bridge, fmt):
    c, w = M.fixture_config_and_weights(fixture)
    m = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST, fmt=fmt)
    assert m.weight_summary()[0] == (32 if fmt == E.BF16_EXACT else 0)
    run = m.new_run(len(fixture["ids"]))
    s = O.Oracle(w).new_state()
    for tok in fixture["ids"]:
        logits, rec = run.step(tok, capture=True)
        want, orec = s.step(tok, O.REFERENCE, trace=True)
        assert np.array_equal(logits, want)
        omap = {(l, n): v for (l, n, v) in orec}
        names = {"input_norm": "input_norm", "mixed": "mixer", "after_mixer": "after_mixer", "post_norm": "post_norm",
                 "ffn_product": "ffn.product", "ffn": "ffn.output", "output": "layer"}
        seen = 0
        for (layer, name, v) in rec:
            if name in names:
                assert np.array_equal(v, omap[(layer, names[name])]), (layer, name)
                seen += 1
        assert seen == 7 * c.num_layers
    for layer in range(c.num_layers):
        for which in range(4):
            assert np.array_equal(run.state(layer, which), s.part(layer, which))


@pytest.mark.parametrize("bridge", BRIDGES)
def test_tiny_greedy_prefill_chunks_and_decode(tiny, bridge):
    """Config 1: prompt of 16 IDs, greedy 32 tokens, bit-exact against the
    oracle; every prefill chunk size gives the same logits and state."""
    c, w = tiny
    ids = tiny_prompt()
    o = O.Oracle(w)
    s = o.new_state()
    for t in ids:
        last = s.step(t, O.REFERENCE)
    want_ids = [O.select_greedy(last)]
    for _ in range(31):
        want_ids.append(O.select_greedy(s.step(want_ids[-1], O.REFERENCE)))
    m = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST)
    for chunk in (1, 7, 16):
        run = m.new_run(64, chunk=chunk)
        logits = run.prefill(ids)
        assert np.array_equal(logits, o_last := last) or chunk > 1
        got, _ = run.decode_greedy(O.select_greedy(logits), 32)
        assert got == want_ids, chunk
        del o_last


@pytest.mark.parametrize("bridge", BRIDGES)
def test_tiny_teacher_forced_walk_bitwise(tiny, bridge):
    """Config 1's greedy continuation is a fixed point for every prompt (the
    tied embedding makes a token's own logit the largest at N(0, 0.02):
    seeds 1-29 all repeat one token), so identical greedy ids alone
    discriminate little. Here the model is fed 48 random ids after the
    prompt instead: every step's logits bit-exact against the oracle, and
    its pick with them."""
    c, w = tiny
    ids = tiny_prompt()
    walk = [int(v) for v in np.random.default_rng(101).integers(0, c.vocab_size, 48)]
    s = O.Oracle(w).new_state()
    for t in ids:
        s.step(t, O.REFERENCE)
    run = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST).new_run(96, chunk=16)
    run.prefill(ids)
    picks = set()
    for t in walk:
        want = s.step(t, O.REFERENCE)
        got = run.step(t)
        assert np.array_equal(got, want), t
        picks.add(O.select_greedy(got))
    assert len(picks) > 24  # the walk's picks vary (each tends to repeat its input)


def config_gqa():
    """A small hybrid whose attention has 2 KV heads for 8 query heads and a
    16-wide rotary part of a 32-wide head (theta 1e6), and whose DeltaNet
    has 2 key heads feeding 4 value heads: the head-to-group mappings and the
    RoPE frequencies for i > 0 that the fixture and the tiny model (1 KV head,
    rotary 2 or 8) leave unexercised."""
    return M.make_config(hidden=64, intermediate=128, vocab=256,
                         layer_types=["linear_attention", "full_attention", "linear_attention", "full_attention"],
                         heads=8, kv_heads=2, head_dim=32, rotary_dim=16, key_heads=2, value_heads=4, key_dim=16,
                         value_dim=8, conv_kernel=4, max_positions=256, eps=1e-6, theta=1e6)


@pytest.mark.parametrize("bridge", BRIDGES)
def test_gqa_config_bitwise(bridge):
    """The engine's op sequence on the CPU bridges (ours, and the reference's
    own) equals the oracle's Backend::Reference forward bit for bit on the
    GQA config: logits of every prompt position, the greedy continuation and
    every state part."""
    c = config_gqa()
    w = M.synthetic_weights(c, seed=3, std=0.1)
    ids = [int(v) for v in np.random.default_rng(9).integers(0, c.vocab_size, 40)]
    s = O.Oracle(w).new_state()
    run = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST).new_run(64)
    for t in ids:
        assert np.array_equal(run.step(t), s.step(t, O.REFERENCE))
    want = []
    logits = None
    for i in range(8):
        logits = s.step(want[-1] if want else ids[-1], O.REFERENCE)
        want.append(O.select_greedy(logits))
    run2 = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST).new_run(64, chunk=16)
    run2.prefill(ids)
    got, _ = run2.decode_greedy(ids[-1], 9)
    assert got[1:] == want
    for layer in range(c.num_layers):
        for which in range(4):
            assert np.array_equal(run2.state(layer, which), s.part(layer, which)), (layer, which)


@pytest.mark.parametrize("bridge", BRIDGES)
def test_verify_rollback_and_accept(tiny, bridge):
    """verify_rollback + accept(k) leaves exactly the state of k sequential
    steps (reference src/device/tests.rs:1001-1041)."""
    c, w = tiny
    ids = tiny_prompt()
    m = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST)
    draft = [5, 17, 300, 42]
    for k in range(1, 5):
        a = m.new_run(64, snapshots=3)
        a.prefill(ids)
        rows = a.verify_rollback(draft)
        a.accept(k)
        b = m.new_run(64)
        b.prefill(ids)
        for r, t in enumerate(draft[:k]):
            assert np.array_equal(b.step(t), rows[r])
        assert a.position == b.position == len(ids) + k
        for layer in range(c.num_layers):
            for which in range(4):
                assert np.array_equal(a.state(layer, which), b.state(layer, which)), (k, layer, which)
        # the next step continues from the accepted prefix
        assert np.array_equal(a.step(9), b.step(9))
    g = m.new_run(64, snapshots=3)
    g.prefill(ids)
    picks = g.verify_rollback_greedy(draft)
    assert picks == [O.select_greedy(r) for r in rows]


@pytest.mark.parametrize("bridge", BRIDGES)
def test_fusion_fallbacks_agree(tiny, bridge):
    """Optional symbols absent (src/device.rs:368-441) change nothing."""
    c, w = tiny
    ids = tiny_prompt()
    ref = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST).new_run(32)
    want = ref.prefill(ids)
    for disable in (E.NO_FUSED_OPS, E.NO_ARGMAX | E.NO_DELTA_MIXER, 63):
        run = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST, disable=disable).new_run(32)
        assert np.array_equal(run.prefill(ids), want)
        assert run.step_greedy(3) == ref.step_greedy(3) if disable == 63 else True


def test_checkpoint_restore_reset_and_poison(tiny):
    c, w = tiny
    m = E.Model(w, bridge=OPS_BRIDGE, kind=E.KIND_CPU_TEST)
    run = m.new_run(20)
    ids = tiny_prompt()
    run.prefill(ids[:8])
    cp = run.checkpoint()
    a = run.prefill(ids[8:12])
    run.restore(cp)
    assert run.position == 8
    assert np.array_equal(run.prefill(ids[8:12]), a)
    run.restore(run.initial_checkpoint())
    assert run.position == 0
    first = run.prefill(ids[:8])
    fresh = m.new_run(20)
    assert np.array_equal(fresh.prefill(ids[:8]), first)
    # capacity overflow is refused before anything is enqueued; a failed forward poisons
    with pytest.raises(E.EngineError):
        run.prefill(list(range(13)))
    assert run.position == 8
    with pytest.raises(E.EngineError):
        run.step(10**6)
    run.reset()
    assert run.position == 0
    assert np.array_equal(run.prefill(ids[:8]), first)


def test_int8_quantiser_matches_oracle(tiny):
    c, w = tiny
    a = w.tensors[0]
    s1, q1 = E.quantize_int8_rows(a, c.vocab_size, c.hidden_size)
    s2, q2 = O.quantize_int8_rows(a, c.vocab_size, c.hidden_size)
    assert np.array_equal(s1, s2) and np.array_equal(q1, q2)


def dequantised(c, w):
    """The oracle on the int8 run's weights (the CPU path on
    the dequantised weights): every projection matrix as scale * q, the
    vocabulary projection as the dequantised embedding, the lookup rows exact."""
    t = dict(w.tensors)
    for spec in M.tensor_specs(c):
        if spec.kind == "matrix" and spec.index != 0:
            rows, cols = spec.shape
            s, q = O.quantize_int8_rows(t[spec.index], rows, cols)
            t[spec.index] = O.dequantize_int8_rows(s, q, rows, cols)
    o = O.Oracle(M.Weights(c, t))
    s, q = O.quantize_int8_rows(w.tensors[0], c.vocab_size, c.hidden_size)
    o.set_lm_head(O.dequantize_int8_rows(s, q, c.vocab_size, c.hidden_size))
    return o


def test_int8_against_dequantised_oracle(tiny):
    c, w = tiny
    ids = tiny_prompt()
    run = E.Model(w, bridge=OPS_BRIDGE, kind=E.KIND_CPU_TEST, fmt=E.INT8).new_run(32)
    st = dequantised(c, w).new_state()
    for t in ids:
        want = st.step(t, O.REFERENCE)
    parity(run.prefill(ids), want, rtol=INT8_RTOL, where="int8 logits")
    for t in (3, 77, 500):
        parity(run.step(t), st.step(t, O.REFERENCE), rtol=INT8_RTOL, where="int8 decode")


class Replay:
    """A draft source that proposes a known continuation (`want`: the plain
    greedy tokens after the prompt), with the tokens at `wrong` indices of
    `want` replaced, so that their verify rows reject them."""

    def __init__(self, prompt_len, want, wrong=(), vocab=512):
        self.prompt_len, self.want, self.wrong, self.vocab = prompt_len, want, set(wrong), vocab
        self.absorbed = 0

    def absorb(self, tokens):
        self.absorbed += len(tokens)

    def draft(self, k):
        known = self.absorbed - (self.prompt_len - 1)
        out = []
        for i in range(known, min(known + k, len(self.want))):
            out.append((self.want[i] + 1) % self.vocab if i in self.wrong else self.want[i])
        return out


@pytest.mark.parametrize("bridge", BRIDGES)
@pytest.mark.parametrize("depth", [1, 2, 3])
def test_speculative_equals_greedy(tiny, bridge, depth):
    """generate (reference src/device/speculative.rs:53-160): the output equals
    plain greedy decoding whatever the drafts (all right, some wrong, the
    prompt-lookup draft); a fully right draft has every offered token
    accepted; an eos token stops it (emitted, then nothing more)."""
    c, w = tiny
    ids = tiny_prompt()
    m = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST)
    plain = m.new_run(64)
    want, _ = plain.decode_greedy(O.select_greedy(plain.prefill(ids)), 24)
    for draft in (Replay(len(ids), want), Replay(len(ids), want, wrong=range(1, 24, 3)), "ngram"):
        run = m.new_run(64, chunk=16, snapshots=depth)
        got, st = run.speculative_generate(ids, 24, depth, draft=draft)
        assert got == want
        assert run.position == len(ids) + 23
        if isinstance(draft, Replay) and not draft.wrong:
            assert st["accepted"] == st["offered"] and st["passes"] <= -(-23 // (depth + 1)) + 1
    stop = want[5]
    run = m.new_run(64, chunk=16, snapshots=depth)
    got, _ = run.speculative_generate(ids, 24, depth, draft=Replay(len(ids), want), eos=[stop])
    assert got == want[:want.index(stop) + 1]
    with pytest.raises(E.EngineError):
        m.new_run(64, chunk=16, snapshots=depth - 1).speculative_generate(ids, 24, depth)


def fixture_edits(hidden):
    """The reference's device edit test manifest (src/device/tests.rs:212-243):
    unit 3 of layer 1 disabled, and the direction d = e_0 - 0.5 e_{hidden-1}
    removed from columns 0 and 5 of layer 2's down matrix with coefficient 0.7."""
    d = np.zeros(hidden, np.float32)
    d[0], d[hidden - 1] = 1.0, -0.5
    return [dict(layer=1, columns=[3], direction=None, coefficient=1.0),
            dict(layer=2, columns=[0, 5], direction=d, coefficient=0.7)]


@pytest.mark.parametrize("bridge", BRIDGES)
@pytest.mark.parametrize("fmt", [E.F32, E.BF16_EXACT])
def test_edit_overlay_matches_oracle(fixture, bridge, fmt):
    """cpu_bridge_edit_overlay_matches_cpu (reference src/device/tests.rs:208-300):
    the engine's edit overlay equals the CPU model's edited run bit for bit
    (captured intervened product, FFN output, logits) in decode, in chunked
    prefill, after reset, and removing it restores the plain run; invalid
    manifests are refused."""
    c, w = M.fixture_config_and_weights(fixture)
    ids = fixture["ids"]
    edits = fixture_edits(c.hidden_size)
    plain_o, edited_o = O.Oracle(w), O.Oracle(w)
    edited_o.set_edit(edits)
    ps, es = plain_o.new_state(), edited_o.new_state()
    plain, edited = [], []
    for tok in ids:
        plain.append(ps.step(tok, O.REFERENCE))
        edited.append(es.step(tok, O.REFERENCE, trace=True))
    assert np.max(np.abs(plain[-1] - edited[-1][0])) > 1e-3, "the edit must matter"
    m = E.Model(w, bridge=bridge, kind=E.KIND_CPU_TEST, fmt=fmt)
    run = m.new_run(len(ids))
    run.set_edit(edits)
    for p, tok in enumerate(ids):
        logits, rec = run.step(tok, capture=True)
        want, orec = edited[p]
        omap = {(l, n): v for (l, n, v) in orec}
        got = {(l, n): v for (l, n, v) in rec}
        for layer in (1, 2):
            assert np.array_equal(got[(layer, "ffn_intervened_product")], omap[(layer, "ffn.intervened_product")])
            assert np.array_equal(got[(layer, "ffn")], omap[(layer, "ffn.output")])
        assert (0, "ffn_intervened_product") not in got
        assert np.array_equal(logits, want)
    run = m.new_run(len(ids), chunk=3)
    run.set_edit(edits)
    assert np.array_equal(run.prefill(ids), edited[-1][0])
    run.reset()
    assert np.array_equal(run.prefill(ids), edited[-1][0])
    run.reset()
    run.set_edit([])
    assert np.array_equal(run.prefill(ids), plain[-1])
    bad = [dict(edits[0], tensor_name="model.language_model.layers.0.mlp.down_proj.weight")]
    with pytest.raises(E.EngineError, match="target"):
        run.set_edit(bad)
    with pytest.raises(E.EngineError, match="duplicate"):
        run.set_edit([dict(edits[0], columns=[3, 3])])
    with pytest.raises(E.EngineError, match="direction"):
        run.set_edit([dict(edits[1], direction=np.zeros(c.hidden_size, np.float32))])


def test_bf16_weights_round_like_torch(tiny):
    """model.bf16_weights (the BF16-exact model of the BF16 decode tests and
    the bench) rounds every tensor as torch's float32 -> bfloat16 conversion
    does (nearest, ties to even), including values exactly halfway."""
    import torch
    c, w = tiny
    b = M.bf16_weights(w)
    for i, t in w.tensors.items():
        want = torch.from_numpy(t).to(torch.bfloat16).to(torch.float32).numpy()
        assert np.array_equal(b.tensors[i].view(np.uint32), want.view(np.uint32)), i
    ties = np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 2.0 ** -130 * 3], dtype=np.float32)
    tw = M.Weights(c, {**w.tensors, 0: np.resize(ties, w.tensors[0].size).astype(np.float32)})
    got = M.bf16_weights(tw).tensors[0][:4]
    want = torch.from_numpy(ties).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
