"""Pins the oracle's op bridge (oracle/ops_bridge.cpp, the scalar restatement
of the reference's op bodies that every HIP kernel is checked against) op by
op against the reference's own CPU test bridge (native/rocm/bridge.cpp +
reference.h built with -DQR_CPU_TEST from the reference's sources into
oracle/_ref by oracle/Makefile), bit for bit, at the Qwen3.5-0.8B op shapes:
head_dim 256, rotary 64, theta 1e7, 8 query / 2 KV heads (so the GQA head ->
KV head mapping and the RoPE frequency exponent for i > 0 are exercised),
DeltaRule 16 x 128 x 128 with snapshots, multi-row AttentionRead, the
6144-channel conv with snapshots, and every projection kind."""
import numpy as np
import pytest

from bridges import both, rnd
from conftest import ROOT
from qwen_mi355x.bridge import Bridge, pack_bf16, pack_int8

import oracle as O

OPS = ROOT / "oracle" / "lib" / "libqwen_ops_bridge.so"
REF = ROOT / "oracle" / "_ref" / "libqwen_rocm_test.so"

pytestmark = pytest.mark.skipif(not REF.exists(), reason="reference CPU bridge not built (no reference tree here)")


@pytest.fixture(scope="module")
def ours():
    b = Bridge(OPS, kind=0)
    yield b
    b.close()


@pytest.fixture(scope="module")
def ref():
    b = Bridge(REF, kind=0)
    yield b
    b.close()


def same(a, b, where):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, where
    eq = a.view(np.uint32) == b.view(np.uint32)
    assert eq.all(), f"{where}: first difference at {np.argmin(eq)}: {a[~eq][:3]} vs {b[~eq][:3]}"


def check(ours, ref, op, count, inputs, outputs, n=(), f=()):
    g, c = both(ours, ref, op, count, inputs, outputs, n, f)
    for s in outputs:
        same(g[s], c[s], f"{op} slot {s}")


@pytest.mark.parametrize("d,groups", [(1024, 3), (256, 8), (128, 16), (8, 5)])
def test_norm_family(ours, ref, d, groups):
    rng = np.random.default_rng(d + groups)
    x, w, u, z = rnd(rng, d * groups), rnd(rng, d, 0.1), rnd(rng, d * groups), rnd(rng, d * groups)
    check(ours, ref, "RMS_NORM", groups, {1: x, 2: w}, {0: d * groups}, [d], [1e-6, 1.0])
    check(ours, ref, "ADD_RMS_NORM", groups, {1: x, 2: u, 4: w}, {0: d * groups, 3: d * groups}, [d], [1e-6, 1.0])
    check(ours, ref, "RMS_NORM_GATE", groups, {1: x, 2: w, 3: z}, {0: d * groups}, [d], [1e-6, 0.0])


def test_elementwise_gates_embed_argmax(ours, ref):
    rng = np.random.default_rng(5)
    n = 3584
    a, b = rnd(rng, n, 3), rnd(rng, n)
    check(ours, ref, "ADD", n, {1: a, 2: b}, {0: n})
    check(ours, ref, "SILU_PRODUCT", n, {1: a, 2: b}, {0: n})
    # DeltaGates: the reference's boundary values (src/device/tests.rs:368-400), then 16 heads x 5 tokens
    av = np.array([100, -100, 0, 10], np.float32)
    bv = np.array([-100, 100, 0, 1], np.float32)
    dt = np.array([0, 0, 1, -1], np.float32)
    al = np.array([-20, 0, 1, 2], np.float32)
    check(ours, ref, "DELTA_GATES", 4, {1: av, 2: bv, 3: dt, 4: al}, {0: 4, 5: 4})
    check(ours, ref, "DELTA_GATES", 80, {1: rnd(rng, 80, 4), 2: rnd(rng, 80, 4), 3: rnd(rng, 16), 4: rnd(rng, 16)},
          {0: 80, 5: 80}, [16])
    emb = rnd(rng, 300 * 1024)
    packed = pack_bf16(emb).view(np.float32)
    check(ours, ref, "EMBED_BF16", 1024, {1: packed}, {0: 1024}, [299, 1024])
    picks = np.array([3, 0, 298, 0, 17, 0], np.float32)
    check(ours, ref, "EMBED_BF16_PICKED", 3 * 1024, {1: packed, 2: picks}, {0: 3 * 1024}, [0, 1024])
    row = rnd(rng, 248320, 5)
    row[[7, 4096, 100000]] = [np.nan, np.inf, -np.inf]
    row[200000] = 40.0
    row[200001] = 40.0
    logits = np.concatenate([row, np.full(248320, np.nan, np.float32), np.roll(row, 1013)])
    check(ours, ref, "ARGMAX", 3, {1: logits}, {0: 6}, [248320])


@pytest.mark.parametrize("k,tokens,snaps", [(4, 1, 0), (4, 5, 0), (4, 4, 3), (3, 2, 1)])
def test_conv_silu(ours, ref, k, tokens, snaps):
    rng = np.random.default_rng(k * 10 + tokens)
    ch = 6144 if k == 4 else 24
    x, w, h = rnd(rng, tokens * ch), rnd(rng, ch * k, 0.5), rnd(rng, ch * (k - 1) * (1 + snaps))
    check(ours, ref, "CONV_SILU", ch, {1: x, 2: w, 3: h}, {0: tokens * ch, 3: h.size}, [k, tokens, ch, snaps])


@pytest.mark.parametrize("kh,vh,d,tokens", [(16, 16, 128, 1), (16, 16, 128, 3), (2, 4, 3, 1)])
def test_delta_qk(ours, ref, kh, vh, d, tokens):
    rng = np.random.default_rng(d + tokens)
    stride = 2 * kh * d + vh * d
    x = rnd(rng, tokens * stride)
    check(ours, ref, "DELTA_QK", vh * tokens, {1: x}, {0: vh * tokens * d, 2: vh * tokens * d}, [kh, vh, d, stride])


@pytest.mark.parametrize("tokens,snaps,gated", [(1, 0, True), (4, 3, True), (5, 0, False), (2, 1, False)])
def test_delta_rule(ours, ref, tokens, snaps, gated):
    kd = vd = 128
    heads = 16
    rng = np.random.default_rng(tokens * 3 + snaps)
    stride = 2 * heads * kd + heads * vd
    q, k = rnd(rng, tokens * heads * kd, 0.1), rnd(rng, tokens * heads * kd, 0.1)
    v = rnd(rng, tokens * stride, 2.0)
    state = rnd(rng, heads * kd * vd * (1 + snaps))
    if gated:
        ins = {1: q, 2: k, 3: v, 4: state, 5: rnd(rng, tokens * heads), 6: rnd(rng, tokens * heads),
               7: rnd(rng, 2 * heads, 0.5)}
        op = "DELTA_RULE_GATED"
    else:
        decay = (-0.1 - np.abs(rnd(rng, tokens * heads, 0.1))).astype(np.float32)
        beta = (0.5 + rnd(rng, tokens * heads, 0.2)).clip(0, 1).astype(np.float32)
        ins = {1: q, 2: k, 3: v, 4: state, 5: decay, 6: beta}
        op = "DELTA_RULE"
    check(ours, ref, op, heads * vd, ins, {0: tokens * heads * vd, 4: state.size},
          [kd, vd, heads, heads, tokens, stride, snaps])


@pytest.mark.parametrize("d,rot,heads,kv,tokens,pos,theta", [(256, 64, 8, 2, 1, 453, 1e7), (256, 64, 8, 2, 3, 8190, 1e7),
                                                              (16, 8, 4, 2, 2, 7, 1e4), (256, 64, 8, 2, 2, 0, 1e7)])
def test_attention_query_kv(ours, ref, d, rot, heads, kv, tokens, pos, theta):
    rng = np.random.default_rng(d + pos)
    cap = pos + tokens + 1
    mixed, key, value = rnd(rng, tokens * heads * 2 * d), rnd(rng, tokens * kv * d), rnd(rng, tokens * kv * d)
    qkn = rnd(rng, 2 * d, 0.1)
    keys, values = np.zeros(cap * kv * d, np.float32), np.zeros(cap * kv * d, np.float32)
    check(ours, ref, "ATTENTION_QUERY_KV", (heads + kv) * tokens,
          {1: mixed, 2: qkn, 4: keys, 5: key, 6: value, 7: values},
          {0: tokens * heads * d, 3: tokens * heads * d, 4: keys.size, 7: values.size},
          [d, rot, pos, heads, kv, tokens], [1e-6, theta])
    # the split query / KV ops (8, 9) the engine uses without the fused op
    check(ours, ref, "ATTENTION_QUERY", heads * tokens, {1: mixed, 2: qkn[:d]}, {0: tokens * heads * d,
                                                                                3: tokens * heads * d},
          [d, rot, pos, heads], [1e-6, theta])
    check(ours, ref, "ATTENTION_KV", kv * tokens, {1: key, 2: qkn[d:], 3: value, 0: keys, 4: values},
          {0: keys.size, 4: values.size}, [d, rot, pos, kv], [1e-6, theta])


@pytest.mark.parametrize("d,heads,kv,length,tokens", [(256, 8, 2, 454, 1), (256, 8, 2, 100, 4), (256, 8, 2, 1, 3),
                                                      (16, 4, 2, 17, 2), (16, 8, 2, 5, 1)])
def test_attention_read(ours, ref, d, heads, kv, length, tokens):
    rng = np.random.default_rng(d + length + tokens)
    cap = length + tokens + 64
    q = rnd(rng, tokens * heads * d)
    keys, values = rnd(rng, cap * kv * d), rnd(rng, cap * kv * d)
    gate = rnd(rng, tokens * heads * d)
    n6 = max(cap, (cap + 31) // 32 * (d + 2))
    check(ours, ref, "ATTENTION_READ", heads, {1: q, 2: keys, 3: values, 4: gate, 5: np.zeros(n6 * heads, np.float32)},
          {0: tokens * heads * d}, [d, heads, kv, length, cap, tokens, n6])


@pytest.mark.parametrize("rows,cols,batch", [(6144, 1024, 1), (1024, 3584, 2), (16, 1024, 4), (7, 12, 3)])
def test_projections(ours, ref, rows, cols, batch):
    rng = np.random.default_rng(rows + cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    outs = []
    for br in (ours, ref):
        a, xb = br.upload(w), br.upload(x)
        y1, y2, y3 = br.alloc(batch * rows), br.alloc(batch * rows), br.alloc(batch * rows)
        if batch == 1:
            br.gemv(y1, a, xb, rows, cols)
        else:
            br.gemm(y1, a, xb, rows, cols, batch)
        br.gemm(y2, br.upload(pack_bf16(w).view(np.float32)), xb, rows, cols, batch, kind="bf16")
        br.gemm(y3, br.upload(pack_int8(*O.quantize_int8_rows(w, rows, cols)).view(np.float32)), xb, rows, cols, batch,
                kind="i8")
        outs.append([y.read() for y in (y1, y2, y3)])
    for name, a, b in zip(("f32", "bf16", "i8"), *outs):
        same(a, b, f"projection {name} {rows}x{cols} batch {batch}")
