"""Each HIP kernel of the MI355X bridge, called through the C ABI, against the
CPU op bridge (the restatement of the reference's op bodies) on the same
seeded inputs, or against fp64 for the projections; argmax and the
embedding ops bit-exact."""
import numpy as np
import pytest

from bridges import both, rnd
from conftest import ROOT
from parity import FP32_RTOL, dot_bound, parity
from qwen_mi355x.bridge import Bridge, pack_bf16, pack_int8

import oracle as O

pytestmark = pytest.mark.gpu
OPS = ROOT / "oracle" / "lib" / "libqwen_ops_bridge.so"


@pytest.fixture(scope="module")
def gpu():
    b = Bridge()
    print("bridge:", b.info, flush=True)
    yield b
    b.close()


@pytest.fixture(scope="module")
def cpu():
    b = Bridge(OPS, kind=0)
    yield b
    b.close()


SHAPES_08B = [(6144, 1024), (2048, 1024), (16, 1024), (4096, 1024), (512, 1024), (1024, 2048), (3584, 1024),
              (1024, 3584)]
SHAPES_SMALL = [(24, 8), (8, 16), (16, 8), (19, 8), (64, 64), (256, 64), (64, 256), (512, 64), (7, 12), (33, 20)]


@pytest.mark.parametrize("rows,cols", SHAPES_08B + SHAPES_SMALL)
@pytest.mark.parametrize("batch", [1, 2, 4, 5, 8, 40])
def test_gemm_f32(gpu, rows, cols, batch):
    print(f"gemm f32 {rows}x{cols} batch {batch}", flush=True)
    rng = np.random.default_rng(rows * 31 + cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    a, xb, y = gpu.upload(w), gpu.upload(x), gpu.alloc(batch * rows)
    if batch == 1:
        gpu.gemv(y, a, xb, rows, cols)
    else:
        gpu.gemm(y, a, xb, rows, cols, batch)
    got = y.read().reshape(batch, rows)
    W = w.reshape(rows, cols)
    X = x.reshape(batch, cols)
    want = X.astype(np.float64) @ W.T.astype(np.float64)
    bound = np.abs(X.astype(np.float64)) @ np.abs(W.T.astype(np.float64)) * 2e-5 + 1e-30
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("batch", [1, 4])
def test_gemm_f32_lm_head_shape(gpu, batch):
    """The tied lm_head (248,320 x 1024, 1 GB of fp32) as the op path runs it:
    one logit row (GEMV) and the 4 rows of a verify pass, against fp64."""
    test_gemm_f32(gpu, 248320, 1024, batch)


@pytest.mark.parametrize("rows,cols", SHAPES_08B + [(33, 20), (7, 12), (3, 260), (12, 64), (5, 192)])
@pytest.mark.parametrize("batch", [127, 130, 257])
def test_gemm_f32_prefill_tiles(gpu, rows, cols, batch):
    """Prefill batches across the 128-token MFMA tile edge (and odd widths on
    the FMA kernel; few-row matrices on the 16-token MFMA tiles with their
    rows past the matrix masked)."""
    test_gemm_f32(gpu, rows, cols, batch)


@pytest.mark.parametrize("kind", ["bf16", "i8"])
@pytest.mark.parametrize("rows,cols", [(6144, 1024), (1024, 3584), (3584, 1024), (16, 1024), (24, 8), (64, 64),
                                       (256, 64), (8, 16)])
@pytest.mark.parametrize("batch", [1, 3, 4, 8, 24])
def test_gemm_bf16_int8(gpu, kind, rows, cols, batch):
    print(f"gemm {kind} {rows}x{cols} batch {batch}", flush=True)
    rng = np.random.default_rng(rows + 7 * cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    if kind == "bf16":
        packed = pack_bf16(w)
        dense = ((w.view(np.uint32) >> 16) << 16).view(np.float32)
        scales = np.ones(rows, np.float64)
        q = dense
    else:
        s, qi = O.quantize_int8_rows(w, rows, cols)
        packed = pack_int8(s, qi)
        scales = s.astype(np.float64)
        q = qi.astype(np.float32)
    a, xb, y = gpu.upload(packed), gpu.upload(x), gpu.alloc(batch * rows)
    if batch == 1 and kind == "bf16":
        gpu.gemv(y, a, xb, rows, cols, kind="bf16")
    else:
        gpu.gemm(y, a, xb, rows, cols, batch, kind=kind)
    got = y.read().reshape(batch, rows)
    Q = q.reshape(rows, cols).astype(np.float64)
    X = x.reshape(batch, cols).astype(np.float64)
    want = (X @ Q.T) * scales[None, :]
    bound = (np.abs(X) @ np.abs(Q.T)) * np.abs(scales)[None, :] * 2e-5 + 1e-30
    assert np.all(np.abs(got - want) <= bound)


@pytest.mark.parametrize("rows,cols,batch", [(100, 64, 37), (64, 1024, 129), (3584, 1024, 130), (8, 12, 5)])
def test_glu_f32_fused_edges(gpu, rows, cols, batch):
    """The fused fp32 GLU kernel (64-row gate/up tiles, silu in the epilogue)
    at ragged row, token and K edges, against fp64."""
    print(f"glu f32 {rows}x{cols} batch {batch}", flush=True)
    rng = np.random.default_rng(rows + cols + batch)
    gw = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    uw = (rng.standard_normal(rows * cols) * 0.05).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    prod, gy, uy = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.glu(prod, gy, uy, gpu.upload(gw), gpu.upload(uw), gpu.upload(x), rows, cols, batch)
    X = x.reshape(batch, cols).astype(np.float64)
    G, U = X @ gw.reshape(rows, cols).astype(np.float64).T, X @ uw.reshape(rows, cols).astype(np.float64).T
    want = G / (1 + np.exp(-G)) * U
    bound = dot_bound(gw.reshape(rows, cols), X.T).T * (np.abs(U) + 1) + dot_bound(uw.reshape(rows, cols), X.T).T * \
        (np.abs(G) + 1)
    got = prod.read().reshape(batch, rows)
    assert np.all(np.abs(got - want) <= bound + 1e-6 * np.abs(want)), np.max(np.abs(got - want) - bound)


@pytest.mark.parametrize("kind", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("batch", [1, 4, 6, 20, 130])
def test_group_glu_equal_separate_calls(gpu, kind, batch):
    """Grouped / GLU projections equal the separate projections (reference
    native/rocm/bridge.cpp:657-729); fp32 arms are this bridge's own."""
    print(f"group/glu {kind} batch {batch}", flush=True)
    rng = np.random.default_rng(11 + batch)
    cols = 1024
    shapes = [6144, 2048, 16, 16]

    def pack(w, rows):
        if kind == "f32":
            return w
        if kind == "bf16":
            return pack_bf16(w)
        s, q = O.quantize_int8_rows(w, rows, cols)
        return pack_int8(s, q)

    mats = [gpu.upload(pack((rng.standard_normal(r * cols) * 0.02).astype(np.float32), r)) for r in shapes]
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32))
    ys = [gpu.alloc(batch * r) for r in shapes]
    gpu.group(list(zip(ys, mats, shapes)), x, cols, batch, kind=kind)
    for y, m, r in zip(ys, mats, shapes):
        one = gpu.alloc(batch * r)
        gpu.gemm(one, m, x, r, cols, batch, kind=kind)
        assert np.array_equal(y.read(), one.read()) or batch > 4
        parity(y.read(), one.read(), where=f"group {r}")
    rows = 3584
    g = gpu.upload(pack((rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rows))
    u = gpu.upload(pack((rng.standard_normal(rows * cols) * 0.02).astype(np.float32), rows))
    prod, gy, uy = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch, kind=kind)
    g1, u1 = gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.gemm(g1, g, x, rows, cols, batch, kind=kind)
    gpu.gemm(u1, u, x, rows, cols, batch, kind=kind)
    gv, uv = g1.read().astype(np.float64), u1.read().astype(np.float64)
    want = gv / (1 + np.exp(-gv)) * uv
    parity(prod.read(), want, where="glu")


@pytest.mark.parametrize("rows,cols,batch", [(6144, 1024, 2644), (1024, 2048, 130), (1024, 3584, 64), (512, 1024, 454),
                                            (4096, 1024, 10240), (40, 12, 65), (2048, 1024, 63),
                                            (4096, 1024, 2644), (1024, 3584, 2644), (3584, 1024, 2644),
                                            (1024, 2048, 10240), (256, 64, 300), (48, 1024, 200),
                                            (96, 32, 130), (320, 96, 257)])
def test_gemm_f32_prepared(gpu, rows, cols, batch):
    """qr_gemm_f32_prepare: the projection of a prepared matrix (the P3 GEMM of
    gemm_p3.hip from 64 tokens: whole tiles, and the tiles past the last whole
    round of 256 blocks split along K and summed in chunk order; K loops of
    one step (cols 32: only the last step, which issues no DMA) and of three;
    the
    split-BF16 kernel below 64 tokens or for cols % 32 != 0) against fp64 with
    the fp32 dot-product bound on sampled rows (the last row always among
    them), twice bitwise-equal, and within the bound of the unprepared
    kernel's result."""
    print(f"gemm f32 prepared {rows}x{cols} batch {batch}", flush=True)
    rng = np.random.default_rng(rows + 3 * cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    a, xb = gpu.upload(w), gpu.upload(x)
    plain, y1, y2 = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.gemm(plain, a, xb, rows, cols, batch)
    gpu.prepare(a, rows, cols)
    gpu.gemm(y1, a, xb, rows, cols, batch)
    gpu.gemm(y2, a, xb, rows, cols, batch)
    got = y1.read().reshape(batch, rows)
    assert np.array_equal(got, y2.read().reshape(batch, rows))
    idx = np.unique(np.append(np.random.default_rng(0).integers(0, batch, 64), batch - 1))
    X, W = x.reshape(batch, cols)[idx].astype(np.float64), w.reshape(rows, cols).astype(np.float64)
    want = X @ W.T
    bound = np.abs(X) @ np.abs(W.T) * 2e-5 + 1e-30
    assert np.all(np.abs(got[idx] - want) <= bound), np.max(np.abs(got[idx] - want) / bound)
    other = plain.read().reshape(batch, rows)[idx]
    assert np.all(np.abs(got[idx] - other) <= 2 * bound)


def test_prepared_group_glu_and_invalidation(gpu):
    """Prepared matrices in a group (x split once) equal the separate prepared
    projections bitwise; a prepared GLU (gate and up as one GEMM over their
    planes side by side, then silu(gate) * up; gate_y / up_y untouched, as the
    fused GLU) follows the separate projections to the fp32 bound; a qr_write
    into a prepared matrix drops its planes (and the GLU pair's copy), so the
    next projection follows the new values; release and free are accepted."""
    rng = np.random.default_rng(5)
    cols, batch = 1024, 300
    shapes = [6144, 2048, 16, 16]
    ws = [(rng.standard_normal(r * cols) * 0.02).astype(np.float32) for r in shapes]
    mats = [gpu.upload(w) for w in ws]
    for m, r in zip(mats, shapes):
        if r > 16:
            gpu.prepare(m, r, cols)
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32))
    ys = [gpu.alloc(batch * r) for r in shapes]
    gpu.group(list(zip(ys, mats, shapes)), x, cols, batch)
    for y, m, r in zip(ys, mats, shapes):
        one = gpu.alloc(batch * r)
        gpu.gemm(one, m, x, r, cols, batch)
        assert np.array_equal(y.read(), one.read()), r
    rows = 3584
    gw, uw = [(rng.standard_normal(rows * cols) * 0.02).astype(np.float32) for _ in range(2)]
    g, u = gpu.upload(gw), gpu.upload(uw)
    gpu.prepare(g, rows, cols)
    gpu.prepare(u, rows, cols)
    prod, gy, uy = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch)
    g1, u1 = gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.gemm(g1, g, x, rows, cols, batch)
    gpu.gemm(u1, u, x, rows, cols, batch)
    assert not gy.read().any() and not uy.read().any()  # untouched
    gv, uv = g1.read().astype(np.float64), u1.read().astype(np.float64)
    parity(prod.read(), gv / (1 + np.exp(-gv)) * uv, where="prepared glu")
    # a write into gate drops its planes and the pair's: the GLU follows the new gate
    gw2 = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    g.write(gw2)
    gpu.prepare(g, rows, cols)
    gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch)
    gpu.gemm(g1, g, x, rows, cols, batch)
    gv = g1.read().astype(np.float64)
    parity(prod.read(), gv / (1 + np.exp(-gv)) * uv, where="prepared glu after a write")
    # rewrite the first matrix: its planes are dropped, the projection follows the new weights
    new = (rng.standard_normal(shapes[0] * cols) * 0.02).astype(np.float32)
    mats[0].write(new)
    y = gpu.alloc(batch * shapes[0])
    gpu.gemm(y, mats[0], x, shapes[0], cols, batch)
    X = x.read().reshape(batch, cols)[:16].astype(np.float64)
    W = new.reshape(shapes[0], cols).astype(np.float64)
    bound = np.abs(X) @ np.abs(W.T) * 2e-5 + 1e-30
    assert np.all(np.abs(y.read().reshape(batch, shapes[0])[:16] - X @ W.T) <= bound)
    gpu.release(mats[1])
    gpu.release(mats[1])  # releasing twice (or an unprepared matrix) is accepted


@pytest.mark.gpu
def test_prepared_inside_freed_allocation(gpu):
    """A matrix prepared at an offset inside a larger allocation loses its planes
    when that allocation is freed: a new allocation of the same size (the
    runtime usually returns the same address), its values put there by a kernel
    (an ADD, which drops no planes itself) and prepared again at the same
    offset, is multiplied with the new values, not the old planes."""
    import ctypes
    rng = np.random.default_rng(23)
    rows, cols, batch = 512, 1024, 128
    off = rows * cols
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32))
    X = x.read().reshape(batch, cols).astype(np.float64)
    y = gpu.alloc(batch * rows)
    addrs = []
    for rep in range(2):
        w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
        big = gpu.alloc(2 * off)
        addrs.append(big.ptr)
        wb, zero = gpu.upload(w), gpu.alloc(off)
        gpu.run("ADD", off, p=(big.at(off), wb, zero))
        inner = ctypes.c_void_p(big.at(off))
        gpu._check(gpu.L.qr_gemm_f32_prepare(gpu.ctx, inner, rows, cols))
        gpu._check(gpu.L.qr_gemm(gpu.ctx, ctypes.c_void_p(y.ptr), inner, ctypes.c_void_p(x.ptr), rows, cols, batch))
        W = w.reshape(rows, cols).astype(np.float64)
        bound = np.abs(X) @ np.abs(W.T) * 2e-5 + 1e-30
        assert np.all(np.abs(y.read().reshape(batch, rows) - X @ W.T) <= bound), (rep, addrs)
        del big  # qr_free of the whole allocation
    print("allocation addresses", [hex(a) for a in addrs])


def _bf16_or_i8(kind, w, rows, cols):
    """(packed upload, exact values as a float64 matrix, per-row scales)."""
    if kind == "bf16":
        dense = ((w.view(np.uint32) >> 16) << 16).view(np.float32)  # the values pack_bf16 keeps
        return pack_bf16(w), dense.reshape(rows, cols).astype(np.float64), np.ones(rows)
    sc, q = O.quantize_int8_rows(w, rows, cols)
    return pack_int8(sc, q), q.reshape(rows, cols).astype(np.float64), sc.astype(np.float64)


@pytest.mark.parametrize("kind", ["bf16", "i8"])
@pytest.mark.parametrize("rows,cols,batch", [(6144, 1024, 2644), (1024, 3584, 130), (3584, 1024, 257),
                                            (512, 1024, 454), (1024, 2048, 64), (48, 1024, 200), (96, 32, 130),
                                            (4096, 1024, 10240), (37, 64, 70)])
def test_gemm_bf16_prepared(gpu, kind, rows, cols, batch):
    """qr_gemm_bf16_prepare / qr_gemm_i8_prepare: the projection of a prepared
    BF16 or int8 matrix (one plane of its exact values in fragment order,
    three part products x_p w on the plane kernels: whole tiles, K-split
    tiles, 128- and 256-row weight tiles; int8 rows scaled after the sum; an
    odd-row int8 matrix, whose values sit off 8-byte alignment, keeps the
    split-BF16 kernel)
    against fp64 over the matrix's values with the fp32 dot-product bound on
    sampled rows (the last among them), twice bitwise-equal, and within the
    bound of the unprepared split-BF16 kernel's result."""
    print(f"gemm {kind} prepared {rows}x{cols} batch {batch}", flush=True)
    rng = np.random.default_rng(rows + 5 * cols + batch)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    packed, W, scales = _bf16_or_i8(kind, w, rows, cols)
    x = rng.standard_normal(batch * cols).astype(np.float32)
    a, xb = gpu.upload(packed), gpu.upload(x)
    plain, y1, y2 = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.gemm(plain, a, xb, rows, cols, batch, kind=kind)
    gpu.prepare(a, rows, cols, kind=kind)
    gpu.gemm(y1, a, xb, rows, cols, batch, kind=kind)
    gpu.gemm(y2, a, xb, rows, cols, batch, kind=kind)
    got = y1.read().reshape(batch, rows)
    assert np.array_equal(got, y2.read().reshape(batch, rows))
    idx = np.unique(np.append(np.random.default_rng(0).integers(0, batch, 64), batch - 1))
    X = x.reshape(batch, cols)[idx].astype(np.float64)
    want = (X @ W.T) * scales[None, :]
    bound = (np.abs(X) @ np.abs(W.T)) * np.abs(scales)[None, :] * 2e-5 + 1e-30
    assert np.all(np.abs(got[idx] - want) <= bound), np.max(np.abs(got[idx] - want) / bound)
    other = plain.read().reshape(batch, rows)[idx]
    assert np.all(np.abs(got[idx] - other) <= 2 * bound)


@pytest.mark.parametrize("kind", ["bf16", "i8"])
def test_prepared_bf16_group_glu_and_invalidation(gpu, kind):
    """Prepared BF16 (int8) matrices in a group equal their separate prepared
    projections bitwise (the 16-row a / b matrices unprepared beside them); a
    prepared BF16 (int8: the rows' scales after the sums) GLU (gate and up in one kernel over their interleaved planes
    with the silu product; rows % 128 != 0: two prepared projections and the
    silu product) follows the separate projections to the fp32 bound, gate_y /
    up_y untouched by the fused form; a qr_write into a prepared matrix drops
    its plane, so the next projection follows the new values."""
    rng = np.random.default_rng(15)
    cols, batch = 1024, 300
    shapes = [6144, 2048, 16, 16]
    ws = [(rng.standard_normal(r * cols) * 0.02).astype(np.float32) for r in shapes]
    mats = [gpu.upload(_bf16_or_i8(kind, w, r, cols)[0]) for w, r in zip(ws, shapes)]
    for m, r in zip(mats, shapes):
        if r > 16:
            gpu.prepare(m, r, cols, kind=kind)
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32))
    ys = [gpu.alloc(batch * r) for r in shapes]
    gpu.group(list(zip(ys, mats, shapes)), x, cols, batch, kind=kind)
    for y, m, r in zip(ys, mats, shapes):
        one = gpu.alloc(batch * r)
        gpu.gemm(one, m, x, r, cols, batch, kind=kind)
        assert np.array_equal(y.read(), one.read()), r
    for rows in (3584, 320):
        gw, uw = [(rng.standard_normal(rows * cols) * 0.02).astype(np.float32) for _ in range(2)]
        g, u = gpu.upload(_bf16_or_i8(kind, gw, rows, cols)[0]), gpu.upload(_bf16_or_i8(kind, uw, rows, cols)[0])
        gpu.prepare(g, rows, cols, kind=kind)
        gpu.prepare(u, rows, cols, kind=kind)
        prod, gy, uy = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
        gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch, kind=kind)
        g1, u1 = gpu.alloc(batch * rows), gpu.alloc(batch * rows)
        gpu.gemm(g1, g, x, rows, cols, batch, kind=kind)
        gpu.gemm(u1, u, x, rows, cols, batch, kind=kind)
        if rows % 128 == 0:
            assert not gy.read().any() and not uy.read().any()  # untouched
        gv, uv = g1.read().astype(np.float64), u1.read().astype(np.float64)
        parity(prod.read(), gv / (1 + np.exp(-gv)) * uv, where=f"prepared {kind} glu {rows}")
    # rewrite the first matrix: its plane is dropped, the projection follows the new weights
    new = (rng.standard_normal(shapes[0] * cols) * 0.02).astype(np.float32)
    packed, W, sc = _bf16_or_i8(kind, new, shapes[0], cols)
    mats[0].write(packed)
    y = gpu.alloc(batch * shapes[0])
    gpu.gemm(y, mats[0], x, shapes[0], cols, batch, kind=kind)
    X = x.read().reshape(batch, cols)[:16].astype(np.float64)
    bound = (np.abs(X) @ np.abs(W.T)) * np.abs(sc)[None, :] * 2e-5 + 1e-30
    assert np.all(np.abs(y.read().reshape(batch, shapes[0])[:16] - (X @ W.T) * sc[None, :]) <= bound)
    gpu.release(mats[1])


@pytest.mark.parametrize("rows,batch", [(3584, 2644), (3584, 64), (256, 300), (384, 130), (320, 130)])
def test_prepared_glu_shapes(gpu, rows, batch):
    """A GLU of two prepared matrices (rows % 128 == 0: gate, up and the silu
    product in one P3 kernel, whole tiles and K-split tiles; else two prepared
    projections and the silu product) against the silu product of the
    prepared projections in float64, gate_y / up_y untouched by the fused
    form, twice bitwise-equal."""
    print(f"prepared glu {rows} rows batch {batch}", flush=True)
    rng = np.random.default_rng(rows + batch)
    cols = 1024
    g = gpu.upload((rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    u = gpu.upload((rng.standard_normal(rows * cols) * 0.02).astype(np.float32))
    x = gpu.upload(rng.standard_normal(batch * cols).astype(np.float32))
    gpu.prepare(g, rows, cols)
    gpu.prepare(u, rows, cols)
    prod, gy, uy = gpu.alloc(batch * rows), gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch)
    first = prod.read()
    gpu.glu(prod, gy, uy, g, u, x, rows, cols, batch)
    assert np.array_equal(first, prod.read())
    if rows % 128 == 0:
        assert not gy.read().any() and not uy.read().any()
    g1, u1 = gpu.alloc(batch * rows), gpu.alloc(batch * rows)
    gpu.gemm(g1, g, x, rows, cols, batch)
    gpu.gemm(u1, u, x, rows, cols, batch)
    gv, uv = g1.read().astype(np.float64), u1.read().astype(np.float64)
    parity(first, gv / (1 + np.exp(-gv)) * uv, where=f"prepared glu {rows}x{batch}")


def test_planes_from_producers(gpu):
    """A norm over >= 64 rows whose width a prepared matrix takes, and a
    prepared GLU whose product width one does, leave their output's split
    planes for the very next call: that projection equals the same projection
    of a copy (split afresh) bitwise. Any call in between (here a sync or a
    write into the output) makes the next projection split again, so it
    follows what the buffer holds then."""
    rng = np.random.default_rng(11)
    h, inter, batch = 1024, 3584, 130
    w_in = gpu.upload((rng.standard_normal(2048 * h) * 0.02).astype(np.float32))
    gate = gpu.upload((rng.standard_normal(inter * h) * 0.02).astype(np.float32))
    up = gpu.upload((rng.standard_normal(inter * h) * 0.02).astype(np.float32))
    down = gpu.upload((rng.standard_normal(h * inter) * 0.02).astype(np.float32))
    gpu.prepare(w_in, 2048, h)
    gpu.prepare(gate, inter, h)
    gpu.prepare(up, inter, h)
    gpu.prepare(down, h, inter)
    x = gpu.upload(rng.standard_normal(batch * h).astype(np.float32))
    res = gpu.upload(rng.standard_normal(batch * h).astype(np.float32))
    nw = gpu.upload((rng.standard_normal(h) * 0.1).astype(np.float32))

    def proj_of_copy(src, a, rows, cols):
        cp, out = gpu.alloc(batch * cols), gpu.alloc(batch * rows)
        gpu.copy(cp, src, batch * cols)
        gpu.gemm(out, a, cp, rows, cols, batch)
        return out.read()

    # RmsNorm -> projection
    y = gpu.alloc(batch * h)
    gpu.run("RMS_NORM", batch, [y, x, nw], [h], [1e-6, 1.0])
    out = gpu.alloc(batch * 2048)
    gpu.gemm(out, w_in, y, 2048, h, batch)
    assert np.array_equal(out.read(), proj_of_copy(y, w_in, 2048, h))
    # AddRmsNorm -> GLU -> down projection
    s_, y2 = gpu.alloc(batch * h), gpu.alloc(batch * h)
    gpu.run("ADD_RMS_NORM", batch, [s_, x, res, y2, nw], [h], [1e-6, 1.0])
    prod, gy, uy = gpu.alloc(batch * inter), gpu.alloc(batch * inter), gpu.alloc(batch * inter)
    gpu.glu(prod, gy, uy, gate, up, y2, inter, h, batch)
    o1 = gpu.alloc(batch * h)
    gpu.gemm(o1, down, prod, h, inter, batch)
    o2 = gpu.alloc(batch * h)
    gpu.sync()  # a call in between: the down projection splits the product again
    gpu.gemm(o2, down, prod, h, inter, batch)
    assert np.array_equal(o1.read(), o2.read())
    assert np.array_equal(o1.read(), proj_of_copy(prod, down, h, inter))
    g1, u1 = gpu.alloc(batch * inter), gpu.alloc(batch * inter)
    gpu.gemm(g1, gate, y2, inter, h, batch)
    gpu.gemm(u1, up, y2, inter, h, batch)
    gv, uv = g1.read().astype(np.float64), u1.read().astype(np.float64)
    parity(prod.read(), gv / (1 + np.exp(-gv)) * uv, where="glu product with planes")
    # a write between the norm and the projection: the projection follows the new values
    gpu.run("RMS_NORM", batch, [y, x, nw], [h], [1e-6, 1.0])
    new = rng.standard_normal(batch * h).astype(np.float32)
    y.write(new)
    gpu.gemm(out, w_in, y, 2048, h, batch)
    X = new.reshape(batch, h)[:8].astype(np.float64)
    W = w_in.read().reshape(2048, h).astype(np.float64)
    bound = np.abs(X) @ np.abs(W.T) * 2e-5 + 1e-30
    assert np.all(np.abs(out.read().reshape(batch, 2048)[:8] - X @ W.T) <= bound)
    # RmsNormGate (groups of 128, 16 per token) -> a projection of width 2048:
    # the first pair teaches the bridge the width, the next norm writes planes
    heads, d = 16, 128
    core = gpu.upload(rng.standard_normal(batch * heads * d).astype(np.float32))
    z = gpu.upload(rng.standard_normal(batch * heads * d).astype(np.float32))
    gw = gpu.upload((rng.standard_normal(d) * 0.1 + 1.0).astype(np.float32))
    w_o = gpu.upload((rng.standard_normal(h * heads * d) * 0.02).astype(np.float32))
    gpu.prepare(w_o, h, heads * d)
    gated, o3 = gpu.alloc(batch * heads * d), gpu.alloc(batch * h)
    for _ in range(3):
        gpu.run("RMS_NORM_GATE", batch * heads, [gated, core, gw, z], [d], [1e-6, 0.0])
        gpu.gemm(o3, w_o, gated, h, heads * d, batch)
        assert np.array_equal(o3.read(), proj_of_copy(gated, w_o, h, heads * d))
    G = gated.read().reshape(batch, heads * d)[:8].astype(np.float64)
    W = w_o.read().reshape(h, heads * d).astype(np.float64)
    bound = np.abs(G) @ np.abs(W.T) * 2e-5 + 1e-30
    assert np.all(np.abs(o3.read().reshape(batch, h)[:8] - G @ W.T) <= bound)


@pytest.mark.parametrize("kind", ["f32", "bf16", "i8"])
@pytest.mark.parametrize("rows,cols", [(1024, 2048), (1024, 3584), (64, 256), (8, 16)])
def test_add_norm_tail(gpu, cpu, kind, rows, cols):
    """GEMV + Add + RmsNorm tail equals GEMV then op AddRmsNorm (bridge.cpp:797-827)."""
    print(f"add_norm {kind} {rows}x{cols}", flush=True)
    rng = np.random.default_rng(rows + cols)
    w = (rng.standard_normal(rows * cols) * 0.02).astype(np.float32)
    if kind == "bf16":
        packed = pack_bf16(w)
    elif kind == "i8":
        packed = pack_int8(*O.quantize_int8_rows(w, rows, cols))
    else:
        packed = w
    xv = rng.standard_normal(cols).astype(np.float32)
    uv = rng.standard_normal(rows).astype(np.float32)
    wn = (rng.standard_normal(rows) * 0.1).astype(np.float32)
    for repeat in range(3):  # the ticket must be back at 0 after every launch
        a, x, y = gpu.upload(packed), gpu.upload(xv), gpu.alloc(rows)
        u, s, norm, weight = gpu.upload(uv), gpu.alloc(rows), gpu.alloc(rows), gpu.upload(wn)
        gpu.add_norm(y, a, x, rows, cols, s, u, y, weight, norm, 1e-6, 1.0, kind=kind)
        y2 = gpu.alloc(rows)
        gpu.gemm(y2, a, x, rows, cols, 1, kind=kind)
        yv = y2.read()
        parity(y.read(), yv, where="tail gemv")
        sv = (uv + yv).astype(np.float32)
        parity(s.read(), sv, where="tail sum")
        r = 1 / np.sqrt(np.mean(sv.astype(np.float64) ** 2) + 1e-6)
        parity(norm.read(), sv * r * (wn.astype(np.float64) + 1), where="tail norm")


def argmax_cases():
    """The reference's argmax known answers (src/device/tests.rs:1117-1184):
    ties across slices, NaN/+-Inf, a row with no finite value, lengths around
    the one-block / two-pass switch."""
    seed = [0x2545F4914F6CDD1D]

    def nxt():
        s = seed[0]
        s ^= (s << 13) & 0xFFFFFFFFFFFFFFFF
        s ^= s >> 7
        s ^= (s << 17) & 0xFFFFFFFFFFFFFFFF
        seed[0] = s
        return np.float32((s >> 40) / float(1 << 24) * 20.0 - 10.0)

    cases = []
    for n in [1, 4095, 8191, 8192, 8193, 70000, 248320]:
        cases.append(np.array([nxt() for _ in range(n)], np.float32))
    tie = np.array([nxt() for _ in range(248320)], np.float32)
    for i in [248000, 70000, 5000, 300]:
        tie[i] = 50.0
    cases.append(tie)
    odd = np.array([nxt() for _ in range(248320)], np.float32)
    for k, i in enumerate([7, 4096, 4097, 100000, 248319]):
        odd[i] = [np.nan, np.inf, -np.inf][k % 3]
    odd[200000] = 30.0
    cases.append(odd)
    cases.append(np.full(20000, np.nan, np.float32))
    return cases


def argmax_rule(v):
    fin = np.isfinite(v)
    bad = int((~fin).sum())
    if not fin.any():
        return [np.float32(4294967295.0), np.float32(bad)]
    best = np.max(v[fin])
    return [np.float32(np.flatnonzero(fin & (v == best))[0]), np.float32(bad)]


def test_argmax_known_answers(gpu):
    for row in argmax_cases():
        n = row.size
        for rows in (1, 3):
            logits = np.concatenate([np.roll(row, -r * 1013) for r in range(rows)]).astype(np.float32)
            want = np.array(sum((argmax_rule(np.roll(row, -r * 1013)) for r in range(rows)), []), np.float32)
            buf = gpu.alloc(logits.size).write(logits.view(np.uint32))
            out = gpu.alloc(2 * rows)
            gpu.run("ARGMAX", rows, [out, buf], [n])
            assert np.array_equal(out.read(), want), (n, rows)


@pytest.mark.parametrize("d,groups", [(1024, 1), (1024, 3), (128, 16), (128, 48), (8, 5), (256, 8), (2048, 5), (512, 7),
                                      (1024, 9), (64, 3)])
def test_rms_family(gpu, cpu, d, groups):
    """RmsNorm, AddRmsNorm, RmsNormGate: the register form (d = 64 PER for
    PER 2..32, ragged last block of 4 groups) and the generic forms."""
    rng = np.random.default_rng(d + groups)
    x, w, u, z = rnd(rng, d * groups), rnd(rng, d, 0.1), rnd(rng, d * groups), rnd(rng, d * groups)
    g, c = both(gpu, cpu, "RMS_NORM", groups, {1: x, 2: w}, {0: d * groups}, [d], [1e-6, 1.0])
    parity(g[0], c[0], where="rms_norm")
    g, c = both(gpu, cpu, "ADD_RMS_NORM", groups, {1: x, 2: u, 4: w}, {0: d * groups, 3: d * groups}, [d], [1e-6, 1.0])
    parity(g[0], c[0], where="add")
    parity(g[3], c[3], where="add_rms_norm")
    g, c = both(gpu, cpu, "RMS_NORM_GATE", groups, {1: x, 2: w, 3: z}, {0: d * groups}, [d], [1e-6, 0.0])
    parity(g[0], c[0], where="rms_norm_gate")


def test_elementwise_and_embed(gpu, cpu):
    rng = np.random.default_rng(5)
    n = 3584 * 3
    a, b = rnd(rng, n, 3), rnd(rng, n)
    g, c = both(gpu, cpu, "ADD", n, {1: a, 2: b}, {0: n})
    assert np.array_equal(g[0], c[0])
    g, c = both(gpu, cpu, "SILU_PRODUCT", n, {1: a, 2: b}, {0: n})
    parity(g[0], c[0], where="silu_product")
    # DeltaGates with the reference's boundary values (src/device/tests.rs:368-400)
    av = np.array([100, -100, 0, 10], np.float32)
    bv = np.array([-100, 100, 0, 1], np.float32)
    dt = np.array([0, 0, 1, -1], np.float32)
    al = np.array([-20, 0, 1, 2], np.float32)
    g, c = both(gpu, cpu, "DELTA_GATES", 4, {1: av, 2: bv, 3: dt, 4: al}, {0: 4, 5: 4})
    parity(g[0], c[0], where="gates g")
    parity(g[5], c[5], where="gates beta")
    emb = rnd(rng, 19 * 8)
    packed = pack_bf16(emb)
    g, c = both(gpu, cpu, "EMBED_BF16", 8, {1: packed.view(np.float32)}, {0: 8}, [5, 8])
    assert np.array_equal(g[0], c[0])
    picks = np.array([3, 0, 18, 0], np.float32)
    g, c = both(gpu, cpu, "EMBED_BF16_PICKED", 16, {1: packed.view(np.float32), 2: picks}, {0: 16}, [0, 8])
    assert np.array_equal(g[0], c[0])


@pytest.mark.parametrize("width,n", [(1024, 1000), (1000, 3), (8, 481)])
def test_embed_rows(gpu, width, n):
    """qr_embed_rows (several launches past 480 ids) equals the per-row gather,
    bit for bit, for fp32 and packed BF16 tables; a bad id is refused before
    anything is queued."""
    rng = np.random.default_rng(width + n)
    rows = 300
    table = rnd(rng, rows * width)
    ids = rng.integers(0, rows, n).astype(np.int32)
    ids[0], ids[-1] = 0, rows - 1
    dst = gpu.alloc(n * width)
    gpu.embed_rows(dst, gpu.upload(table), rows, width, ids)
    assert np.array_equal(dst.read().reshape(n, width), table.reshape(rows, width)[ids])
    packed = gpu.upload(pack_bf16(table).view(np.float32))
    gpu.embed_rows(dst, packed, rows, width, ids, bf16=True)
    widened = ((table.view(np.uint32) >> 16) << 16).view(np.float32).reshape(rows, width)
    assert np.array_equal(dst.read().reshape(n, width), widened[ids])
    with pytest.raises(Exception, match="out of range"):
        gpu.embed_rows(dst, packed, rows, width, np.array([0, rows], np.int32), bf16=True)


@pytest.mark.parametrize("k,tokens,snaps", [(4, 1, 0), (4, 5, 0), (4, 4, 3), (3, 2, 1), (1, 1, 0),
                                             (4, 37, 5), (4, 130, 0), (3, 9, 8), (1, 7, 2), (17, 6, 2), (4, 33, 33),
                                             (4, 21, 2)])
def test_conv_silu(gpu, cpu, k, tokens, snaps):
    """ConvSilu: one thread per channel walking the tokens (<= 4 tokens), the
    16-token window kernel over prefill chunks (6146 channels: a ragged last
    block), snapshots of the history per token."""
    rng = np.random.default_rng(k * 10 + tokens)
    ch = (6146 if tokens == 21 else 6144) if k == 4 else 24
    x, w, h = rnd(rng, tokens * ch), rnd(rng, ch * k, 0.5), rnd(rng, ch * max(k - 1, 1) * (1 + snaps))
    g, c = both(gpu, cpu, "CONV_SILU", ch, {1: x, 2: w, 3: h}, {0: tokens * ch, 3: h.size}, [k, tokens, ch, snaps])
    parity(g[0], c[0], where="conv out")
    parity(g[3], c[3], where="conv history")


@pytest.mark.parametrize("kh,vh,d,tokens", [(16, 16, 128, 1), (16, 16, 128, 3), (2, 4, 3, 1), (4, 4, 16, 2),
                                             (8, 16, 128, 37)])
def test_delta_qk(gpu, cpu, kh, vh, d, tokens):
    rng = np.random.default_rng(d + tokens)
    stride = 2 * kh * d + vh * d
    x = rnd(rng, tokens * stride)
    g, c = both(gpu, cpu, "DELTA_QK", vh * tokens, {1: x}, {0: vh * tokens * d, 2: vh * tokens * d},
                [kh, vh, d, stride])
    parity(g[0], c[0], where="q")
    parity(g[2], c[2], where="k")


@pytest.mark.parametrize("kd,vd,heads,tokens,snaps,gated",
                         [(128, 128, 16, 1, 0, True), (128, 128, 16, 5, 0, True), (128, 128, 16, 4, 3, True),
                          (64, 5, 2, 3, 0, False), (128, 3, 2, 3, 0, False), (16, 16, 4, 7, 2, True),
                          (4, 4, 2, 5, 0, True), (3, 2, 4, 1, 0, False)])
def test_delta_rule(gpu, cpu, kd, vd, heads, tokens, snaps, gated):
    """Includes the reference's partially filled column groups (kd 64 with 5
    columns, kd 128 with 3; src/device/tests.rs:1214-1284)."""
    print(f"delta_rule kd={kd} vd={vd} heads={heads} tokens={tokens} snaps={snaps}", flush=True)
    rng = np.random.default_rng(kd + vd + tokens)
    stride = 2 * heads * kd + heads * vd
    q = rnd(rng, tokens * heads * kd, 0.2)
    k = rnd(rng, tokens * heads * kd, 0.2)
    v = rnd(rng, tokens * stride, 2.0)
    state = rnd(rng, heads * kd * vd * (1 + snaps))
    if gated:
        a, b = rnd(rng, tokens * heads), rnd(rng, tokens * heads)
        gates = rnd(rng, 2 * heads, 0.5)
        ins = {1: q, 2: k, 3: v, 4: state, 5: a, 6: b, 7: gates}
        op = "DELTA_RULE_GATED"
    else:
        decay = (-0.1 - np.abs(rnd(rng, tokens * heads, 0.1))).astype(np.float32)
        beta = (0.5 + rnd(rng, tokens * heads, 0.2)).clip(0, 1).astype(np.float32)
        ins = {1: q, 2: k, 3: v, 4: state, 5: decay, 6: beta}
        op = "DELTA_RULE"
    g, c = both(gpu, cpu, op, heads * vd, ins, {0: tokens * heads * vd, 4: state.size},
                [kd, vd, heads, heads, tokens, stride, snaps])
    parity(g[0], c[0], where="core")
    parity(g[4], c[4], where="state+snapshots")


def _unit_rows(rng, rows, d, scale=1.0):
    x = rng.standard_normal((rows, d))
    return (x / np.linalg.norm(x, axis=1, keepdims=True) * scale).astype(np.float32).ravel()


@pytest.mark.parametrize("tokens,gated,a_log,heads", [(16, True, 0.0, 16), (63, True, 0.0, 16), (64, True, 0.0, 16),
                                                      (65, False, 0.0, 16), (130, True, 0.0, 16), (300, False, 0.0, 16),
                                                      (200, True, 3.0, 16), (64 * 64 + 37, True, 0.0, 16),
                                                      (64 * 70 + 5, False, 0.0, 16), (64 * 66 + 3, True, 0.0, 4)])
def test_delta_rule_chunked(gpu, cpu, tokens, gated, a_log, heads):
    """Prefill lengths take the chunked (WY form, MFMA) path: 64-token chunks,
    ragged last chunks, heavy decay (A_log 3: g ~ -14 per token), and past 64
    chunks the grouped walk (65 chunks: five groups of 13; 71: four of 15 and
    one of 11), each group's scan beside the next group's prep in one launch
    (with 4 heads: 32 scan blocks beside 224 prep blocks). q and k are unit
    rows (q also / sqrt(dk)) as DeltaQk hands them to the rule; the CPU side
    is the token-by-token recurrence."""
    kd = vd = 128
    print(f"delta_rule_chunked tokens={tokens} gated={gated} a_log={a_log} heads={heads}", flush=True)
    rng = np.random.default_rng(tokens + 7 * gated)
    stride = 2 * heads * kd + heads * vd
    q = _unit_rows(rng, tokens * heads, kd, 1 / np.sqrt(kd))
    k = _unit_rows(rng, tokens * heads, kd)
    v = rnd(rng, tokens * stride, 1.0)
    state = rnd(rng, heads * kd * vd, 0.5)
    if gated:
        a, b = rnd(rng, tokens * heads), rnd(rng, tokens * heads)
        gates = np.concatenate([rnd(rng, heads, 0.5), np.full(heads, a_log, np.float32) + rnd(rng, heads, 0.5)])
        ins = {1: q, 2: k, 3: v, 4: state, 5: a, 6: b, 7: gates}
        op = "DELTA_RULE_GATED"
    else:
        decay = (-0.05 - np.abs(rnd(rng, tokens * heads, 0.1))).astype(np.float32)
        beta = (0.5 + rnd(rng, tokens * heads, 0.2)).clip(0, 1).astype(np.float32)
        ins = {1: q, 2: k, 3: v, 4: state, 5: decay, 6: beta}
        op = "DELTA_RULE"
    g, c = both(gpu, cpu, op, heads * vd, ins, {0: tokens * heads * vd, 4: state.size},
                [kd, vd, heads, heads, tokens, stride, 0])
    parity(g[0], c[0], where="core")
    parity(g[4], c[4], where="state")


@pytest.mark.parametrize("d,rot,heads,kv,tokens,pos", [(256, 64, 8, 2, 1, 453), (256, 64, 8, 2, 3, 8190),
                                                       (16, 8, 4, 1, 2, 7), (4, 2, 2, 1, 1, 0)])
def test_attention_query_kv(gpu, cpu, d, rot, heads, kv, tokens, pos):
    rng = np.random.default_rng(d + pos)
    cap = pos + tokens + 1
    mixed, key, value = rnd(rng, tokens * heads * 2 * d), rnd(rng, tokens * kv * d), rnd(rng, tokens * kv * d)
    qkn = rnd(rng, 2 * d, 0.1)
    keys, values = np.zeros(cap * kv * d, np.float32), np.zeros(cap * kv * d, np.float32)
    g, c = both(gpu, cpu, "ATTENTION_QUERY_KV", (heads + kv) * tokens,
                {1: mixed, 2: qkn, 4: keys, 5: key, 6: value, 7: values},
                {0: tokens * heads * d, 3: tokens * heads * d, 4: keys.size, 7: values.size},
                [d, rot, pos, heads, kv, tokens], [1e-6, 1e7 if d == 256 else 1e4])
    parity(g[0], c[0], where="query")
    assert np.array_equal(g[3], c[3])
    parity(g[4], c[4], where="keys")
    assert np.array_equal(g[7], c[7])


@pytest.mark.parametrize("d,heads,kv,length,tokens", [(256, 8, 2, 454, 1), (256, 8, 2, 8192, 1), (256, 8, 2, 1, 1),
                                                      (256, 8, 2, 100, 4), (256, 8, 2, 40, 24), (16, 4, 1, 17, 1),
                                                      (16, 4, 1, 5, 16), (4, 2, 1, 3, 2), (256, 8, 2, 1, 700),
                                                      (256, 8, 2, 77, 33), (128, 8, 2, 1, 64), (128, 4, 2, 10, 100),
                                                      (128, 8, 1, 3, 40), (64, 2, 2, 1, 65), (64, 8, 1, 5, 129),
                                                      (256, 16, 2, 1, 40), (256, 8, 2, 1, 8)])
def test_attention_read(gpu, cpu, d, heads, kv, length, tokens):
    """Decode (one row, split-K), a verify pass (rows 2..8, one decode read
    per row) and prefill chunks (causal rows: the MFMA flash kernel for head
    dims 64 / 128 / 256 and GQA groups 1, 2, 4, 8, ragged 32-row tiles, a
    cached prefix before the chunk; the per-row kernel for the rest)."""
    print(f"attention_read d={d} len={length} rows={tokens}", flush=True)
    rng = np.random.default_rng(d + length + tokens)
    cap = length + tokens + 64
    q = rnd(rng, tokens * heads * d)
    keys, values = rnd(rng, cap * kv * d), rnd(rng, cap * kv * d)
    gate = rnd(rng, tokens * heads * d)
    n6 = max(cap, (cap + 31) // 32 * (d + 2))
    g, c = both(gpu, cpu, "ATTENTION_READ", heads, {1: q, 2: keys, 3: values, 4: gate, 5: np.zeros(n6 * heads, np.float32)},
                {0: tokens * heads * d}, [d, heads, kv, length, cap, tokens, n6])
    parity(g[0], c[0], where="attention")


@pytest.mark.parametrize("tokens,kh,vh", [(1, 16, 16), (150, 16, 16), (70, 4, 8), (64 * 66 + 3, 4, 4)])
def test_delta_mixer_matches_four_ops(gpu, cpu, tokens, kh, vh):
    """qr_delta_mixer equals ConvSilu, DeltaQk, DeltaRuleGated, RmsNormGate
    (reference native/rocm/bridge.cpp:730-796): one token (the fused decode
    mixer) and prefill lengths, where the chunked rule normalises the
    convolution's q / k rows itself and stores them to query / key (key
    heads shared by two value heads; past 64 chunks the grouped walk, whose
    later groups' preps run beside the scan)."""
    print(f"delta_mixer tokens={tokens} kh={kh} vh={vh}", flush=True)
    rng = np.random.default_rng(99 + tokens)
    k, t = 4, tokens
    ch = (2 * kh + vh) * 128
    data = dict(projected=rnd(rng, t * ch), conv_w=rnd(rng, ch * k, 0.3), conv_state=rnd(rng, ch * (k - 1)),
                recurrent=rnd(rng, vh * 128 * 128, 0.5), a=rnd(rng, t * vh), b=rnd(rng, t * vh),
                gates=rnd(rng, 2 * vh, 0.3), norm_w=(1 + rnd(rng, 128, 0.1)).astype(np.float32),
                z=rnd(rng, t * vh * 128))
    outs = dict(convolved=t * ch, query=t * vh * 128, key=t * vh * 128, core=t * vh * 128, gated=t * vh * 128)
    res = []
    for br in (gpu, cpu):
        bufs = {n: br.upload(v) for n, v in data.items()}
        bufs.update({n: br.alloc(s) for n, s in outs.items()})
        if br is gpu:
            br.delta_mixer(**bufs, key_heads=kh, value_heads=vh, key_dim=128, value_dim=128, kernel=k, tokens=t,
                           channels=ch, eps=1e-6)
        else:
            br.run("CONV_SILU", ch, [bufs["convolved"], bufs["projected"], bufs["conv_w"], bufs["conv_state"]],
                   [k, t, ch])
            br.run("DELTA_QK", vh * t, [bufs["query"], bufs["convolved"], bufs["key"]], [kh, vh, 128, ch])
            br.run("DELTA_RULE_GATED", vh * 128, [bufs["core"], bufs["query"], bufs["key"], bufs["convolved"],
                                                  bufs["recurrent"], bufs["a"], bufs["b"], bufs["gates"]],
                   [128, 128, kh, vh, t, ch])
            br.run("RMS_NORM_GATE", vh * t, [bufs["gated"], bufs["core"], bufs["norm_w"], bufs["z"]], [128],
                   [1e-6, 0.0])
        res.append({n: bufs[n].read() for n in list(outs) + ["conv_state", "recurrent"]})
    for n in res[0]:
        parity(res[0][n], res[1][n], where=n)
