"""qr_argmax_fixed (the argmax with its partials in a fixed device array, for
callers that cannot allocate) against qr_run's Argmax op (partials in
library-allocated memory), bit for bit, through the C ABI: the reference's
argmax known answers, then two calls in a row with the second on a smaller
input (the array keeps the first call's partials), and the size limits."""
import ctypes

import numpy as np
import pytest

from qwen_mi355x.bridge import Bridge, Params
from test_gpu_ops import argmax_cases

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def gpu():
    b = Bridge()
    b.L.qr_argmax_fixed.restype = ctypes.c_int
    yield b
    b.close()


def fixed(gpu, out, logits, rows, n):
    a = Params()
    a.p[0], a.p[1], a.n[0] = out.ptr, logits.ptr, n
    return gpu.L.qr_argmax_fixed(gpu.ctx, rows, ctypes.byref(a))


def both(gpu, logits, rows, n):
    buf = gpu.alloc(logits.size).write(logits.view(np.uint32))
    want, got = gpu.alloc(2 * rows), gpu.alloc(2 * rows)
    gpu.run("ARGMAX", rows, [want, buf], [n])
    assert fixed(gpu, got, buf, rows, n) == 0, gpu.L.qr_error(gpu.ctx)
    return got.read(), want.read()


def test_argmax_fixed_equals_argmax_op(gpu):
    for row in argmax_cases():
        n = row.size
        for rows in (1, 3, 8):
            logits = np.concatenate([np.roll(row, -r * 1013) for r in range(rows)]).astype(np.float32)
            got, want = both(gpu, logits, rows, n)
            assert np.array_equal(got, want), (n, rows)


def test_argmax_fixed_second_call_smaller(gpu):
    rng = np.random.default_rng(21)
    big = rng.standard_normal(8 * 248320).astype(np.float32)
    got, want = both(gpu, big, 8, 248320)
    assert np.array_equal(got, want)
    small = rng.standard_normal(2 * 9000).astype(np.float32)
    small[9000 + 3345] = 50.0  # row 1, entry 3345
    got, want = both(gpu, small, 2, 9000)
    assert np.array_equal(got, want)
    assert got[2] == 3345 and got[3] == 0


def test_argmax_fixed_refuses_beyond_its_array(gpu):
    buf, out = gpu.alloc(16), gpu.alloc(18)
    assert fixed(gpu, out, buf, 9, 1) != 0
    assert b"rows must be 1..8" in gpu.L.qr_error(gpu.ctx)
    assert fixed(gpu, out, buf, 1, (1 << 20) + 1) != 0
    assert fixed(gpu, out, buf, 1, 0) != 0
