"""Parity metric of the GPU path against the CPU oracle.

fp32: |a - b| <= rtol * (|b| + rms(b)) with rtol = 1e-4 (the north-star
tolerance, relative; the rms(b) term is the absolute floor that a relative
bound needs for elements near zero, scaled to the tensor). int8 against the
oracle run on the dequantised weights: rtol = 1e-2. The reference's own
`compare` (src/validation.rs:10-51) is |a - b| <= atol + rtol * |b|."""
import numpy as np

FP32_RTOL = 1e-4
INT8_RTOL = 1e-2


def parity(actual, expected, rtol=FP32_RTOL, where=""):
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    b = np.asarray(expected, dtype=np.float64).reshape(-1)
    assert a.shape == b.shape, f"{where}: shape {a.shape} != {b.shape}"
    assert np.all(np.isfinite(a)), f"{where}: non-finite values"
    floor = float(np.sqrt(np.mean(b * b))) if b.size else 0.0
    err = np.abs(a - b)
    bound = rtol * (np.abs(b) + floor)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(bad))
        raise AssertionError(f"{where}: first divergence [{i}] actual={a[i]} expected={b[i]} "
                             f"err={err[i]:.3e} bound={bound[i]:.3e}; max rel err {np.max(err / (np.abs(b) + floor)):.3e}")
    return float(np.max(err / (np.abs(b) + floor))) if b.size else 0.0


def dot_bound(w, x, rel=2e-5):
    """Error bound of an fp32 dot product against fp64: rel * sum |w_j x_j|."""
    return rel * (np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))) + 1e-30


def bf16_round(a):
    """Round-to-nearest-even float32 -> BF16, returned widened to float32."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def bf16_weights(c, w):
    """The weights with every tensor rounded to BF16 (a BF16-exact model: every
    matrix uploads as BF16 under fmt=BF16_EXACT, the embedding and tied LM head
    included)."""
    from qwen_mi355x import model as M
    return M.bf16_weights(w)
