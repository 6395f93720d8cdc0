"""Runs one qr_* op on two bridges with the same inputs (a HIP bridge and a
CPU bridge, or two CPU bridges) and returns both sets of outputs."""
import numpy as np


def rnd(rng, n, scale=1.0):
    return (rng.standard_normal(n) * scale).astype(np.float32)


def both(first, second, op, count, inputs, outputs, n=(), f=()):
    """Run `op` on both bridges. inputs: {slot: array}; outputs: {slot: size}
    (an output slot may also be an input). Returns ({slot: first}, {slot: second})."""
    res = []
    for br in (first, second):
        bufs = {}
        for s, arr in inputs.items():
            bufs[s] = br.upload(np.ascontiguousarray(arr))
        for s, size in outputs.items():
            if s not in bufs:
                bufs[s] = br.alloc(size)
        p = [bufs.get(i, 0) for i in range(8)]
        br.run(op, count, p, n, f)
        res.append({s: bufs[s].read(size) for s, size in outputs.items()})
    return res
