"""Seeded random shapes through the C ABI against the oracle: every format,
row counts from 1 up, K at every block granularity, M from 1 to 40 (vector,
matrix-core and multi-launch paths), fp16 and fp32 activations; and the int(8)
sum at both steps, bit for bit."""
import os

import numpy as np
import pytest

import oracle
from rqmv import synth

pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
BLOCK = {"q8_0": 32, "q4_0": 32, "q4_k": 256, "q6_k": 256}
SEED = {"q8_0": 11, "q4_0": 12, "q4_k": 13, "q6_k": 14}


def _cases(fmt, count, seed):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(count):
        rows = int(rng.integers(1, 700))
        cols = BLOCK[fmt] * int(rng.integers(1, 6144 // BLOCK[fmt] + 1))
        m = int(rng.choice([1, 1, 2, 3, 5, 8, 13, 16, 21, 32, 40]))
        xdt = "f16" if rng.random() < 0.5 else "f32"
        out.append((rows, cols, m, xdt, int(rng.integers(1, 1 << 30))))
    return out


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_random_matvec_shapes(gpu, fmt):
    for rows, cols, m, xdt, seed in _cases(fmt, 12, seed=SEED[fmt]):
        w = synth.weights(fmt, rows, cols, seed=seed)
        W = gpu.Weight(fmt, rows, cols, w)
        if xdt == "f16":
            xh = synth.activations_f16(m * cols, seed=seed + 1).reshape(m, cols)
            x32, dt = synth.fp16_to_f32(xh), gpu.DTYPE_F16
        else:
            xh = synth.activations_f32(m * cols, seed=seed + 1).reshape(m, cols)
            x32, dt = xh, gpu.DTYPE_F32
        xb = gpu.DeviceBuffer.from_array(xh)
        yb = gpu.DeviceBuffer(4 * m * rows)
        print(f"{fmt} rows={rows} cols={cols} m={m} x={xdt}", flush=True)
        W.matvec(xb, dt, m, cols, yb, rows)
        gpu.synchronize()
        y = yb.download(np.float32).reshape(m, rows)
        ref = oracle.matvec_recipe_f32(fmt, w, rows, cols, x32, threads=THREADS)
        limit = 5e-4 if rows * cols < 4096 else 2e-4
        assert _rel(y, ref) <= limit, (fmt, rows, cols, m, xdt, _rel(y, ref))
        W.close()


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_random_int8_shapes(gpu, fmt):
    for rows, cols, m, _, seed in _cases(fmt, 6, seed=SEED[fmt] + 100):
        m = min(m, 6)
        w = synth.weights(fmt, rows, cols, seed=seed)
        W = gpu.Weight(fmt, rows, cols, w)
        x = np.stack([synth.activations_f32(cols, seed=seed + 1 + i) for i in range(m)])
        for step in (32, 256):
            print(f"int8 {fmt} rows={rows} cols={cols} m={m} step={step}", flush=True)
            got = gpu.contract_int8(W, x, step)
            want = oracle.int8_matvec(fmt, w, rows, cols, x, step)
            assert np.array_equal(np.asarray(got, np.float32).view(np.uint32),
                                  np.asarray(want, np.float32).view(np.uint32)), (fmt, rows, cols, m, step)
        W.close()
