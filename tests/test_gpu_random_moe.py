"""Seeded random gguf_moe configurations through the C ABI against the f64
oracle: formats, model and hidden widths, expert counts, top-k, softmax or
sigmoid scoring with or without renormalisation, a gated shared expert or
none, fp16 or fp32 activations, one position or a batch (each position also
bit-identical to its one-position call)."""
import numpy as np
import pytest

import oracle
from rqmv import synth

pytestmark = pytest.mark.gpu

BLOCK = {"q8_0": 32, "q4_0": 32, "q4_k": 256, "q6_k": 256}


def _case(rng):
    fmt = str(rng.choice(list(BLOCK)))
    blk = BLOCK[fmt]
    chunk = {"q8_0": 32, "q4_0": 64}.get(fmt, 256)  # the bank format's chunk
    dstep = max(chunk, 64)  # and the F16 router packs rows in 64-value chunks
    d = dstep * int(rng.integers(1, 1024 // dstep + 1))
    H = chunk * int(rng.integers(1, 512 // chunk + 1))
    E = int(rng.integers(2, 65))
    top = int(rng.integers(1, min(8, E) + 1))
    HS = H if rng.random() < 0.5 else 0
    m = int(rng.choice([1, 3, 7]))
    return dict(fmt=fmt, d=d, H=H, E=E, top=top, HS=HS, m=m, scoring=int(rng.integers(0, 2)),
                renorm=bool(rng.integers(0, 2)), xdt="f16" if rng.random() < 0.5 else "f32",
                seed=int(rng.integers(1, 1 << 30)))


def _rel(a, b):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def run_cases(gpu, count, seed):
    rng = np.random.default_rng(seed)
    for _ in range(count):
        c = _case(rng)
        fmt, d, H, E, top, HS, m, s = c["fmt"], c["d"], c["H"], c["E"], c["top"], c["HS"], c["m"], c["seed"]
        print(f"moe {c}", flush=True)
        router = synth.f16_weights(E, d, 0.02, seed=s, tag="router")
        gate = synth.weights(fmt, E * H, d, seed=s + 1, tag="gate")
        up = synth.weights(fmt, E * H, d, seed=s + 2, tag="up")
        down = synth.weights(fmt, E * d, H, seed=s + 3, tag="down")
        kw, okw = {}, {}
        if HS:
            sg = synth.f16_weights(1, d, 0.02, seed=s + 4, tag="sg")
            gs, us = synth.weights(fmt, HS, d, seed=s + 5, tag="gs"), synth.weights(fmt, HS, d, seed=s + 6, tag="us")
            ds = synth.weights(fmt, d, HS, seed=s + 7, tag="ds")
            kw = dict(shared_gate_inp=gpu.Weight("f16", 1, d, sg), gate_sh=gpu.Weight(fmt, HS, d, gs),
                      up_sh=gpu.Weight(fmt, HS, d, us), down_sh=gpu.Weight(fmt, d, HS, ds))
            okw = dict(hidden_shared=HS, shared_gate_bits=sg.view(np.uint16), gate_sh=gs, up_sh=us, down_sh=ds)
        moe = gpu.Moe(gpu.Weight("f16", E, d, router), gpu.Weight(fmt, H, d, gate, experts=E),
                      gpu.Weight(fmt, H, d, up, experts=E), gpu.Weight(fmt, d, H, down, experts=E), top,
                      scoring=c["scoring"], renormalize=c["renorm"], **kw)
        if c["xdt"] == "f16":
            xh = synth.activations_f16(m * d, seed=s + 8).reshape(m, d)
            x32 = synth.fp16_to_f32(xh)
        else:
            xh = synth.activations_f32(m * d, seed=s + 8).reshape(m, d)
            x32 = xh
        y, route = moe(xh if m > 1 else xh[0])
        y, route = np.reshape(y, (m, d)), np.reshape(route, (m, E))
        for p in range(m):
            y_ref, rw_ref = oracle.moe_f64(fmt, d, E, top, H, router.view(np.uint16), gate, up, down,
                                           x32[p].astype(np.float64), scoring=c["scoring"],
                                           renormalize=c["renorm"], **okw)
            assert np.array_equal(route[p] != 0, rw_ref != 0), (c, p)
            assert np.allclose(route[p], rw_ref, rtol=1e-5, atol=1e-7), (c, p)
            assert _rel(y[p], y_ref) <= 1e-3, (c, p, _rel(y[p], y_ref))
            if m > 1:
                y1, r1 = moe(xh[p])
                assert np.array_equal(y1, y[p]) and np.array_equal(r1, route[p]), (c, p)


def test_random_moe_configurations(gpu):
    run_cases(gpu, 8, seed=5)
