"""Writes the small golden fixtures under tests/golden/ from the CPU oracle.

Each fixture holds seeded GGUF weight bytes, activations, and what the oracle
computes for them: the fp32 dequantized weights, the exact (f64) matvec and
recipe's fp32-accumulate matvec, and for the MoE case the routing weights and
output. The oracle is pinned by tests/test_oracle.py; these files freeze its
answers so that a later change to the oracle or to the GPU path is caught
against fixed data.

Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "recipe-dev_amd")]

import oracle  # noqa: E402
from rqmv import synth  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))

# (format, rows, cols): Q8_0/Q4_0 with an odd block count, K-quants with two superblocks
MATVEC_CASES = [("q8_0", 8, 288), ("q4_0", 8, 288), ("q4_k", 8, 512), ("q6_k", 8, 512), ("f16", 8, 256)]


def matvec_fixture(fmt, rows, cols, seed=23):
    w = synth.weights(fmt, rows, cols, seed=seed, tag="golden-w") if fmt != "f16" else \
        synth.f16_weights(rows, cols, 0.05, seed=seed, tag="golden-w")
    x_bits = synth.activations_f16(2 * cols, seed=seed, tag="golden-x").reshape(2, cols)
    x32 = synth.fp16_to_f32(x_bits)
    wb = np.ascontiguousarray(w).view(np.uint8).reshape(-1)
    deq = oracle.dequant_rows(fmt, wb, rows, cols).astype(np.float32)
    y64 = np.stack([oracle.matvec_f64(fmt, wb, rows, cols, x32[m].astype(np.float64)) for m in range(2)])
    y32 = oracle.matvec_recipe_f32(fmt, wb, rows, cols, x32)
    np.savez_compressed(os.path.join(HERE, f"matvec_{fmt}.npz"), fmt=np.array(fmt), rows=rows, cols=cols, w=wb,
                        x_bits=x_bits, deq=deq, y64=y64, y32=y32)


def moe_fixture(seed=29):
    fmt, d, E, top, H = "q8_0", 128, 6, 2, 64
    router = synth.f16_weights(E, d, 0.02, seed=seed, tag="golden-router")
    gate = synth.weights(fmt, E * H, d, seed=seed + 1, tag="golden-gate")
    up = synth.weights(fmt, E * H, d, seed=seed + 2, tag="golden-up")
    down = synth.weights(fmt, E * d, H, seed=seed + 3, tag="golden-down")
    sg = synth.f16_weights(1, d, 0.02, seed=seed + 4, tag="golden-sg")
    gs = synth.weights(fmt, H, d, seed=seed + 5, tag="golden-gs")
    us = synth.weights(fmt, H, d, seed=seed + 6, tag="golden-us")
    ds = synth.weights(fmt, d, H, seed=seed + 7, tag="golden-ds")
    x_bits = synth.activations_f16(d, seed=seed, tag="golden-moe-x")
    x64 = synth.fp16_to_f32(x_bits).astype(np.float64)
    y, rw = oracle.moe_f64(fmt, d, E, top, H, router.view(np.uint16), gate, up, down, x64, scoring=0,
                           renormalize=True, hidden_shared=H, shared_gate_bits=sg.view(np.uint16), gate_sh=gs,
                           up_sh=us, down_sh=ds)
    np.savez_compressed(os.path.join(HERE, "moe_q8_0.npz"), fmt=np.array(fmt), d=d, experts=E, top=top, hidden=H,
                        router=router.view(np.uint16), gate=gate, up=up, down=down, shared_gate=sg.view(np.uint16),
                        gate_sh=gs, up_sh=us, down_sh=ds, x_bits=x_bits, y=y, route=rw)


if __name__ == "__main__":
    for case in MATVEC_CASES:
        matvec_fixture(*case)
    moe_fixture()
    print("wrote", sorted(f for f in os.listdir(HERE) if f.endswith(".npz")))
