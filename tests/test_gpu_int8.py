"""GPU parity of recipe's int(8) sum: rqmv_matvec_int8 and rqmv_q8_records
against the oracle (orc_int8_matvec, orc_q8_records), bit for bit, through the
C ABI. Covers both steps (32: the default profile; 256: the llama.cpp profile),
the four block formats, ragged shapes (partial lane rounds, odd block counts,
a partial last 256-step group), batches with the 256-step Q4_K quarter rule and
the tail flag, the order-sensitive constructions of the oracle's pins, an
expert bank, and the full 14336 x 4096 projection."""
import numpy as np
import pytest

import oracle
from rqmv import synth
from test_oracle_int8 import _exact_weights, _exact_x, _q6k_chain_case, _q8_0_row

pytestmark = pytest.mark.gpu

FMTS = ["q8_0", "q4_0", "q4_k", "q6_k"]


def _bits_equal(got, want):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    return got.shape == want.shape and np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _shapes(fmt):
    if fmt in ("q4_k", "q6_k"):
        return [(1, 256), (17, 768), (300, 4096), (33, 5120)]
    return [(1, 32), (5, 96), (9, 160), (300, 4096), (33, 5120)]


@pytest.mark.parametrize("step", [32, 256])
def test_records_bit_exact(gpu, step):
    for k, seed in ((32, 1), (96, 2), (256, 3), (4096 + 96, 4), (14336, 5)):
        x = synth.activations_f32(k, seed=seed) * np.float32(2.5)
        x[::97] = 0.0
        if k >= 256:
            x[:32] = 0.0  # an all-zero record
        d, c = gpu.q8_records(x, step)
        dw, cw = oracle.q8_records(x, step)
        print(f"records step={step} k={k}", flush=True)
        assert _bits_equal(d, dw) and np.array_equal(c, cw), (step, k)


def test_records_tie_rules(gpu):
    x = np.zeros(256, np.float32)
    x[0], x[32] = -5.0, 5.0
    for step in (32, 256):
        d, c = gpu.q8_records(x, step)
        dw, cw = oracle.q8_records(x, step)
        assert _bits_equal(d, dw) and np.array_equal(c, cw), step
    x[1] = 5.0
    d, c = gpu.q8_records(x, 256)
    dw, cw = oracle.q8_records(x, 256)
    assert _bits_equal(d, dw) and np.array_equal(c, cw)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("step", [32, 256])
def test_matvec_int8_bit_exact(gpu, fmt, step):
    for rows, cols in _shapes(fmt):
        w = synth.weights(fmt, rows, cols, seed=rows * 3 + cols)
        W = gpu.Weight(fmt, rows, cols, w)
        for m in (1, 3):
            x = np.stack([synth.activations_f32(cols, seed=100 + i + cols) for i in range(m)])
            print(f"int8 {fmt} step={step} {rows}x{cols} m={m}", flush=True)
            got = gpu.contract_int8(W, x, step)
            want = oracle.int8_matvec(fmt, w, rows, cols, x, step)
            assert _bits_equal(got, want), (fmt, step, rows, cols, m)
        W.close()


@pytest.mark.parametrize("tail", [False, True])
def test_q4k_256_batch_rule_bit_exact(gpu, tail):
    rows, cols = 70, 1536
    w = synth.q4_k(rows, cols, seed=9)
    W = gpu.Weight("q4_k", rows, cols, w)
    for m in (4, 5, 6, 8):
        x = np.stack([synth.activations_f32(cols, seed=40 + i) for i in range(m)])
        got = gpu.contract_int8(W, x, 256, tail)
        want = oracle.int8_matvec("q4_k", w, rows, cols, x, 256, tail=tail)
        assert _bits_equal(got, want), (m, tail)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("step", [32, 256])
def test_exact_cases(gpu, fmt, step):
    rows, cols = 24, 512
    w = _exact_weights(fmt, rows, cols, seed=5)
    x = np.stack([_exact_x(cols, step, seed=s) for s in (1, 2, 3)])
    W = gpu.Weight(fmt, rows, cols, w)
    assert _bits_equal(gpu.contract_int8(W, x, step), oracle.int8_matvec(fmt, w, rows, cols, x, step))


def test_summation_order_cases(gpu):
    for cols, slices in ((512, {0: 2 ** 24, 2: 1, 16: -2 ** 24}), (1024, {0: 2 ** 24, 32: 1, 16: -2 ** 24, 48: 1})):
        w, x = _q8_0_row(cols, slices)
        W = gpu.Weight("q8_0", 1, cols, w)
        got = gpu.contract_int8(W, x[None, :], 32)
        assert got[0, 0] == 1.0 and _bits_equal(got, oracle.int8_matvec("q8_0", w, 1, cols, x[None, :], 32))
    for chain2 in (False, True):
        w, x = _q6k_chain_case(chain2)
        W = gpu.Weight("q6_k", 1, 512, w)
        got = gpu.contract_int8(W, x[None, :], 256)
        assert _bits_equal(got, oracle.int8_matvec("q6_k", w, 1, 512, x[None, :], 256)), chain2


def test_expert_bank_rows(gpu):
    experts, rows, cols = 4, 40, 1024
    w = synth.q4_k(experts * rows, cols, seed=13)
    bank = gpu.Weight("q4_k", rows, cols, w, experts=experts)
    x = synth.activations_f32(cols, seed=14)[None, :]
    for step in (32, 256):
        want = oracle.int8_matvec("q4_k", w, experts * rows, cols, x, step)
        assert _bits_equal(gpu.contract_int8(bank, x, step), want), step


@pytest.mark.parametrize("step", [32, 256])
def test_full_size_q4k_up_projection(gpu, step):
    rows, cols = 14336, 4096
    w = synth.q4_k(rows, cols, seed=2)
    W = gpu.Weight("q4_k", rows, cols, w)
    x = synth.activations_f32(cols, seed=3)[None, :]
    got = gpu.contract_int8(W, x, step)
    want = oracle.int8_matvec("q4_k", w, rows, cols, x, step)
    assert _bits_equal(got, want), step


def test_argument_errors(gpu):
    w = synth.q4_k(4, 256, seed=1)
    W = gpu.Weight("q4_k", 4, 256, w)
    xb = gpu.DeviceBuffer(4 * 256)
    yb = gpu.DeviceBuffer(4 * 4)
    for step, flags in ((64, False), (0, False)):
        with pytest.raises(gpu.RqmvError, match="step"):
            gpu.matvec_int8(W, xb, 1, 256, yb, 4, step, flags)
    with pytest.raises(gpu.RqmvError, match="ldx"):
        gpu.matvec_int8(W, xb, 1, 128, yb, 4, 32)
    F = gpu.Weight("f16", 4, 64, synth.f16_weights(4, 64, 0.02, seed=2))
    with pytest.raises(gpu.RqmvError, match="Q4_K, Q6_K, Q8_0 or Q4_0"):
        gpu.matvec_int8(F, xb, 1, 64, yb, 4, 32)


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "f16", "q8_0", "q4_k"])
@pytest.mark.parametrize("step", [32, 256])
def test_int8_profile_storage(gpu, fmt, step):
    """recipe's int(8) profile end to end: the weight in the storage the profile
    gives it (Q4_K and Q8_0 kept, F16/Q4_0/Q6_K re-encoded to Q8_0), then the
    int(8) product, bit for bit against the oracle's composition."""
    rows, cols = 96, 1024
    w = synth.f16_weights(rows, cols, 0.02, seed=6) if fmt == "f16" else synth.weights(fmt, rows, cols, seed=6)
    W = gpu.int8_weight(fmt, rows, cols, w)
    kept = fmt in ("q4_k", "q8_0")
    assert W.info()["format"] == (gpu.FORMATS[fmt] if kept else gpu.FORMATS["q8_0"])
    stored = w if kept else oracle.requantize_q8_0(fmt, w, rows, cols)
    sfmt = fmt if kept else "q8_0"
    x = np.stack([synth.activations_f32(cols, seed=20 + i) for i in range(2)])
    assert _bits_equal(gpu.contract_int8(W, x, step), oracle.int8_matvec(sfmt, stored, rows, cols, x, step))
    assert np.array_equal(W.unpack(), stored)
