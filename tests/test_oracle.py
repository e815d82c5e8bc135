"""Pins the CPU oracle (oracle/oracle.c) against formulations that do not share
its code: IEEE binary16 in numpy, exact rational arithmetic, ggml's textbook
loop-form block decoders, recipe's own Q8_0 known answer (suite.rs:186-193),
the independent Q4_K x Q8_1 algebra of evidence/2026-10-10-m60-p2p/bench.rs,
brute force, and invariants that a dropped term or a swapped index breaks."""
import math
from fractions import Fraction

import numpy as np
import pytest

import oracle
from rqmv import synth


# ---------------------------------------------------------------- fp16 ----

def test_unfp16_matches_ieee_binary16_exhaustively():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib().orc_f32_from_fp16(int(b)) for b in bits], dtype=np.float32)
    finite = ~np.isnan(ref)
    assert np.array_equal(got[finite].view(np.uint32), ref[finite].view(np.uint32))
    assert np.isnan(got[~finite]).all()


def _fp16_rational_model(x: float) -> int:
    """recipe.rs:15098-15113 stated arithmetically for finite |x| < 65504 + half an ulp."""
    f = Fraction(x)
    sign = 0x8000 if math.copysign(1.0, x) < 0 else 0
    a = abs(f)
    if a == 0:
        return sign
    if a < Fraction(1, 2 ** 14):
        # truncate to 2^-37, then round half to even on the 2^-24 grid
        v = (a * 2 ** 37).numerator // (a * 2 ** 37).denominator
        q, r = divmod(v, 2 ** 13)
        if r > 2 ** 12 or (r == 2 ** 12 and q & 1):
            q += 1
        return sign | q
    # normal: round half to even to 11 significant bits
    e = 0
    while a >= 2:
        a /= 2
        e += 1
    while a < 1:
        a *= 2
        e -= 1
    m = a * 1024
    q = m.numerator // m.denominator
    r = m - q
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and q & 1):
        q += 1
    if q == 2048:
        q, e = 1024, e + 1
    if e + 15 >= 31:
        return sign | 0x7C00
    return sign | ((e + 15) << 10) | (q - 1024)


def test_fp16_conversion_against_rational_model_and_numpy():
    rng = np.random.default_rng(5)
    normal = rng.standard_normal(3000).astype(np.float32) * np.float32(3.0)
    tiny = (rng.standard_normal(3000) * 2.0 ** -16).astype(np.float32)  # subnormal fp16 range
    edge = np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 6.1035156e-05, 5.9604645e-08, 2.9802322e-08,
                     2.9802326e-08, 8.940697e-08, -1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11], dtype=np.float32)
    vals = np.concatenate([normal, tiny, edge])
    got = oracle.fp16_from_f32(vals)
    model = np.array([_fp16_rational_model(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, model)
    # on the normal range the conversion is IEEE round-half-even
    assert np.array_equal(got[:3000], normal.astype(np.float16).view(np.uint16))
    # the vectorised restatement used by the workload generator agrees
    assert np.array_equal(synth.fp16_bits(vals), got)


def test_fp16_large_values_follow_recipe():
    # finite values at 2^16 and beyond: inf when the f32 mantissa is zero, NaN bits otherwise
    vals = np.array([65536.0, 70000.0, -131072.0, 1e30, np.inf, -np.inf], dtype=np.float32)
    got = oracle.fp16_from_f32(vals)
    assert list(got) == [0x7C00, 0x7C01, 0xFC00, 0x7C01, 0x7C00, 0xFC00]
    assert np.array_equal(synth.fp16_bits(vals), got)


# ------------------------------------------------------- textbook decode ----

def _h(b2):
    return b2.copy().view(np.float16).astype(np.float64).reshape(-1)


def ggml_q8_0(raw, n):
    blk = raw.reshape(-1, 34)
    d = _h(blk[:, 0:2])
    q = blk[:, 2:].view(np.int8).astype(np.float64)
    return (q * d[:, None]).reshape(-1)


def ggml_q4_0(raw, n):
    blk = raw.reshape(-1, 18)
    d = _h(blk[:, 0:2])
    qs = blk[:, 2:].astype(np.int64)
    y = np.empty((blk.shape[0], 32))
    for j in range(16):
        y[:, j] = ((qs[:, j] & 0x0F) - 8) * d
        y[:, j + 16] = ((qs[:, j] >> 4) - 8) * d
    return y.reshape(-1)


def _scale_min_k4(j, q):
    if j < 4:
        return q[:, j] & 63, q[:, j + 4] & 63
    return (q[:, j + 4] & 0xF) | ((q[:, j - 4] >> 6) << 4), (q[:, j + 4] >> 4) | ((q[:, j] >> 6) << 4)


def ggml_q4_k(raw, n):
    blk = raw.reshape(-1, 144)
    d, dmin = _h(blk[:, 0:2]), _h(blk[:, 2:4])
    scales = blk[:, 4:16].astype(np.int64)
    qs = blk[:, 16:].astype(np.int64)
    y = np.empty((blk.shape[0], 256))
    is_ = 0
    for j in range(0, 256, 64):
        q = qs[:, (j // 64) * 32:(j // 64) * 32 + 32]
        sc, m = _scale_min_k4(is_, scales)
        d1, m1 = d * sc, dmin * m
        sc, m = _scale_min_k4(is_ + 1, scales)
        d2, m2 = d * sc, dmin * m
        y[:, j:j + 32] = d1[:, None] * (q & 0xF) - m1[:, None]
        y[:, j + 32:j + 64] = d2[:, None] * (q >> 4) - m2[:, None]
        is_ += 2
    return y.reshape(-1)


def ggml_q6_k(raw, n):
    blk = raw.reshape(-1, 210)
    d = _h(blk[:, 208:210])
    out = np.empty((blk.shape[0], 256))
    for half in range(2):
        ql = blk[:, 64 * half:64 * half + 64].astype(np.int64)
        qh = blk[:, 128 + 32 * half:128 + 32 * half + 32].astype(np.int64)
        sc = blk[:, 192 + 8 * half:192 + 8 * half + 8].view(np.int8).astype(np.int64)
        y = out[:, 128 * half:128 * half + 128]
        for l in range(32):
            is_ = l // 16
            q1 = ((ql[:, l] & 0xF) | (((qh[:, l] >> 0) & 3) << 4)) - 32
            q2 = ((ql[:, l + 32] & 0xF) | (((qh[:, l] >> 2) & 3) << 4)) - 32
            q3 = ((ql[:, l] >> 4) | (((qh[:, l] >> 4) & 3) << 4)) - 32
            q4 = ((ql[:, l + 32] >> 4) | (((qh[:, l] >> 6) & 3) << 4)) - 32
            y[:, l] = d * sc[:, is_] * q1
            y[:, l + 32] = d * sc[:, is_ + 2] * q2
            y[:, l + 64] = d * sc[:, is_ + 4] * q3
            y[:, l + 96] = d * sc[:, is_ + 6] * q4
    return out.reshape(-1)


TEXTBOOK = {"q8_0": ggml_q8_0, "q4_0": ggml_q4_0, "q4_k": ggml_q4_k, "q6_k": ggml_q6_k}


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_dequant_bit_exact_against_ggml_textbook(fmt):
    rows, cols = 48, 512
    w = synth.weights(fmt, rows, cols, seed=3)
    got = oracle.dequant_rows(fmt, w, rows, cols).reshape(-1)
    ref = TEXTBOOK[fmt](w, rows * cols).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_dequant_with_extreme_scales(fmt):
    """Subnormal, zero, negative and large fp16 scales, all code values."""
    rows, cols = 16, 256
    w = synth.weights(fmt, rows, cols, seed=11).copy()
    bv, bb = synth.BLOCK[fmt]
    blk = w.reshape(-1, bb)
    scale_bits = np.array([0x0001, 0x03FF, 0x0000, 0x8001, 0x7BFF, 0xFBFF, 0x3C00, 0x2400], dtype=np.uint16)
    at = 208 if fmt == "q6_k" else 0
    for i in range(blk.shape[0]):
        blk[i, at:at + 2] = scale_bits[i % 8:i % 8 + 1].view(np.uint8)
        if fmt == "q4_k":
            blk[i, 2:4] = scale_bits[(i + 3) % 8:(i + 3) % 8 + 1].view(np.uint8)
    got = oracle.dequant_rows(fmt, w, rows, cols).reshape(-1)
    ref = TEXTBOOK[fmt](w, rows * cols).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_q4k_every_scale_and_minimum_code():
    """All 64 x 64 (scale, minimum) codes in every sub-block position round-trip
    through the k_scale packing (recipe.rs:15204-15210)."""
    sc = np.array([[(i + j) % 64 for j in range(8)] for i in range(64)], dtype=np.int64)
    for mshift in range(0, 64, 7):
        mn = (sc * 5 + mshift) % 64
        blk = np.zeros((64, 144), np.uint8)
        blk[:, 0:2] = np.uint16(0x3C00).reshape(1).view(np.uint8)  # d = 1
        blk[:, 2:4] = np.uint16(0x3800).reshape(1).view(np.uint8)  # dmin = 0.5
        blk[:, 4:16] = synth.pack_k_scales(sc, mn)
        blk[:, 16:] = 0x21  # low nibble 1, high nibble 2
        vals = oracle.dequant_rows("q4_k", blk.reshape(-1), 64, 256).reshape(64, 8, 32)
        q = np.array([1, 2] * 4)
        expect = sc * q[None, :] - 0.5 * mn
        assert np.array_equal(vals[:, :, 0], expect.astype(np.float32))
        assert (vals == vals[:, :, :1]).all()


def test_recipe_q8_0_known_answer():
    """recipe's stepper fixture (suite.rs:186-193): d = 0x2400 (2^-6), codes 32,
    96, -80, 48 per row decode to 0.5, 1.5, -1.25, 0.75."""
    blk = np.zeros((4, 34), np.uint8)
    for r, code in enumerate([32, 96, -80, 48]):
        blk[r, 0:2] = np.uint16(0x2400).reshape(1).view(np.uint8)
        blk[r, 2:] = np.int8(code).view(np.uint8)
    w = blk.reshape(-1)
    vals = oracle.dequant_rows("q8_0", w, 4, 32)
    assert np.array_equal(vals, np.repeat(np.array([[0.5], [1.5], [-1.25], [0.75]], np.float32), 32, axis=1))
    y = oracle.matvec_recipe_f32("q8_0", w, 4, 32, np.ones(32, np.float32))
    assert list(y[0]) == [16.0, 48.0, -40.0, 24.0]
    y64 = oracle.matvec_f64("q8_0", w, 4, 32, np.ones(32))
    assert list(y64[0]) == [16.0, 48.0, -40.0, 24.0]


@pytest.mark.parametrize("source", ["xorshift", "synth"])
def test_q4k_against_bench_rs_q81_algebra(source):
    """A second reference-held algorithm for Q4_K: bench.rs's integer dot over
    Q8_1-style activation records with f64 block scales must equal the f64
    dequantized matvec on the same (quantized) activations."""
    rows, cols = 64, 4096
    if source == "xorshift":
        w = oracle.q4k_xorshift_rows(0x1234567, rows, 0x2400)
    else:
        w = synth.q4_k(rows, cols, seed=21)
    x = synth.activations_f32(cols, seed=4)
    y_ref, x_used = oracle.q4k_q81_reference(w, rows, cols, x)
    y = oracle.matvec_f64("q4_k", w, rows, cols, x_used)[0]
    assert np.allclose(y, y_ref, rtol=2e-6, atol=1e-6 * np.abs(y_ref).max())


# ---------------------------------------------------------------- matvec ----

@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k", "f16"])
def test_matvec_f64_brute_force(fmt):
    rows, cols = 24, 512
    w = synth.f16_weights(rows, cols, 0.05, seed=2) if fmt == "f16" else synth.weights(fmt, rows, cols, seed=2)
    x = np.random.default_rng(1).standard_normal((3, cols))
    if fmt == "f16":
        W = w.view(np.float16).astype(np.float64).reshape(rows, cols)
    else:  # f64 weights: Q4_K's d*sc*q - dmin*m need not be an fp32 value
        W = TEXTBOOK[fmt](w, rows * cols).reshape(rows, cols)
    y = oracle.matvec_f64(fmt, w, rows, cols, x)
    assert np.allclose(y, x @ W.T, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_matvec_recipe_f32_close_to_f64(fmt):
    rows, cols = 64, 1024
    w = synth.weights(fmt, rows, cols, seed=8)
    x = synth.fp16_to_f32(synth.activations_f16(2 * cols, seed=9)).reshape(2, cols)
    y32 = oracle.matvec_recipe_f32(fmt, w, rows, cols, x)
    y64 = oracle.matvec_f64(fmt, w, rows, cols, x.astype(np.float64))
    rel = np.linalg.norm(y32 - y64) / np.linalg.norm(y64)
    assert rel < 1e-6
    # threaded rows give the identical result
    assert np.array_equal(oracle.matvec_recipe_f32(fmt, w, rows, cols, x, threads=5), y32)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("rows,m,threads", [(1, 1, 1), (13, 2, 1), (77, 3, 4), (300, 1, 7)])
def test_matvec_recipe_fast_bit_identical(fmt, rows, m, threads):
    """The timed CPU baseline (recipe's compiled schedule: eight rows per lane
    group, headers decoded once per block) gives the per-value path's bits,
    ragged row groups and extreme activations included."""
    cols = 768
    rng = np.random.default_rng(rows * 10 + m)
    w = synth.weights(fmt, rows, cols, seed=rows + m)
    x = (rng.standard_normal((m, cols)) * 10.0 ** rng.integers(-3, 4, (m, cols))).astype(np.float32)
    want = oracle.matvec_recipe_f32(fmt, w, rows, cols, x)
    got = oracle.matvec_recipe_fast(fmt, w, rows, cols, x, threads=threads)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
def test_matvec_scales_exactly_with_block_scale(fmt):
    """Doubling every fp16 block scale (exponent + 1) doubles y exactly."""
    rows, cols = 16, 512
    w = synth.weights(fmt, rows, cols, seed=12).copy()
    bv, bb = synth.BLOCK[fmt]
    blk = w.reshape(-1, bb)
    offs = [208] if fmt == "q6_k" else ([0, 2] if fmt == "q4_k" else [0])
    for o in offs:
        h = blk[:, o:o + 2].copy().view(np.uint16).reshape(-1)
        h = np.where((h & 0x7C00) != 0, h + 0x0400, h * 2).astype(np.uint16)  # subnormals double too
        blk[:, o:o + 2] = h.view(np.uint8).reshape(-1, 2)
    x = np.random.default_rng(3).standard_normal(cols)
    y1 = oracle.matvec_f64(fmt, synth.weights(fmt, rows, cols, seed=12), rows, cols, x)
    y2 = oracle.matvec_f64(fmt, w, rows, cols, x)
    assert np.array_equal(y2, 2 * y1)


def test_matvec_linear_and_row_independent():
    rows, cols = 32, 512
    w = synth.q6_k(rows, cols, seed=14)
    rng = np.random.default_rng(6)
    a, b = rng.standard_normal(cols), rng.standard_normal(cols)
    ya = oracle.matvec_f64("q6_k", w, rows, cols, a)
    yb = oracle.matvec_f64("q6_k", w, rows, cols, b)
    yab = oracle.matvec_f64("q6_k", w, rows, cols, 2 * a - 3 * b)
    assert np.allclose(yab, 2 * ya - 3 * yb, rtol=1e-12, atol=1e-11)
    # rows are independent: row 5 alone equals row 5 of the whole
    row = w.reshape(rows, -1)[5]
    assert np.allclose(oracle.matvec_f64("q6_k", row, 1, cols, a)[0, 0], ya[0, 5], rtol=0, atol=0)


# ------------------------------------------------------------------ topk ----

def _topk_brute(scores, top, scoring, renorm):
    order = np.argsort(-scores, kind="stable")  # ties: lower index first
    kept = np.sort(order[:top])
    out = np.zeros_like(scores)
    if scoring == 0:
        if renorm:
            m = scores[kept].max()
            e = np.exp(scores[kept] - m)
            out[kept] = e / e.sum()
        else:
            m = scores.max()
            e = np.exp(scores - m)
            out[kept] = e[kept] / e.sum()
    else:
        s = 1 / (1 + np.exp(-scores))
        out[kept] = s[kept] / (s[kept].sum() if renorm else 1.0)
    return out


@pytest.mark.parametrize("scoring", [0, 1])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_brute_force(scoring, renorm):
    rng = np.random.default_rng(scoring * 2 + renorm)
    for trial in range(20):
        e = int(rng.integers(4, 300))
        top = int(rng.integers(1, min(e, 16) + 1))
        s = np.round(rng.standard_normal(e), 1)  # many ties
        got = oracle.topk(s, top, scoring, renorm)
        ref = _topk_brute(s, top, scoring, renorm)
        assert np.array_equal(got != 0, ref != 0)
        assert np.allclose(got, ref, rtol=1e-13, atol=1e-15)


def _topk_biased_brute(scores, top, scoring, renorm, bias):
    """The selection by probability + bias (probability: the sigmoid, or the
    softmax over every expert), by a stable sort instead of repeated scans;
    the weights from the unbiased scores, as _topk_brute computes them."""
    if scoring == 0:
        e = np.exp(scores - scores.max())
        prob = e / e.sum()
    else:
        prob = 1 / (1 + np.exp(-scores))
    order = np.argsort(-(prob + bias), kind="stable")
    kept = np.sort(order[:top])
    out = np.zeros_like(scores)
    if scoring == 0:
        m = scores[kept].max() if renorm else scores.max()
        ex = np.exp(scores - m)
        out[kept] = ex[kept] / (ex[kept].sum() if renorm else ex.sum())
    else:
        sg = 1 / (1 + np.exp(-scores))
        out[kept] = sg[kept] / (sg[kept].sum() if renorm else 1.0)
    return out


@pytest.mark.parametrize("scoring", [0, 1])
@pytest.mark.parametrize("renorm", [True, False])
def test_topk_selection_bias_brute_force(scoring, renorm):
    """A selection bias changes which experts are kept, never the weights
    given to them (topk_key, amd-nv-cpu.ll:4653-4660)."""
    rng = np.random.default_rng(40 + scoring * 2 + renorm)
    changed = 0
    for trial in range(30):
        e = int(rng.integers(4, 300))
        top = int(rng.integers(1, min(e, 16) + 1))
        s = rng.standard_normal(e)
        bias = rng.standard_normal(e) * (0.5 if trial % 2 else 0.02)
        got = oracle.topk(s, top, scoring, renorm, bias=bias)
        ref = _topk_biased_brute(s, top, scoring, renorm, bias)
        assert np.array_equal(got != 0, ref != 0)
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-15)
        changed += not np.array_equal(got != 0, oracle.topk(s, top, scoring, renorm) != 0)
    assert changed > 5  # the bias does move the selection
    # equal keys: the lower expert wins; a bias that only lifts one expert's key above the others' picks it
    s = np.zeros(6)
    assert list(np.nonzero(oracle.topk(s, 2, scoring, renorm, bias=np.zeros(6)))[0]) == [0, 1]
    b = np.zeros(6)
    b[4] = 1e-3
    assert list(np.nonzero(oracle.topk(s, 2, scoring, renorm, bias=b))[0]) == [0, 4]


@pytest.mark.parametrize("name", ["linear", "relu", "sigmoid", "silu", "tanh", "gelu", "elu", "selu", "softplus",
                                  "leak", "exp", "cos", "sqrt", "ln", "log", "huber", "tan", "prelu", "scale"])
def test_activation_against_independent_forms(name):
    """The oracle's activation programs against torch's CPU implementations
    or textbook closed forms written differently (expit, logaddexp, erf-based
    GELU within the tanh approximation's known error)."""
    import torch
    import torch.nn.functional as F
    from scipy.special import erf, expit
    x = np.concatenate([np.linspace(-12, 12, 961), [0.0, -0.0, 1e-30, -1e-30, 40.0, -40.0]])
    if name in ("sqrt",):
        x = np.abs(x)
    got = oracle.activation(name, x, factor=0.3)
    t = torch.from_numpy(x)
    ref = {
        "linear": lambda: x,
        "relu": lambda: np.maximum(x, 0),
        "sigmoid": lambda: expit(x),
        "silu": lambda: x * expit(x),
        "tanh": lambda: np.tanh(x),
        "gelu": lambda: F.gelu(t, approximate="tanh").numpy(),
        "elu": lambda: F.elu(t).numpy(),
        "selu": lambda: F.selu(t).numpy(),
        "softplus": lambda: np.logaddexp(0, x),
        "leak": lambda: F.leaky_relu(t, 0.01).numpy(),
        "exp": lambda: np.exp(x),
        "cos": lambda: np.cos(x),
        "sqrt": lambda: np.sqrt(x),
        "ln": lambda: np.sign(x) * np.log1p(np.abs(x)),
        "log": lambda: np.sign(x) * np.log10(1 + np.abs(x)),
        "huber": lambda: np.where(np.abs(x) <= 1, 0.5 * x * x, np.abs(x) - 0.5),
        "tan": lambda: np.tan(x),
        "prelu": lambda: np.where(x > 0, x, 0.3 * x),
        "scale": lambda: 0.3 * x,
    }[name]()
    assert np.allclose(got, ref, rtol=1e-12, atol=1e-14), name
    if name == "gelu":  # the tanh form stays within 5e-4 of the exact erf GELU
        assert np.max(np.abs(got - 0.5 * x * (1 + erf(x / np.sqrt(2))))) < 5e-4


def test_activation_gelu_fp16_table():
    """Gelu under the gelu table: the fp16-rounded input through the tanh form,
    the result rounded to fp16, inside (-10, 10); x itself above 10, 0 below -10."""
    x = np.concatenate([np.linspace(-11, 11, 2201), [10.0, -10.0, 10.5, -10.5]])
    got = oracle.activation("gelu_fp16", x)
    h = x.astype(np.float16).astype(np.float64)
    inner = oracle.activation("gelu", h)
    ref = np.where(x > 10, x, np.where(x < -10, 0.0, inner.astype(np.float32).astype(np.float16).astype(np.float64)))
    assert np.array_equal(got, ref)
    assert np.array_equal(got[(x > -10) & (x < 10)].astype(np.float16).astype(np.float64), got[(x > -10) & (x < 10)])


# ------------------------------------------------------------------- moe ----

def test_moe_against_numpy_composition():
    d, E, top, H, HS = 256, 8, 2, 256, 512
    fmt = "q4_k"
    router = synth.f16_weights(E, d, 0.05, seed=1, tag="router")
    gate = synth.q4_k(E * H, d, seed=2, tag="gate")
    up = synth.q4_k(E * H, d, seed=3, tag="up")
    down = synth.q4_k(E * d, H, seed=4, tag="down")
    sg = synth.f16_weights(1, d, 0.05, seed=5, tag="sg")
    gs, us, ds = synth.q4_k(HS, d, seed=6, tag="gs"), synth.q4_k(HS, d, seed=7, tag="us"), synth.q4_k(d, HS, seed=8, tag="ds")
    x = synth.fp16_to_f32(synth.activations_f16(d, seed=9)).astype(np.float64)
    y, rw = oracle.moe_f64(fmt, d, E, top, H, router.view(np.uint16), gate, up, down, x, hidden_shared=HS,
                           shared_gate_bits=sg.view(np.uint16), gate_sh=gs, up_sh=us, down_sh=ds)
    R = synth.fp16_to_f32(router.view(np.uint16)).astype(np.float64).reshape(E, d)
    scores = R @ x
    w = _topk_brute(scores, top, 0, True)
    assert np.allclose(rw, w, rtol=1e-12)
    G = ggml_q4_k(gate, 0).reshape(E, H, d)
    U = ggml_q4_k(up, 0).reshape(E, H, d)
    D = ggml_q4_k(down, 0).reshape(E, d, H)
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    ref = np.zeros(d)
    for e in np.nonzero(w)[0]:
        ref += w[e] * (D[e] @ (silu(G[e] @ x) * (U[e] @ x)))
    SGv = synth.fp16_to_f32(sg.view(np.uint16)).astype(np.float64)
    g = 1 / (1 + np.exp(-(SGv @ x)))
    GS = ggml_q4_k(gs, 0).reshape(HS, d)
    US = ggml_q4_k(us, 0).reshape(HS, d)
    DS = ggml_q4_k(ds, 0).reshape(d, HS)
    ref += g * (DS @ (silu(GS @ x) * (US @ x)))
    assert np.allclose(y, ref, rtol=1e-10, atol=1e-10 * np.abs(ref).max())


@pytest.mark.parametrize("act,gate_act,biased,gated", [("gelu", "sigmoid", True, True), ("relu", "tanh", False, True),
                                                        ("silu", "linear", True, False)])
def test_moe_activation_bias_and_ungated_shared(act, gate_act, biased, gated):
    """gguf_moe's activation, the shared gate's activation, the selection
    bias and an ungated shared expert, against a numpy composition of the
    dequantized tensors (textbook decoders), torch's activations and the
    brute-force biased selection."""
    import torch
    import torch.nn.functional as F
    from scipy.special import expit
    d, E, top, H, HS = 256, 8, 3, 256, 256
    fmt = "q4_k"
    router = synth.f16_weights(E, d, 0.05, seed=11, tag="router")
    gate = synth.q4_k(E * H, d, seed=12, tag="gate")
    up = synth.q4_k(E * H, d, seed=13, tag="up")
    down = synth.q4_k(E * d, H, seed=14, tag="down")
    sg = synth.f16_weights(1, d, 0.05, seed=15, tag="sg")
    gs, us, ds = synth.q4_k(HS, d, seed=16, tag="gs"), synth.q4_k(HS, d, seed=17, tag="us"), synth.q4_k(d, HS, seed=18, tag="ds")
    x = synth.fp16_to_f32(synth.activations_f16(d, seed=19)).astype(np.float64)
    bias = np.random.default_rng(20).standard_normal(E) * 0.3 if biased else None
    y, rw = oracle.moe_f64(fmt, d, E, top, H, router.view(np.uint16), gate, up, down, x, scoring=1, hidden_shared=HS,
                           shared_gate_bits=sg.view(np.uint16) if gated else None, gate_sh=gs, up_sh=us, down_sh=ds,
                           activation=act, shared_gate_activation=gate_act, selection_bias=bias)
    R = synth.fp16_to_f32(router.view(np.uint16)).astype(np.float64).reshape(E, d)
    scores = R @ x
    w = _topk_biased_brute(scores, top, 1, True, bias) if biased else _topk_brute(scores, top, 1, True)
    assert np.allclose(rw, w, rtol=1e-12)
    torch_act = {"gelu": lambda v: F.gelu(torch.from_numpy(v), approximate="tanh").numpy(),
                 "relu": lambda v: np.maximum(v, 0), "silu": lambda v: v * expit(v), "sigmoid": expit,
                 "tanh": np.tanh, "linear": lambda v: v}
    G = ggml_q4_k(gate, 0).reshape(E, H, d)
    U = ggml_q4_k(up, 0).reshape(E, H, d)
    D = ggml_q4_k(down, 0).reshape(E, d, H)
    f = torch_act[act]
    ref = np.zeros(d)
    for e in np.nonzero(w)[0]:
        ref += w[e] * (D[e] @ (f(G[e] @ x) * (U[e] @ x)))
    SGv = synth.fp16_to_f32(sg.view(np.uint16)).astype(np.float64)
    g = float(torch_act[gate_act](np.array([SGv @ x]))[0]) if gated else 1.0
    GS = ggml_q4_k(gs, 0).reshape(HS, d)
    US = ggml_q4_k(us, 0).reshape(HS, d)
    DS = ggml_q4_k(ds, 0).reshape(d, HS)
    ref += g * (DS @ (f(GS @ x) * (US @ x)))
    assert np.allclose(y, ref, rtol=1e-10, atol=1e-10 * np.abs(ref).max())
