"""Pins the oracle's restatement of recipe's int(8) sum (oracle.c, orc_q8_records
and orc_int8_matvec; amd-nv-cpu.ll:1231-2241, build.rs:743-915).

The reference holds no golden vectors for this path and its IR needs recipe's
Rust build to run, so the pins are: hand-worked record cases (round half to
even, the sign convention, the tie rules), the records' error bound, exact
cases where every fp32 operation is exact so the result must equal the f64
product of the dequantized weights and the coded activations (a dropped term,
a wrong scale or record index fails them), cases whose answer depends on the
summation order (the lane partition and the butterfly), and consistency of the
256-step Q4_K batch rule."""
import numpy as np
import pytest

import oracle
from rqmv import synth

F16_2M6 = np.float16(2.0 ** -6).view(np.uint16)


# ------------------------------------------------------------- records ----

def test_records_round_half_to_even_and_sign():
    x = np.zeros(32, np.float32)
    x[:7] = [127.0, 2.5, 3.5, -2.5, 0.5, 1.5, -126.5]
    d, codes = oracle.q8_records(x, 32)
    # extreme 127 -> inverse -1 exactly, d = -1; codes are -x rounded half to even
    assert d[0] == np.float32(-1.0)
    assert list(codes[:7]) == [-127, -2, -4, 2, 0, -2, 126]
    assert not codes[7:].any()


def test_records_tie_prefers_the_positive_extreme():
    x = np.zeros(32, np.float32)
    x[3], x[20] = -5.0, 5.0
    d, codes = oracle.q8_records(x, 32)
    assert codes[20] == -127 and codes[3] == 127 and d[0] < 0
    x[3], x[20] = 5.0, -5.0
    d2, codes2 = oracle.q8_records(x, 32)
    assert codes2[3] == -127 and d2[0] == d[0]


def test_records_256_step_lane_keeps_its_first_extreme():
    # lane 0 meets -5 (block 0) before +5 (block 1) and keeps -5; no other lane
    # holds a 5, so the step's extreme is -5 (amd-nv-cpu.ll:1422-1440).
    x = np.zeros(256, np.float32)
    x[0], x[32] = -5.0, 5.0
    d, codes = oracle.q8_records(x, 256)
    assert codes[0] == -127 and codes[32] == 127 and d[0] > 0
    # +5 in another lane wins the cross-lane tie.
    x[1] = 5.0
    d, codes = oracle.q8_records(x, 256)
    assert codes[1] == -127 and d[0] < 0
    assert np.all(d == d[0])  # one step shared by the eight records


def test_records_zero_step():
    x = np.zeros(64, np.float32)
    x[40] = 3.0
    d, codes = oracle.q8_records(x, 32)
    assert d[0] == 0 and not codes[:32].any()
    assert d[1] != 0 and codes[40] == -127


@pytest.mark.parametrize("step", [32, 256])
def test_records_error_bound(step):
    x = synth.activations_f32(4096 + 96, seed=11) * 3.0
    d, codes = oracle.q8_records(x, step)
    dd = np.repeat(d.astype(np.float64), 32)
    err = np.abs(codes.astype(np.float64) * dd - x.astype(np.float64))
    assert np.all(err <= np.abs(dd) * (0.5 + 2.0 ** -18))
    span = step // 32
    for g in range(0, x.size // 32, span):
        seg = x[g * 32:min(x.size, (g + span) * 32)]
        i = int(np.argmax(np.abs(seg)))
        assert abs(int(codes[g * 32 + i])) == 127
        assert np.all(d[g:g + span] == d[g])


# -------------------------------------------------------- exact cases ----

def _exact_x(cols: int, step: int, seed: int) -> np.ndarray:
    """Codes in [-4, 4] times a power-of-two step per group, one +-127 per group:
    every record's extreme is 127 times its power of two, so the records are exact."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(-4, 5, cols).astype(np.float64)
    x = np.empty(cols, np.float64)
    for g0 in range(0, cols, step):
        g1 = min(cols, g0 + step)
        codes[g0 + rng.integers(0, g1 - g0)] = 127.0 * rng.choice([-1.0, 1.0])
        x[g0:g1] = codes[g0:g1] * 2.0 ** int(rng.integers(-2, 1))
    return x.astype(np.float32)


def _exact_weights(fmt: str, rows: int, cols: int, seed: int) -> np.ndarray:
    """Synthetic blocks with power-of-two block scales and small sub-scales, so
    that every fp32 operation of the int(8) sum is exact at these sizes."""
    rng = np.random.default_rng(seed)
    w = synth.weights(fmt, rows, cols, seed=seed)
    if fmt in ("q8_0", "q4_0"):
        blk = w.reshape(-1, 34 if fmt == "q8_0" else 18)
        blk[:, 0:2] = np.full((blk.shape[0], 1), F16_2M6, np.uint16).view(np.uint8)
    elif fmt == "q4_k":
        blk = w.reshape(-1, 144)
        blk[:, 0:4] = np.full((blk.shape[0], 2), F16_2M6, np.uint16).view(np.uint8)
        sc = rng.integers(0, 16, (blk.shape[0], 8))
        mn = rng.integers(0, 16, (blk.shape[0], 8))
        blk[:, 4:16] = synth.pack_k_scales(sc, mn)
    else:
        blk = w.reshape(-1, 210)
        blk[:, 192:208] = rng.integers(-8, 8, (blk.shape[0], 16)).astype(np.int8).view(np.uint8)
        blk[:, 208:210] = np.full((blk.shape[0], 1), F16_2M6, np.uint16).view(np.uint8)
    return w


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("step", [32, 256])
def test_exact_cases_equal_the_f64_product(fmt, step):
    rows, cols = 24, 512
    w = _exact_weights(fmt, rows, cols, seed=5)
    xs = np.stack([_exact_x(cols, step, seed=s) for s in (1, 2, 3, 4, 5)])
    got = oracle.int8_matvec(fmt, w, rows, cols, xs, step)
    for m in range(xs.shape[0]):
        d, codes = oracle.q8_records(xs[m], step)
        used = codes.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
        assert np.array_equal(used, xs[m].astype(np.float64))  # the records are exact here
        want = oracle.matvec_f64(fmt, w, rows, cols, used[None, :])[0]
        assert np.array_equal(got[m].astype(np.float64), want), (fmt, step, m)


@pytest.mark.parametrize("fmt", ["q8_0", "q4_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("step", [32, 256])
def test_random_cases_within_fp32_bound(fmt, step):
    rows, cols = 16, 2048
    w = synth.weights(fmt, rows, cols, seed=8)
    x = synth.activations_f32(cols, seed=9)
    got = oracle.int8_matvec(fmt, w, rows, cols, x[None, :], step)[0].astype(np.float64)
    d, codes = oracle.q8_records(x, step)
    used = codes.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
    want = oracle.matvec_f64(fmt, w, rows, cols, used[None, :])[0]
    deq = oracle.dequant_rows(fmt, w, rows, cols).astype(np.float64)
    scale = np.abs(deq) @ np.abs(used)
    assert np.all(np.abs(got - want) <= scale * 2.0 ** -19), (fmt, step)


# ------------------------------------------------------ summation order ----

def _q8_0_row(cols: int, slices: dict) -> tuple:
    """A one-row Q8_0 weight and an activation column whose slice values are the
    given powers of two: slice s (block s//2, half s%2) gets one weight against
    a code of 64, the block's d chosen so the slice's value is exactly v; every
    touched block holds 127 in a weight-free place so its record step is -1."""
    nb = cols // 32
    blk = np.zeros((nb, 34), np.uint8)
    x = np.zeros(cols, np.float32)
    for s, v in slices.items():
        b, h = divmod(s, 2)
        d, w = (2.0 ** 12, -64 if v > 0 else 64) if abs(v) == 2 ** 24 else (2.0 ** -6, -1 if v > 0 else 1)
        blk[b, 0:2] = np.array([np.float16(d)]).view(np.uint8)
        blk[b, 2 + h * 16] = np.int8(w).view(np.uint8)
        x[b * 32 + h * 16] = -64.0
        x[b * 32 + (1 - h) * 16 + 5] = 127.0
    return blk.reshape(-1), x


def test_butterfly_pairs_lane_16_with_lane_0_first():
    # v0 = 2^24, v2 = 1, v16 = -2^24: the butterfly adds lanes 0 and 16 first
    # (exactly 0), then lane 2's 1 -> 1; a sequential sum loses the 1 -> 0.
    w, x = _q8_0_row(512, {0: 2 ** 24, 2: 1, 16: -2 ** 24})
    assert oracle.int8_matvec("q8_0", w, 1, 512, x[None, :], 32)[0, 0] == 1.0


def test_lane_partition_adds_slice_32_on_lane_0():
    # lane 0 holds slices 0 and 32 (2^24 + 1 rounds to 2^24), lane 16 holds 16
    # and 48 (-2^24 + 1 is exact); they meet as 1. A sequential sum gives 2.
    w, x = _q8_0_row(1024, {0: 2 ** 24, 32: 1, 16: -2 ** 24, 48: 1})
    assert oracle.int8_matvec("q8_0", w, 1, 1024, x[None, :], 32)[0, 0] == 1.0


# ------------------------------------------------ 256-step Q4_K batches ----

def test_q4k_256_batch_rule():
    rows, cols = 64, 1024
    w = synth.q4_k(rows, cols, seed=21)
    xs = np.stack([synth.activations_f32(cols, seed=30 + m) for m in range(5)])
    single = np.stack([oracle.int8_matvec("q4_k", w, rows, cols, xs[m:m + 1], 256)[0] for m in range(5)])
    batch = oracle.int8_matvec("q4_k", w, rows, cols, xs, 256)
    # positions 0..3 take four fmas per block; position 4 (past 4*(5//4)) the whole block
    assert np.array_equal(batch[4], single[4])
    assert not np.array_equal(batch[:4], single[:4])
    assert np.allclose(batch[:4], single[:4], rtol=1e-5, atol=1e-4)
    tail = oracle.int8_matvec("q4_k", w, rows, cols, xs[:4], 256, tail=True)
    assert np.array_equal(tail[3], single[3]) and np.array_equal(tail[:3], batch[:3])
    # the slice path (32 step) has no batch rule
    s32 = oracle.int8_matvec("q4_k", w, rows, cols, xs, 32)
    assert np.array_equal(s32[2], oracle.int8_matvec("q4_k", w, rows, cols, xs[2:3], 32)[0])


# ------------------------------------------------ 256-step Q6_K chains ----

def _q6k_block(codes: np.ndarray, scales, d: float) -> np.ndarray:
    """One Q6_K block from 256 six-bit codes (ggml's field positions)."""
    blk = np.zeros(210, np.uint8)
    for n, q in enumerate(codes):
        chunk, local, within = n // 128, (n % 128) // 32, n % 32
        blk[chunk * 64 + within + 32 * (local & 1)] |= (int(q) & 15) << (4 * (local >> 1))
        blk[128 + chunk * 32 + within] |= ((int(q) >> 4) & 3) << (2 * local)
    blk[192:208] = np.asarray(scales, np.int8).view(np.uint8)
    blk[208:210] = np.array([np.float16(d)]).view(np.uint8)
    return blk


def _q6k_chain_case(chain2: bool):
    """Block 0 (step -1 after records, d = 1): group 0's word 0 (values 0..3,
    codes 63 against -127) makes chain 0's word part -2048256 * scale 64.
    Without chain2 the group-0 code sums (sum part of chain 0) cancel it in the
    int; with chain2 they are zero and group 2 puts the opposite value on chain 2.
    Block 1 (d = 2^-6) puts a small value on chain 4 through group 4."""
    q0, s0 = np.zeros(256, np.int64), np.zeros(16, np.int64)
    x = np.zeros(512, np.float32)
    q0[0:4] = 63
    x[0:4] = 127.0
    s0[0] = 64
    if not chain2:
        x[4:16] = 41.0   # codes -41: group 0's sums reach -1000 with x[16]
        x[16] = 1.0
        s0[1] = 8
    else:
        x[16:20] = 127.0  # q = 0 there: only the sums, cancelling slice 0's
        s0[1] = -64
        q0[72:76] = 63
        x[72:76] = 127.0
        x[64:68] = 0.0
        s0[4], s0[5] = -64, 64
        x[80:84] = 127.0
    q1, s1 = np.zeros(256, np.int64), np.zeros(16, np.int64)
    q1[144] = 33
    s1[9] = 1
    x[256 + 144] = 1.0
    w = np.concatenate([_q6k_block(q0, s0, 1.0), _q6k_block(q1, s1, 2.0 ** -6)])
    return w, x


def test_q6k_256_chain_takes_its_words_and_its_group_sums():
    w, x = _q6k_chain_case(chain2=False)
    d, codes = oracle.q8_records(x, 256)
    assert d[0] == -1.0 and codes[0] == -127 and codes[16] == -1
    got = oracle.int8_matvec("q6_k", w, 1, 512, x[None, :], 256)[0, 0]
    # chain 0 cancels in its int; chain 4 alone is nonzero
    small = np.float32(np.float32(d[8] * np.float32(2.0 ** -6)) * np.float32(-127.0))
    assert got == small and small != 0


def test_q6k_256_chains_meet_in_the_fixed_tree():
    w, x = _q6k_chain_case(chain2=True)
    # chains 0 and 2 hold +-2048256 and chain 4 a value below their half ulp:
    # (f0 + f4) rounds to f0 and meets f2 + f6 = -f0 -> 0; a sequential sum of
    # the chains keeps the small value.
    assert oracle.int8_matvec("q6_k", w, 1, 512, x[None, :], 256)[0, 0] == 0.0


@pytest.mark.parametrize("fmt", ["q4_k", "q6_k"])
def test_256_step_blocks_meet_their_accumulator_with_fma(fmt):
    """Block 1 repeats block 0's weights against the negated activations: its
    codes are the same and its step the opposite, so its product is -P for
    block 0's P. A fused multiply-add leaves P's rounding error (nonzero, below
    half an ulp of P per chain); a rounded product added separately leaves exactly 0."""
    rows = 8
    one = synth.weights(fmt, rows, 256, seed=41).reshape(rows, -1)
    if fmt == "q4_k":
        sc = synth.uniform_int(41, "sc", rows * 8, 1, 63).reshape(rows, 8)
        one[:, 4:16] = synth.pack_k_scales(sc, np.zeros_like(sc))  # no minimum chain
    w = np.concatenate([one, one], axis=1).reshape(-1)
    half = synth.activations_f32(256, seed=42)
    x = np.concatenate([half, -half])
    got = oracle.int8_matvec(fmt, w, rows, 512, x[None, :], 256)[0].astype(np.float64)
    d, codes = oracle.q8_records(half, 256)
    used = codes.astype(np.float64) * np.repeat(d.astype(np.float64), 32)
    terms = np.abs(oracle.dequant_rows(fmt, one.reshape(-1), rows, 256).astype(np.float64)) @ np.abs(used)
    assert np.count_nonzero(got) >= rows - 1
    assert np.all(np.abs(got) <= terms * 2.0 ** -21)


# ------------------------------------------- Q8_0 storage under int(8) ----

def test_fp16_rne_matches_ieee():
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2 ** 32, 200000, dtype=np.uint64).astype(np.uint32)
    vals = bits.view(np.float32)
    vals = vals[np.isfinite(vals)]
    edge = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 1e9, 2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001,
                     2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -12), 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 3.0e-8],
                    np.float32)
    for v in np.concatenate([vals, edge, -edge]):
        want = np.array([v], np.float32).astype(np.float16).view(np.uint16)[0]
        assert oracle.lib().orc_fp16_rne(float(v)) == want, v


def _q8_block(d, codes):
    return np.concatenate([np.array([np.float16(d)]).view(np.uint8), np.asarray(codes, np.int8).view(np.uint8)])


def test_requantize_rounds_half_away_through_fp32():
    # An F16 row holding 127 (scale 1, inverse 1) and halves: 2.5 -> 3, -2.5 -> -3,
    # 1.5 -> 2, -0.5 -> -1 (round half away from zero, recipe.rs:8023, 8072-8078).
    v = np.zeros(32, np.float32)
    v[:6] = [127.0, 2.5, -2.5, 1.5, -0.5, -127.0]
    out = oracle.requantize_q8_0("f16", v.astype(np.float16).view(np.uint8), 1, 32)
    assert out[:2].view(np.float16)[0] == 1.0
    assert list(out[2:8].view(np.int8)) == [127, 3, -3, 2, -1, -127]
    # A Q8_0 source holding 127 and -128 (d = 1): the extreme is -128, the scale
    # 128/127; 127 * (1/scale) = 126.0078 -> 126, -128 -> -127; d = fp16(128/127).
    out = oracle.requantize_q8_0("q8_0", _q8_block(1.0, [127, -128] + [0] * 30), 1, 32)
    assert out[:2].view(np.float16)[0] == np.float16(np.float32(128.0) / np.float32(127.0))
    assert list(out[2:4].view(np.int8)) == [126, -127]


def test_requantize_q8_0_is_idempotent_on_full_range_blocks():
    rng = np.random.default_rng(9)
    blocks = []
    for _ in range(64):
        codes = rng.integers(-127, 128, 32)
        codes[rng.integers(0, 32)] = rng.choice([-127, 127])
        d = np.float16(np.abs(rng.standard_normal()) * 0.01 + 1e-3)
        blocks.append(_q8_block(d, codes))
    w = np.concatenate(blocks)
    assert np.array_equal(oracle.requantize_q8_0("q8_0", w, 8, 256), w)


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "f16"])
def test_requantize_error_bound(fmt):
    rows, cols = 12, 512
    w = synth.f16_weights(rows, cols, 0.02, seed=3) if fmt == "f16" else synth.weights(fmt, rows, cols, seed=3)
    out = oracle.requantize_q8_0(fmt, w, rows, cols)
    src = (synth.fp16_to_f32(w.view(np.uint16)).reshape(rows, cols) if fmt == "f16"
           else oracle.dequant_rows(fmt, w, rows, cols)).astype(np.float64)
    back = oracle.dequant_rows("q8_0", out, rows, cols).astype(np.float64)
    blk = out.reshape(-1, 34)
    d16 = blk[:, :2].copy().view(np.float16).astype(np.float64).reshape(rows, cols // 32)
    scale = np.abs(src.reshape(rows, cols // 32, 32)).max(axis=2) / 127.0
    codes = blk[:, 2:].view(np.int8).astype(np.float64).reshape(rows, cols // 32, 32)
    # the codes are the scaled values rounded to within half a step (the step before its fp16 rounding) ...
    assert np.all(np.abs(codes * scale[..., None] - src.reshape(rows, cols // 32, 32)) <= scale[..., None] * (0.5 + 1e-5))
    # ... and the block's largest value takes code +-127
    assert np.all(np.abs(codes).max(axis=2) == 127)
    # the stored step is the fp16 rounding of the scale
    assert np.array_equal(d16, scale.astype(np.float32).astype(np.float16).astype(np.float64))
    assert np.allclose(back, src, atol=np.abs(src).max() / 127 * 0.51)
