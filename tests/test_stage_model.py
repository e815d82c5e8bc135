"""The activation encoding of the integer kernels, restated on the CPU
(tests/stage_model.py): its error bound, and why up to four outliers per
32-value block are taken out and multiplied exactly (host only, no device)."""
import numpy as np
import pytest

import stage_model as sm

RNG = np.random.default_rng(11)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("threshold", [None, sm.RATIO])
def test_every_value_within_half_a_step(threshold):
    for scale in (1e-6, 1.0, 1e4):
        x = (RNG.standard_normal(4096) * scale).astype(np.float32)
        x[::97] *= 300  # a few outliers
        eff = sm.effective_row(x, threshold)
        bound = sm.block_bound(x, threshold)
        assert np.all(np.abs(eff.astype(np.float64) - x) <= bound)


def test_bound_is_relative_to_the_block_maximum_without_extraction():
    """Without extraction an outlier coarsens its whole block: the other
    values' error grows with the outlier, up to 1/61166 of it."""
    x = RNG.standard_normal(32).astype(np.float32)
    x[5] = 1000.0
    err = np.abs(sm.effective_row(x, None) - x)
    err[5] = 0
    assert err.max() > 1000.0 / 61166 / 4  # of the order of the outlier's step
    err_x = np.abs(sm.effective_row(x, sm.RATIO) - x)
    assert err_x[5] == 0.0  # exact
    assert err_x.max() <= np.abs(np.delete(x, 5)).max() / 61166 * 1.02


def test_outliers_on_zero_weight_columns_need_extraction():
    """The hard case: a 1000x outlier in every 32-block, on a column whose
    weights are all zero. Without extraction the other values' rounding
    (scaled by the outliers) is the whole error and exceeds the 1e-3 bar;
    with it the product stays near 1e-5."""
    rows, k = 64, 4096
    W = RNG.standard_normal((rows, k))
    x = RNG.standard_normal(k).astype(np.float32)
    cols = np.arange(0, k, 32) + RNG.integers(0, 32, k // 32)
    x[cols] *= 1000
    W[:, cols] = 0
    y = W @ x.astype(np.float64)
    plain = _rel(W @ sm.effective_row(x, None).astype(np.float64), y)
    extracted = _rel(W @ sm.effective_row(x, sm.RATIO).astype(np.float64), y)
    assert plain > 1e-3
    assert extracted < 1e-4


def test_gaussian_blocks_never_extract():
    """N(0, 1) blocks never have at most four values at or above 1/16 of
    their largest, so ordinary activations keep the plain encoding."""
    x = RNG.standard_normal(32 * 20000).astype(np.float32)
    hits = 0
    for b in range(0, x.size, 32):
        hits += len(sm.encode_block(x[b:b + 32], sm.RATIO)[2]) > 0
    assert hits == 0


def test_heavy_tailed_blocks_rarely_extract():
    """Heavy-tailed activations (a SiLU-gated product, the input of a
    gated FFN's down projection; Student-t with 3 degrees of freedom) have
    values taken out in under 1 % of their blocks: extraction is for
    outliers, not for tails, so these keep the fast path."""
    rng = np.random.default_rng(12)
    g, u = rng.standard_normal(32 * 4000) * 2, rng.standard_normal(32 * 4000) * 2
    for x in (g / (1 + np.exp(-g)) * u, rng.standard_t(3, 32 * 4000)):
        x = x.astype(np.float32)
        hits = sum(len(sm.encode_block(x[b:b + 32], sm.RATIO)[2]) > 0 for b in range(0, x.size, 32))
        assert hits < 0.01 * (x.size // 32)


def test_ties_and_single_values():
    # two equal largest values and nothing else: both are taken out, exactly
    x = np.zeros(32, np.float32)
    x[3] = x[9] = 5.0
    eff, s, taken, vals = sm.encode_block(x, sm.RATIO)
    assert taken == [3, 9] and np.array_equal(eff, x) and s == 0
    # one nonzero value: it is the outlier and the rest encodes to zero, exactly
    x = np.zeros(32, np.float32)
    x[17] = -3.25
    eff, s, taken, vals = sm.encode_block(x, sm.RATIO)
    assert taken == [17] and vals == [np.float32(-3.25)] and np.array_equal(eff, x)


def _zero_weight_outliers(per_block, scale, rng, ordinary_weights=False):
    """A 64 x 4096 product whose activations carry `per_block` outliers of
    `scale` times an N(0, 1) value in every 32-value block, on columns whose
    weights are all zero (or ordinary). Returns the rel-L2 of the product
    with and without extraction, against the exact product."""
    rows, k = 64, 4096
    W = rng.standard_normal((rows, k))
    x = rng.standard_normal(k).astype(np.float32)
    cols = np.concatenate([b + rng.choice(32, per_block, replace=False) for b in range(0, k, 32)])
    x[cols] *= np.float32(scale)
    if not ordinary_weights:
        W[:, cols] = 0
    y = W @ x.astype(np.float64)
    plain = _rel(W @ sm.effective_row(x, None).astype(np.float64), y)
    extracted = _rel(W @ sm.effective_row(x, sm.RATIO).astype(np.float64), y)
    return plain, extracted


@pytest.mark.parametrize("per_block,scale", [(1, 1000), (2, 100), (2, 1000), (3, 100), (3, 1000), (4, 1000)])
def test_several_outliers_per_block_on_zero_weight_columns(per_block, scale):
    """Up to four outliers per block, each on a column whose weights are
    zero: without extraction the other values' rounding (scaled by the
    outliers) is the whole error; with it the product stays near 1e-5, well
    inside 2e-4."""
    plain, extracted = _zero_weight_outliers(per_block, scale, np.random.default_rng(100 * per_block + scale))
    assert plain > 5e-4
    assert extracted < 2e-4


def test_outliers_on_ordinary_columns_stay_accurate():
    for per_block in (1, 2, 3, 5, 8):
        _, extracted = _zero_weight_outliers(per_block, 1000, np.random.default_rng(per_block), True)
        assert extracted < 1e-4


def test_nested_outliers_are_taken_out_in_rounds():
    """A block of ordinary values with one 1000x and one 50x value: the
    first round takes the 1000 alone (50 < 1000 / 16), the second the 50,
    and the rest is scaled by its own largest magnitude."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal(32).astype(np.float32)
    x[4], x[20] = 1000.0, -50.0
    eff, s, taken, vals = sm.encode_block(x, sm.RATIO)
    assert taken == [4, 20] and vals == [np.float32(1000.0), np.float32(-50.0)]
    rest = np.abs(np.delete(x, [4, 20])).max()
    assert s == np.float32(rest * sm.INV_XMAX)


def test_step_is_bounded_by_the_fifth_largest_magnitude():
    """Whatever the block: the scale is at most 16 / 30583 of the block's
    fifth largest magnitude (four slots, ratio 16), and every value keeps its
    half-step bound. Blocks with 0-8 outliers at mixed magnitudes."""
    rng = np.random.default_rng(9)
    for trial in range(3000):
        x = rng.standard_normal(32).astype(np.float32)
        n = rng.integers(0, 9)
        idx = rng.choice(32, n, replace=False)
        x[idx] *= (10.0 ** rng.uniform(0, 4, n)).astype(np.float32)
        if trial % 7 == 0:
            x[rng.choice(32, rng.integers(0, 28), replace=False)] = 0  # sparse blocks
        eff, s, taken, _ = sm.encode_block(x, sm.RATIO)
        fifth = np.sort(np.abs(x))[::-1][4]
        assert s <= np.float32(sm.RATIO) * fifth * sm.INV_XMAX * np.float32(1 + 2 ** -20) or s == np.float32(2.0 ** -126)
        assert len(taken) <= sm.SLOTS
        err = np.abs(eff.astype(np.float64) - x)
        assert np.all(err <= 0.51 * float(s) + 1e-45)
        assert np.all(err[taken] == 0)


def test_five_outliers_per_block_is_the_limit():
    """Five comparable outliers in a block exceed the four slots: the block
    is scaled by its fifth largest value at least (the stated limit of the
    encoding), so on zero-weight columns the error grows past the bar."""
    plain, extracted = _zero_weight_outliers(5, 1000, np.random.default_rng(55))
    assert extracted > 1e-3


def test_extreme_block_magnitudes():
    """Blocks at the ends of the fp32 range. The largest keep the half-step
    bound (the reciprocal of their step stays a normal float); blocks whose
    step would fall below the smallest normal float take the step 2^-126,
    so their values keep an absolute error of at most 2^-127."""
    for scale in (1e37, 7.5e37):
        x = (RNG.uniform(-1, 1, 32) * scale).astype(np.float32)
        eff, s, _, _ = sm.encode_block(x)
        assert np.isfinite(s) and s > 0
        assert np.all(np.abs(eff.astype(np.float64) - x) <= 0.51 * float(s))
    for scale in (1e-35, 1e-38, 1e-44):
        x = (RNG.uniform(-1, 1, 32) * scale).astype(np.float32)
        eff, s, _, _ = sm.encode_block(x)
        assert s == np.float32(2.0 ** -126)
        assert np.all(np.abs(eff.astype(np.float64) - x) <= 2.0 ** -127)
    eff, s, _, _ = sm.encode_block(np.zeros(32, np.float32))
    assert s == 0 and not eff.any()
