"""The activation encoding of the integer kernels, restated on the CPU
(tests/stage_model.py): its error bound, and why one outlier per 32-value
block is taken out and multiplied exactly (host only, no device)."""
import numpy as np
import pytest

import stage_model as sm

RNG = np.random.default_rng(11)


def _rel(a, b):
    return float(np.linalg.norm(a - b) / np.linalg.norm(b))


@pytest.mark.parametrize("threshold", [None, 4.0])
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
    err_x = np.abs(sm.effective_row(x, 4.0) - x)
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
    extracted = _rel(W @ sm.effective_row(x, 4.0).astype(np.float64), y)
    assert plain > 1e-3
    assert extracted < 1e-4


def test_gaussian_blocks_never_extract():
    """N(0, 1) blocks essentially never have a largest magnitude 4x the
    second largest, so ordinary activations keep the plain encoding."""
    x = RNG.standard_normal(32 * 20000).astype(np.float32)
    hits = 0
    for b in range(0, x.size, 32):
        hits += sm.encode_block(x[b:b + 32], 4.0)[2] >= 0
    assert hits == 0


def test_ties_and_single_values():
    # two equal largest values: no outlier (the second largest equals the largest)
    x = np.zeros(32, np.float32)
    x[3] = x[9] = 5.0
    assert sm.encode_block(x, 4.0)[2] == -1
    # one nonzero value: it is the outlier and the rest encodes to zero, exactly
    x = np.zeros(32, np.float32)
    x[17] = -3.25
    eff, s, i, v = sm.encode_block(x, 4.0)
    assert i == 17 and v == np.float32(-3.25) and np.array_equal(eff, x)


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
