"""A CPU restatement of the activation encoding of the integer matvec
kernels (recipe-dev_amd/csrc/stage.h), test infrastructure.

Every 32-value block of an activation row becomes 16-bit integers
x_i = rint(v_i / s) with the block scale s = amax * fp32(1 / 30583) (2^-126 for
blocks whose step would fall below the smallest normal float), rounded once
from the exact product of v_i and 1 / s (the kernels form 1 / s with the
hardware reciprocal, within one ulp; the model divides); the kernels' products are exact integer dots of
these against the weights' integer codes, scaled per block in fp32, so the
activation a kernel multiplies is s * x_i. With outlier extraction, a block takes out its large values before it is
scaled: when at most `slots` (4) of its values are at or above amax / threshold
(amax its largest magnitude; threshold RATIO = 16), they go to the block's slots
(encoded as 0) and are multiplied exactly (in fp32) with their weights; the
test repeats on the values left, with their own largest magnitude, until the
slots are used up or more large values remain than slots are left. So the
block's scale is at most threshold / 30583 of its fifth largest magnitude.
The ratio is wide enough that heavy-tailed activations (a SiLU-gated product,
Student-t) almost never have values taken out (under 1 % of blocks), and
narrow enough that outliers 100x the rest always are.

The functions return the effective activations and the error bound they
obey: |v_i - s x_i| <= 0.51 s for every encoded value (half a step, plus the
fp32 roundings of v * inv and of s, and the reciprocal's error, each below
2^-22 * 30583 steps), i.e.
about (the block's scaling magnitude) / 60000.
"""
from __future__ import annotations

import numpy as np

XMAX = np.float32(30583.0)
INV_XMAX = np.float32(1.0) / XMAX
SLOTS = 4
RATIO = 16.0


def encode_block(v: np.ndarray, threshold: float | None = None, slots: int = SLOTS):
    """One block (32 fp32 values) -> (effective values, scale s, indices taken
    out, their values). Arithmetic in fp32 as the kernel does it; the slots
    are filled round by round, each round's values in index order."""
    v = np.asarray(v, dtype=np.float32).copy()
    a = np.abs(v)
    amax = np.float32(a.max()) if a.size else np.float32(0)
    taken_i, taken_v = [], []
    if threshold is not None and np.isfinite(v).all():
        mask = np.zeros(v.size, bool)
        cur = amax
        ratio = np.float32(1.0) / np.float32(threshold)
        while len(taken_i) < slots and cur > 0:
            big = ~mask & (a >= np.float32(cur * ratio))
            if int(big.sum()) > slots - len(taken_i):
                break
            for i in np.nonzero(big)[0]:
                taken_i.append(int(i))
                taken_v.append(v[i])
            mask |= big
            cur = np.float32(np.where(mask, np.float32(0), a).max())
        if taken_i:
            v[mask] = 0
            amax = cur
    if not np.isfinite(amax) or not np.isfinite(v).all():
        return np.full(v.shape, np.nan, np.float32), np.float32(np.nan), [], []
    s = np.float32(amax * INV_XMAX)
    if s < np.float32(2.0 ** -126):  # zero or tiny blocks: the step 2^-126
        s = np.float32(2.0 ** -126) if amax > 0 else np.float32(0)
    inv = np.float32(1) / s if s > 0 else np.float32(0)
    # one rounding of the exact product (the kernel's fma); no clamp is needed
    x = np.rint(v.astype(np.float64) * np.float64(inv)).astype(np.float32)
    assert np.abs(x).max(initial=0) <= 30583
    eff = (s * x).astype(np.float32)
    for i, tv in zip(taken_i, taken_v):
        eff[i] = tv
    return eff, s, taken_i, taken_v


def effective_row(x: np.ndarray, threshold: float | None = None) -> np.ndarray:
    """The activation row a kernel multiplies, block by block (len(x) a
    multiple of 32)."""
    x = np.asarray(x, dtype=np.float32)
    out = np.empty_like(x)
    for b in range(0, x.size, 32):
        out[b:b + 32] = encode_block(x[b:b + 32], threshold)[0]
    return out


def block_bound(x: np.ndarray, threshold: float | None = None) -> np.ndarray:
    """Per-value error bound |v - eff|: 0.51 s (s the block's scale), 0 for
    a value taken out."""
    x = np.asarray(x, dtype=np.float32)
    out = np.empty(x.size, np.float64)
    for b in range(0, x.size, 32):
        blk = x[b:b + 32]
        eff, s, taken, _ = encode_block(blk, threshold)
        out[b:b + 32] = 0.51 * float(s) + 1e-45
        for i in taken:
            out[b + i] = 0.0
    return out
