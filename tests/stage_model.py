"""A CPU restatement of the activation encoding of the integer matvec
kernels (recipe-dev_amd/csrc/stage.h), test infrastructure.

Every 32-value block of an activation row becomes 16-bit integers
x_i = rint(v_i / s) with the block scale s = amax * fp32(1 / 30583) (2^-126 for
blocks whose step would fall below the smallest normal float), rounded once
from the exact product of v_i and 1 / s (the kernels form 1 / s with the
hardware reciprocal, within one ulp; the model divides); the kernels' products are exact integer dots of
these against the weights' integer codes, scaled per block in fp32, so the
activation a kernel multiplies is s * x_i. With outlier extraction, a block
whose largest magnitude exceeds `threshold` times its second largest has that
one value (the lowest index among equal magnitudes) taken out: it is encoded
as 0, the block is scaled by the second largest magnitude, and the value
itself is multiplied exactly (in fp32) with its weight.

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


def encode_block(v: np.ndarray, threshold: float | None = None):
    """One block (32 fp32 values) -> (effective values, scale s, outlier index
    or -1, outlier value). Arithmetic in fp32 as the kernel does it."""
    v = np.asarray(v, dtype=np.float32)
    a = np.abs(v)
    amax = np.float32(a.max()) if a.size else np.float32(0)
    out_i, out_v = -1, np.float32(0)
    if threshold is not None and amax > 0:
        i = int(np.argmax(a))  # lowest index among the largest
        rest = a.copy()
        rest[i] = 0
        amax2 = np.float32(rest.max())
        if amax > np.float32(threshold) * amax2:
            out_i, out_v = i, v[i]
            v = v.copy()
            v[i] = 0
            amax = amax2
    if not np.isfinite(amax) or not np.isfinite(v).all():
        return np.full(v.shape, np.nan, np.float32), np.float32(np.nan), -1, np.float32(0)
    s = np.float32(amax * INV_XMAX)
    if s < np.float32(2.0 ** -126):  # zero or tiny blocks: the step 2^-126
        s = np.float32(2.0 ** -126) if amax > 0 else np.float32(0)
    inv = np.float32(1) / s if s > 0 else np.float32(0)
    # one rounding of the exact product (the kernel's fma); no clamp is needed
    x = np.rint(v.astype(np.float64) * np.float64(inv)).astype(np.float32)
    assert np.abs(x).max(initial=0) <= 30583
    eff = (s * x).astype(np.float32)
    if out_i >= 0:
        eff[out_i] = out_v
    return eff, s, out_i, out_v


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
    an extracted outlier."""
    x = np.asarray(x, dtype=np.float32)
    out = np.empty(x.size, np.float64)
    for b in range(0, x.size, 32):
        blk = x[b:b + 32]
        eff, s, oi, _ = encode_block(blk, threshold)
        out[b:b + 32] = 0.51 * float(s) + 1e-45
        if oi >= 0:
            out[b + oi] = 0.0
    return out
