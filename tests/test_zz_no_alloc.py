"""rqmv_moe_batch_noalloc: the gguf_moe batch on the library's own per-GPU
scratch, for callers that cannot allocate. Called through the C ABI and
checked bit for bit against rqmv_moe_batch (the same kernels on a caller
workspace), on two calls in a row, the second with fewer positions, plus the
size limit and a check against the f64 oracle."""
import numpy as np
import pytest

import oracle
from rqmv import synth

pytestmark = pytest.mark.gpu


def _block(gpu, fmt, d, E, top, H, HS, seed):
    router = synth.f16_weights(E, d, 0.02, seed=seed, tag="router")
    gate = synth.weights(fmt, E * H, d, seed=seed + 1, tag="gate")
    up = synth.weights(fmt, E * H, d, seed=seed + 2, tag="up")
    down = synth.weights(fmt, E * d, H, seed=seed + 3, tag="down")
    sg = synth.f16_weights(1, d, 0.02, seed=seed + 4, tag="sg")
    gs = synth.weights(fmt, HS, d, seed=seed + 5, tag="gs")
    us = synth.weights(fmt, HS, d, seed=seed + 6, tag="us")
    ds = synth.weights(fmt, d, HS, seed=seed + 7, tag="ds")
    moe = gpu.Moe(gpu.Weight("f16", E, d, router), gpu.Weight(fmt, H, d, gate, experts=E),
                  gpu.Weight(fmt, H, d, up, experts=E), gpu.Weight(fmt, d, H, down, experts=E), top,
                  shared_gate_inp=gpu.Weight("f16", 1, d, sg), gate_sh=gpu.Weight(fmt, HS, d, gs),
                  up_sh=gpu.Weight(fmt, HS, d, us), down_sh=gpu.Weight(fmt, d, HS, ds))
    ref_args = (router, gate, up, down, sg, gs, us, ds)
    return moe, ref_args


def _both(gpu, moe, m, seed):
    d, E = moe.d_model, moe.experts
    xh = synth.activations_f16(m * d, seed=seed).reshape(m, d)
    X = gpu.DeviceBuffer.from_array(xh)
    ya, yb = gpu.DeviceBuffer(4 * m * d), gpu.DeviceBuffer(4 * m * d)
    ra, rb = gpu.DeviceBuffer(4 * m * E), gpu.DeviceBuffer(4 * m * E)
    moe.run_batch(X, 1, m, d, ya, d, ra)
    moe.run_batch_noalloc(X, 1, m, d, yb, d, rb)
    gpu.synchronize()
    out = [b.download(np.float32).reshape(m, -1) for b in (ya, yb, ra, rb)]
    return xh, out


def test_noalloc_matches_the_workspace_entry_point(gpu):
    fmt, d, E, top, H, HS = "q4_k", 2048, 256, 8, 512, 512  # the gguf_moe decode workload's block
    moe, (router, gate, up, down, sg, gs, us, ds) = _block(gpu, fmt, d, E, top, H, HS, seed=61)
    for m, seed in ((5, 62), (2, 63)):  # the second call smaller than the first
        xh, (ya, yb, ra, rb) = _both(gpu, moe, m, seed)
        assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32)), m
        assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32)), m
        x0 = synth.fp16_to_f32(xh[0]).astype(np.float64)
        y_ref, rw_ref = oracle.moe_f64(fmt, d, E, top, H, router.view(np.uint16), gate, up, down, x0,
                                       hidden_shared=HS, shared_gate_bits=sg.view(np.uint16), gate_sh=gs, up_sh=us,
                                       down_sh=ds)
        assert np.array_equal(rb[0] != 0, rw_ref != 0)
        assert np.linalg.norm(yb[0] - y_ref) / np.linalg.norm(y_ref) <= 1e-3


def test_noalloc_refuses_batches_past_its_scratch(gpu):
    fmt, d, E, top, H, HS = "q4_k", 2048, 256, 8, 512, 512
    moe, _ = _block(gpu, fmt, d, E, top, H, HS, seed=71)
    per = moe.workspace.nbytes
    m = (1 << 20) // per + 1  # one position more than the 1 MiB scratch holds
    X = gpu.DeviceBuffer(2 * m * d)
    Y, R = gpu.DeviceBuffer(4 * m * d), gpu.DeviceBuffer(4 * m * E)
    with pytest.raises(gpu.RqmvError, match="scratch"):
        moe.run_batch_noalloc(X, 1, m, d, Y, d, R)
    # the largest batch that fits still runs, and matches the workspace form
    xh, (ya, yb, ra, rb) = _both(gpu, moe, m - 1, seed=72)
    assert np.array_equal(ya.view(np.uint32), yb.view(np.uint32))
    assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32))
