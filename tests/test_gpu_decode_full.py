"""The single-token decode step of the full 32-layer decoder at its own
configuration, against the oracle's f64 decoder, through the C ABI.

Configuration: 32 layers, d 4096, 32 query and 8 key-value heads of 128,
SiLU-GLU of 14336, Q4_K projections, the 128256-row Q8_0 head, an fp16 KV
cache prefilled to 4096 positions, decoding position 4096 (Placed::step,
recipe.rs:21314-21470; lower_attention, recipe.rs:23056-23150).

Teacher-forced: the oracle's layer i takes the device's input of layer i (the
stream an early-exit step of i layers hands its head), so every layer is
checked on its own at rel-L2 1e-3, the projections' bar, and so is the key
and value the device appended to each layer's cache at the position. The
oracle's own chain from the embedding row is held to the same bar against
the device's logits, and so is the head applied to the device's final
stream; the chosen token is the argmax of the logits. The head's product is
also compared alone with the oracle's restatement of recipe's fp32 path.
"""
import os
import sys
import time

import numpy as np
import pytest

import oracle
from oracle import decode as ref
from rqmv import synth
from rqmv.decode import DecodeModel, DecoderShape

pytestmark = pytest.mark.gpu

THREADS = max(1, min(16, os.cpu_count() or 1))
CTX = 4096  # prefilled positions; the step decodes position CTX
TOKEN = 91237
BAR = 1e-3


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _progress(msg):
    sys.__stderr__.write(f"[decode 32-layer] {msg}\n")
    sys.__stderr__.flush()


@pytest.fixture(scope="module")
def full(gpu):
    s = DecoderShape()
    assert (s.layers, s.d, s.q_heads, s.kv_heads, s.head_dim, s.ffn, s.vocab, s.proj_fmt, s.head_fmt) == \
        (32, 4096, 32, 8, 128, 14336, 128256, "q4_k", "q8_0")
    t0 = time.perf_counter()
    D = synth.DecoderSynth(s, seed=29, norm_std=0.1)
    embed, out_norm, head = D.embed(), D.out_norm(), D.head()
    model = DecodeModel(s, CTX + 1, embed, out_norm, head)
    layers, caches = [], []
    for i in range(s.layers):
        t, kv = D.layer(i), D.cache(i, CTX)
        model.set_layer(i, t)
        model.set_cache(i, *kv)
        layers.append(t)
        caches.append(kv)
    gpu.synchronize()
    _progress(f"model built in {time.perf_counter() - t0:.1f} s")
    return {"shape": s, "model": model, "embed": embed, "out_norm": out_norm, "head": head, "layers": layers,
            "caches": caches}


def _cache_row(model, buf, pos):
    """fp16 entries at `pos` of every kv head of one layer's cache, as float64."""
    s = model.shape
    row = 2 * s.head_dim
    out = [buf.view((h * model.max_ctx + pos) * row, row).download(np.uint16) for h in range(s.kv_heads)]
    return np.stack(out).view(np.float16).astype(np.float64)


def test_full_decoder_step_teacher_forced(gpu, full):
    s, model = full["shape"], full["model"]
    pos = CTX
    t0 = time.perf_counter()
    # the device's input of every layer: layer 0 takes the embedding row; layer
    # i > 0 the stream an early-exit step of i layers hands its head
    inputs = [full["embed"][TOKEN].astype(np.float64)]
    for depth in range(1, s.layers):
        model.set_position(TOKEN, pos)
        model.enqueue_step(layers=depth)
        gpu.synchronize()
        inputs.append(model.read_hidden().astype(np.float64))
    model.set_position(TOKEN, pos)
    model.enqueue_step()
    gpu.synchronize()
    final = model.read_hidden().astype(np.float64)
    logits, token = model.read_logits(), model.read_token()
    assert model.read_position() == pos + 1
    kv_dev = [(_cache_row(model, model.k_cache[i], pos), _cache_row(model, model.v_cache[i], pos))
              for i in range(s.layers)]
    _progress(f"device steps done in {time.perf_counter() - t0:.1f} s")
    outputs = inputs[1:] + [final]

    x_own = inputs[0].copy()  # the oracle's own chain
    errs = []
    for i in range(s.layers):
        L = ref.QuantLayer(s, full["layers"][i], THREADS)
        k_bits, v_bits = full["caches"][i]
        forced = (ref.f64_cache(k_bits, pos + 1), ref.f64_cache(v_bits, pos + 1))
        own = (forced[0].copy(), forced[1].copy())
        Y = ref.layer_forward(s, L, L.attn_norm, L.ffn_norm, [forced, own], np.stack([inputs[i], x_own]), pos)
        e = rel_err(outputs[i], Y[0])
        errs.append(e)
        assert e < BAR, (i, e)
        assert rel_err(kv_dev[i][0], forced[0][:, pos]) < BAR, i
        assert rel_err(kv_dev[i][1], forced[1][:, pos]) < BAR, i
        x_own = Y[1]
        if i % 8 == 7:
            _progress(f"layers 0..{i} checked, worst rel-L2 {max(errs):.2e} ({time.perf_counter() - t0:.1f} s)")
    H = oracle.matvec_f64(s.head_fmt, full["head"], s.vocab, s.d,
                          np.stack([ref.rmsnorm(final, full["out_norm"], s.eps),
                                    ref.rmsnorm(x_own, full["out_norm"], s.eps)]), THREADS)
    e_head, e_chain = rel_err(logits, H[0]), rel_err(logits, H[1])
    _progress(f"head rel-L2 {e_head:.2e}, own chain {e_chain:.2e}, layers worst {max(errs):.2e}")
    assert e_head < BAR
    assert e_chain < BAR
    assert token == int(np.argmax(logits))


def test_head_product_full_vocabulary(gpu, full):
    """The 128256x4096 Q8_0 head alone: the device's product of an N(0, 1)
    stream within 1e-3 of recipe's fp32 path (the oracle's restatement) and of
    the f64 product, and the device argmax over all rows equal to numpy's."""
    s, model = full["shape"], full["model"]
    x = synth.activations_f32(s.d, seed=17)
    X, Y = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * s.vocab)
    model.head.matvec(X, gpu.DTYPE_F32, 1, s.d, Y, s.vocab)
    gpu.synchronize()
    y = Y.download(np.float32)
    want32 = oracle.matvec_recipe_f32(s.head_fmt, full["head"], s.vocab, s.d, x, threads=THREADS)[0]
    want64 = oracle.matvec_f64(s.head_fmt, full["head"], s.vocab, s.d, x.astype(np.float64), THREADS)[0]
    assert rel_err(y, want32) < BAR
    assert rel_err(y, want64) < BAR
    assert rel_err(want32, want64) < 1e-5  # the restatement of recipe's fp32 path against f64
    O, ws = gpu.DeviceBuffer(4), gpu.argmax_workspace()
    gpu.argmax(Y, s.vocab, O, ws)
    gpu.synchronize()
    assert int(O.download(np.int32, 1)[0]) == int(np.argmax(y))
