"""Pins the oracle's decode-step reference (oracle/decode.py) with closed forms
and independent formulations: complex multiplication for the rotary, scipy's
softmax for attention, scipy's logistic function for SiLU, and decoders whose
projections are zero so that the whole step reduces to the head applied to
the normalised embedding."""
import numpy as np
import pytest
from scipy.special import expit, softmax

from oracle import decode as ref
from rqmv import synth
from rqmv.decode import DecoderShape, LayerTensors

RNG = np.random.default_rng(5)


def test_rmsnorm_constant_vector_closed_form():
    n, c, eps = 64, 3.0, 1e-5
    out = ref.rmsnorm(np.full(n, c), np.full(n, 2.0), eps)
    assert np.allclose(out, c / np.sqrt(c * c + eps) * 2.0, rtol=0, atol=1e-15)


def test_rmsnorm_scale_invariant_without_eps():
    x = RNG.standard_normal(100)
    s = RNG.standard_normal(100)
    assert np.allclose(ref.rmsnorm(x, s, 0.0), ref.rmsnorm(37.5 * x, s, 0.0), rtol=1e-14)
    y = ref.rmsnorm(x, np.ones(100), 0.0)
    assert abs(np.mean(y * y) - 1.0) < 1e-14


@pytest.mark.parametrize("pos", [0, 1, 17, 4095])
@pytest.mark.parametrize("dims", [2, 64, 128])
def test_rope_is_a_complex_rotation_per_pair(pos, dims):
    base = 500000.0
    h = RNG.standard_normal((3, dims))
    got = ref.rope_neox(h, pos, base)
    half = dims // 2
    z = h[:, :half] + 1j * h[:, half:]
    theta = pos * base ** (-np.arange(half) * 2.0 / dims)
    w = z * np.exp(1j * theta)
    assert np.allclose(got[:, :half], w.real, rtol=1e-12, atol=1e-12)
    assert np.allclose(got[:, half:], w.imag, rtol=1e-12, atol=1e-12)
    if pos == 0:
        assert np.array_equal(got, h)


def test_rope_scores_depend_on_relative_position_only():
    q = RNG.standard_normal(128)
    k = RNG.standard_normal(128)
    s1 = ref.rope_neox(q, 100, 1e4) @ ref.rope_neox(k, 90, 1e4)
    s2 = ref.rope_neox(q, 1010, 1e4) @ ref.rope_neox(k, 1000, 1e4)
    assert abs(s1 - s2) < 1e-9 * max(1.0, abs(s1))


def test_attention_single_position_returns_its_value():
    q = RNG.standard_normal((4, 64))
    k = RNG.standard_normal((2, 5, 64))
    v = RNG.standard_normal((2, 5, 64))
    out = ref.attention(q, k, v, 1)
    assert np.allclose(out[:2], v[0, 0]) and np.allclose(out[2:], v[1, 0])


def test_attention_identical_keys_average_values():
    q = RNG.standard_normal((2, 64))
    k = np.repeat(RNG.standard_normal((1, 1, 64)), 7, axis=1)
    v = RNG.standard_normal((1, 7, 64))
    out = ref.attention(q, k, v, 7)
    assert np.allclose(out, v[0].mean(axis=0)[None, :], rtol=1e-12, atol=1e-12)


def test_attention_matches_scipy_softmax_and_group_mapping():
    nq, nkv, hd, n = 8, 2, 64, 33
    q = RNG.standard_normal((nq, hd))
    k = RNG.standard_normal((nkv, 40, hd))
    v = RNG.standard_normal((nkv, 40, hd))
    out = ref.attention(q, k, v, n)
    for h in range(nq):
        kh = h // (nq // nkv)
        w = softmax(k[kh, :n] @ q[h] / 8.0)
        assert np.allclose(out[h], w @ v[kh, :n], rtol=1e-12, atol=1e-12)


def test_silu_mul_matches_logistic():
    g = np.concatenate([RNG.standard_normal(50) * 5, [0.0, 60.0, -60.0]])
    u = RNG.standard_normal(g.size)
    # recipe's form 0.5 (tanh(v / 2) + 1) cancels for v -> -inf: an absolute
    # error of a few f64 ulps of 1 times |g u|
    assert np.all(np.abs(ref.silu_mul(g, u) - g * expit(g) * u) <= 1e-15 * np.abs(g * u) + 1e-14 * np.abs(g * expit(g) * u))
    assert ref.silu_mul(np.array([0.0]), np.array([3.0]))[0] == 0.0


def _zero_scales(fmt, blocks):
    lo, hi = synth._SCALE_BYTES[fmt]
    b = blocks.reshape(-1, synth.BLOCK[fmt][1]).copy()
    b[:, lo:hi] = 0
    return b.reshape(-1)


def test_decoder_with_zero_projections_is_head_of_normed_embedding():
    s = DecoderShape(layers=2, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=256, vocab=64)
    D = synth.DecoderSynth(s, seed=3, norm_std=0.2)
    layers = []
    for i in range(s.layers):
        t = D.layer(i)
        layers.append(LayerTensors(t.attn_norm, t.qkv, _zero_scales(s.proj_fmt, t.o), t.ffn_norm, t.gate, t.up,
                                   _zero_scales(s.proj_fmt, t.down)))
    embed = D.embed()[: s.vocab]
    R = ref.DecoderReference(s, embed, D.out_norm(), D.head(), layers, [D.cache(i, 4) for i in range(s.layers)], 8)
    import oracle
    head = oracle.dequant_rows(s.head_fmt, D.head(), s.vocab, s.d).reshape(s.vocab, s.d).astype(np.float64)
    for pos, tok in ((4, 9), (5, 70)):
        got = R.step(tok, pos)
        x = embed[tok % s.vocab].astype(np.float64)
        want = head @ (x / np.sqrt(np.mean(x * x) + s.eps) * D.out_norm())
        assert np.allclose(got, want, rtol=1e-12, atol=1e-9)
        # the step still appended its key and value (fp16) at pos
        assert np.any(R.k[0][:, pos] != 0) and np.all(R.k[0][:, pos + 1:] == 0)


def test_layer_variants_keep_block_scales_and_differ():
    a = synth.weights("q4_k", 4, 512, seed=1)
    v1 = synth.layer_variant("q4_k", a, 1, "t.l0")
    v2 = synth.layer_variant("q4_k", a, 1, "t.l1")
    for v in (v1, v2):
        assert np.array_equal(v.reshape(-1, 144)[:, :4], a.reshape(-1, 144)[:, :4])
    assert not np.array_equal(v1, v2)
    assert np.array_equal(synth.layer_variant("q4_k", v1, 1, "t.l0"), a)  # an involution


def test_streaming_layers_equal_the_dequantized_decoder():
    """The streaming form used for decoders too large to dequantize whole
    (QuantLayer: the oracle's f64 row products on threads, several streams per
    layer) equals the dequantized decoder's step, with a Q4_K_M-style QKV of
    mixed formats in one layer."""
    import oracle
    s = DecoderShape(layers=2, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=64)
    D = synth.DecoderSynth(s, seed=8, norm_std=0.2)
    layers = [D.layer(i) for i in range(s.layers)]
    t = layers[1]
    q_rows, kv_rows = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
    v6 = synth.weights("q6_k", kv_rows, s.d, seed=4)
    qkv = t.qkv.reshape(q_rows + 2 * kv_rows, -1)
    layers[1] = LayerTensors(t.attn_norm, None, t.o, t.ffn_norm, t.gate, t.up, t.down,
                             qkv_parts=[("q4_k", q_rows, qkv[:q_rows].reshape(-1)),
                                        ("q4_k", kv_rows, qkv[q_rows:q_rows + kv_rows].reshape(-1)),
                                        ("q6_k", kv_rows, v6)])
    embed, caches, ctx = D.embed()[: s.vocab], [D.cache(i, 6) for i in range(s.layers)], 6
    R = ref.DecoderReference(s, embed, D.out_norm(), D.head(), layers, caches, 8)
    want = R.step(5, ctx)
    x = np.stack([embed[5].astype(np.float64)] * 2)
    for i in range(s.layers):
        L = ref.QuantLayer(s, layers[i], threads=3)
        c = [(ref.f64_cache(caches[i][0], 8), ref.f64_cache(caches[i][1], 8)) for _ in range(2)]
        x = ref.layer_forward(s, L, L.attn_norm, L.ffn_norm, c, x, ctx)
        assert np.array_equal(c[0][0], c[1][0]) and np.array_equal(c[0][0][:, ctx], R.k[i][:, ctx])
    head = oracle.matvec_f64(s.head_fmt, D.head(), s.vocab, s.d, ref.rmsnorm(x[0], D.out_norm(), s.eps), 2)[0]
    assert np.array_equal(x[0], x[1])
    # the dequantized decoder holds each weight rounded to fp32, the row
    # products the f64 value of the decoder's formula: 1e-7 covers that
    assert np.allclose(head, want, rtol=1e-7, atol=1e-7 * np.abs(want).max())
