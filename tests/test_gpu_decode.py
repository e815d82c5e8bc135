"""GPU parity of the decode-step helpers and of a whole decode step against the
oracle's f64 decode reference (oracle/decode.py), through the C ABI.

Bars: residual adds bit-exact (one fp32 add, as numpy does it); the helpers
within rel 1e-5 (norm, rotary, attention, SiLU-GLU); cache appends within one
fp16 rounding of the reference; logits of a whole step within rel-L2 1e-3 of
the f64 reference (the projections' own bar), steps replayed from a captured
HIP graph included; argmax bit-exact with ties to the lowest index.
"""
import numpy as np
import pytest

from oracle import decode as ref
from rqmv import synth
from rqmv.decode import DecodeModel, DecoderShape

pytestmark = pytest.mark.gpu

RNG = np.random.default_rng(11)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def _i32(gpu, v):
    return gpu.DeviceBuffer.from_array(np.array([v], dtype=np.int32))


@pytest.mark.parametrize("n", [1, 100, 4096, 5120])
def test_add_rmsnorm(gpu, n):
    x = RNG.standard_normal(n).astype(np.float32) * 40
    delta = RNG.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * RNG.standard_normal(n)).astype(np.float32)
    X, D, W, O = (gpu.DeviceBuffer.from_array(a) for a in (x, delta, w, np.zeros(n, np.float32)))
    gpu.add_rmsnorm(X, D, W, n, 1e-5, O)
    gpu.synchronize()
    xs = x + delta
    assert np.array_equal(X.download(np.float32), xs)
    assert rel_err(O.download(np.float32), ref.rmsnorm(xs, w, 1e-5)) < 1e-5
    gpu.add_rmsnorm(X, None, W, n, 1e-5, O)  # no delta: x unchanged
    gpu.synchronize()
    assert np.array_equal(X.download(np.float32), xs)


@pytest.mark.parametrize("nq,nkv,hd", [(4, 2, 64), (32, 8, 128), (8, 8, 256)])
@pytest.mark.parametrize("pos", [0, 7, 4095])
def test_rope_kv(gpu, nq, nkv, hd, pos):
    max_ctx = 4100
    qkv = RNG.standard_normal((nq + 2 * nkv) * hd).astype(np.float32)
    Q = gpu.DeviceBuffer.from_array(qkv)
    cache_bytes = nkv * max_ctx * hd * 2
    K, V = gpu.DeviceBuffer(cache_bytes), gpu.DeviceBuffer(cache_bytes)
    K.fill_zero()
    V.fill_zero()
    gpu.rope_kv(Q, _i32(gpu, pos), nq, nkv, hd, 500000.0, K, V, max_ctx)
    gpu.synchronize()
    got = Q.download(np.float32)
    q_ref = ref.rope_neox(qkv[:nq * hd].reshape(nq, hd), pos, 500000.0).reshape(-1)
    k_ref = ref.rope_neox(qkv[nq * hd:(nq + nkv) * hd].reshape(nkv, hd), pos, 500000.0)
    assert rel_err(got[:nq * hd], q_ref) < 1e-5
    assert rel_err(got[nq * hd:(nq + nkv) * hd], k_ref.reshape(-1)) < 1e-5
    assert np.array_equal(got[(nq + nkv) * hd:], qkv[(nq + nkv) * hd:])  # values untouched
    kc = K.download(np.uint16).reshape(nkv, max_ctx, hd).view(np.float16)
    vc = V.download(np.uint16).reshape(nkv, max_ctx, hd).view(np.float16)
    # the cache holds fp16 of the fp32 results: within one fp16 rounding of the f64 reference
    k16 = k_ref.astype(np.float16).astype(np.float64)
    assert np.all(np.abs(kc[:, pos].astype(np.float64) - k16) <= np.abs(k16) * 2 ** -10 + 2 ** -24)
    assert np.array_equal(vc[:, pos], qkv[(nq + nkv) * hd:].reshape(nkv, hd).astype(np.float16))
    others = np.ones(max_ctx, bool)
    others[pos] = False
    assert not np.any(kc.view(np.uint16)[:, others]) and not np.any(vc.view(np.uint16)[:, others])


def test_rope_kv_position_outside_cache_writes_nothing(gpu):
    nq, nkv, hd, max_ctx = 4, 2, 64, 16
    qkv = RNG.standard_normal((nq + 2 * nkv) * hd).astype(np.float32)
    Q = gpu.DeviceBuffer.from_array(qkv)
    K, V = gpu.DeviceBuffer(nkv * max_ctx * hd * 2), gpu.DeviceBuffer(nkv * max_ctx * hd * 2)
    K.fill_zero()
    V.fill_zero()
    gpu.rope_kv(Q, _i32(gpu, max_ctx), nq, nkv, hd, 1e4, K, V, max_ctx)
    gpu.synchronize()
    assert not np.any(K.download(np.uint16)) and not np.any(V.download(np.uint16))


@pytest.mark.parametrize("nq,nkv,hd", [(4, 2, 64), (32, 8, 128), (8, 1, 128), (4, 4, 256), (12, 4, 128), (24, 4, 64)])
@pytest.mark.parametrize("length", [1, 127, 128, 129, 300])
def test_attention(gpu, nq, nkv, hd, length):
    max_ctx = 384
    q = RNG.standard_normal((nq, hd)).astype(np.float32)
    kc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    vc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    Q = gpu.DeviceBuffer.from_array(q)
    K = gpu.DeviceBuffer.from_array(kc.view(np.uint16))
    V = gpu.DeviceBuffer.from_array(vc.view(np.uint16))
    ws = gpu.attention_workspace(nq, nkv, hd, max_ctx)
    O = gpu.DeviceBuffer(nq * hd * 4)
    gpu.attention(Q, K, V, _i32(gpu, length - 1), nq, nkv, hd, max_ctx, ws, O)
    gpu.synchronize()
    want = ref.attention(q, kc.astype(np.float64), vc.astype(np.float64), length)
    assert rel_err(O.download(np.float32), want.reshape(-1)) < 1e-5


def test_attention_long_context(gpu):
    nq, nkv, hd, max_ctx = 32, 8, 128, 4160
    q = (RNG.standard_normal((nq, hd)) * 0.2).astype(np.float32)
    kc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    vc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    Q = gpu.DeviceBuffer.from_array(q)
    K = gpu.DeviceBuffer.from_array(kc.view(np.uint16))
    V = gpu.DeviceBuffer.from_array(vc.view(np.uint16))
    ws = gpu.attention_workspace(nq, nkv, hd, max_ctx)
    O = gpu.DeviceBuffer(nq * hd * 4)
    for length in (4096, 4097, max_ctx):
        gpu.attention(Q, K, V, _i32(gpu, length - 1), nq, nkv, hd, max_ctx, ws, O)
        gpu.synchronize()
        want = ref.attention(q, kc.astype(np.float64), vc.astype(np.float64), length)
        assert rel_err(O.download(np.float32), want.reshape(-1)) < 1e-5, length


@pytest.mark.parametrize("n", [1, 300, 14336])
def test_silu_mul(gpu, n):
    gu = (RNG.standard_normal(2 * n) * 6).astype(np.float32)
    G, O = gpu.DeviceBuffer.from_array(gu), gpu.DeviceBuffer(4 * n)
    gpu.silu_mul(G, n, O)
    gpu.synchronize()
    got = O.download(np.float32).astype(np.float64)
    want = ref.silu_mul(gu[:n], gu[n:])
    # recipe's sigmoid is 0.5 (tanh(v / 2) + 1) in fp32 (recipe.rs:22662-22668):
    # near v -> -inf the sum cancels, so each element carries an absolute error
    # of a few fp32 ulps of 1 times |g u| besides its relative rounding
    g, u = gu[:n].astype(np.float64), gu[n:].astype(np.float64)
    assert np.all(np.abs(got - want) <= 2.0 ** -22 * np.abs(g * u) + 1e-6 * np.abs(want))
    if n >= 300:
        assert rel_err(got, want) < 1e-5


@pytest.mark.parametrize("n", [1, 1000, 1025, 128256])
def test_argmax_lowest_index_on_ties(gpu, n):
    v = RNG.standard_normal(n).astype(np.float32)
    if n > 10:
        v[n // 3] = v[n - 2] = v.max() + 1.0  # a tie: the lower index wins
        v[5] = -np.inf
    V, O = gpu.DeviceBuffer.from_array(v), gpu.DeviceBuffer(4)
    ws = gpu.argmax_workspace()
    for _ in range(2):  # a second call over the same workspace
        gpu.argmax(V, n, O, ws)
        gpu.synchronize()
        assert int(O.download(np.int32, 1)[0]) == int(np.argmax(v))


def test_embed_row(gpu):
    rows, n = 50, 4096
    table = RNG.standard_normal((rows, n)).astype(np.float32)
    T, O = gpu.DeviceBuffer.from_array(table), gpu.DeviceBuffer(4 * n)
    for tok in (0, 49, 123):
        gpu.embed_row(T, rows, n, _i32(gpu, tok), O)
        gpu.synchronize()
        assert np.array_equal(O.download(np.float32), table[tok % rows])


# ------------------------------------------------------ whole decode step ----

def _small_decoder(gpu, shape, ctx, max_ctx, seed):
    D = synth.DecoderSynth(shape, seed=seed, norm_std=0.1)
    layers = [D.layer(i) for i in range(shape.layers)]
    caches = [D.cache(i, ctx) for i in range(shape.layers)]
    embed = D.embed()
    model = DecodeModel(shape, max_ctx, embed, D.out_norm(), D.head())
    for i in range(shape.layers):
        model.set_layer(i, layers[i])
        model.set_cache(i, *caches[i])
    R = ref.DecoderReference(shape, embed, D.out_norm(), D.head(), layers, caches, max_ctx)
    return model, R


@pytest.mark.parametrize("proj_fmt,head_fmt", [("q4_k", "q8_0"), ("q6_k", "q4_0")])
def test_decode_steps_match_reference(gpu, proj_fmt, head_fmt):
    shape = DecoderShape(layers=2, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=512,
                         proj_fmt=proj_fmt, head_fmt=head_fmt)
    ctx, max_ctx = 16, 24
    model, R = _small_decoder(gpu, shape, ctx, max_ctx, seed=21)
    stream = gpu.Stream()
    token, pos = 7, ctx
    model.set_position(token, pos)
    # one eager step, then steps replayed from a captured graph (teacher-forced:
    # the reference decodes the token the device chose)
    model.enqueue_step(stream)
    stream.synchronize()
    steps = [(token, pos, model.read_logits(), model.read_token())]
    graph = model.capture(stream)
    for _ in range(3):
        token, pos = steps[-1][3], steps[-1][1] + 1
        graph.launch(stream)
        stream.synchronize()
        steps.append((token, pos, model.read_logits(), model.read_token()))
    assert model.read_position() == ctx + 4
    for token, pos, logits, chosen in steps:
        want = R.step(token, pos)
        assert rel_err(logits, want) < 1e-3, (token, pos, rel_err(logits, want))
        assert chosen == int(np.argmax(logits))
    graph.close()
    stream.close()


def test_decode_refuses_steps_past_the_cache(gpu):
    """recipe refuses a step whose token window lies outside the placement's
    capacity (recipe.rs:21330-21331): set_position checks the position, step()
    and replay() count steps on the host and raise before one would run past
    the cache, and the results of a graph launched directly past the end are
    refused when read. (A step past the end reads and writes only inside the
    cache: the kernels clamp the position.)"""
    shape = DecoderShape(layers=1, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=256)
    ctx, max_ctx = 4, 6
    model, _ = _small_decoder(gpu, shape, ctx, max_ctx, seed=2)
    for bad in (max_ctx, max_ctx + 5, -1):
        with pytest.raises(ValueError):
            model.set_position(1, bad)
    stream = gpu.Stream()
    with pytest.raises(RuntimeError):
        model.step(stream)  # no position yet
    model.set_position(1, ctx)  # positions 4 and 5 fit
    model.step(stream)
    graph = model.capture(stream)
    with pytest.raises(ValueError):
        model.replay(graph, stream, 2)
    model.replay(graph, stream)  # position 5, the cache's last
    stream.synchronize()
    assert np.isfinite(model.read_logits()).all()
    with pytest.raises(ValueError):
        model.step(stream)
    with pytest.raises(ValueError):
        model.replay(graph, stream)
    assert model.read_position() == max_ctx
    graph.launch(stream)  # bypasses the host count
    stream.synchronize()
    with pytest.raises(RuntimeError):
        model.read_logits()
    with pytest.raises(RuntimeError):
        model.read_token()
    graph.close()
    stream.close()


def test_decode_real_head_shapes(gpu):
    """One step at the full decoder's attention and projection widths (two
    layers, smaller vocab), against the f64 reference."""
    shape = DecoderShape(layers=2, d=4096, q_heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=2048)
    ctx, max_ctx = 300, 320
    model, R = _small_decoder(gpu, shape, ctx, max_ctx, seed=5)
    model.set_position(3, ctx)
    model.enqueue_step()
    gpu.synchronize()
    logits = model.read_logits()
    want = R.step(3, ctx)
    assert rel_err(logits, want) < 1e-3
    assert model.read_token() == int(np.argmax(logits))


# ------------------------------------------------------- fused products ----

def _mv_ref(fmt, w, rows, cols, x):
    import oracle
    return oracle.dequant_rows(fmt, w, rows, cols).reshape(rows, cols).astype(np.float64) @ np.asarray(x, np.float64)


@pytest.mark.parametrize("fmt,rows,cols", [("q4_k", 6144, 4096), ("q8_0", 4096, 4096), ("q6_k", 512, 1024),
                                           ("q4_0", 300, 4096), ("q4_k", 256, 14336), ("q8_0", 1001, 544),
                                           ("q8_0", 3, 32), ("q4_k", 6143, 4096), ("q6_k", 6145, 1024),
                                           ("q4_0", 6142, 512), ("q6_k", 4096, 5120), ("q4_0", 4100, 4096)])
@pytest.mark.parametrize("with_delta", [False, True])
def test_fused_norm_prologue(gpu, fmt, rows, cols, with_delta):
    w = synth.weights(fmt, rows, cols, seed=rows + cols)
    W = gpu.Weight(fmt, rows, cols, w)
    x = (RNG.standard_normal(cols) * 30).astype(np.float32)
    d = (RNG.standard_normal(cols) * 5).astype(np.float32)
    nw = (1 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    X, D, NW, Y = (gpu.DeviceBuffer.from_array(a) for a in (x, d, nw, np.zeros(rows, np.float32)))
    XO = gpu.DeviceBuffer(4 * cols)
    if with_delta:
        gpu.matvec_fused(W, X, Y, gpu.EPI_PLAIN, NW, 1e-5, D, XO)
        u = x + d  # one fp32 add, as the kernel takes it
    else:
        gpu.matvec_fused(W, X, Y, gpu.EPI_PLAIN, NW, 1e-5)
        u = x
    gpu.synchronize()
    want = _mv_ref(fmt, w, rows, cols, ref.rmsnorm(u, nw, 1e-5))
    assert rel_err(Y.download(np.float32), want) < 1e-3
    if with_delta:
        assert np.array_equal(XO.download(np.float32), u)
    assert np.array_equal(X.download(np.float32), x)  # x itself is not modified


@pytest.mark.parametrize("fmt,n,cols", [("q4_k", 14336, 4096), ("q4_k", 512, 256), ("q8_0", 1000, 512),
                                        ("q6_k", 2048, 5120), ("q8_0", 2048, 4096), ("q4_0", 2050, 4096)])
def test_fused_glu_epilogue(gpu, fmt, n, cols):
    g = synth.weights(fmt, n, cols, seed=3)
    u = synth.weights(fmt, n, cols, seed=4)
    W = gpu.glu_weight(fmt, n, cols, g, u)
    x = RNG.standard_normal(cols).astype(np.float32)
    X, Y = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * n)
    gpu.matvec_fused(W, X, Y, gpu.EPI_GLU)
    gpu.synchronize()
    want = ref.silu_mul(_mv_ref(fmt, g, n, cols, x), _mv_ref(fmt, u, n, cols, x))
    assert rel_err(Y.download(np.float32), want) < 1e-3
    # a plain product over the pair weight writes the rows interleaved
    Z = gpu.DeviceBuffer(8 * n)
    W.matvec(X, gpu.DTYPE_F32, 1, cols, Z, 2 * n)
    gpu.synchronize()
    z = Z.download(np.float32)
    assert rel_err(z[0::2], _mv_ref(fmt, g, n, cols, x)) < 1e-3
    assert rel_err(z[1::2], _mv_ref(fmt, u, n, cols, x)) < 1e-3


@pytest.mark.parametrize("fmt,n,cols", [("q4_k", 14336, 4096), ("q6_k", 2048, 5120), ("q4_k", 300, 4096)])
def test_fused_norm_and_glu(gpu, fmt, n, cols):
    """The decode step's gate/up form: the norm prologue (with a delta and
    x_out) and the GLU epilogue in one launch, at sizes that take the
    two-waves-per-tile form (the pairs 2i, 2i + 1 of a tile) and one that
    does not."""
    g = synth.weights(fmt, n, cols, seed=5)
    u = synth.weights(fmt, n, cols, seed=6)
    W = gpu.glu_weight(fmt, n, cols, g, u)
    x = (RNG.standard_normal(cols) * 30).astype(np.float32)
    d = (RNG.standard_normal(cols) * 5).astype(np.float32)
    nw = (1 + 0.1 * RNG.standard_normal(cols)).astype(np.float32)
    X, D, NW, Y = (gpu.DeviceBuffer.from_array(a) for a in (x, d, nw, np.zeros(n, np.float32)))
    XO = gpu.DeviceBuffer(4 * cols)
    gpu.matvec_fused(W, X, Y, gpu.EPI_GLU, NW, 1e-5, D, XO)
    gpu.synchronize()
    un = ref.rmsnorm(x + d, nw, 1e-5)
    want = ref.silu_mul(_mv_ref(fmt, g, n, cols, un), _mv_ref(fmt, u, n, cols, un))
    assert rel_err(Y.download(np.float32), want) < 1e-3
    assert np.array_equal(XO.download(np.float32), x + d)


@pytest.mark.parametrize("epi", ["plain", "glu"])
@pytest.mark.parametrize("fmt,n,cols", [("q4_k", 3072, 4096), ("q6_k", 2048, 5120), ("q4_k", 150, 4096)])
@pytest.mark.parametrize("bad", [np.nan, np.inf])
def test_fused_norm_non_finite(gpu, epi, fmt, n, cols, bad):
    """A NaN or an infinity in x + delta makes the norm's sum of squares, so
    every output of the product, non-finite (recipe's rmsnorm gives NaN there
    too), in both forms of the fused kernel and with either epilogue; x_out
    still receives x + delta as it is."""
    g = synth.weights(fmt, n, cols, seed=8)
    u = synth.weights(fmt, n, cols, seed=9)
    W = gpu.glu_weight(fmt, n, cols, g, u) if epi == "glu" else gpu.Weight(fmt, 2 * n, cols,
                                                                            np.concatenate([g, u]))
    x = RNG.standard_normal(cols).astype(np.float32)
    x[cols // 3] = bad
    d = RNG.standard_normal(cols).astype(np.float32)
    nw = np.ones(cols, np.float32)
    rows_out = n if epi == "glu" else 2 * n
    X, D, NW, Y = (gpu.DeviceBuffer.from_array(a) for a in (x, d, nw, np.zeros(rows_out, np.float32)))
    XO = gpu.DeviceBuffer(4 * cols)
    gpu.matvec_fused(W, X, Y, gpu.EPI_GLU if epi == "glu" else gpu.EPI_PLAIN, NW, 1e-5, D, XO)
    gpu.synchronize()
    assert not np.isfinite(Y.download(np.float32)).any()
    np.testing.assert_array_equal(XO.download(np.float32), x + d)  # (NaN where x + d is NaN)


@pytest.mark.parametrize("fmt,rows,cols", [("q8_0", 1001, 544), ("q8_0", 4096, 4096), ("q4_0", 77, 128),
                                           ("q4_k", 6143, 4096), ("q4_k", 4096, 14336), ("q4_0", 1001, 14336),
                                           ("q4_k", 4097, 8448)])
def test_fused_plain_without_norm(gpu, fmt, rows, cols):
    """The fused entry point with neither prologue nor epilogue equals the plain
    product bit for bit (one launch shape per format and row count; long Q4_K
    and Q4_0 rows take the two-waves-per-tile form up to 4,096 rows in both)."""
    w = synth.weights(fmt, rows, cols, seed=rows)
    W = gpu.Weight(fmt, rows, cols, w)
    x = RNG.standard_normal(cols).astype(np.float32)
    X, Y, Z = gpu.DeviceBuffer.from_array(x), gpu.DeviceBuffer(4 * rows), gpu.DeviceBuffer(4 * rows)
    gpu.matvec_fused(W, X, Y, gpu.EPI_PLAIN)
    W.matvec(X, gpu.DTYPE_F32, 1, cols, Z, rows)
    gpu.synchronize()
    y = Y.download(np.float32)
    assert rel_err(y, _mv_ref(fmt, w, rows, cols, x)) < 1e-3
    assert np.array_equal(y.view(np.uint32), Z.download(np.float32).view(np.uint32))


def test_fused_rejects_bad_arguments(gpu):
    w = synth.weights("q4_k", 64, 256, seed=1)
    W = gpu.Weight("q4_k", 64, 256, w)
    X, Y, D = gpu.DeviceBuffer(4 * 256), gpu.DeviceBuffer(4 * 64), gpu.DeviceBuffer(4 * 256)
    with pytest.raises(gpu.RqmvError):
        gpu.matvec_fused(W, X, Y, gpu.EPI_GLU)  # not a pair weight
    with pytest.raises(gpu.RqmvError):
        gpu.matvec_fused(W, X, Y, gpu.EPI_PLAIN, delta=D)  # a delta without the norm
    with pytest.raises(gpu.RqmvError):
        gpu.matvec_fused(W, X, Y, gpu.EPI_PLAIN, D, 1e-5, D, X)  # x_out over x


@pytest.mark.parametrize("nq,nkv,hd", [(32, 8, 128), (4, 2, 64), (8, 1, 256), (12, 4, 128), (24, 4, 64)])
@pytest.mark.parametrize("pos", [0, 63, 64, 300, 4099])
def test_attention_rope_fused(gpu, nq, nkv, hd, pos):
    """Rotary, cache append and attention in one call, against the f64
    reference (the new key and value rounded to fp16 as the cache holds them)."""
    max_ctx, base = 4100, 500000.0
    qkv = RNG.standard_normal((nq + 2 * nkv) * hd).astype(np.float32)
    kc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    vc = RNG.standard_normal((nkv, max_ctx, hd)).astype(np.float16)
    Q = gpu.DeviceBuffer.from_array(qkv)
    K = gpu.DeviceBuffer.from_array(kc.view(np.uint16))
    V = gpu.DeviceBuffer.from_array(vc.view(np.uint16))
    T = gpu.rope_table(hd, base, max_ctx)
    ws = gpu.attention_workspace(nq, nkv, hd, max_ctx)
    O = gpu.DeviceBuffer(nq * hd * 4)
    gpu.attention_rope(Q, T, K, V, _i32(gpu, pos), nq, nkv, hd, max_ctx, ws, O)
    gpu.synchronize()
    assert np.array_equal(Q.download(np.float32), qkv)  # qkv is not modified
    q_ref = ref.rope_neox(qkv[:nq * hd].reshape(nq, hd), pos, base)
    k_ref = ref.rope_neox(qkv[nq * hd:(nq + nkv) * hd].reshape(nkv, hd), pos, base)
    v_new = qkv[(nq + nkv) * hd:].reshape(nkv, hd)
    k_all = kc.astype(np.float64)
    v_all = vc.astype(np.float64)
    k_all[:, pos] = k_ref.astype(np.float32).astype(np.float16)
    v_all[:, pos] = v_new.astype(np.float16)
    want = ref.attention(q_ref, k_all, v_all, pos + 1)
    assert rel_err(O.download(np.float32), want.reshape(-1)) < 1e-5
    kg = K.download(np.uint16).reshape(nkv, max_ctx, hd).view(np.float16)
    vg = V.download(np.uint16).reshape(nkv, max_ctx, hd).view(np.float16)
    k16 = k_ref.astype(np.float16).astype(np.float64)
    assert np.all(np.abs(kg[:, pos].astype(np.float64) - k16) <= np.abs(k16) * 2 ** -10 + 2 ** -24)
    assert np.array_equal(vg[:, pos], v_new.astype(np.float16))
    others = np.ones(max_ctx, bool)
    others[pos] = False
    assert np.array_equal(kg[:, others], kc[:, others]) and np.array_equal(vg[:, others], vc[:, others])


def test_rope_table_matches_rope_kv(gpu):
    hd, base, rows = 128, 500000.0, 300
    T = gpu.rope_table(hd, base, rows)
    gpu.synchronize()
    t = T.download(np.float32).reshape(rows, hd // 2, 2)
    i = np.arange(hd // 2)
    for p in (0, 1, 77, 299):
        ang = p * np.exp(-(2.0 * i / hd) * np.log(base))
        assert np.array_equal(t[p, :, 0], np.cos(ang).astype(np.float32))
        assert np.array_equal(t[p, :, 1], np.sin(ang).astype(np.float32))


# ------------------------------------------------------------------ GGUF ----

def _write_llama_gguf(path, shape, D, layers_t, head, embed):
    import gguf_writer as gw
    from rqmv.decode import DecoderShape  # noqa: F401
    gt = {"q4_0": 2, "q8_0": 8, "q4_k": 12, "q6_k": 14}
    s = shape
    qkv_rows = s.qkv_rows
    meta = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.U32, s.layers),
            ("llama.embedding_length", gw.U32, s.d), ("llama.attention.head_count", gw.U32, s.q_heads),
            ("llama.attention.head_count_kv", gw.U32, s.kv_heads), ("llama.feed_forward_length", gw.U32, s.ffn),
            ("llama.rope.freq_base", gw.F32, s.rope_base), ("llama.attention.layer_norm_rms_epsilon", gw.F32, s.eps)]
    tensors = [("token_embd.weight", [s.d, s.vocab], 0, embed.astype(np.float32).tobytes())]
    pf = gt[s.proj_fmt]
    for i, t in enumerate(layers_t):
        rb = t.qkv.nbytes // qkv_rows
        nq, nk = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
        q, k, v = t.qkv[:nq * rb], t.qkv[nq * rb:(nq + nk) * rb], t.qkv[(nq + nk) * rb:]
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", [s.d], 0, t.attn_norm.astype(np.float32).tobytes()),
                    (p + "attn_q.weight", [s.d, nq], pf, q.tobytes()),
                    (p + "attn_k.weight", [s.d, nk], pf, k.tobytes()),
                    (p + "attn_v.weight", [s.d, nk], pf, v.tobytes()),
                    (p + "attn_output.weight", [s.d, s.d], pf, t.o.tobytes()),
                    (p + "ffn_norm.weight", [s.d], 0, t.ffn_norm.astype(np.float32).tobytes()),
                    (p + "ffn_gate.weight", [s.d, s.ffn], pf, t.gate.tobytes()),
                    (p + "ffn_up.weight", [s.d, s.ffn], pf, t.up.tobytes()),
                    (p + "ffn_down.weight", [s.ffn, s.d], pf, t.down.tobytes())]
    tensors += [("output_norm.weight", [s.d], 0, D.out_norm().astype(np.float32).tobytes()),
                ("output.weight", [s.d, s.vocab], gt[s.head_fmt], head.tobytes())]
    gw.write(path, meta, tensors)


def test_decode_from_gguf_matches_reference(gpu, tmp_path):
    from rqmv.decode import from_gguf
    shape = DecoderShape(layers=2, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=384)
    D = synth.DecoderSynth(shape, seed=8, norm_std=0.1)
    layers = [D.layer(i) for i in range(shape.layers)]
    head, embed = D.head(), D.embed()
    path = str(tmp_path / "tiny-llama.gguf")
    _write_llama_gguf(path, shape, D, layers, head, embed)
    max_ctx = 8
    model = from_gguf(path, max_ctx)
    assert model.shape.proj_fmt == "q4_k" and model.shape.kv_heads == 2 and model.shape.vocab == 384
    R = ref.DecoderReference(shape, embed, D.out_norm(), head, layers,
                             [(np.zeros((2, 0, 64), np.uint16), np.zeros((2, 0, 64), np.uint16))] * 2, max_ctx)
    stream = gpu.Stream()
    model.set_position(5, 0)
    token, pos = 5, 0
    for _ in range(3):  # a fresh sequence from position 0
        model.enqueue_step(stream)
        stream.synchronize()
        logits = model.read_logits()
        assert rel_err(logits, R.step(token, pos)) < 1e-3
        token, pos = model.read_token(), pos + 1
    stream.close()


def test_gguf_weight_matches_bytes(gpu, tmp_path):
    import gguf_writer as gw
    path = str(tmp_path / "w.gguf")
    w = synth.q6_k(48, 1024, seed=3)
    bank = synth.q4_k(3 * 64, 512, seed=4)
    gw.write(path, [], [("blk.0.ffn_down.weight", [1024, 48], 14, w.tobytes()),
                        ("blk.0.ffn_up_exps.weight", [512, 64, 3], 12, bank.tobytes())])
    g = gpu.Gguf(path)
    W = g.weight("blk.0.ffn_down.weight")
    assert W.info()["rows"] == 48 and W.info()["cols"] == 1024
    assert np.array_equal(W.unpack(), w)
    B = g.weight("blk.0.ffn_up_exps.weight")
    assert B.info()["experts"] == 3 and B.info()["rows"] == 64
    assert np.array_equal(B.unpack(), bank)
    x = RNG.standard_normal(1024).astype(np.float32)
    import oracle
    assert rel_err(gpu.contract(W, x), oracle.matvec_f64("q6_k", w, 48, 1024, x)[0]) < 1e-3
    with pytest.raises(gpu.RqmvError):
        g.weight("absent")


def _scaled_q6_k(rows, cols, seed, factor=0.25):
    """Q6_K blocks whose fp16 d is scaled, so their values stay near the Q4_K ones."""
    w = synth.q6_k(rows, cols, seed=seed).reshape(-1, 210)
    d = w[:, 208:210].copy().view(np.float16).astype(np.float32) * factor
    w[:, 208:210] = d.astype(np.float16).view(np.uint8)
    return w.reshape(-1)


def test_decode_from_q4_k_m_style_gguf(gpu, tmp_path):
    """A file laid out as llama.cpp's Q4_K_M mixes formats: Q4_K token_embd and
    attn_q / attn_k, Q6_K attn_v and (in some layers) ffn_down, a Q6_K output.
    Every projection keeps its own format; Q, K and V of two formats run as two
    products into one QKV vector; token_embd is decoded on the device."""
    import gguf_writer as gw
    from rqmv.decode import from_gguf
    shape = DecoderShape(layers=2, d=256, q_heads=4, kv_heads=2, head_dim=64, ffn=512, vocab=384,
                         head_fmt="q6_k")
    D = synth.DecoderSynth(shape, seed=12, norm_std=0.1)
    s = shape
    nq, nk = s.q_heads * s.head_dim, s.kv_heads * s.head_dim
    embed = synth.q4_k(s.vocab, s.d, seed=31)
    head = _scaled_q6_k(s.vocab, s.d, seed=32)
    meta = [("general.architecture", gw.STRING, "llama"), ("llama.block_count", gw.U32, s.layers),
            ("llama.embedding_length", gw.U32, s.d), ("llama.attention.head_count", gw.U32, s.q_heads),
            ("llama.attention.head_count_kv", gw.U32, s.kv_heads), ("llama.feed_forward_length", gw.U32, s.ffn),
            ("llama.rope.freq_base", gw.F32, s.rope_base), ("llama.attention.layer_norm_rms_epsilon", gw.F32, s.eps)]
    tensors = [("token_embd.weight", [s.d, s.vocab], 12, embed.tobytes())]
    layers = []
    for i in range(s.layers):
        t = D.layer(i)
        rb = t.qkv.nbytes // s.qkv_rows
        q, k = t.qkv[:nq * rb], t.qkv[nq * rb:(nq + nk) * rb]
        v = _scaled_q6_k(nk, s.d, seed=40 + i)
        down_fmt = "q6_k" if i == 0 else "q4_k"
        down = _scaled_q6_k(s.d, s.ffn, seed=50 + i) if i == 0 else t.down
        p = f"blk.{i}."
        tensors += [(p + "attn_norm.weight", [s.d], 0, t.attn_norm.astype(np.float32).tobytes()),
                    (p + "attn_q.weight", [s.d, nq], 12, q.tobytes()), (p + "attn_k.weight", [s.d, nk], 12, k.tobytes()),
                    (p + "attn_v.weight", [s.d, nk], 14, v.tobytes()),
                    (p + "attn_output.weight", [s.d, s.d], 12, t.o.tobytes()),
                    (p + "ffn_norm.weight", [s.d], 0, t.ffn_norm.astype(np.float32).tobytes()),
                    (p + "ffn_gate.weight", [s.d, s.ffn], 12, t.gate.tobytes()),
                    (p + "ffn_up.weight", [s.d, s.ffn], 12, t.up.tobytes()),
                    (p + "ffn_down.weight", [s.ffn, s.d], 14 if i == 0 else 12, down.tobytes())]
        layers.append(type(t)(attn_norm=t.attn_norm, qkv=None, o=t.o, ffn_norm=t.ffn_norm, gate=t.gate, up=t.up,
                              down=down, fmts={"down": down_fmt},
                              qkv_parts=[("q4_k", nq, q), ("q4_k", nk, k), ("q6_k", nk, v)]))
    tensors += [("output_norm.weight", [s.d], 0, D.out_norm().astype(np.float32).tobytes()),
                ("output.weight", [s.d, s.vocab], 14, head.tobytes())]
    path = str(tmp_path / "q4km.gguf")
    gw.write(path, meta, tensors)
    max_ctx = 8
    model = from_gguf(path, max_ctx)
    assert model.shape.head_fmt == "q6_k" and len(model.layers[0]["qkv"]) == 2
    R = ref.DecoderReference(shape, ("q4_k", embed), D.out_norm(), head, layers,
                             [(np.zeros((2, 0, 64), np.uint16), np.zeros((2, 0, 64), np.uint16))] * 2, max_ctx)
    stream = gpu.Stream()
    token, pos = 7, 0
    model.set_position(token, pos)
    for _ in range(3):
        model.enqueue_step(stream)
        stream.synchronize()
        logits = model.read_logits()
        want = R.step(token, pos)
        assert np.isfinite(want).all() and rel_err(logits, want) < 1e-3, pos
        token, pos = model.read_token(), pos + 1
    # and captured: a graph replay continues the sequence
    g = model.capture(stream)
    g.launch(stream)
    stream.synchronize()
    assert rel_err(model.read_logits(), R.step(token, pos)) < 1e-3
    g.close()
    stream.close()
