"""f64 restatement of one single-token decode step of a llama-style decoder.

TEST INFRASTRUCTURE ONLY: the checker of the device decode step (tests/ and
smoke()); the product never imports it.

Semantics (recipe's attention block and feed-forward, one position at a time):
- RMSNorm: x / sqrt(mean(x^2) + eps) * scale (lower_normalize,
  recipe.rs:23190-23210; emit_normalize_stats, recipe.rs:6836-6870).
- Fused QKV projection laid out [q heads | k heads | v heads]; rotary on
  queries and keys; scores q.k / sqrt(head_dim); softmax over positions
  0..pos; weighted sum of values; output projection (lower_attention,
  recipe.rs:23056-23150).
- NeoX rotary without yarn (rope_pair, amd-nv-cpu.ll:3719-3780): pair i of a
  head is (x_i, x_{i+half}), angle = pos * exp(-(2i/dims) * log(base)),
  lower = a cos - b sin, upper = b cos + a sin.
- SiLU-GLU: silu(gate) * up with silu(v) = v * sigmoid(v) and the sigmoid
  taken as 0.5 (tanh(v / 2) + 1) (recipe.rs:23279-23286, 22662-22668).
- The KV cache stores fp16: the appended key (after rotation) and value are
  rounded to fp16 (round to nearest even), as the device cache holds them.
Projection weights are dequantized with the oracle's bit-exact decoders and
every product, sum and transcendental is taken in float64.

Pins (tests/test_oracle_decode.py): RMSNorm of a constant vector and its
scale invariance; the rotary equal to multiplying each pair, as a complex
number, by exp(i pos base^(-2i/dims)), the identity at pos 0, and scores that
depend on the relative position only; attention over one position returning
its value, over identical keys returning the mean of the values, and equal to
scipy's softmax with the query-to-kv-head grouping; SiLU-GLU against scipy's
logistic function; a decoder whose output and down projections are zero
reducing to the head applied to the normalised embedding.
"""
from __future__ import annotations

import numpy as np

from . import dequant_rows, matvec_f64


def rmsnorm(x: np.ndarray, scale: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, dtype=np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(scale, dtype=np.float64)


def rope_neox(heads: np.ndarray, pos: int, base: float) -> np.ndarray:
    """Rotate each row (a head of even width) by the NeoX rotary at `pos`."""
    h = np.array(heads, dtype=np.float64, copy=True)
    dims = h.shape[-1]
    half = dims // 2
    i = np.arange(half, dtype=np.float64)
    angle = float(pos) * np.exp(-(2.0 * i / dims) * np.log(base))
    c, s = np.cos(angle), np.sin(angle)
    a, b = h[..., :half].copy(), h[..., half:].copy()
    h[..., :half] = a * c - b * s
    h[..., half:] = b * c + a * s
    return h


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, length: int) -> np.ndarray:
    """q [nq, hd]; k, v [nkv, >= length, hd]; query head h reads kv head h // (nq / nkv)."""
    nq, hd = q.shape
    nkv = k.shape[0]
    group = nq // nkv
    out = np.empty((nq, hd), dtype=np.float64)
    for h in range(nq):
        kh = h // group
        s = (k[kh, :length].astype(np.float64) @ q[h].astype(np.float64)) / np.sqrt(hd)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[kh, :length].astype(np.float64)
    return out


def silu_mul(gate: np.ndarray, up: np.ndarray) -> np.ndarray:
    g = np.asarray(gate, dtype=np.float64)
    return g * (0.5 * (np.tanh(0.5 * g) + 1.0)) * np.asarray(up, dtype=np.float64)


def _fp16_round(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)


def layer_forward(s, mv, attn_norm, ffn_norm, caches, X, pos: int) -> np.ndarray:
    """One decoder layer at `pos` for each row of X (m residual streams,
    float64). mv(name, A) multiplies projection `name` ("qkv", "o", "gate",
    "up", "down") by each row of A and returns the products as rows;
    caches[j] = (k, v), float64 arrays [kv_heads, > pos, head_dim] of stream j,
    which receive that stream's key and value at pos. Returns the streams
    after the layer."""
    hd, nq, nkv = s.head_dim, s.q_heads, s.kv_heads
    X = np.atleast_2d(np.asarray(X, dtype=np.float64))
    QKV = mv("qkv", np.stack([rmsnorm(x, attn_norm, s.eps) for x in X]))
    A = []
    for j, qkv in enumerate(QKV):
        q = rope_neox(qkv[:nq * hd].reshape(nq, hd), pos, s.rope_base)
        k = rope_neox(qkv[nq * hd:(nq + nkv) * hd].reshape(nkv, hd), pos, s.rope_base)
        v = qkv[(nq + nkv) * hd:].reshape(nkv, hd)
        kc, vc = caches[j]
        kc[:, pos] = _fp16_round(k)
        vc[:, pos] = _fp16_round(v)
        A.append(attention(q, kc, vc, pos + 1).reshape(-1))
    X = X + mv("o", np.stack(A))
    XN = np.stack([rmsnorm(x, ffn_norm, s.eps) for x in X])
    return X + mv("down", silu_mul(mv("gate", XN), mv("up", XN)))


def f64_cache(bits: np.ndarray, max_ctx: int) -> np.ndarray:
    """fp16 bits [kv_heads, n, head_dim] -> float64 [kv_heads, max_ctx, head_dim], zero past n."""
    bits = np.asarray(bits, dtype=np.uint16)
    out = np.zeros((bits.shape[0], max_ctx, bits.shape[2]))
    out[:, :bits.shape[1]] = bits.view(np.float16).astype(np.float64)
    return out


class QuantLayer:
    """One layer's projections as stored (GGUF blocks), multiplied by the
    oracle's f64 row products on `threads` threads, without dequantizing the
    whole matrix: the checker of decoders too large to hold as float64."""

    def __init__(self, s, t, threads: int = 1):
        fmts = getattr(t, "fmts", None) or {}
        f = lambda name: fmts.get(name, s.proj_fmt)  # noqa: E731
        qkv_rows = (s.q_heads + 2 * s.kv_heads) * s.head_dim
        parts = getattr(t, "qkv_parts", None) or [(f("qkv"), qkv_rows, t.qkv)]
        self.parts = {"qkv": [(fmt, rows, s.d, blocks) for fmt, rows, blocks in parts],
                      "o": [(f("o"), s.d, s.d, t.o)], "gate": [(f("gate"), s.ffn, s.d, t.gate)],
                      "up": [(f("up"), s.ffn, s.d, t.up)], "down": [(f("down"), s.d, s.ffn, t.down)]}
        self.attn_norm = np.asarray(t.attn_norm, dtype=np.float64)
        self.ffn_norm = np.asarray(t.ffn_norm, dtype=np.float64)
        self.threads = threads

    def __call__(self, name: str, A: np.ndarray) -> np.ndarray:
        return np.hstack([matvec_f64(fmt, blocks, rows, cols, A, self.threads)
                          for fmt, rows, cols, blocks in self.parts[name]])


class DecoderReference:
    """The decoder's weights dequantized once; `step` advances one token.

    `shape` has layers, d, q_heads, kv_heads, head_dim, ffn, vocab, rope_base,
    eps, proj_fmt, head_fmt. Caches are float64 arrays [kv_heads, max_ctx,
    head_dim] holding fp16 values."""

    def __init__(self, shape, embed, out_norm, head, layers, caches, max_ctx: int):
        s = self.shape = shape
        if isinstance(embed, tuple):  # (format, blocks) of a quantized token_embd
            self.embed = dequant_rows(embed[0], embed[1], s.vocab, s.d).reshape(s.vocab, s.d).astype(np.float64)
        else:
            self.embed = np.asarray(embed, dtype=np.float64)
        self.out_norm = np.asarray(out_norm, dtype=np.float64)
        self.head = dequant_rows(s.head_fmt, head, s.vocab, s.d).reshape(s.vocab, s.d).astype(np.float64)
        qkv_rows = (s.q_heads + 2 * s.kv_heads) * s.head_dim
        self.layers = []

        def deq(fmt, blocks, rows, cols):
            return dequant_rows(fmt, blocks, rows, cols).reshape(rows, cols).astype(np.float64)

        for t in layers:
            # per-tensor formats (a Q4_K_M file) where the layer names them
            fmts = getattr(t, "fmts", None) or {}
            f = lambda name: fmts.get(name, s.proj_fmt)  # noqa: E731
            parts = getattr(t, "qkv_parts", None)
            if parts:
                qkv = np.vstack([deq(fmt, blocks, rows, s.d) for fmt, rows, blocks in parts])
            else:
                qkv = deq(f("qkv"), t.qkv, qkv_rows, s.d)
            self.layers.append({
                "attn_norm": np.asarray(t.attn_norm, dtype=np.float64),
                "qkv": qkv,
                "o": deq(f("o"), t.o, s.d, s.d),
                "ffn_norm": np.asarray(t.ffn_norm, dtype=np.float64),
                "gate": deq(f("gate"), t.gate, s.ffn, s.d),
                "up": deq(f("up"), t.up, s.ffn, s.d),
                "down": deq(f("down"), t.down, s.d, s.ffn),
            })
        self.k = [f64_cache(kc, max_ctx) for kc, _ in caches]
        self.v = [f64_cache(vc, max_ctx) for _, vc in caches]

    def step(self, token: int, pos: int) -> np.ndarray:
        """Logits of the token at `pos` (its key and value join the caches)."""
        s = self.shape
        x = self.embed[token % s.vocab].copy()
        for i, L in enumerate(self.layers):
            x = layer_forward(s, lambda name, A, L=L: A @ L[name].T, L["attn_norm"], L["ffn_norm"],
                              [(self.k[i], self.v[i])], x, pos)[0]
        return self.head @ rmsnorm(x, self.out_norm, s.eps)
