"""Single-token decode of a llama-style decoder on the device.

One step runs, for a token held in device memory at a position held in device
memory (so that a captured step replays at the next position):

    x = embed[token]
    per layer:  qkv = W_qkv rmsnorm(x) * attn_norm        (one fused projection, [q | k | v] heads)
                rotate q, k (NeoX); append k, v (fp16) to the layer's cache at pos
                a = attention(q, cache[0..pos])          (grouped-query, 1/sqrt(head_dim))
                x += W_o a
                h = silu(W_gate xn) * (W_up xn),  xn = rmsnorm(x) * ffn_norm
                x += W_down h
    logits = W_head rmsnorm(x) * out_norm;  token = argmax(logits);  pos += 1

This is recipe's attention block and SiLU-GLU feed-forward (lower_attention,
recipe.rs:23056-23150; lower_normalize, recipe.rs:23190-23210; silu(gate) * up,
recipe.rs:23279-23286, 22662-22668) run one position at a time. Every
projection is a quantized matrix-vector product of librqmv, with the norms,
the SiLU-GLU product and the residual adds folded into the products
(rqmv_matvec_fused): a product's output is added to the residual stream by the
next product's prologue, which also takes the sum of squares for its norm and
writes the updated stream (two buffers, alternating); the rotary and the cache
append are folded into attention (rqmv_attention_rope). Six launches per
layer: QKV, attention (two), output, gate/up, down. The residual stream and every activation are fp32; the KV cache is fp16.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import (EPI_GLU, EPI_PLAIN, DeviceBuffer, Graph, Stream, Weight, advance, argmax, argmax_workspace,
               attention_rope, attention_workspace, embed_row, glu_weight, matvec_fused, rope_table)


@dataclass(frozen=True)
class DecoderShape:
    layers: int = 32
    d: int = 4096
    q_heads: int = 32
    kv_heads: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    rope_base: float = 500000.0
    eps: float = 1e-5
    proj_fmt: str = "q4_k"
    head_fmt: str = "q8_0"

    @property
    def qkv_rows(self) -> int:
        return (self.q_heads + 2 * self.kv_heads) * self.head_dim

    def validate(self):
        if self.d % 256 or self.ffn % 256:
            raise ValueError("d and ffn must be multiples of 256 (one K-quant superblock)")
        if self.q_heads * self.head_dim != self.d:
            raise ValueError("q_heads * head_dim must equal d")
        if self.q_heads % self.kv_heads or self.q_heads // self.kv_heads > 8:
            raise ValueError("q_heads must be a multiple of kv_heads, at most 8 per kv head")
        if self.head_dim not in (64, 128, 256):
            raise ValueError("head_dim must be 64, 128 or 256")


@dataclass
class LayerTensors:
    """One layer's tensors as the file stores them: fp32 norm scales and GGUF
    blocks (rows of W_q, W_k, W_v stacked as one QKV projection; W_gate and
    W_up as ffn_gate and ffn_up). Every projection is in the shape's proj_fmt
    unless `fmts` names its own ("qkv", "o", "gate", "up", "down"). A QKV
    projection whose parts differ in format (a Q4_K_M file's Q6_K attn_v) comes
    as `qkv_parts`: (format, rows, blocks) for Q, K and V in order; consecutive
    parts of one format run as one product."""
    attn_norm: np.ndarray
    qkv: np.ndarray | None
    o: np.ndarray
    ffn_norm: np.ndarray
    gate: np.ndarray
    up: np.ndarray
    down: np.ndarray
    fmts: dict | None = None
    qkv_parts: list | None = None

    def fmt(self, name: str, default: str) -> str:
        return (self.fmts or {}).get(name, default)

    def qkv_runs(self, default: str, q_rows: int, kv_rows: int) -> list:
        """[(format, rows, blocks)] for the QKV projection, runs of one format merged."""
        parts = self.qkv_parts
        if parts is None:
            return [(self.fmt("qkv", default), q_rows + 2 * kv_rows, self.qkv)]
        runs = []
        for fmt, rows, blocks in parts:
            blocks = np.ascontiguousarray(blocks).view(np.uint8).reshape(-1)
            if runs and runs[-1][0] == fmt:
                runs[-1] = (fmt, runs[-1][1] + rows, np.concatenate([runs[-1][2], blocks]))
            else:
                runs.append((fmt, rows, blocks))
        if sum(r for _, r, _ in runs) != q_rows + 2 * kv_rows:
            raise ValueError("qkv_parts must hold the Q, K and V rows")
        return runs


class DecodeModel:
    """The device state of one decoder: weights, caches and step buffers."""

    def __init__(self, shape: DecoderShape, max_ctx: int, embed, out_norm: np.ndarray, head: np.ndarray):
        """embed: the fp32 table [vocab, d], or (format, GGUF blocks) of a
        quantized token_embd, decoded once to fp32 on the device."""
        shape.validate()
        self.shape, self.max_ctx = shape, int(max_ctx)
        s = shape
        if isinstance(embed, tuple):
            fmt, blocks = embed
            table = Weight(fmt, s.vocab, s.d, blocks)
            self.embed = DeviceBuffer(4 * s.vocab * s.d)
            table.dequantize(self.embed)
            table.close()
        else:
            embed = np.ascontiguousarray(embed, dtype=np.float32)
            if embed.shape != (s.vocab, s.d):
                raise ValueError(f"embedding table must be {(s.vocab, s.d)}, got {embed.shape}")
            self.embed = DeviceBuffer.from_array(embed)
        self.out_norm = DeviceBuffer.from_array(np.ascontiguousarray(out_norm, dtype=np.float32))
        self.head = Weight(s.head_fmt, s.vocab, s.d, head)
        self.layers: list[dict | None] = [None] * s.layers
        cache_bytes = s.kv_heads * self.max_ctx * s.head_dim * 2
        self.k_cache = [DeviceBuffer(cache_bytes) for _ in range(s.layers)]
        self.v_cache = [DeviceBuffer(cache_bytes) for _ in range(s.layers)]
        f32 = 4
        self.xs = [DeviceBuffer(s.d * f32), DeviceBuffer(s.d * f32)]  # the residual stream, alternating
        self.qkv = DeviceBuffer(s.qkv_rows * f32)
        self.attn = DeviceBuffer(s.d * f32)
        self.y_o = DeviceBuffer(s.d * f32)  # output projection, added by the next prologue
        self.h = DeviceBuffer(s.ffn * f32)
        self.y_f = DeviceBuffer(s.d * f32)  # down projection, added by the next prologue
        self.logits = DeviceBuffer(s.vocab * f32)
        self.token = DeviceBuffer(4)
        self.pos = DeviceBuffer(4)
        self.workspace = attention_workspace(s.q_heads, s.kv_heads, s.head_dim, self.max_ctx)
        self.argmax_ws = argmax_workspace()
        self.rope = rope_table(s.head_dim, s.rope_base, self.max_ctx)
        self._pos: int | None = None  # host count of the position (set_position, step, replay)
        self._hidden: DeviceBuffer | None = None  # the buffer the head's prologue writes the stream to

    # ---------------------------------------------------------------- setup
    def set_layer(self, index: int, t: LayerTensors):
        s = self.shape
        gate_fmt, up_fmt = t.fmt("gate", s.proj_fmt), t.fmt("up", s.proj_fmt)
        if gate_fmt != up_fmt:
            raise ValueError("ffn_gate and ffn_up must share a format (they run as one pair weight)")
        runs, at = [], 0
        for fmt, rows, blocks in t.qkv_runs(s.proj_fmt, s.q_heads * s.head_dim, s.kv_heads * s.head_dim):
            runs.append((Weight(fmt, rows, s.d, blocks), self.qkv.view(4 * at, 4 * rows)))
            at += rows
        self.layers[index] = {
            "attn_norm": DeviceBuffer.from_array(np.ascontiguousarray(t.attn_norm, dtype=np.float32)),
            "qkv": runs,
            "o": Weight(t.fmt("o", s.proj_fmt), s.d, s.d, t.o),
            "ffn_norm": DeviceBuffer.from_array(np.ascontiguousarray(t.ffn_norm, dtype=np.float32)),
            "gate_up": glu_weight(gate_fmt, s.ffn, s.d, t.gate, t.up),
            "down": Weight(t.fmt("down", s.proj_fmt), s.d, s.ffn, t.down),
        }

    def set_cache(self, index: int, k: np.ndarray, v: np.ndarray):
        """Prefill layer `index`'s cache: k, v are fp16 bits [kv_heads, n, head_dim]
        for positions 0..n-1."""
        s = self.shape
        for buf, src in ((self.k_cache[index], k), (self.v_cache[index], v)):
            src = np.asarray(src, dtype=np.uint16)
            n = src.shape[1]
            if src.shape != (s.kv_heads, n, s.head_dim) or n > self.max_ctx:
                raise ValueError(f"cache prefill must be [kv_heads, n <= max_ctx, head_dim], got {src.shape}")
            full = np.zeros((s.kv_heads, self.max_ctx, s.head_dim), dtype=np.uint16)
            full[:, :n] = src
            buf.upload(full)

    def set_position(self, token: int, pos: int):
        """The next step decodes `token` at `pos`; pos must lie inside the
        cache (recipe refuses a step whose token window is outside the
        placement's capacity, recipe.rs:21330-21331)."""
        if not 0 <= pos < self.max_ctx:
            raise ValueError(f"position {pos} is outside the cache (0..{self.max_ctx - 1}): the token window is "
                             "outside the placement capacity")
        self.token.upload(np.array([token], dtype=np.int32))
        self.pos.upload(np.array([pos], dtype=np.int32))
        self._pos = pos

    def _room(self, steps: int):
        """Raises unless `steps` more steps stay inside the cache (host count
        of the steps run through step() and replay())."""
        if self._pos is None:
            raise RuntimeError("set_position must come before the first step")
        if self._pos + steps > self.max_ctx:
            raise ValueError(f"{steps} step(s) from position {self._pos} run past the cache's {self.max_ctx} "
                             "positions: the token window is outside the placement capacity")

    def step(self, stream: Stream | None = None):
        """One eager step at the current position; raises before a step past the cache."""
        self._room(1)
        self.enqueue_step(stream)
        self._pos += 1

    def replay(self, graph: Graph, stream: Stream, times: int = 1):
        """`times` replays of a captured step; raises before any would run past the cache."""
        self._room(times)
        for _ in range(times):
            graph.launch(stream)
        self._pos += times

    def _check_inside(self):
        """The device position after a step is at most max_ctx; beyond it a
        step ran past the cache (a graph launched directly, past the end), and
        its results are refused."""
        p = self.read_position()
        if p > self.max_ctx:
            raise RuntimeError(f"a step ran at position {p - 1}, outside the cache (0..{self.max_ctx - 1}): the "
                               "token window is outside the placement capacity")

    # ----------------------------------------------------------------- step
    def enqueue_step(self, stream: Stream | None = None, layers: int | None = None):
        """Enqueue one decode step on `stream` (capturable: no allocation, no
        host synchronisation). `layers` < the decoder's depth runs only the
        first `layers` layers before the head (an early exit); read_hidden()
        then returns the stream that layer `layers` would take as input."""
        s = self.shape
        if any(layer is None for layer in self.layers):
            raise RuntimeError("every layer must be set before a step")
        depth = s.layers if layers is None else int(layers)
        if not 1 <= depth <= s.layers:
            raise ValueError(f"layers must be 1..{s.layers}, got {layers}")
        xs = self.xs
        embed_row(self.embed, s.vocab, s.d, self.token, xs[0], stream)
        cur, pending = 0, None  # pending: the down projection not yet added to the stream
        for i, L in enumerate(self.layers[:depth]):
            (w0, y0), rest = L["qkv"][0], L["qkv"][1:]
            if pending is None:
                matvec_fused(w0, xs[cur], y0, EPI_PLAIN, L["attn_norm"], s.eps, stream=stream)
            else:
                matvec_fused(w0, xs[cur], y0, EPI_PLAIN, L["attn_norm"], s.eps, pending, xs[1 - cur], stream=stream)
                cur = 1 - cur
            for w, y in rest:  # further format runs of Q, K, V read the updated stream
                matvec_fused(w, xs[cur], y, EPI_PLAIN, L["attn_norm"], s.eps, stream=stream)
            attention_rope(self.qkv, self.rope, self.k_cache[i], self.v_cache[i], self.pos, s.q_heads, s.kv_heads,
                           s.head_dim, self.max_ctx, self.workspace, self.attn, stream)
            matvec_fused(L["o"], self.attn, self.y_o, EPI_PLAIN, stream=stream)
            matvec_fused(L["gate_up"], xs[cur], self.h, EPI_GLU, L["ffn_norm"], s.eps, self.y_o, xs[1 - cur],
                         stream=stream)
            cur = 1 - cur
            matvec_fused(L["down"], self.h, self.y_f, EPI_PLAIN, stream=stream)
            pending = self.y_f
        matvec_fused(self.head, xs[cur], self.logits, EPI_PLAIN, self.out_norm, s.eps, pending, xs[1 - cur],
                     stream=stream)
        self._hidden = xs[1 - cur]
        argmax(self.logits, s.vocab, self.token, self.argmax_ws, stream)
        advance(self.pos, stream)

    def capture(self, stream: Stream) -> Graph:
        """A HIP graph of one step; each launch decodes the next token."""
        return Graph(stream, lambda: self.enqueue_step(stream))

    def read_logits(self) -> np.ndarray:
        self._check_inside()
        return self.logits.download(np.float32, self.shape.vocab)

    def read_token(self) -> int:
        self._check_inside()
        return int(self.token.download(np.int32, 1)[0])

    def read_hidden(self) -> np.ndarray:
        """The residual stream after the last layer of the latest step (the
        head's input, before its norm)."""
        if self._hidden is None:
            raise RuntimeError("no step has been enqueued")
        self._check_inside()
        return self._hidden.download(np.float32, self.shape.d)

    def read_position(self) -> int:
        return int(self.pos.download(np.int32, 1)[0])

    def weight_bytes(self) -> int:
        """GGUF bytes of every projection and the head (what one step streams)."""
        total = self.head.gguf_nbytes
        for L in self.layers:
            total += sum(L[k].gguf_nbytes for k in ("o", "gate_up", "down")) + sum(w.gguf_nbytes for w, _ in L["qkv"])
        return total


# ------------------------------------------------------------- from GGUF ----

_GGML_FORMAT = {2: "q4_0", 8: "q8_0", 12: "q4_k", 14: "q6_k"}


def _f32_vector(g, name: str) -> np.ndarray:
    t = g.tensor(name)
    if t is None:
        raise ValueError(f"{name} is absent")
    raw = g.data(name)
    if t.ggml_type == 0:
        return raw.view(np.float32).copy()
    if t.ggml_type == 1:
        return raw.view(np.float16).astype(np.float32)
    raise ValueError(f"{name} must be F32 or F16, not GGML type {t.ggml_type}")


def from_gguf(path: str, max_ctx: int) -> DecodeModel:
    """A DecodeModel from a llama-style GGUF file, with recipe's tensor names
    (token_embd, blk.N.attn_norm / attn_q / attn_k / attn_v or attn_qkv /
    attn_output / ffn_norm / ffn_gate / ffn_up / ffn_down, output_norm,
    output; recipe.rs:14382-14457, 17798-17860) and hyperparameters
    (<arch>.block_count, embedding_length, attention.head_count(_kv),
    feed_forward_length, rope.freq_base (default 10000),
    attention.layer_norm_rms_epsilon (default 1e-5); recipe.rs:17806-17936).
    Separate Q, K and V projections of one format are stacked into one QKV
    weight (of different formats, as in a Q4_K_M file's Q6_K attn_v, they run
    as consecutive products into the QKV vector); gate and up become one pair
    weight; every projection keeps its own format; a quantized token_embd is
    decoded to fp32 once on the device; blocks are uploaded from the mapped
    file."""
    from . import Gguf

    g = Gguf(path)
    arch = g.get_string("general.architecture")

    def meta_int(key):
        return g.get_int(f"{arch}.{key}")

    def meta_float(key, default):
        try:
            return g.get_float(f"{arch}.{key}")
        except Exception:
            return default

    layers = meta_int("block_count")
    d = meta_int("embedding_length")
    nq = meta_int("attention.head_count")
    try:
        nkv = meta_int("attention.head_count_kv")
    except Exception:
        nkv = nq
    ffn = meta_int("feed_forward_length")
    embed_info = g.tensor("token_embd.weight")
    if embed_info is None or embed_info.shape[0] != d:
        raise ValueError("token_embd.weight must be [embedding_length, vocabulary]")
    vocab = embed_info.shape[1]
    head_info = g.tensor("output.weight")
    if head_info is None:
        raise ValueError("output.weight is absent")
    q0 = g.tensor("blk.0.attn_qkv.weight") or g.tensor("blk.0.attn_q.weight")
    if q0 is None or q0.ggml_type not in _GGML_FORMAT or head_info.ggml_type not in _GGML_FORMAT:
        raise ValueError("projections and the head must be Q4_0, Q8_0, Q4_K or Q6_K")
    shape = DecoderShape(layers=layers, d=d, q_heads=nq, kv_heads=nkv, head_dim=d // nq, ffn=ffn, vocab=vocab,
                         rope_base=meta_float("rope.freq_base", 10000.0),
                         eps=meta_float("attention.layer_norm_rms_epsilon", 1e-5),
                         proj_fmt=_GGML_FORMAT[q0.ggml_type], head_fmt=_GGML_FORMAT[head_info.ggml_type])
    if embed_info.ggml_type == 0:
        embed = g.data("token_embd.weight").view(np.float32).reshape(vocab, d)
    elif embed_info.ggml_type == 1:
        embed = g.data("token_embd.weight").view(np.float16).astype(np.float32).reshape(vocab, d)
    elif embed_info.ggml_type in _GGML_FORMAT:  # decoded to fp32 once, on the device
        embed = (_GGML_FORMAT[embed_info.ggml_type], g.data("token_embd.weight"))
    else:
        raise ValueError("token_embd.weight must be F32, F16, Q4_0, Q8_0, Q4_K or Q6_K")
    model = DecodeModel(shape, max_ctx, embed, _f32_vector(g, "output_norm.weight"), g.data("output.weight"))
    hd = d // nq
    for i in range(layers):
        p = f"blk.{i}."

        def fmt_of(name):
            t = g.tensor(p + name)
            if t is None:
                raise ValueError(f"{p + name} is absent")
            if t.ggml_type not in _GGML_FORMAT:
                raise ValueError(f"{p + name} must be Q4_0, Q8_0, Q4_K or Q6_K")
            return _GGML_FORMAT[t.ggml_type]

        fmts = {k: fmt_of(f"{n}.weight") for k, n in (("o", "attn_output"), ("gate", "ffn_gate"), ("up", "ffn_up"),
                                                      ("down", "ffn_down"))}
        qkv, parts = None, None
        if g.tensor(p + "attn_qkv.weight") is not None:
            fmts["qkv"] = fmt_of("attn_qkv.weight")
            qkv = g.data(p + "attn_qkv.weight")
        else:
            f3 = [fmt_of(f"attn_{n}.weight") for n in "qkv"]
            data = [g.data(p + f"attn_{n}.weight") for n in "qkv"]
            if f3[0] == f3[1] == f3[2]:
                fmts["qkv"] = f3[0]
                qkv = np.concatenate(data)
            else:  # a Q4_K_M file: attn_v in Q6_K beside Q4_K attn_q / attn_k
                parts = [(f3[0], nq * hd, data[0]), (f3[1], nkv * hd, data[1]), (f3[2], nkv * hd, data[2])]
        model.set_layer(i, LayerTensors(attn_norm=_f32_vector(g, p + "attn_norm.weight"), qkv=qkv,
                                        o=g.data(p + "attn_output.weight"), ffn_norm=_f32_vector(g, p + "ffn_norm.weight"),
                                        gate=g.data(p + "ffn_gate.weight"), up=g.data(p + "ffn_up.weight"),
                                        down=g.data(p + "ffn_down.weight"), fmts=fmts, qkv_parts=parts))
    g.close()
    return model
