"""Seeded synthetic GGUF workloads for the quantized matrix-vector path.

Every draw comes from a counter-based splitmix64 stream: value i of stream s
under seed S is splitmix64's output for the state S' + (i + 1) * 0x9E3779B97F4A7C15,
with S' a mix of S and s. Uniform integers take the top 53 bits scaled to the
range; normals are Box-Muller over two uniforms. fp16 values are produced by
recipe's own float-to-half conversion (recipe.rs:15098-15113), restated here
vectorised. The default seed is recipe's (Cargo.toml:113).

The distributions follow the workload definitions: weights' integer fields
uniform over their range, fp16 block scales |N(0,1)| * 0.01 (Q4_K dmin
|N(0,1)| * 0.005), activations N(0,1), the MoE router N(0, 0.02).
"""
from __future__ import annotations

import numpy as np

DEFAULT_SEED = 17
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

BLOCK = {"q4_0": (32, 18), "q8_0": (32, 34), "q4_k": (256, 144), "q6_k": (256, 210), "f16": (1, 2)}
GGML_TYPE = {"f16": 1, "q4_0": 2, "q8_0": 8, "q4_k": 12, "q6_k": 14}


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_u64(seed: int, stream: str, count: int) -> np.ndarray:
    """`count` 64-bit draws of the named stream."""
    key = np.uint64(0)
    for ch in stream.encode():
        key = _mix(np.array([key ^ np.uint64(ch)], dtype=np.uint64))[0]
    base = _mix(np.array([np.uint64(seed) ^ key], dtype=np.uint64))[0]
    with np.errstate(over="ignore"):
        idx = np.arange(1, count + 1, dtype=np.uint64)
        return _mix(base + idx * _GOLDEN)


def uniform_int(seed: int, stream: str, count: int, lo: int, hi: int) -> np.ndarray:
    """Integers uniform over lo..hi inclusive."""
    u53 = stream_u64(seed, stream, count) >> np.uint64(11)
    span = np.uint64(hi - lo + 1)
    return (lo + ((u53 * span) >> np.uint64(53)).astype(np.int64)).astype(np.int64)


def random_bytes(seed: int, stream: str, count: int) -> np.ndarray:
    words = stream_u64(seed, stream, (count + 7) // 8)
    return words.view(np.uint8)[:count].copy()


def normal(seed: int, stream: str, count: int) -> np.ndarray:
    """N(0, 1) in float64 by Box-Muller over draws 2i and 2i + 1."""
    u = stream_u64(seed, stream, 2 * count) >> np.uint64(11)
    u1 = (u[0::2].astype(np.float64) + 1.0) * 2.0 ** -53
    u2 = u[1::2].astype(np.float64) * 2.0 ** -53
    return np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)


def fp16_bits(values) -> np.ndarray:
    """recipe's `fp16` (recipe.rs:15098-15113) on float32 inputs, as uint16 bits."""
    v = np.asarray(values, dtype=np.float32)
    bits = v.view(np.uint32).astype(np.int64)
    sign = (bits >> 16) & 0x8000
    exponent = ((bits >> 23) & 0xFF) - 112
    mantissa = bits & 0x7FFFFF
    out = np.zeros(bits.shape, dtype=np.int64)
    # normal range
    rounded = mantissa + 0xFFF + ((mantissa >> 13) & 1)
    carry = (rounded & 0x800000) != 0
    normal_val = np.where(carry, sign | (np.minimum(exponent + 1, 31) << 10), sign | (exponent << 10) | (rounded >> 13))
    # subnormal range: truncate to the scaled grid, then round
    shift = np.clip(1 - exponent, 0, 31)
    sv = (mantissa | 0x800000) >> shift
    sub_val = sign | ((sv + 0xFFF + ((sv >> 13) & 1)) >> 13)
    big = sign | 0x7C00 | (mantissa != 0).astype(np.int64)
    out = np.where(exponent <= 0, np.where(exponent < -10, sign, sub_val), np.where(exponent >= 31, big, normal_val))
    return (out & 0xFFFF).astype(np.uint16)


def fp16_to_f32(bits) -> np.ndarray:
    return np.asarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def _scale_fp16(seed: int, stream: str, count: int, factor: float) -> np.ndarray:
    return fp16_bits((np.abs(normal(seed, stream, count)) * factor).astype(np.float32))


def gguf_bytes(fmt: str, rows: int, cols: int) -> int:
    bv, bb = BLOCK[fmt]
    return rows * (cols // bv) * bb


def q8_0(rows: int, cols: int, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    """Q8_0 blocks: codes uniform in [-127, 127], d = fp16(|N(0,1)| * 0.01)."""
    nb = rows * (cols // 32)
    blk = np.zeros((nb, 34), dtype=np.uint8)
    blk[:, 0:2] = _scale_fp16(seed, tag + ".q8_0.d", nb, 0.01).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = uniform_int(seed, tag + ".q8_0.q", nb * 32, -127, 127).astype(np.int8).view(np.uint8).reshape(nb, 32)
    return blk.reshape(-1)


def q4_0(rows: int, cols: int, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    """Q4_0 blocks: 4-bit codes uniform over 0..15, d = fp16(|N(0,1)| * 0.01)."""
    nb = rows * (cols // 32)
    blk = np.zeros((nb, 18), dtype=np.uint8)
    blk[:, 0:2] = _scale_fp16(seed, tag + ".q4_0.d", nb, 0.01).view(np.uint8).reshape(nb, 2)
    blk[:, 2:] = random_bytes(seed, tag + ".q4_0.q", nb * 16).reshape(nb, 16)
    return blk.reshape(-1)


def pack_k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """8 six-bit scales and minimums per superblock -> the 12 bytes that
    k_scale (recipe.rs:15204-15210) unpacks."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    out = np.zeros(sc.shape[:-1] + (12,), dtype=np.uint8)
    for j in range(4):
        out[..., j] = (sc[..., j] & 63) | ((sc[..., j + 4] >> 4) << 6)
        out[..., j + 4] = (mn[..., j] & 63) | ((mn[..., j + 4] >> 4) << 6)
        out[..., j + 8] = (sc[..., j + 4] & 15) | ((mn[..., j + 4] & 15) << 4)
    return out


def q4_k(rows: int, cols: int, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    """Q4_K superblocks: nibbles uniform 0..15, six-bit sub-scales and sub-mins
    uniform 0..63, d = fp16(|N| * 0.01), dmin = fp16(|N| * 0.005)."""
    nb = rows * (cols // 256)
    blk = np.zeros((nb, 144), dtype=np.uint8)
    blk[:, 0:2] = _scale_fp16(seed, tag + ".q4_k.d", nb, 0.01).view(np.uint8).reshape(nb, 2)
    blk[:, 2:4] = _scale_fp16(seed, tag + ".q4_k.dmin", nb, 0.005).view(np.uint8).reshape(nb, 2)
    sc = uniform_int(seed, tag + ".q4_k.sc", nb * 8, 0, 63).reshape(nb, 8)
    mn = uniform_int(seed, tag + ".q4_k.m", nb * 8, 0, 63).reshape(nb, 8)
    blk[:, 4:16] = pack_k_scales(sc, mn)
    blk[:, 16:] = random_bytes(seed, tag + ".q4_k.q", nb * 128).reshape(nb, 128)
    return blk.reshape(-1)


def q6_k(rows: int, cols: int, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    """Q6_K superblocks: six-bit codes uniform 0..63 (uniform ql/qh bytes),
    int8 scales uniform in [-32, 31], d = fp16(|N| * 0.01)."""
    nb = rows * (cols // 256)
    blk = np.zeros((nb, 210), dtype=np.uint8)
    blk[:, 0:192] = random_bytes(seed, tag + ".q6_k.q", nb * 192).reshape(nb, 192)
    blk[:, 192:208] = uniform_int(seed, tag + ".q6_k.sc", nb * 16, -32, 31).astype(np.int8).view(np.uint8).reshape(nb, 16)
    blk[:, 208:210] = _scale_fp16(seed, tag + ".q6_k.d", nb, 0.01).view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def f16_weights(rows: int, cols: int, std: float, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    """fp16 weights N(0, std^2) as GGUF F16 bytes."""
    v = (normal(seed, tag + ".f16", rows * cols) * std).astype(np.float32)
    return fp16_bits(v).view(np.uint8).copy()


GENERATORS = {"q4_0": q4_0, "q8_0": q8_0, "q4_k": q4_k, "q6_k": q6_k}


def weights(fmt: str, rows: int, cols: int, seed: int = DEFAULT_SEED, tag: str = "w") -> np.ndarray:
    return GENERATORS[fmt](rows, cols, seed, tag)


def activations_f16(count: int, seed: int = DEFAULT_SEED, tag: str = "x") -> np.ndarray:
    """fp16 N(0, 1) activations as uint16 bits."""
    return fp16_bits(normal(seed, tag + ".f16", count).astype(np.float32))


def activations_f32(count: int, seed: int = DEFAULT_SEED, tag: str = "x") -> np.ndarray:
    return normal(seed, tag + ".f32", count).astype(np.float32)


# ------------------------------------------------------------- decoder ----
# A random-init decoder for the single-token decode step. Projection weights
# of one layer are drawn with the generators above; every layer then holds
# those blocks with a layer-specific byte pattern XORed over the code and
# sub-scale bytes (the fp16 block scales are kept), which keeps each field's
# distribution uniform over its range while giving every layer its own bytes
# (so no layer's weights can be served from another's cache lines). KV-cache
# prefill is N(0, 1) in fp16, one layer drawn and the others given per-layer
# random signs. A large output head is drawn for its first eighth of rows and
# the other eighths are keyed variants of it, like the layers. The embedding
# table (fp32, not a quantized tensor; one row is read per token) is N(0, 1)
# from numpy's PCG64 under the seed for its first 8192 rows, repeated over the
# vocabulary with a random sign per row.

_SCALE_BYTES = {"q4_0": (0, 2), "q8_0": (0, 2), "q4_k": (0, 4), "q6_k": (208, 210)}


def _payload_mask(fmt: str) -> np.ndarray:
    """Per block byte: True for the code and sub-scale bytes a layer key may flip."""
    bb = BLOCK[fmt][1]
    keep = np.ones(bb, dtype=bool)
    lo, hi = _SCALE_BYTES[fmt]
    keep[lo:hi] = False
    return keep


def layer_variant(fmt: str, blocks: np.ndarray, seed: int, tag: str) -> np.ndarray:
    """`blocks` with the layer key `tag` XORed over every block's payload bytes."""
    bb = BLOCK[fmt][1]
    key = random_bytes(seed, tag + ".key", bb)
    key[~_payload_mask(fmt)] = 0
    return (blocks.reshape(-1, bb) ^ key[None, :]).reshape(-1)


def fp16_normal(count: int, seed: int, tag: str) -> np.ndarray:
    return fp16_bits(normal(seed, tag, count).astype(np.float32))


class DecoderSynth:
    """Seeded tensors of a random-init decoder of the given shape (an object
    with layers, d, q_heads, kv_heads, head_dim, ffn, vocab, proj_fmt,
    head_fmt). `norm_std` = 0 gives identity RMSNorm scales (recipe's
    initial value, recipe.rs:23206-23208); tests draw them N(1, norm_std^2)."""

    def __init__(self, shape, seed: int = DEFAULT_SEED, norm_std: float = 0.0):
        self.shape, self.seed, self.norm_std = shape, seed, norm_std
        s = shape
        qkv_rows = (s.q_heads + 2 * s.kv_heads) * s.head_dim
        f = s.proj_fmt
        self._base = {
            "qkv": (qkv_rows, s.d, weights(f, qkv_rows, s.d, seed, "dec.qkv")),
            "o": (s.d, s.d, weights(f, s.d, s.d, seed, "dec.o")),
            "gate": (s.ffn, s.d, weights(f, s.ffn, s.d, seed, "dec.gate")),
            "up": (s.ffn, s.d, weights(f, s.ffn, s.d, seed, "dec.up")),
            "down": (s.d, s.ffn, weights(f, s.d, s.ffn, seed, "dec.down")),
        }
        self._kv_base = None

    def _norm(self, tag: str) -> np.ndarray:
        n = self.shape.d
        if self.norm_std == 0.0:
            return np.ones(n, dtype=np.float32)
        return (1.0 + self.norm_std * normal(self.seed, tag, n)).astype(np.float32)

    def layer(self, index: int):
        from .decode import LayerTensors
        f = self.shape.proj_fmt
        w = {k: layer_variant(f, b, self.seed, f"dec.l{index}.{k}") for k, (_, _, b) in self._base.items()}
        return LayerTensors(attn_norm=self._norm(f"dec.l{index}.attn_norm"), qkv=w["qkv"], o=w["o"],
                            ffn_norm=self._norm(f"dec.l{index}.ffn_norm"), gate=w["gate"], up=w["up"], down=w["down"])

    def cache(self, index: int, ctx: int):
        """fp16 bits [kv_heads, ctx, head_dim] of keys and values for layer `index`."""
        s = self.shape
        n = s.kv_heads * ctx * s.head_dim
        if self._kv_base is None or self._kv_base[0].size != n:
            self._kv_base = (fp16_normal(n, self.seed, "dec.kcache"), fp16_normal(n, self.seed, "dec.vcache"))
        out = []
        for j, base in enumerate(self._kv_base):
            signs = random_bytes(self.seed, f"dec.l{index}.signs{j}", 2 * n).view(np.uint16) & np.uint16(0x8000)
            out.append((base ^ signs).reshape(s.kv_heads, ctx, s.head_dim))
        return out[0], out[1]

    def out_norm(self) -> np.ndarray:
        return self._norm("dec.out_norm")

    def head(self) -> np.ndarray:
        s = self.shape
        if s.vocab < 16384 or s.vocab % 8:
            return weights(s.head_fmt, s.vocab, s.d, self.seed, "dec.head")
        base = weights(s.head_fmt, s.vocab // 8, s.d, self.seed, "dec.head")
        parts = [base] + [layer_variant(s.head_fmt, base, self.seed, f"dec.head{c}") for c in range(1, 8)]
        return np.concatenate(parts)

    def embed(self) -> np.ndarray:
        s = self.shape
        rng = np.random.Generator(np.random.PCG64(self.seed))
        base = rng.standard_normal((min(s.vocab, 8192), s.d), dtype=np.float32)
        if s.vocab <= base.shape[0]:
            return base
        reps = -(-s.vocab // base.shape[0])
        table = np.tile(base, (reps, 1))[: s.vocab]
        signs = np.where(rng.integers(0, 2, s.vocab) == 1, np.float32(-1.0), np.float32(1.0))
        table *= signs[:, None]
        return table
