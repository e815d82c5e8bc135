"""CPU tests of librqmv: the library loads, exports every entry point that
include/rqmv.h declares, and its host-only loader functions (repack, unpack,
layout sizes, argument checks) behave. No GPU call is made here."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

import rqmv
from rqmv import synth

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
FMTS = ["q8_0", "q4_0", "q4_k", "q6_k"]


def _declared():
    text = open(os.path.join(ROOT, "include", "rqmv.h")).read()
    return sorted(set(re.findall(r"\b(rqmv_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    names = _declared()
    assert "rqmv_matvec" in names and "rqmv_moe" in names and len(names) >= 15
    lib = ctypes.CDLL(rqmv.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_missing_library_raises_instead_of_falling_back():
    """Without librqmv.so every entry fails with RqmvError; there is no CPU
    path to fall back to (checked in a fresh interpreter)."""
    code = (
        "import sys; sys.path[:0] = [%r, %r]\n"
        "import numpy as np, rqmv\n"
        "rqmv.LIB_PATH = '/nonexistent/librqmv.so'\n"
        "for call in (lambda: rqmv.init(0), lambda: rqmv.Weight('q4_k', 1, 256, np.zeros(144, np.uint8)),\n"
        "             lambda: rqmv.layout_bytes('q4_k', 1, 256)):\n"
        "    try:\n"
        "        call()\n"
        "    except rqmv.RqmvError as e:\n"
        "        assert 'not built' in str(e), e\n"
        "    else:\n"
        "        raise SystemExit('no error')\n"
        "print('raised')\n" % (ROOT, os.path.join(ROOT, "recipe-dev_amd")))
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0 and "raised" in out.stdout, out.stdout + out.stderr


def _shapes(fmt):
    if fmt in ("q4_k", "q6_k"):
        return [(1, 256), (3, 768), (17, 4096), (5, 14336)]
    return [(1, 32), (3, 96), (17, 4096), (5, 160), (2, 14336)]  # odd Q4_0 block counts included


@pytest.mark.parametrize("fmt", FMTS)
def test_host_repack_round_trip(fmt):
    for rows, cols in _shapes(fmt):
        w = synth.weights(fmt, rows, cols, seed=rows + cols)
        packed = rqmv.repack_host(fmt, rows, cols, w)
        back = rqmv.unpack_host(fmt, rows, cols, packed, w.nbytes)
        assert np.array_equal(back, w), (fmt, rows, cols)


def test_host_repack_f16_round_trip():
    rows, cols = 7, 2048
    w = synth.f16_weights(rows, cols, 0.02, seed=1)
    packed = rqmv.repack_host("f16", rows, cols, w)
    assert packed.nbytes == w.nbytes
    assert np.array_equal(rqmv.unpack_host("f16", rows, cols, packed, w.nbytes), w)


@pytest.mark.parametrize("fmt", FMTS)
def test_layout_carries_gguf_bytes(fmt):
    """The repacked rows hold exactly the GGUF bytes when rows are whole 16-byte
    multiples; otherwise only row padding is added."""
    rows, cols = 9, 4096
    assert rqmv.layout_bytes(fmt, rows, cols) == synth.gguf_bytes(fmt, rows, cols)
    rows, cols = 5, 96 if fmt in ("q8_0", "q4_0") else 768
    extra = rqmv.layout_bytes(fmt, rows, cols) - synth.gguf_bytes(fmt, rows, cols)
    assert 0 <= extra <= rows * (16 + 18)


def _nibbles(b16):
    """32 four-bit codes in natural order from 16 packed bytes (each XOR 8)."""
    b = np.asarray(b16, np.uint8)
    out = np.empty(32, np.int64)
    out[0::2] = (b & 15) ^ 8
    out[1::2] = (b >> 4) ^ 8
    return out


def test_layout_parts_are_contiguous_per_wave():
    """Part h of 64 consecutive chunks forms one contiguous 1 KiB run; part h of
    Q4_K chunk c holds sub-block 2(c % 4) + h's codes in order; each
    superblock's 16 scale bytes carry its 6-bit scales and minimums as one
    24-bit field per chunk."""
    rows, cols = 1, 4096  # Q4_K: 64 chunks of 64 weights, 2 parts each
    w = synth.q4_k(rows, cols, seed=5)
    code = rqmv.repack_host("q4_k", rows, cols, w)
    blk = w.reshape(16, 144)
    for c in range(64):
        sb, p = divmod(c, 4)
        for h in range(2):
            got = _nibbles(code[(h * 64 + c) * 16:(h * 64 + c) * 16 + 16])
            want = (blk[sb, 16 + 32 * p:16 + 32 * p + 32].astype(np.int64) >> (4 * h)) & 15
            assert np.array_equal(got, want), (c, h)
    # the group's scale bytes follow its two code parts: d and dmin as stored,
    # then chunk p's 24-bit field at bit 24p holding scale(2p), min(2p),
    # scale(2p+1), min(2p+1), against get_scale_min_k4 of the block's 12 bytes
    meta = code[2048:2304].reshape(16, 16)
    assert np.array_equal(meta[:, :4], blk[:, :4])
    for sb in range(16):
        s = blk[sb, 4:16].astype(np.int64)
        want = []
        for j in range(8):
            if j < 4:
                want += [s[j] & 63, s[j + 4] & 63]
            else:
                want += [(s[j + 4] & 15) | ((s[j - 4] >> 6) << 4), (s[j + 4] >> 4) | ((s[j] >> 6) << 4)]
        v = int.from_bytes(bytes(meta[sb, 4:16]), "little")
        got = [(v >> (6 * i)) & 63 for i in range(16)]  # fields back to back: sc, m per sub-block
        assert got == want, sb


def test_q6k_layout_decodes_each_code():
    """Every 6-bit code is its low nibble (parts 0-1) plus 16 times its high
    field (part 2, expanded by H & 0x33333333 and (H >> 2) & 0x33333333)."""
    rows, cols = 1, 256
    w = synth.q6_k(rows, cols, seed=9)
    code = rqmv.repack_host("q6_k", rows, cols, w)
    assert np.array_equal(code[192:208], w[192:208]) and np.array_equal(code[208:210], w[208:210])
    blk = w.reshape(210)
    ql, qh = blk[:128].astype(np.int64), blk[128:192].astype(np.int64)

    def q_of(i):  # recipe.rs:3743-3780 field positions
        ch, loc = divmod(i, 128)
        g, j = divmod(loc, 32)
        lo = (ql[64 * ch + j + 32 * (g & 1)] >> (4 * (g // 2))) & 15
        hi = (qh[32 * ch + j] >> (2 * g)) & 3
        return lo | (hi << 4)

    for c in range(4):  # one 64-chunk group of 4 chunks: part p of chunk c at (p * 4 + c) * 16
        lo = np.concatenate([_nibbles(code[(0 * 4 + c) * 16:(0 * 4 + c + 1) * 16]),
                             _nibbles(code[(1 * 4 + c) * 16:(1 * 4 + c + 1) * 16])])
        H = code[(2 * 4 + c) * 16:(2 * 4 + c + 1) * 16].view(np.uint32).astype(np.int64)
        for g in range(4):
            he, ho = H[g] & 0x33333333, (H[g] >> 2) & 0x33333333
            for j in range(16):
                h = ((he >> (4 * j)) & 15) if j < 8 else ((ho >> (4 * (j - 8))) & 15)
                e = 16 * g + j
                assert lo[e] + 16 * h == q_of(64 * c + e), (c, g, j)


def test_q6k_byte_words_hold_each_code():
    """The integer dot's byte words (chunk.h q6k_bytes, restated here on the
    repacked words): for scale group g of a chunk, word 0 holds the codes of
    the group's weights 0, 2, 4, 6, word 1 of 1, 3, 5, 7, word 2 of 8, 10, 12,
    14 and word 3 of 9, 11, 13, 15, one 6-bit code q = l + 16 h per byte; the
    activation staging writes its byte planes in the same order."""
    rows, cols = 2, 512
    w = synth.q6_k(rows, cols, seed=21)
    code = rqmv.repack_host("q6_k", rows, cols, w)
    row_bytes = rqmv.layout_bytes("q6_k", 1, cols)
    nch = cols // 64
    order = [[0, 2, 4, 6], [1, 3, 5, 7], [8, 10, 12, 14], [9, 11, 13, 15]]
    for r in range(rows):
        blk = w.reshape(rows, -1)[r]
        rb = code[r * row_bytes:(r + 1) * row_bytes]

        def q_of(i):  # recipe.rs:3743-3780 field positions
            sb, k = divmod(i, 256)
            ch, loc = divmod(k, 128)
            g, j = divmod(loc, 32)
            ql, qh = blk[sb * 210:sb * 210 + 128].astype(np.int64), blk[sb * 210 + 128:sb * 210 + 192].astype(np.int64)
            lo = (ql[64 * ch + j + 32 * (g & 1)] >> (4 * (g // 2))) & 15
            hi = (qh[32 * ch + j] >> (2 * g)) & 3
            return int(lo | (hi << 4))

        for c in range(nch):  # one group of nch chunks: part p of chunk c at (p * nch + c) * 16
            part = [rb[(p * nch + c) * 16:(p * nch + c + 1) * 16].view(np.uint32).astype(np.uint64) for p in range(3)]
            for g in range(4):
                L0 = int(part[g >> 1][(g & 1) * 2]) ^ 0x88888888
                L1 = int(part[g >> 1][(g & 1) * 2 + 1]) ^ 0x88888888
                H = int(part[2][g])
                W = [(L0 & 0x0F0F0F0F) | ((H << 4) & 0x30303030),
                     ((L0 >> 4) & 0x0F0F0F0F) | (H & 0x30303030),
                     (L1 & 0x0F0F0F0F) | ((H << 2) & 0x30303030),
                     ((L1 >> 4) & 0x0F0F0F0F) | ((H >> 2) & 0x30303030)]
                for t in range(4):
                    got = [(W[t] >> (8 * k)) & 0xFF for k in range(4)]
                    want = [q_of(64 * c + 16 * g + e) for e in order[t]]
                    assert got == want, (r, c, g, t)


@pytest.mark.parametrize("fmt,rows,cols", [("q4_k", 4, 100), ("q8_0", 2, 31), ("q6_k", 0, 256), (99, 2, 256)])
def test_bad_shapes_are_rejected(fmt, rows, cols):
    with pytest.raises(rqmv.RqmvError):
        rqmv.layout_bytes(fmt, rows, cols)


@pytest.mark.parametrize("fmt,rows,cols", [("f16", 2 ** 31, 64), ("q4_k", 1, 2 ** 30 + 256), ("q8_0", -5, 32),
                                           ("q6_k", 2 ** 62, 2 ** 30)])
def test_shapes_past_the_kernels_limits_are_rejected(fmt, rows, cols):
    """Row indices are 32-bit in the kernels and sizes are checked for
    overflow, so an oversized shape is an error, never a wrapped size."""
    with pytest.raises(rqmv.RqmvError):
        rqmv.layout_bytes(fmt, rows, cols)
    out = np.zeros(16, np.uint8)
    assert rqmv.lib().lib.rqmv_repack_host(rqmv._fmt(fmt), rows, cols,
                                           out.ctypes.data, out.ctypes.data) == -1


def test_weight_create_refuses_overflowing_shapes_before_any_copy():
    """experts x rows that wraps in 64 bits, or a bank past 2^31 rows, is
    refused from the shape alone (the byte buffer is never read)."""
    L = rqmv.lib().lib
    h = ctypes.c_void_p()
    data = np.zeros(128, np.uint8)
    for experts, rows in ((2 ** 40, 2 ** 40), (2 ** 20, 2 ** 12), (1, 2 ** 31)):
        rc = L.rqmv_expert_bank_create(1, experts, rows, 64, data.ctypes.data, 128, ctypes.byref(h))
        assert rc == -1 and h.value is None
        assert b"2^31" in L.rqmv_last_error() or b"overflow" in L.rqmv_last_error()


def test_last_error_names_the_failure():
    L = rqmv.lib().lib
    rc = L.rqmv_layout_bytes(12, 4, 100, None, None, None)
    assert rc == -1
    assert b"shape" in L.rqmv_last_error()
    h = ctypes.c_void_p()
    rc = L.rqmv_weight_create(12, 4, 256, None, 0, ctypes.byref(h))
    assert rc == -1 and h.value is None


@pytest.mark.parametrize("fmt", ["q4_0", "q6_k", "q8_0", "f16"])
def test_host_requantize_q8_0_matches_oracle(fmt):
    """The library's int(8) storage re-encoding (rqmv_requantize_q8_0_host)
    against the oracle's restatement of recipe's device Q8_0 quantizer."""
    import oracle

    shapes = [(1, 256), (7, 512), (33, 4096)] if fmt in ("q6_k",) else [(1, 64), (9, 128), (33, 4096)]
    for rows, cols in shapes:
        if fmt == "f16":
            w = synth.f16_weights(rows, cols, 0.02, seed=rows + cols)
        else:
            w = synth.weights(fmt, rows, cols, seed=rows + cols)
        got = rqmv.requantize_q8_0_host(fmt, rows, cols, w)
        assert np.array_equal(got, oracle.requantize_q8_0(fmt, w, rows, cols)), (fmt, rows, cols)


def test_host_requantize_extremes():
    import oracle

    # zero blocks, ties of magnitude, tiny and large fp16 values through an F16 source
    v = np.zeros((4, 64), np.float32)
    v[1, :32] = 3.0
    v[1, 5] = -3.0
    v[2, :] = np.float32(6.1e-5)
    v[2, 7] = np.float32(-65504.0)
    v[3, :] = np.linspace(-1, 1, 64, dtype=np.float32) * np.float32(1e-3)
    w = v.astype(np.float16).view(np.uint8).reshape(-1)
    got = rqmv.requantize_q8_0_host("f16", 4, 64, w)
    assert np.array_equal(got, oracle.requantize_q8_0("f16", w, 4, 64))
    assert not got[:68].any()  # the zero row: d = 0 and zero codes


def test_host_requantize_rejects_bad_arguments():
    w = synth.q4_k(1, 256, seed=1)
    with pytest.raises(rqmv.RqmvError, match="F16, Q8_0, Q4_0 or Q6_K"):
        rqmv.requantize_q8_0_host("q4_k", 1, 256, w)
    with pytest.raises(rqmv.RqmvError, match="expected"):
        rqmv.requantize_q8_0_host("q4_0", 2, 64, synth.q4_0(1, 64, seed=1))


def test_capability_row_for_gfx950():
    v, m = rqmv.capability("int8")
    assert "v_dot4_i32_i8" in v and m is None
    v, m = rqmv.capability("fp16")
    assert "v_dot8_i32_i4" in v and "v_mfma_f32_16x16x32_f16" in m
    with pytest.raises(rqmv.RqmvError, match=r"gfx950 has no fp8 instruction. Vector: int8 fp16 fp32. Matrix: fp16 fp32."):
        rqmv.capability("fp8")
    with pytest.raises(rqmv.RqmvError, match="no int7 capability entry"):
        rqmv.capability("int7")
