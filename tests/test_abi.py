"""CPU tests of librqmv: the library loads, exports every entry point that
include/rqmv.h declares, and its host-only loader functions (repack, unpack,
layout sizes, argument checks) behave. No GPU call is made here."""
import ctypes
import os
import re

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


def _shapes(fmt):
    if fmt in ("q4_k", "q6_k"):
        return [(1, 256), (3, 768), (17, 4096), (5, 14336)]
    return [(1, 32), (3, 96), (17, 4096), (5, 160), (2, 14336)]  # odd Q4_0 block counts included


@pytest.mark.parametrize("fmt", FMTS)
def test_host_repack_round_trip(fmt):
    for rows, cols in _shapes(fmt):
        w = synth.weights(fmt, rows, cols, seed=rows + cols)
        code, m0, m1 = rqmv.repack_host(fmt, rows, cols, w)
        back = rqmv.unpack_host(fmt, rows, cols, code, m0, m1, w.nbytes)
        assert np.array_equal(back, w), (fmt, rows, cols)


def test_host_repack_f16_round_trip():
    rows, cols = 7, 2048
    w = synth.f16_weights(rows, cols, 0.02, seed=1)
    code, m0, m1 = rqmv.repack_host("f16", rows, cols, w)
    assert m0.size == 0 and m1.size == 0
    assert np.array_equal(rqmv.unpack_host("f16", rows, cols, code, m0, m1, w.nbytes), w)


@pytest.mark.parametrize("fmt", FMTS)
def test_layout_carries_gguf_bytes_without_padding(fmt):
    """The repacked planes hold exactly the GGUF bytes (Q4_0 pads an odd block)."""
    rows, cols = 9, 4096
    code, m0, m1 = rqmv.layout_bytes(fmt, rows, cols)
    assert code + m0 + m1 == synth.gguf_bytes(fmt, rows, cols)


def test_layout_parts_are_contiguous_per_wave():
    """Part p of 64 consecutive chunks forms one contiguous 1 KiB run."""
    rows, cols = 1, 4096  # Q4_K: 64 chunks of 64 weights, 2 parts each
    w = synth.q4_k(rows, cols, seed=5)
    code, m0, _ = rqmv.repack_host("q4_k", rows, cols, w)
    blk = w.reshape(16, 144)
    for c in range(64):
        sb, p = divmod(c, 4)
        for h in range(2):
            got = code[(h * 64 + c) * 16:(h * 64 + c) * 16 + 16]
            assert np.array_equal(got, blk[sb, 16 + 32 * p + 16 * h:16 + 32 * p + 16 * h + 16])
    assert np.array_equal(m0.reshape(16, 16), blk[:, :16])


def test_q6k_group_packing_decodes_each_code():
    """Every 6-bit code lands where the kernels' mask-and-or reads it back."""
    rows, cols = 1, 256
    w = synth.q6_k(rows, cols, seed=9)
    code, _, _ = rqmv.repack_host("q6_k", rows, cols, w)
    blk = w.reshape(210)
    ql, qh = blk[:128].astype(np.int64), blk[128:192].astype(np.int64)

    def q_of(i):  # recipe.rs:3743-3780 field positions
        ch, loc = divmod(i, 128)
        g, j = divmod(loc, 32)
        lo = (ql[64 * ch + j + 32 * (g & 1)] >> (4 * (g // 2))) & 15
        hi = (qh[32 * ch + j] >> (2 * g)) & 3
        return lo | (hi << 4)

    def rotr(v, s):
        return ((v >> s) | (v << (32 - s))) & 0xFFFFFFFF

    for c in range(4):
        words = [int(v) for v in code[c * 16:(c + 1) * 16].view(np.uint32)]  # part 0 (one 64-chunk group)
        words += [int(v) for v in code[(4 + c) * 16:(4 + c + 1) * 16].view(np.uint32)]  # part 1
        H = [int(v) for v in code[(8 + c) * 16:(8 + c + 1) * 16].view(np.uint32)]  # part 2
        for g in range(4):
            A, B, h = words[2 * g], words[2 * g + 1], H[g]
            pairs = [
                (A & 0x000F000F) | (h & 0x00300030), ((A >> 8) & 0x000F000F) | ((h >> 2) & 0x00300030),
                (B & 0x000F000F) | (rotr(h, 8) & 0x00300030), ((B >> 8) & 0x000F000F) | (rotr(h, 10) & 0x00300030),
                (A & 0x00F000F0) | (h & 0x03000300), ((A >> 8) & 0x00F000F0) | ((h >> 2) & 0x03000300),
                (B & 0x00F000F0) | (rotr(h, 8) & 0x03000300), ((B >> 8) & 0x00F000F0) | (rotr(h, 10) & 0x03000300)]
            for j, v in enumerate(pairs):
                lo, hi = v & 0xFFFF, v >> 16
                if j >= 4:
                    lo, hi = lo // 16, hi // 16
                e = 64 * c + 16 * g + 2 * j
                assert (lo, hi) == (q_of(e), q_of(e + 1)), (c, g, j)


@pytest.mark.parametrize("fmt,rows,cols", [("q4_k", 4, 100), ("q8_0", 2, 31), ("q6_k", 0, 256), (99, 2, 256)])
def test_bad_shapes_are_rejected(fmt, rows, cols):
    with pytest.raises(rqmv.RqmvError):
        rqmv.layout_bytes(fmt, rows, cols)


def test_last_error_names_the_failure():
    L = rqmv.lib().lib
    rc = L.rqmv_layout_bytes(12, 4, 100, None, None, None)
    assert rc == -1
    assert b"shape" in L.rqmv_last_error()
    h = ctypes.c_void_p()
    rc = L.rqmv_weight_create(12, 4, 256, None, 0, ctypes.byref(h))
    assert rc == -1 and h.value is None
