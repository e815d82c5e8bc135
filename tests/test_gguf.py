"""The GGUF v3 reader in librqmv (host only, no device), against files written
by tests/gguf_writer.py, with recipe's rules (mod gguf, recipe.rs:9783-10327):
metadata of every value type, tensor descriptors and aligned data, the
general.alignment key, split models, and every error the reference raises."""
import os

import numpy as np
import pytest

import rqmv
from rqmv import synth

import gguf_writer as gw

RNG = np.random.default_rng(3)


def _rand(n):
    return RNG.integers(0, 256, n, dtype=np.uint8).tobytes()


META = [
    ("general.architecture", gw.STRING, "llama"),
    ("llama.block_count", gw.U32, 32),
    ("u8", gw.U8, 200), ("i8", gw.I8, -5), ("u16", gw.U16, 60000), ("i16", gw.I16, 1234),
    ("i32", gw.I32, 7), ("u64", gw.U64, 2 ** 40), ("i64", gw.I64, 2 ** 33), ("flag", gw.BOOL, 1),
    ("eps", gw.F32, 1e-5), ("base", gw.F64, 500000.0),
    ("ints", gw.ARRAY, (gw.I32, [3, 1, 4, 1, 5])),
    ("words", gw.ARRAY, (gw.STRING, ["a", "bc", "", "déf"])),
    ("nested", gw.ARRAY, (gw.ARRAY, [(gw.U8, [1, 2]), (gw.U8, [])])),
]


def _tensors():
    specs = [("token_embd.weight", [64, 10], 0), ("blk.0.attn_q.weight", [512, 8], 12),
             ("blk.0.ffn_down.weight", [256, 3], 14), ("output.weight", [64, 5], 8), ("q40", [96, 2], 2),
             ("halves", [33], 1), ("bf", [7, 3], 30), ("bytes", [5], 24)]
    return [(n, s, t, _rand(gw.tensor_bytes(t, s))) for n, s, t in specs]


def test_round_trip_every_value_type_and_tensor(tmp_path):
    path = str(tmp_path / "m.gguf")
    tensors = _tensors()
    gw.write(path, META, tensors)
    g = rqmv.Gguf(path)
    assert [k for k, _ in g.keys()] == [k for k, _, _ in META]
    assert g.get_string("general.architecture") == "llama"
    assert g.get_int("llama.block_count") == 32
    for key, want in (("u8", 200), ("u16", 60000), ("i16", 1234), ("i32", 7), ("u64", 2 ** 40), ("i64", 2 ** 33),
                      ("flag", None)):
        if want is None:
            continue
        assert g.get_int(key) == want
    with pytest.raises(rqmv.RqmvError):
        g.get_int("i8")  # negative: not a nonnegative integer (GgufValue::integer)
    assert g.get_float("eps") == np.float32(1e-5)
    assert g.get_float("base") == 500000.0
    with pytest.raises(rqmv.RqmvError):
        g.get_float("u8")
    assert g.get_array("ints") == [3, 1, 4, 1, 5]
    assert g.get_array("words") == ["a", "bc", "", "déf"]
    with pytest.raises(rqmv.RqmvError):
        g.get_int("absent.key")
    got = g.tensors()
    assert [t.name for t in got] == [n for n, _, _, _ in tensors]
    for t, (name, shape, ty, data) in zip(got, tensors):
        assert t.shape == tuple(shape) and t.ggml_type == ty and t.nbytes == len(data)
        assert g.data(name).tobytes() == data
    assert g.tensor("nope") is None
    g.close()


@pytest.mark.parametrize("alignment", [1, 32, 64, 4096])
def test_alignment_key(tmp_path, alignment):
    path = str(tmp_path / "a.gguf")
    tensors = _tensors()[:3]
    meta = [("general.alignment", gw.U32, alignment)]
    start = gw.write(path, meta, tensors, alignment=alignment)
    assert start % alignment == 0
    g = rqmv.Gguf(path)
    for name, _, _, data in tensors:
        assert g.data(name).tobytes() == data


@pytest.mark.parametrize("case,message", [
    ("magic", "not a GGUF file"),
    ("version", "version 2"),
    ("truncated", "truncated"),
    ("past_end", "runs past the end"),
    ("alignment", "alignment 48"),
    ("value_type", "value type 13"),
    ("tensor_type", "tensor type 99"),
    ("partial_block", "not a multiple of its 256-element block"),
])
def test_errors(tmp_path, case, message):
    path = str(tmp_path / "bad.gguf")
    tensors = _tensors()[:2]
    if case == "magic":
        gw.write(path, META[:2], tensors, magic=b"GGUG")
    elif case == "version":
        gw.write(path, META[:2], tensors, version=2)
    elif case == "truncated":
        gw.write(path, META, tensors, truncate=40)
    elif case == "past_end":
        start = gw.write(path, META[:2], tensors)
        os.truncate(path, start + 100)
    elif case == "alignment":
        gw.write(path, [("general.alignment", gw.U32, 48)], tensors)
    elif case == "value_type":
        with open(path, "wb") as f:
            import struct
            f.write(b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13))
    elif case == "tensor_type":
        gw.write(path, [], [("t", [32], 99, b"")])
    elif case == "partial_block":
        gw.write(path, [], [("t", [100], 12, b"")])
    with pytest.raises(rqmv.RqmvError, match=message):
        rqmv.Gguf(path)


def test_missing_file_raises(tmp_path):
    with pytest.raises(rqmv.RqmvError, match="cannot open"):
        rqmv.Gguf(str(tmp_path / "none.gguf"))


def _split(tmp_path, count=3, wrong_no=None, declared=None, name="model"):
    tensors = _tensors()
    per = [tensors[i::count] for i in range(count)]
    paths = []
    for i in range(count):
        meta = [("split.no", gw.U16, wrong_no if (wrong_no is not None and i == 1) else i),
                ("split.count", gw.U16, count),
                ("split.tensors.count", gw.I32, declared if declared is not None else len(tensors))]
        p = str(tmp_path / f"{name}-{i + 1:05d}-of-{count:05d}.gguf")
        gw.write(p, meta if i else META + meta, per[i])
        paths.append(p)
    return paths, per


def test_split_model(tmp_path):
    paths, per = _split(tmp_path)
    g = rqmv.Gguf(paths[0])
    names = [t.name for t in g.tensors()]
    assert names == [n for shard in per for n, _, _, _ in shard]  # shard by shard, file order
    for shard in per:
        for name, _, _, data in shard:
            assert g.data(name).tobytes() == data
    assert g.get_string("general.architecture") == "llama"  # the first shard's metadata


def test_split_errors(tmp_path):
    paths, _ = _split(tmp_path, wrong_no=5, name="a")
    with pytest.raises(rqmv.RqmvError, match="shard 5, expected shard 1"):
        rqmv.Gguf(paths[0])
    paths, _ = _split(tmp_path, declared=99, name="b")
    with pytest.raises(rqmv.RqmvError, match="declares 99 tensors"):
        rqmv.Gguf(paths[0])
    paths, _ = _split(tmp_path, name="c")
    os.remove(paths[2])
    with pytest.raises(rqmv.RqmvError, match="cannot open"):
        rqmv.Gguf(paths[0])
    bad = str(tmp_path / "plain.gguf")
    gw.write(bad, [("split.count", gw.U16, 2)], [])
    with pytest.raises(rqmv.RqmvError, match="not named"):
        rqmv.Gguf(bad)


def test_synthetic_blocks_through_the_file(tmp_path):
    """Quantized blocks written into a file read back byte for byte."""
    path = str(tmp_path / "q.gguf")
    w = synth.q4_k(16, 512, seed=4)
    gw.write(path, [], [("blk.0.ffn_up.weight", [512, 16], 12, w.tobytes())])
    g = rqmv.Gguf(path)
    assert np.array_equal(g.data("blk.0.ffn_up.weight"), w)


def test_shape_whose_byte_count_wraps_is_refused(tmp_path):
    """An F16 tensor [64, 2^57 + 1] holds 2^63 + 64 elements: its byte count,
    2^64 + 128, would wrap to 128 in 64-bit arithmetic and match a 128-byte
    data section. The reader counts in 128 bits and refuses the shape."""
    path = str(tmp_path / "wrap.gguf")
    gw.write(path, [], [("wrap", [64, 2 ** 57 + 1], 1, bytes(128))])
    with pytest.raises(rqmv.RqmvError, match="overflows"):
        rqmv.Gguf(path)
