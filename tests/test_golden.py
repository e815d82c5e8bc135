"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle): the oracle still reproduces
them, the host repack round-trips their bytes, and the GPU path matches
them (dequant bit-exact, outputs within rel-L2 1e-3)."""
import glob
import os

import numpy as np
import pytest

import oracle

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
MATVEC = sorted(glob.glob(os.path.join(HERE, "matvec_*.npz")))
MOE = sorted(glob.glob(os.path.join(HERE, "moe_*.npz")))
REL_L2 = 1e-3


def _load(path):
    return np.load(path, allow_pickle=False)


def _x32(bits):
    return oracle.f32_from_fp16(bits.reshape(-1)).reshape(bits.shape)


def _rel(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


def test_fixtures_present():
    assert len(MATVEC) == 5 and len(MOE) == 1


@pytest.mark.parametrize("path", MATVEC, ids=os.path.basename)
def test_oracle_reproduces_matvec_fixture(path):
    f = _load(path)
    fmt, rows, cols = str(f["fmt"]), int(f["rows"]), int(f["cols"])
    deq = oracle.dequant_rows(fmt, f["w"], rows, cols).astype(np.float32)
    assert np.array_equal(deq.view(np.uint32), f["deq"].view(np.uint32))
    x32 = _x32(f["x_bits"])
    for m in range(x32.shape[0]):
        assert np.array_equal(oracle.matvec_f64(fmt, f["w"], rows, cols, x32[m].astype(np.float64)), f["y64"][m])
    assert np.array_equal(oracle.matvec_recipe_f32(fmt, f["w"], rows, cols, x32), f["y32"])


@pytest.mark.parametrize("path", MATVEC, ids=os.path.basename)
def test_repack_round_trips_fixture(path):
    import rqmv

    f = _load(path)
    fmt, rows, cols = str(f["fmt"]), int(f["rows"]), int(f["cols"])
    packed = rqmv.repack_host(fmt, rows, cols, f["w"])
    assert np.array_equal(rqmv.unpack_host(fmt, rows, cols, packed, f["w"].size), f["w"])


@pytest.mark.parametrize("path", MOE, ids=os.path.basename)
def test_oracle_reproduces_moe_fixture(path):
    f = _load(path)
    fmt = str(f["fmt"])
    y, rw = oracle.moe_f64(fmt, int(f["d"]), int(f["experts"]), int(f["top"]), int(f["hidden"]), f["router"],
                           f["gate"], f["up"], f["down"], _x32(f["x_bits"]).astype(np.float64), scoring=0,
                           renormalize=True, hidden_shared=int(f["hidden"]), shared_gate_bits=f["shared_gate"],
                           gate_sh=f["gate_sh"], up_sh=f["up_sh"], down_sh=f["down_sh"])
    assert np.array_equal(y, f["y"]) and np.array_equal(rw, f["route"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", MATVEC, ids=os.path.basename)
def test_gpu_matches_matvec_fixture(gpu, path):
    f = _load(path)
    fmt, rows, cols = str(f["fmt"]), int(f["rows"]), int(f["cols"])
    W = gpu.Weight(fmt, rows, cols, f["w"])
    out = gpu.DeviceBuffer(4 * rows * cols)
    W.dequantize(out)
    gpu.synchronize()
    deq = out.download(np.float32)
    assert np.array_equal(deq.view(np.uint32), f["deq"].reshape(-1).view(np.uint32))
    y = gpu.contract(W, f["x_bits"])
    err = _rel(y, f["y32"])
    print(f"golden {fmt}: rel-L2 {err:.3e}", flush=True)
    assert err <= REL_L2


@pytest.mark.gpu
@pytest.mark.parametrize("path", MOE, ids=os.path.basename)
def test_gpu_matches_moe_fixture(gpu, path):
    f = _load(path)
    fmt, d, E, top, H = str(f["fmt"]), int(f["d"]), int(f["experts"]), int(f["top"]), int(f["hidden"])
    moe = gpu.Moe(gpu.Weight("f16", E, d, f["router"]), gpu.Weight(fmt, H, d, f["gate"], experts=E),
                  gpu.Weight(fmt, H, d, f["up"], experts=E), gpu.Weight(fmt, d, H, f["down"], experts=E), top,
                  scoring=gpu.SCORE_SOFTMAX, renormalize=True,
                  shared_gate_inp=gpu.Weight("f16", 1, d, f["shared_gate"]), gate_sh=gpu.Weight(fmt, H, d, f["gate_sh"]),
                  up_sh=gpu.Weight(fmt, H, d, f["up_sh"]), down_sh=gpu.Weight(fmt, d, H, f["down_sh"]))
    y, route = moe(f["x_bits"])
    assert np.array_equal(route != 0, f["route"] != 0)
    assert np.allclose(route, f["route"], rtol=1e-5, atol=1e-7)
    err = _rel(y, f["y"])
    print(f"golden moe {fmt}: rel-L2 {err:.3e}", flush=True)
    assert err <= REL_L2
