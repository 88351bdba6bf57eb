"""The committed fixtures (tests/golden/golden.npz, made by make_golden.py from
the float64 closed forms) against the C oracle (CPU) and the HIP library (GPU).

Bars: dequantized values bit-exact; GEMV within 1e-3 relative L2 of the float64
dot (the north_star tolerance; observed ~1e-7 for the oracle and ~1e-7 for the
matrix-core kernels).
"""
from pathlib import Path

import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES

GOLDEN = np.load(Path(__file__).resolve().parent / "golden" / "golden.npz")
OUT_DIM, IN_DIM = (int(v) for v in GOLDEN["shape"])
TYPES = sorted(GGML_TYPES)
TOL = 1e-3


def fixture(t):
    return GOLDEN[f"w_{t}"], GOLDEN[f"x_{t}"], GOLDEN[f"deq_{t}"], GOLDEN[f"y_{t}"].reshape(-1)


def test_fixture_covers_every_format():
    assert {int(k[2:]) for k in GOLDEN.files if k.startswith("w_")} == set(TYPES)


@pytest.mark.parametrize("t", TYPES)
def test_oracle_dequant_matches_golden(oracle, t):
    w, _, deq, _ = fixture(t)
    got = oracle.dequant(t, w, OUT_DIM * IN_DIM)
    assert np.array_equal(got.view(np.uint32), deq.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
def test_oracle_gemv_matches_golden(oracle, t):
    w, x, _, y = fixture(t)
    got = oracle.gemv(t, x, w, IN_DIM, OUT_DIM)
    assert cf.rel_l2(got, y) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("t", TYPES)
def test_hip_dequant_matches_golden(qh, t):
    from saient_quartz_amd.api import check
    from saient_quartz_amd.host import GpuBuf

    w, _, deq, _ = fixture(t)
    dw = GpuBuf.upload(w)
    out = GpuBuf.alloc_f32(OUT_DIM * IN_DIM)
    check("hip_dequant", qh.hip_dequant(t, dw.ptr, out.ptr, OUT_DIM * IN_DIM))
    assert np.array_equal(out.download(np.uint32), deq.view(np.uint32))


@pytest.mark.gpu
@pytest.mark.parametrize("t", TYPES)
def test_hip_gemv_matches_golden(qh, t):
    from saient_quartz_amd.host import verify_gemv_hip

    w, x, _, y = fixture(t)
    got = verify_gemv_hip(x, w, t, IN_DIM, OUT_DIM)
    assert cf.rel_l2(got, y) < TOL
