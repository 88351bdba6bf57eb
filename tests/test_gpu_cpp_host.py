"""The C++ host layer (include/quartz_hip.hpp) through tests/cpp/verify_gemv: the
reference's --verify-gemv (src/main.rs:2629-2675) over a GGUF holding one 2-D
tensor per GEMV type and a stacked 3-D expert tensor (src/cuda.rs:250-281)."""
import subprocess
from pathlib import Path

import numpy as np
import pytest

from saient_quartz_amd import synth
from saient_quartz_amd.gguf import GgufWriter

BIN = Path(__file__).resolve().parent / "cpp" / "verify_gemv"

# (type, out_dim, in_dim): K-quants, legacy blocks, IQ formats, f32/f16/bf16
CASES = [(12, 96, 512), (14, 64, 768), (13, 48, 512), (10, 32, 512), (2, 64, 256),
         (3, 64, 256), (6, 64, 256), (7, 64, 256), (8, 64, 256), (20, 64, 256), (21, 64, 512),
         (16, 64, 512), (17, 32, 256), (22, 32, 256), (0, 16, 64), (1, 16, 64), (30, 16, 64)]


def _write(path):
    w = GgufWriter()
    w.add("general.architecture", 8, "test")
    for t, out_dim, in_dim in CASES:
        w.add_tensor(f"blk.{t}.weight", synth.weights(t, out_dim, in_dim, seed=100 + t), [in_dim, out_dim], t)
    experts = np.concatenate([synth.weights(12, 32, 256, seed=200 + e) for e in range(4)])
    w.add_tensor("blk.0.ffn_up_exps.weight", experts, [256, 32, 4], 12)
    w.write(path)


@pytest.mark.gpu
def test_cpp_verify_gemv(tmp_path):
    assert BIN.exists(), "tests/cpp/verify_gemv is not built (run __graft_entry__.build())"
    path = tmp_path / "verify.gguf"
    _write(path)
    r = subprocess.run([str(BIN), str(path)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "MISMATCH" not in r.stdout
    lines = [ln for ln in r.stdout.splitlines() if ln.startswith("type")]
    assert sum(ln.endswith("OK") for ln in lines) == len(CASES) + 4


def test_cpp_verify_gemv_usage():
    """Built and linked (CPU): a wrong argument count is a usage error, exit 2."""
    assert BIN.exists(), "tests/cpp/verify_gemv is not built (run __graft_entry__.build())"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 2 and "usage" in r.stderr
