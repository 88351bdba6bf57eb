"""Build libquartz_hip.so (gfx950) in-tree with hipcc.

    python -m saient_quartz_amd.build        # or build() from Python

The library is one translation unit (csrc/qh_lib.hip).  Flags: -O3, gfx950 only,
packed-FP32 code generation disabled (-packed-fp32-ops), MFMA results in VGPRs.
"""
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
LIB = PKG / "libquartz_hip.so"
SRC = PKG / "csrc" / "qh_lib.hip"
ARCH = os.environ.get("QUARTZ_HIP_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA results in ordinary VGPRs: the GEMV kernels consume every result
    # immediately, so accumulation registers only add copies.
    "-mllvm", "--amdgpu-mfma-vgpr-form",
    # Leading scalar kernel arguments preloaded into SGPRs at wavefront start
    # (gfx950): a kernel's first loads need no round trip to argument memory.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC)")


def build(verbose: bool = False) -> Path:
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *HIPCC_FLAGS, "-o", str(tmp), str(SRC)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + res.stdout + res.stderr)
    if verbose and res.stderr:
        print(res.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
