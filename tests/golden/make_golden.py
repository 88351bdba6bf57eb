"""Write tests/golden/golden.npz: seeded GGUF blocks for every supported format
with their expected dequantized values and GEMV outputs.

    python tests/golden/make_golden.py

Expected values come from tests/closed_form.py, a float64 restatement of the
block formats of src/dequant.rs that shares no code with the C oracle
(oracle/quartz_oracle.c) or the HIP kernels:
  * dequant: float64 decode cast to f32 -- exact, every product has <= 24
    significant bits and the one subtraction (Q4_K/Q5_K/Q2_K mins, Q4_1/Q5_1
    +m) rounds once (53 >= 2*24 + 2, so f64 -> f32 double rounding is
    innocuous);
  * gemv: float64 dot of the float64 decode with x (no f32 rounding at all),
    the reference against which the f32 paths are held to 1e-3 relative L2.
The reference holds no golden vectors for this path (no #[test] in
src/dequant.rs or src/cuda_kernels.cu), so these fixtures are the build's own.
"""
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

import closed_form as cf  # noqa: E402
from saient_quartz_amd import GGML_TYPES, synth  # noqa: E402

OUT_DIM = 8
IN_DIM = 256


def main():
    arrays = {}
    for t in sorted(GGML_TYPES):
        data = synth.weights(t, OUT_DIM, IN_DIM, seed=900 + t)
        x = synth.activations(1, IN_DIM, seed=77)[0]
        deq = cf.decode(t, data).astype(np.float32)
        y = cf.gemv_f64(t, x, data, IN_DIM, OUT_DIM)
        arrays[f"w_{t}"] = data
        arrays[f"x_{t}"] = x
        arrays[f"deq_{t}"] = deq
        arrays[f"y_{t}"] = y
    arrays["shape"] = np.array([OUT_DIM, IN_DIM], dtype=np.int64)
    np.savez_compressed(HERE / "golden.npz", **arrays)
    print(f"wrote {HERE / 'golden.npz'}: {len(GGML_TYPES)} formats, {OUT_DIM}x{IN_DIM}")


if __name__ == "__main__":
    main()
