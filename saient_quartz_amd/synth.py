"""Seeded synthetic GGUF-layout weights and activations.

Distributions follow the benchmark configurations: f16 scales drawn as
|N(0, sigma)|, quant fields uniform random bytes (which gives uniform 4/6-bit
quants, uniform 6-bit Q4_K scale/min fields through the 12-byte packing and
uniform IQ grid indices / sign bits), Q8_0 quants uniform in [-127, 127] and
Q6_K sub-scales uniform in [-64, 63].  Every f16 field is written explicitly so
random bytes never produce Inf/NaN scales.
"""
import numpy as np

from .api import GGML_TYPES

SEED_BASE = 20261201

# f16 scale fields: type -> list of (byte offset, sigma, absolute?)
_F16_FIELDS = {
    2: [(0, 0.01, True)],
    3: [(0, 0.01, True), (2, 0.01, False)],
    6: [(0, 0.01, True)],
    7: [(0, 0.01, True), (2, 0.01, False)],
    8: [(0, 0.02 / 127.0, True)],
    10: [(80, 0.01, True), (82, 0.005, True)],
    12: [(0, 0.01, True), (2, 0.005, True)],
    13: [(0, 0.01, True), (2, 0.005, True)],
    14: [(208, 0.002, True)],
    16: [(0, 0.01, True)],
    17: [(0, 0.01, True)],
    20: [(0, 0.01, True)],
    21: [(0, 0.01, True)],
    22: [(0, 0.01, True)],
}


def rng_for(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def weights(ggml_type: int, out_dim: int, in_dim: int, seed: int) -> np.ndarray:
    """Row-major GGUF blocks for an out_dim x in_dim matrix, as a flat uint8 array."""
    _, qk, bb = GGML_TYPES[ggml_type]
    if in_dim % qk:
        raise ValueError(f"in_dim {in_dim} not a multiple of {qk}")
    rng = rng_for(seed)
    n = out_dim * in_dim
    if ggml_type == 0:
        return rng.normal(0.0, 0.02, n).astype("<f4").view(np.uint8)
    if ggml_type == 1:
        return rng.normal(0.0, 0.02, n).astype("<f2").view(np.uint8)
    if ggml_type == 30:
        f = rng.normal(0.0, 0.02, n).astype("<f4").view("<u4")
        return ((f + 0x7FFF + ((f >> 16) & 1)) >> 16).astype("<u2").view(np.uint8)
    nb = n // qk
    blk = np.frombuffer(rng.bytes(nb * bb), dtype=np.uint8).reshape(nb, bb).copy()
    if ggml_type == 8:
        blk[:, 2:34] = rng.integers(-127, 128, size=(nb, 32), dtype=np.int8).view(np.uint8)
    if ggml_type == 14:
        blk[:, 192:208] = rng.integers(-64, 64, size=(nb, 16), dtype=np.int8).view(np.uint8)
    for off, sigma, absolute in _F16_FIELDS[ggml_type]:
        v = rng.normal(0.0, sigma, nb)
        if absolute:
            v = np.abs(v)
        blk[:, off:off + 2] = v.astype("<f2").view(np.uint8).reshape(nb, 2)
    return blk.reshape(-1)


def activations(n: int, in_dim: int, seed: int) -> np.ndarray:
    """Token-major f32 activations x[n][in_dim] ~ N(0, 1)."""
    return rng_for(seed).standard_normal((n, in_dim), dtype=np.float32)


def verify_x(in_dim: int) -> np.ndarray:
    """The deterministic activation of Quartz's --verify-gemv (src/main.rs:2644-2649)."""
    i = np.arange(in_dim, dtype=np.uint64)
    s = ((i * np.uint64(2654435761)) >> np.uint64(8)) & np.uint64(0x3FF)
    return (s.astype(np.float32) / np.float32(512.0) - np.float32(1.0)).astype(np.float32)
