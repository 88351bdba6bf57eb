"""Seeded synthetic GGUF weights generated directly in device memory (torch RNG),
with the distributions of BASELINE.json's configs.  Used by bench.py and the
decode-step harness, where hundreds of MB to GB of weights make host generation
and upload the slow part.  (saient_quartz_amd.synth is the host-side, numpy
generator the parity tests use; the two streams differ, the distributions match.)
"""
import torch

Q4_K, Q5_K, Q6_K = 12, 13, 14


def _gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def q4k(out_dim: int, in_dim: int, seed: int) -> torch.Tensor:
    """Q4_K: f16 d ~ |N(0,0.01)|, f16 dmin ~ |N(0,0.005)|, scale/min bytes and
    quants uniform random bytes (6-bit fields uniform 0..63, nibbles 0..15)."""
    g = _gen(seed)
    nb = out_dim * in_dim // 256
    blk = torch.randint(0, 256, (nb, 144), dtype=torch.uint8, device="cuda", generator=g)
    d = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.01).half()
    dmin = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.005).half()
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:4] = dmin.view(torch.uint8).view(nb, 2)
    return blk.reshape(-1)


def q5k(out_dim: int, in_dim: int, seed: int) -> torch.Tensor:
    """Q5_K: as Q4_K (176-byte blocks: d, dmin, 12 scale bytes, 32 qh, 128 qs)."""
    g = _gen(seed)
    nb = out_dim * in_dim // 256
    blk = torch.randint(0, 256, (nb, 176), dtype=torch.uint8, device="cuda", generator=g)
    d = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.01).half()
    dmin = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.005).half()
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    blk[:, 2:4] = dmin.view(torch.uint8).view(nb, 2)
    return blk.reshape(-1)


def q6k(out_dim: int, in_dim: int, seed: int) -> torch.Tensor:
    """Q6_K: ql/qh uniform random bytes, 16 int8 sub-scales uniform [-64, 63],
    f16 d ~ |N(0,0.002)|."""
    g = _gen(seed)
    nb = out_dim * in_dim // 256
    blk = torch.randint(0, 256, (nb, 210), dtype=torch.uint8, device="cuda", generator=g)
    sc = torch.randint(-64, 64, (nb, 16), dtype=torch.int8, device="cuda", generator=g)
    d = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.002).half()
    blk[:, 192:208] = sc.view(torch.uint8)
    blk[:, 208:210] = d.view(torch.uint8).view(nb, 2)
    return blk.reshape(-1)


IQ2_XXS, IQ3_S = 16, 21
_IQ_BYTES = {IQ2_XXS: 66, IQ3_S: 110}


def iq(ggml_type: int, out_dim: int, in_dim: int, seed: int) -> torch.Tensor:
    """IQ2_XXS / IQ3_S: random grid indices, sign bits and scale nibbles,
    f16 d ~ |N(0,0.01)| in bytes 0-1 of each block."""
    g = _gen(seed)
    nb = out_dim * in_dim // 256
    bs = _IQ_BYTES[ggml_type]
    blk = torch.randint(0, 256, (nb, bs), dtype=torch.uint8, device="cuda", generator=g)
    d = torch.randn(nb, device="cuda", generator=g).abs_().mul_(0.01).half()
    blk[:, 0:2] = d.view(torch.uint8).view(nb, 2)
    return blk.reshape(-1)


def weights(ggml_type: int, out_dim: int, in_dim: int, seed: int) -> torch.Tensor:
    if ggml_type == Q4_K:
        return q4k(out_dim, in_dim, seed)
    if ggml_type == Q5_K:
        return q5k(out_dim, in_dim, seed)
    if ggml_type == Q6_K:
        return q6k(out_dim, in_dim, seed)
    if ggml_type in _IQ_BYTES:
        return iq(ggml_type, out_dim, in_dim, seed)
    raise ValueError(f"no device generator for ggml type {ggml_type}")
