"""Float64 closed forms of every GGUF block format (test infrastructure).

These decode whole arrays of blocks with numpy bit-field arithmetic in float64
and round ONCE to f32 at the end.  Every value is (f16 scale) x (<=8-bit integer)
x (<=6-bit integer) plus at most one addition, so the float64 result is exact
and the single f64->f32 rounding equals the f32 computation of
src/dequant.rs (double rounding is innocuous: 53 >= 2*24+2).  They are the
independent check the CPU oracle is pinned against; nothing here calls it.

Layouts: src/dequant.rs :1011-1237 (IQ2/IQ3/Q2_K/Q5_K), :1381-1463
(Q5_0/Q5_1/Q8_0), :1482-1519 (Q4_K), :1527-1574 (IQ4_NL), :1583-1631 (Q6_K);
Q4_0/Q4_1 from the public GGUF layout.
"""
import hashlib
import re
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
GRID_HDR = ROOT / "saient_quartz_amd" / "csrc" / "iq_grids.h"


def _grids():
    txt = GRID_HDR.read_text()
    out = {}
    for name in ("IQ2XXS", "IQ2XS", "IQ2S", "IQ3S"):
        m = re.search(r"#define QH_%s_GRID_VALUES \\\n(.*?)\n\n" % name, txt, re.S)
        vals = [int(v.strip().rstrip("ulUL"), 16) for v in re.findall(r"0x[0-9a-fA-F]+u?l*l*", m.group(1))]
        sha = re.search(r'#define QH_%s_GRID_SHA256 "([0-9a-f]+)"' % name, txt).group(1)
        out[name] = (np.array(vals, dtype=np.uint64), sha)
    return out


GRIDS = _grids()


def grid_sha256(name):
    vals, _ = GRIDS[name]
    width = 4 if name == "IQ3S" else 8
    return hashlib.sha256(b"".join(int(v).to_bytes(width, "little") for v in vals)).hexdigest()


def grid_bytes(name) -> np.ndarray:
    """Codebook as signed bytes: (entries, 8) for IQ2*, (entries, 4) for IQ3S."""
    vals, _ = GRIDS[name]
    width = 4 if name == "IQ3S" else 8
    return vals.astype("<u8").view(np.uint8).reshape(-1, 8)[:, :width].astype(np.int8)


def ksigns():
    i = np.arange(128)
    par = np.array([bin(v).count("1") & 1 for v in i])
    return (i | (par << 7)).astype(np.uint8)


def f16(b0, b1):
    """float64 value of little-endian f16 fields (exact)."""
    bits = (np.asarray(b0, np.uint16) | (np.asarray(b1, np.uint16) << 8)).astype("<u2")
    return bits.view(np.float16).astype(np.float64)


def _bits(q, lo, n):
    return (q >> lo) & ((1 << n) - 1)


def _signs_to_pm(signbyte, nbits=8):
    """(..., ) uint8 -> (..., nbits) of +1/-1 (bit j set => -1)."""
    j = np.arange(nbits)
    return np.where((signbyte[..., None].astype(np.int64) >> j) & 1, -1.0, 1.0)


def decode(t: int, data: np.ndarray) -> np.ndarray:
    """Decode a flat uint8 buffer of type-t blocks to float32 (via exact float64)."""
    data = np.asarray(data, dtype=np.uint8)
    if t == 0:
        return data.view("<f4").astype(np.float32)
    if t == 1:
        return data.view("<f2").astype(np.float32)
    if t == 30:
        return (data.view("<u2").astype(np.uint32) << 16).view(np.float32)
    fn = _DECODERS[t]
    return fn(data).astype(np.float32).reshape(-1)


def _blocks(data, nbytes):
    return data.reshape(-1, nbytes).astype(np.int64)


def _q8_0(data):
    b = _blocks(data, 34)
    d = f16(b[:, 0], b[:, 1])
    q = b[:, 2:34].astype(np.uint8).view(np.int8).astype(np.float64)
    return d[:, None] * q


def _q5_common(qs, qh, d, m=None, signed=True):
    j = np.arange(16)
    lo = (qs & 15) | (((qh[:, None] >> j) & 1) << 4)
    hi = (qs >> 4) | (((qh[:, None] >> (j + 16)) & 1) << 4)
    q = np.concatenate([lo, hi], axis=1).astype(np.float64)
    if signed:
        return (q - 16.0) * d[:, None]
    return q * d[:, None] + m[:, None]


def _q5_0(data):
    b = _blocks(data, 22)
    qh = b[:, 2] | (b[:, 3] << 8) | (b[:, 4] << 16) | (b[:, 5] << 24)
    return _q5_common(b[:, 6:22], qh, f16(b[:, 0], b[:, 1]))


def _q5_1(data):
    b = _blocks(data, 24)
    qh = b[:, 4] | (b[:, 5] << 8) | (b[:, 6] << 16) | (b[:, 7] << 24)
    return _q5_common(b[:, 8:24], qh, f16(b[:, 0], b[:, 1]), f16(b[:, 2], b[:, 3]), signed=False)


def _q4_0(data):
    b = _blocks(data, 18)
    q = np.concatenate([b[:, 2:18] & 15, b[:, 2:18] >> 4], axis=1).astype(np.float64)
    return (q - 8.0) * f16(b[:, 0], b[:, 1])[:, None]


def _q4_1(data):
    b = _blocks(data, 20)
    q = np.concatenate([b[:, 4:20] & 15, b[:, 4:20] >> 4], axis=1).astype(np.float64)
    return q * f16(b[:, 0], b[:, 1])[:, None] + f16(b[:, 2], b[:, 3])[:, None]


IQ4NL = np.array([-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113], np.float64)


def _iq4nl(data):
    b = _blocks(data, 18)
    idx = np.concatenate([b[:, 2:18] & 15, b[:, 2:18] >> 4], axis=1)
    return f16(b[:, 0], b[:, 1])[:, None] * IQ4NL[idx]


def k4_scales(sc):
    """(nb, 12) packed bytes -> (nb, 8) scales and (nb, 8) mins (6-bit each)."""
    s = np.zeros((sc.shape[0], 8), np.int64)
    m = np.zeros_like(s)
    s[:, :4] = sc[:, 0:4] & 63
    m[:, :4] = sc[:, 4:8] & 63
    s[:, 4:] = (sc[:, 8:12] & 15) | ((sc[:, 0:4] >> 6) << 4)
    m[:, 4:] = (sc[:, 8:12] >> 4) | ((sc[:, 4:8] >> 6) << 4)
    return s, m


def _q4_k(data):
    b = _blocks(data, 144)
    d, dmin = f16(b[:, 0], b[:, 1]), f16(b[:, 2], b[:, 3])
    s, m = k4_scales(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32)  # sub-block 2i = low, 2i+1 = high
    v = d[:, None, None] * s[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    return v.reshape(-1, 256)


def _q5_k(data):
    b = _blocks(data, 176)
    d, dmin = f16(b[:, 0], b[:, 1]), f16(b[:, 2], b[:, 3])
    s, m = k4_scales(b[:, 4:16])
    qh = b[:, 16:48]
    qs = b[:, 48:176].reshape(-1, 4, 32)
    jb = np.arange(4)[None, :, None]
    lo = (qs & 15) + 16 * ((qh[:, None, :] >> (2 * jb)) & 1)
    hi = (qs >> 4) + 16 * ((qh[:, None, :] >> (2 * jb + 1)) & 1)
    q = np.stack([lo, hi], axis=2).reshape(-1, 8, 32)
    v = d[:, None, None] * s[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    return v.reshape(-1, 256)


def _q6_k(data):
    b = _blocks(data, 210)
    d = f16(b[:, 208], b[:, 209])
    sc = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.float64)
    out = np.zeros((b.shape[0], 256))
    l = np.arange(32)
    for h in range(2):
        ql = b[:, 64 * h:64 * h + 64]
        qh = b[:, 128 + 32 * h:128 + 32 * h + 32]
        qv = [
            (ql[:, :32] & 15) | (_bits(qh, 0, 2) << 4),
            (ql[:, 32:] & 15) | (_bits(qh, 2, 2) << 4),
            (ql[:, :32] >> 4) | (_bits(qh, 4, 2) << 4),
            (ql[:, 32:] >> 4) | (_bits(qh, 6, 2) << 4),
        ]
        for k in range(4):
            scale = sc[:, 8 * h + l // 16 + 2 * k]
            out[:, 128 * h + 32 * k + l] = d[:, None] * scale * (qv[k] - 32)
    return out


def _q2_k(data):
    b = _blocks(data, 84)
    sc = b[:, 0:16]
    qs = b[:, 16:80]
    d, dmin = f16(b[:, 80], b[:, 81]), f16(b[:, 82], b[:, 83])
    out = np.zeros((b.shape[0], 256))
    for n in range(2):
        q = qs[:, 32 * n:32 * n + 32]
        for j in range(4):
            for half in range(2):
                is_ = 8 * n + 2 * j + half
                dl = d * (sc[:, is_] & 15)
                ml = dmin * (sc[:, is_] >> 4)
                vals = (q[:, 16 * half:16 * half + 16] >> (2 * j)) & 3
                base = 128 * n + 32 * j + 16 * half
                out[:, base:base + 16] = dl[:, None] * vals - ml[:, None]
    return out


def _iq2_xxs(data):
    b = _blocks(data, 66)
    d = f16(b[:, 0], b[:, 1])
    g = grid_bytes("IQ2XXS").astype(np.float64)
    ks = ksigns()
    qs = b[:, 2:66].reshape(-1, 8, 8)
    a1 = qs[:, :, 4] | (qs[:, :, 5] << 8) | (qs[:, :, 6] << 16) | (qs[:, :, 7] << 24)
    db = d[:, None] * (0.5 + (a1 >> 28)) * 0.25  # (nb, 8)
    l = np.arange(4)
    idx = qs[:, :, 0:4]  # (nb, 8, 4)
    signs = ks[(a1[:, :, None] >> (7 * l)) & 127]  # (nb, 8, 4)
    vals = g[idx] * _signs_to_pm(signs)  # (nb, 8, 4, 8)
    return (db[:, :, None, None] * vals).reshape(-1, 256)


def _iq2_xs(data):
    b = _blocks(data, 74)
    d = f16(b[:, 0], b[:, 1])
    g = grid_bytes("IQ2XS").astype(np.float64)
    ks = ksigns()
    q = (b[:, 2:66:2] | (b[:, 3:66:2] << 8)).reshape(-1, 8, 4)
    sc = b[:, 66:74]
    db = np.stack([d[:, None] * (0.5 + (sc & 15)) * 0.25, d[:, None] * (0.5 + (sc >> 4)) * 0.25], axis=2)
    dbl = db[:, :, [0, 0, 1, 1]]  # l < 2 -> low nibble scale
    vals = g[q & 511] * _signs_to_pm(ks[q >> 9])
    return (dbl[..., None] * vals).reshape(-1, 256)


def _iq2_s(data):
    b = _blocks(data, 82)
    d = f16(b[:, 0], b[:, 1])
    g = grid_bytes("IQ2S").astype(np.float64)
    qs = b[:, 2:66]
    qh = b[:, 66:74]
    sc = b[:, 74:82]
    l = np.arange(4)
    idx = qs[:, 0:32].reshape(-1, 8, 4) | ((qh[:, :, None] << (8 - 2 * l)) & 0x300)
    signs = qs[:, 32:64].reshape(-1, 8, 4)
    db = np.stack([d[:, None] * (0.5 + (sc & 15)) * 0.25, d[:, None] * (0.5 + (sc >> 4)) * 0.25], axis=2)
    dbl = db[:, :, [0, 0, 1, 1]]
    vals = g[idx] * _signs_to_pm(signs)
    return (dbl[..., None] * vals).reshape(-1, 256)


def _iq3_s(data):
    b = _blocks(data, 110)
    d = f16(b[:, 0], b[:, 1])
    g = grid_bytes("IQ3S").astype(np.float64)
    qs = b[:, 2:66].reshape(-1, 8, 8)  # (nb, ib32, 8 index bytes)
    qh = b[:, 66:74]  # per ib32
    sg = b[:, 74:106].reshape(-1, 8, 4)
    sc = b[:, 106:110]
    scale = np.stack([sc & 15, sc >> 4], axis=2).reshape(-1, 8)  # ib32 -> nibble
    db = d[:, None] * (1.0 + 2.0 * scale)
    l = np.arange(4)
    i0 = qs[:, :, 0::2] | ((qh[:, :, None] << (8 - 2 * l)) & 256)
    i1 = qs[:, :, 1::2] | ((qh[:, :, None] << (7 - 2 * l)) & 256)
    pm = _signs_to_pm(sg)  # (nb, 8, 4, 8)
    v1 = g[i0] * pm[..., 0:4]
    v2 = g[i1] * pm[..., 4:8]
    vals = np.concatenate([v1, v2], axis=3)  # (nb, 8, 4, 8)
    return (db[:, :, None, None] * vals).reshape(-1, 256)


_DECODERS = {
    2: _q4_0, 3: _q4_1, 6: _q5_0, 7: _q5_1, 8: _q8_0, 10: _q2_k, 12: _q4_k, 13: _q5_k, 14: _q6_k,
    16: _iq2_xxs, 17: _iq2_xs, 20: _iq4nl, 21: _iq3_s, 22: _iq2_s,
}


def gemv_f64(t, x, data, in_dim, out_dim):
    """Brute-force float64 dot of the exact dequantized matrix."""
    w = decode(t, data).astype(np.float64).reshape(out_dim, in_dim)
    return w @ np.asarray(x, np.float64).reshape(-1, in_dim).T


def rel_l2(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
