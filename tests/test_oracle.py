"""Pins the CPU oracle (oracle/quartz_oracle.c) -- no GPU needed.

The reference has no tests and no golden vectors on this path (its GEMV code is
Rust/CUDA, neither buildable here), so the oracle is pinned by:
  * f16_to_f32 against IEEE binary16 for all 65536 patterns (numpy),
  * every dequant against float64 closed forms (bit-exact),
  * hand-computed known answers that catch transposed nibbles, wrong scale
    packing, a dropped -32/-16/-8 offset or a wrong sign convention,
  * GEMV/GEMM against a float64 brute-force dot, plus linearity and one-hot
    column checks,
  * the IQ codebooks against their SHA-256 and structural invariants.
"""
import struct

import numpy as np
from pathlib import Path
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES
from saient_quartz_amd import synth

ALL_TYPES = sorted(GGML_TYPES)
QUANT_TYPES = [t for t in ALL_TYPES if GGML_TYPES[t][1] > 1]


def test_f16_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    # through o_dequant(F16), which calls f16_to_f32 per element and writes f32
    # bits to memory (a float return through ctypes would quiet signalling NaNs)
    got = oracle.dequant(1, bits.view(np.uint8), 65536)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # NaN payloads are kept (mant << 13), not quieted: src/dequant.rs:1345-1346
    for b in (0x7C01, 0xFC01, 0x7E00, 0x7DFF):
        v = got[b].view(np.uint32)
        assert v == (((b >> 15) << 31) | 0x7F800000 | ((b & 0x3FF) << 13))


@pytest.mark.parametrize("t", ALL_TYPES)
def test_type_size(oracle, t):
    _, qk, bb = GGML_TYPES[t]
    for n in (qk, 4096 * qk // qk * 1, 14336 * 4096):
        assert oracle.type_size(t, n) == (n // qk) * bb
    assert oracle.type_size(99, 256) == 0


@pytest.mark.parametrize("t", ALL_TYPES)
def test_dequant_matches_closed_form(oracle, t):
    _, qk, _ = GGML_TYPES[t]
    n = 64 * 256
    data = synth.weights(t, 64, 256, seed=1000 + t)
    got = oracle.dequant(t, data, n)
    ref = cf.decode(t, data)
    assert got.shape == ref.shape
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), f"type {t}: not bit-exact"


@pytest.mark.parametrize("t", QUANT_TYPES)
def test_dequant_random_bytes_closed_form(oracle, t):
    """Fully random blocks (random f16 scales too, excluding Inf/NaN) stay bit-exact."""
    _, qk, bb = GGML_TYPES[t]
    rng = np.random.default_rng(77 + t)
    nb = 512
    data = rng.integers(0, 256, size=(nb, bb), dtype=np.uint8)
    # keep f16 fields finite: clear the top exponent bit of every 2-byte scale slot
    for off, _, _ in synth._F16_FIELDS[t]:
        data[:, off + 1] &= 0x3F  # |value| < 2
    data = data.reshape(-1)
    got = oracle.dequant(t, data, nb * qk)
    ref = cf.decode(t, data)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def _f16(v):
    return struct.pack("<e", v)


def test_known_q4_k(oracle):
    # d = 1, dmin = 0.5; scales: j<4 -> sc[j] = j+1, m[j] = 2j; j>=4 -> sc = 5,6,7,8 with
    # high bits from bytes 0..3 (bit 6-7), m = 1.. likewise.
    sc = bytearray(12)
    for j in range(4):
        sc[j] = (j + 1) | (1 << 6)  # low 6 bits: scale j; top 2 bits feed scale j+4 (<<4 -> +16)
        sc[j + 4] = (2 * j) | (0 << 6)
        sc[j + 8] = (5 + j) | ((3 - j) << 4)  # low nibble: scale j+4 low bits; high nibble: min j+4
    qs = bytearray(128)
    qs[0] = 0x21  # weight 0 -> 1 (sub 0), weight 32 -> 2 (sub 1)
    qs[32] = 0xF3  # weight 64 -> 3 (sub 2), weight 96 -> 15 (sub 3)
    qs[127] = 0x4E  # weight 255-32=223 -> 14 (sub 6), weight 255 -> 4 (sub 7)
    blk = _f16(1.0) + _f16(0.5) + bytes(sc) + bytes(qs)
    v = oracle.dequant(12, np.frombuffer(blk, np.uint8), 256)
    scale = [1, 2, 3, 4, 5 + 16, 6 + 16, 7 + 16, 8 + 16]
    mins = [0, 2, 4, 6, 3, 2, 1, 0]
    assert v[0] == 1.0 * scale[0] * 1 - 0.5 * mins[0]
    assert v[1] == -0.5 * mins[0]
    assert v[32] == 1.0 * scale[1] * 2 - 0.5 * mins[1]
    assert v[64] == scale[2] * 3 - 0.5 * mins[2]
    assert v[96] == scale[3] * 15 - 0.5 * mins[3]
    assert v[223] == scale[6] * 14 - 0.5 * mins[6]
    assert v[255] == scale[7] * 4 - 0.5 * mins[7]
    assert v[200] == -0.5 * mins[6]


def test_known_q6_k(oracle):
    ql = bytearray(128)
    qh = bytearray(64)
    sc = bytearray(16)
    for i in range(16):
        sc[i] = (i - 8) & 0xFF  # signed sub-scales -8..7
    ql[0] = 0x5A       # y[0]: low 0xA, y[64]: high 0x5
    qh[0] = 0b11100100  # y[0] +0<<4, y[32] +1<<4, y[64] +2<<4, y[96] +3<<4
    ql[32] = 0x07      # y[32]: low 7, y[96]: high 0
    ql[64 + 17] = 0x3F  # half 1, l=17: y[128+17] low 0xF, y[128+81] high 3
    blk = bytes(ql) + bytes(qh) + bytes(sc) + _f16(0.25)
    v = oracle.dequant(14, np.frombuffer(blk, np.uint8), 256)
    s = [i - 8 for i in range(16)]
    assert v[0] == 0.25 * s[0] * ((0xA | 0 << 4) - 32)
    assert v[32] == 0.25 * s[2] * ((0x7 | 1 << 4) - 32)
    assert v[64] == 0.25 * s[4] * ((0x5 | 2 << 4) - 32)
    assert v[96] == 0.25 * s[6] * ((0x0 | 3 << 4) - 32)
    assert v[1] == 0.25 * s[0] * -32  # all-zero quant -> -32 offset
    assert v[128 + 17] == 0.25 * s[8 + 1] * (0xF - 32)
    assert v[128 + 81] == 0.25 * s[8 + 1 + 4] * (3 - 32)


def test_known_q8_0_q5_0_q4_0(oracle):
    q = bytes(((i - 16) & 0xFF) for i in range(32))
    v = oracle.dequant(8, np.frombuffer(_f16(0.5) + q, np.uint8), 32)
    assert list(v) == [0.5 * (i - 16) for i in range(32)]
    # Q5_0: qh bit j -> +16 on weight j; qs nibbles low -> j, high -> j+16; v = (q - 16) d
    qh = (1 << 0) | (1 << 17)
    qs = bytes([0x21] + [0] * 15)
    v = oracle.dequant(6, np.frombuffer(_f16(2.0) + struct.pack("<I", qh) + qs, np.uint8), 32)
    assert v[0] == 2.0 * ((1 | 16) - 16) and v[16] == 2.0 * (2 - 16)
    assert v[17] == 2.0 * ((0 | 16) - 16) and v[1] == 2.0 * -16
    v = oracle.dequant(2, np.frombuffer(_f16(1.5) + bytes([0xF0] + [0x88] * 15), np.uint8), 32)
    assert v[0] == 1.5 * -8 and v[16] == 1.5 * 7 and v[1] == 0.0 and v[17] == 0.0


def test_known_q5_1_q4_1_iq4nl(oracle):
    qh = 1 << 31
    qs = bytes([0x3C] + [0] * 15)
    v = oracle.dequant(7, np.frombuffer(_f16(0.5) + _f16(-1.0) + struct.pack("<I", qh) + qs, np.uint8), 32)
    assert v[0] == 0.5 * 12 - 1.0 and v[16] == 0.5 * 3 - 1.0 and v[31] == 0.5 * 16 - 1.0
    v = oracle.dequant(3, np.frombuffer(_f16(0.5) + _f16(0.25) + bytes([0x3C] + [0] * 15), np.uint8), 32)
    assert v[0] == 6.25 and v[16] == 1.75 and v[5] == 0.25
    v = oracle.dequant(20, np.frombuffer(_f16(0.5) + bytes([0xF0] + [0x78] * 15), np.uint8), 32)
    assert v[0] == 0.5 * -127 and v[16] == 0.5 * 113 and v[1] == 0.5 * 1 and v[17] == 0.5 * -10


def test_known_iq(oracle):
    # Grid index 0 is 0x08..08 for every IQ2 grid (src/dequant.rs:984-985): all +-8 * db.
    # IQ2_XXS: a1 scale nibble 3 -> db = d * 3.5 * 0.25; sign index 1 -> ksigns[1] = 0b10000001.
    a1 = (3 << 28) | (1 << 0)
    blk = _f16(1.0) + (bytes(4) + struct.pack("<I", a1)) * 8
    v = oracle.dequant(16, np.frombuffer(blk, np.uint8), 256)
    db = 3.5 * 0.25
    assert v[0] == -8 * db and v[7] == -8 * db and v[1] == 8 * db  # bits 0 and 7 set
    assert v[8] == 8 * db  # second quad of the group: sign index 0
    # IQ3_S grid index 0 is 0x01010101: all +-1 * db, db = d * (1 + 2 * nibble)
    blk = _f16(0.5) + bytes(64) + bytes(8) + bytes([0x01] + [0] * 31) + bytes([0x21, 0, 0, 0])
    v = oracle.dequant(21, np.frombuffer(blk, np.uint8), 256)
    assert v[0] == -0.5 * 3 and v[1] == 0.5 * 3 and v[32] == 0.5 * 5 and v[64] == 0.5


def test_ksigns_closed_form():
    ks = cf.ksigns()
    assert ks[0] == 0 and ks[1] == 129 and ks[3] == 3 and ks[127] == 255
    # every entry has even parity over 8 bits
    assert all(bin(int(v)).count("1") % 2 == 0 for v in ks)


def test_iq_grids_pinned(oracle):
    for i, name in enumerate(("IQ2XXS", "IQ2XS", "IQ2S", "IQ3S")):
        vals, sha = cf.GRIDS[name]
        assert cf.grid_sha256(name) == sha
        assert oracle.L.o_grid_sha256(i).decode() == sha
    sizes = {"IQ2XXS": 256, "IQ2XS": 512, "IQ2S": 1024, "IQ3S": 512}
    for name, size in sizes.items():
        g = cf.grid_bytes(name)
        assert g.shape[0] == size
        assert len({tuple(r) for r in g}) == size  # distinct codewords
    for name in ("IQ2XXS", "IQ2XS", "IQ2S"):
        assert set(np.unique(cf.grid_bytes(name))) <= {8, 25, 43}
        assert tuple(cf.grid_bytes(name)[0]) == (8,) * 8
    assert set(np.unique(cf.grid_bytes("IQ3S"))) <= set(range(1, 16, 2))
    assert tuple(cf.grid_bytes("IQ3S")[0]) == (1, 1, 1, 1)


# SHA-256 of each codebook's little-endian values (u64 entries for IQ2*, u32 for
# IQ3S), computed from the reference's tables (src/iq2_tables.rs:3-7,
# src/iq3_tables.rs:2).  Literal here, independent of iq_grids.h, so a wrong
# regeneration of the header fails this test even where the reference is absent.
IQ_GRID_SHA256 = {
    "IQ2XXS": "05826b5d3e472a3a78f196be62ac78acf81df0f909626e12ab9fa2a5d490dd54",
    "IQ2XS": "06e47aaca60b4dc1d9b5a3f34540437058a6b142b4d7a59d5ded769b4d1bf1de",
    "IQ2S": "e1aa1473412b0552c2174c30ef22ab4073f6a181b85a17056e8249bd2932fd88",
    "IQ3S": "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f",
}
REF_SRC = Path("/root/reference/src")


def test_iq_grids_match_pinned_hashes():
    for name, sha in IQ_GRID_SHA256.items():
        assert cf.grid_sha256(name) == sha, name


@pytest.mark.skipif(not (REF_SRC / "iq2_tables.rs").exists(), reason="reference sources not present")
def test_iq_grids_equal_reference_tables():
    """Parse the reference's Rust tables and compare them value by value with
    the header's (and ksigns / kmask with their closed forms)."""
    import re

    def table(fname, ident):
        txt = (REF_SRC / fname).read_text()
        m = re.search(r"pub static %s: \[u\d+; (\d+)\] = \[(.*?)\];" % ident, txt, re.S)
        vals = [int(v, 0) for v in re.findall(r"0x[0-9a-fA-F]+|\b\d+\b", m.group(2))]
        assert len(vals) == int(m.group(1))
        return np.array(vals, dtype=np.uint64)

    for name, (fname, ident) in {"IQ2XXS": ("iq2_tables.rs", "IQ2XXS_GRID"), "IQ2XS": ("iq2_tables.rs", "IQ2XS_GRID"),
                                 "IQ2S": ("iq2_tables.rs", "IQ2S_GRID"), "IQ3S": ("iq3_tables.rs", "IQ3S_GRID")}.items():
        np.testing.assert_array_equal(cf.GRIDS[name][0], table(fname, ident), err_msg=name)
    np.testing.assert_array_equal(table("iq2_tables.rs", "KSIGNS_IQ2XS").astype(np.uint8), cf.ksigns())
    np.testing.assert_array_equal(table("iq2_tables.rs", "KMASK_IQ2XS"), 1 << np.arange(8, dtype=np.uint64))


@pytest.mark.parametrize("t", ALL_TYPES)
@pytest.mark.parametrize("shape", [(8, 256), (3, 512), (17, 1024)])
def test_gemv_vs_f64(oracle, t, shape):
    out_dim, in_dim = shape
    data = synth.weights(t, out_dim, in_dim, seed=2000 + t)
    x = synth.activations(1, in_dim, seed=3000)[0]
    y = oracle.gemv(t, x, data, in_dim, out_dim)
    ref = cf.gemv_f64(t, x, data, in_dim, out_dim)[:, 0]
    assert cf.rel_l2(y, ref) < 1e-5


@pytest.mark.parametrize("t", [8, 12, 14, 21])
def test_gemv_linearity_and_onehot(oracle, t):
    out_dim, in_dim = 16, 512
    data = synth.weights(t, out_dim, in_dim, seed=4000 + t)
    x = synth.activations(1, in_dim, seed=4001)[0]
    y = oracle.gemv(t, x, data, in_dim, out_dim)
    y2 = oracle.gemv(t, 2.0 * x, data, in_dim, out_dim)
    assert np.array_equal(y2, 2.0 * y)  # scaling by 2 is exact
    w = oracle.dequant(t, data, out_dim * in_dim).reshape(out_dim, in_dim)
    for col in (0, 31, 32, 255, 300):
        e = np.zeros(in_dim, np.float32)
        e[col] = 1.0
        assert np.array_equal(oracle.gemv(t, e, data, in_dim, out_dim), w[:, col])


@pytest.mark.parametrize("t", ALL_TYPES)
def test_gemm_rows_equal_gemv(oracle, t):
    out_dim, in_dim, n = 9, 512, 4
    data = synth.weights(t, out_dim, in_dim, seed=5000 + t)
    x = synth.activations(n, in_dim, seed=5001)
    Y = oracle.gemm(t, x, data, in_dim, out_dim, n)
    ref = cf.gemv_f64(t, x, data, in_dim, out_dim).T
    assert cf.rel_l2(Y, ref) < 1e-5
    for k in range(n):
        assert cf.rel_l2(Y[k], oracle.gemv(t, x[k], data, in_dim, out_dim)) < 1e-5


def test_oracle_rejects_bad_input(oracle):
    data = synth.weights(12, 2, 256, seed=1)
    with pytest.raises(ValueError):
        oracle.gemv(12, np.zeros(200, np.float32), data, 200, 2)  # not a multiple of 256
    with pytest.raises(ValueError):
        oracle.gemv(99, np.zeros(256, np.float32), data, 256, 2)


def test_gemv_thread_count_independent(oracle):
    data = synth.weights(12, 64, 1024, seed=9)
    x = synth.activations(1, 1024, seed=10)[0]
    n0 = oracle.threads()
    oracle.set_threads(1)
    a = oracle.gemv(12, x, data, 1024, 64)
    oracle.set_threads(max(2, n0))
    b = oracle.gemv(12, x, data, 1024, 64)
    oracle.set_threads(n0)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("t", [8, 6, 16, 21, 12])
def test_gemv_dequant_matmul_equals_gemv(oracle, t):
    """The whole-matrix dequant + matmul form (timed as the CPU baseline of the
    `_` arm) gives o_gemv's values bit for bit."""
    out_dim, in_dim = 33, 1024
    data = synth.weights(t, out_dim, in_dim, seed=77 + t)
    x = synth.activations(1, in_dim, seed=5)[0]
    a = oracle.gemv(t, x, data, in_dim, out_dim)
    b = oracle.gemv_dequant_matmul(t, x, data, in_dim, out_dim)
    if t == 12:  # fused-row type: same values up to the f32 sum order
        assert cf.rel_l2(a, b) < 1e-5
    else:
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
