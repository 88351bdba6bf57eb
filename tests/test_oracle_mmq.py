"""The oracle's Q8_1 MMQ arithmetic mode (oracle/quartz_oracle.c, restating
src/dequant.rs:202-645), pinned without the reference running:

  * f32 -> f16 round-to-even against numpy's float16 conversion (IEEE
    round-to-nearest-even, a library routine) on 200k random bit patterns,
    subnormals and halfway cases included, and the NaN/Inf encodings;
  * Q8_1 quantisation on closed-form inputs (ramps, a constant, zeros, a block
    whose max is 127);
  * the GEMMs against a float64 sum over the same quantised operands, built here
    with independent code (closed_form's Q4_K scale unpack and Q6_K layout,
    numpy's f16 rounding), 1e-6 relative;
  * the stream-K cut against hand-computed partitions.
No GPU needed."""
import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import synth


def f16r(v):
    return np.asarray(v, np.float32).astype(np.float16).astype(np.float64)


def test_f16_round_to_even_vs_numpy(oracle):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32)
    # bias towards the f16 range and its subnormals / halfway points
    bits[:100_000] = (bits[:100_000] & 0x807FFFFF) | (rng.integers(100, 145, 100_000).astype(np.uint32) << 23)
    bits[100_000:100_100] = (np.arange(100, dtype=np.uint32) << 13) | (0x70 << 23) | 0x1000  # halfway cases
    vals = bits.view(np.float32)
    ok = ~np.isnan(vals)
    want = vals[ok].astype(np.float16).view(np.uint16)
    got = np.array([oracle.f32_to_f16_rne(float(v)) for v in vals[ok]], np.uint16)
    assert np.array_equal(got, want)
    assert oracle.f32_to_f16_rne(float("nan")) == 0x7E00
    assert oracle.f32_to_f16_rne(float("inf")) == 0x7C00
    assert oracle.f32_to_f16_rne(float("-inf")) == 0xFC00
    assert oracle.f32_to_f16_rne(70000.0) == 0x7C00  # overflow rounds to Inf


def test_quantize_q8_1_closed_forms(oracle):
    x = np.zeros((1, 128), np.float32)
    x[0, :32] = np.arange(32)                 # ramp: max 31
    x[0, 32:64] = -127.0                      # constant: every value -127
    x[0, 96:128] = np.arange(32) * 0.25 - 4   # another ramp with negatives
    q, sc, sm = oracle.quantize_q8_1(x, 128, 1, d4=False)
    # ramp 0..31: q_i = round(i * 127/31), half away from zero
    assert np.array_equal(q[0, :32], np.floor(np.arange(32) * (127.0 / 31.0) + 0.5).astype(np.int8))
    assert sc[0, 0] == f16r(31.0 / 127.0)
    assert sm[0, 0] == f16r(np.arange(32).sum())
    assert np.all(q[0, 32:64] == -127) and sc[0, 1] == 1.0 and sm[0, 1] == f16r(-127 * 32)
    assert np.all(q[0, 64:96] == 0) and sc[0, 2] == 0.0 and sm[0, 2] == 0.0     # all zeros
    assert q[0, 96] == -127 and abs(q[0, 127]) <= 127
    q4, sc4, sm4 = oracle.quantize_q8_1(x, 128, 1, d4=True)
    assert np.array_equal(q4, q) and np.all(sm4 == 0)
    assert sc4[0, 0] == np.float32(1.0) / (np.float32(127.0) / np.float32(31.0))  # unrounded 1 / (127/max)


def _q4k_parts(data):
    b = cf._blocks(data, 144)
    d, dmin = cf.f16(b[:, 0], b[:, 1]), cf.f16(b[:, 2], b[:, 3])
    s, m = cf.k4_scales(b[:, 4:16])
    qs = b[:, 16:144].reshape(-1, 4, 32)
    q = np.stack([qs & 15, qs >> 4], axis=2).reshape(-1, 8, 32).astype(np.int64)
    return d, dmin, s, m, q


def _q6k_parts(data):
    b = cf._blocks(data, 210)
    d = cf.f16(b[:, 208], b[:, 209])
    sc = b[:, 192:208].astype(np.uint8).view(np.int8).astype(np.int64)
    q = np.zeros((b.shape[0], 256), np.int64)
    for h in range(2):
        ql, qh = b[:, 64 * h:64 * h + 64].astype(np.int64), b[:, 128 + 32 * h:160 + 32 * h].astype(np.int64)
        for k, (lo, sh) in enumerate(((ql[:, :32] & 15, 0), (ql[:, 32:] & 15, 2), (ql[:, :32] >> 4, 4),
                                      (ql[:, 32:] >> 4, 6))):
            q[:, 128 * h + 32 * k:128 * h + 32 * k + 32] = (lo | (((qh >> sh) & 3) << 4)) - 32
    return d, sc, q


@pytest.mark.parametrize("t", [12, 14])
def test_gemm_q8_1_mmq_vs_f64(oracle, t):
    rows, in_dim, out_dim = 3, 512, 37
    rng = np.random.default_rng(t)
    x = rng.standard_normal((rows, in_dim)).astype(np.float32)
    data = synth.weights(t, out_dim, in_dim, seed=5)
    got = oracle.gemm_q8_1_mmq(t, x, data, in_dim, out_dim, rows)
    qa, sa, ma = oracle.quantize_q8_1(x, in_dim, rows, d4=(t == 14))
    nb = in_dim // 256
    ref = np.zeros((rows, out_dim))
    for c in range(out_dim):
        row_bytes = data.reshape(out_dim, -1)[c]
        for r in range(rows):
            acc = 0.0
            if t == 12:
                d, dmin, s, m, q = _q4k_parts(row_bytes)
                for b in range(nb):
                    for g in range(8):
                        dot = int(np.dot(q[b, g], qa[r, 256 * b + 32 * g:256 * b + 32 * g + 32].astype(np.int64)))
                        cs, cm = f16r(d[b] * s[b, g]), f16r(-dmin[b] * m[b, g])
                        acc += cs * sa[r, 8 * b + g] * dot + cm * ma[r, 8 * b + g]
            else:
                d, sc, q = _q6k_parts(row_bytes)
                for b in range(nb):
                    for g in range(8):
                        xs = qa[r, 256 * b + 32 * g:256 * b + 32 * g + 32].astype(np.int64)
                        d1 = int(np.dot(q[b, 32 * g:32 * g + 16], xs[:16]))
                        d2 = int(np.dot(q[b, 32 * g + 16:32 * g + 32], xs[16:]))
                        acc += d[b] * sa[r, 8 * b + g] * (sc[b, 2 * g] * d1 + sc[b, 2 * g + 1] * d2)
            ref[r, c] = acc
    assert cf.rel_l2(got, ref) < 1e-6
    # the quantised product tracks the float GEMV to the Q8_1 activation precision
    exact = np.stack([cf.gemv_f64(t, x[r], data, in_dim, out_dim) for r in range(rows)])
    assert cf.rel_l2(got, exact) < 3e-2


def test_stream_k_cut_hand_cases(oracle):
    # 3 tiles of 128 columns, 4 superblocks each, 2 multiprocessors: efficiency
    # 100*3/(2*2) = 75% < 90, so grid = 2 and the 12 blocks split at block 6,
    # inside tile 1 (blocks 4..7): its outputs are cut at superblock 2.
    args = dict(in_dim=1024, out_dim=384, reference_rows=128, mps=2)
    assert oracle.stream_k_cut(0, 130, **args) == 2
    assert oracle.stream_k_cut(100, 255, **args) == 2
    assert oracle.stream_k_cut(0, 0, **args) == -1    # tile 0: blocks 0..3, no boundary inside
    assert oracle.stream_k_cut(0, 300, **args) == -1  # tile 2: blocks 8..11
    # tile count a multiple of the grid: no stream-K fixup
    assert oracle.stream_k_cut(0, 0, 1024, 256 * 128, 128, 64) == -1
    # 90% efficiency or more: grid = tile count
    assert oracle.stream_k_cut(0, 0, 1024, 10 * 128, 128, 10) == -1
    assert oracle.stream_k_cut(0, 0, 1000, 384, 128, 2) == -1  # in_dim not a multiple of 256
    # the split result = tail + prefix, equal to the unsplit sum up to f32 rounding
    rng = np.random.default_rng(2)
    x = rng.standard_normal((2, 1024)).astype(np.float32)
    data = synth.weights(12, 384, 1024, seed=3)
    a = oracle.gemm_q8_1_mmq(12, x, data, 1024, 384, 2)
    b = oracle.gemm_q8_1_mmq(12, x, data, 1024, 384, 2, reference_rows=128, mps=2)
    assert np.array_equal(a[:, :128], b[:, :128]) and np.array_equal(a[:, 256:], b[:, 256:])
    assert cf.rel_l2(b[:, 128:256], a[:, 128:256]) < 1e-6
