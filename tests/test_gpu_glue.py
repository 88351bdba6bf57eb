"""GPU parity of the decode-step glue kernels (hip_* twins of the reference's
forward-pass helpers) against oracle/glue_ref.py in float64.

Tolerances (f32 kernels against f64): 1e-5 relative L2 for rms_norm, softmax,
attention and swiglu; RoPE 2e-5 at pos < 64 and 2e-4 at pos 4000 (the f32 angle
pos * inv_freq carries about pos * 2^-24 radians of rounding, as in the
reference's kernel).  hip_embed_lookup is bit-exact against the oracle's
dequant.
"""
import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES, synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import glue_ref as g  # noqa: E402

pytestmark = pytest.mark.gpu


def up(a):
    return GpuBuf.upload_f32(np.ascontiguousarray(a, np.float32).reshape(-1))


def down(b, n):
    return b.download(np.float32)[:n]


def sync(qh):
    check("hip_sync", qh.hip_sync())


@pytest.mark.parametrize("n", [1, 37, 896, 4096, 14336])
def test_rms_norm(qh, n):
    rng = np.random.default_rng(n)
    x, w = rng.standard_normal(n) * 3, rng.standard_normal(n)
    dx, dw, do = up(x), up(w), GpuBuf.alloc_f32(n)
    check("rms_norm", qh.hip_rms_norm(do.ptr, dx.ptr, dw.ptr, n))
    check("rms_norm in place", qh.hip_rms_norm(dx.ptr, dx.ptr, dw.ptr, n))
    sync(qh)
    ref = g.rms_norm(x.astype(np.float32), w.astype(np.float32))
    assert cf.rel_l2(down(do, n), ref) < 1e-5
    assert cf.rel_l2(down(dx, n), ref) < 1e-5


@pytest.mark.parametrize("neox", [0, 1])
@pytest.mark.parametrize("pos, tol", [(0, 2e-5), (17, 2e-5), (4000, 2e-4)])
@pytest.mark.parametrize("yarn", [(1.0, 0), (4.0, 4096)])
def test_rope_yarn(qh, neox, pos, tol, yarn):
    nh, hd = 8, 128
    x = np.random.default_rng(pos + 7 * neox).standard_normal(nh * hd).astype(np.float32)
    dx = up(x)
    check("rope", qh.hip_rope_yarn(dx.ptr, nh, hd, pos, 500000.0, yarn[0], yarn[1], neox))
    sync(qh)
    ref = g.rope_yarn(x, nh, hd, pos, 500000.0, yarn[0], yarn[1], bool(neox))
    assert cf.rel_l2(down(dx, nh * hd), ref) < tol


def test_kv_append_and_vec_ops(qh):
    rng = np.random.default_rng(4)
    kvd, ms = 96, 10
    kc, vc = GpuBuf.alloc_f32(ms * kvd), GpuBuf.alloc_f32(ms * kvd)
    check("zero", qh.hip_vec_zero(kc.ptr, ms * kvd))
    check("zero", qh.hip_vec_zero(vc.ptr, ms * kvd))
    k, v = rng.standard_normal(kvd).astype(np.float32), rng.standard_normal(kvd).astype(np.float32)
    dk, dv = up(k), up(v)  # kept alive until the kernels have run
    check("kv_append", qh.hip_kv_append(kc.ptr, vc.ptr, dk.ptr, dv.ptr, 7, kvd))
    a, b = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    da, db = up(a), up(b)
    check("vec_add", qh.hip_vec_add(da.ptr, db.ptr, 1000))
    check("vec_scale_add", qh.hip_vec_scale_add(da.ptr, db.ptr, C.c_float(0.25), 1000))
    sync(qh)
    K = down(kc, ms * kvd).reshape(ms, kvd)
    V = down(vc, ms * kvd).reshape(ms, kvd)
    assert np.array_equal(K[7], k) and np.array_equal(V[7], v)
    assert not K[:7].any() and not K[8:].any()
    assert np.allclose(down(da, 1000), (a + b) + np.float32(0.25) * b, rtol=1e-6, atol=1e-6)  # FMA or not


@pytest.mark.parametrize("seq", [1, 5, 64, 513, 3000])
@pytest.mark.parametrize("sink", [False, True])
def test_attention_three_kernels_and_fused(qh, seq, sink):
    rng = np.random.default_rng(seq + sink)
    nh, nkv, hd, ms = 32, 8, 128, 3072
    kvd = nkv * hd
    q = rng.standard_normal(nh * hd).astype(np.float32)
    kc = rng.standard_normal((ms, kvd)).astype(np.float32)
    vc = rng.standard_normal((ms, kvd)).astype(np.float32)
    sinks = rng.standard_normal(nh).astype(np.float32) if sink else None
    scale = 1.0 / np.sqrt(hd)
    probs, ref = g.attention(q, kc, vc, nh, nkv, seq, hd, kvd, scale, sinks)
    dq, dk, dv = up(q), up(kc), up(vc)
    ds = up(sinks) if sink else None
    dnone = up(np.full(nh, -1e30, np.float32))  # "no sink" for every head, as the reference passes it
    sinks_arg = ds.ptr if sink else dnone.ptr
    sc, o1, o2 = GpuBuf.alloc_f32(nh * ms), GpuBuf.alloc_f32(nh * hd), GpuBuf.alloc_f32(nh * hd)
    check("score", qh.hip_attn_score_all(sc.ptr, dq.ptr, dk.ptr, nh, nkv, seq, hd, kvd, ms, C.c_float(scale)))
    check("softmax", qh.hip_softmax_sink_all(sc.ptr, nh, seq, ms, sinks_arg))
    check("values", qh.hip_attn_values_all(o1.ptr, sc.ptr, dv.ptr, nh, nkv, seq, hd, kvd, ms))
    check("fused", qh.hip_attention_decode(o2.ptr, dq.ptr, dk.ptr, dv.ptr, ds.ptr if sink else None, nh, nkv, seq, hd,
                                           kvd, C.c_float(scale)))
    sync(qh)
    got_p = down(sc, nh * ms).reshape(nh, ms)[:, :seq]
    assert cf.rel_l2(got_p, probs) < 1e-5
    assert cf.rel_l2(down(o1, nh * hd), ref) < 1e-5
    assert cf.rel_l2(down(o2, nh * hd), ref) < 1e-5


def test_single_head_forms(qh):
    rng = np.random.default_rng(9)
    seq, hd, kvd, off = 40, 64, 256, 128
    q = rng.standard_normal(hd).astype(np.float32)
    kc = rng.standard_normal((seq, kvd)).astype(np.float32)
    vc = rng.standard_normal((seq, kvd)).astype(np.float32)
    sc, out = GpuBuf.alloc_f32(seq), GpuBuf.alloc_f32(hd)
    dq, dk, dv = up(q), up(kc), up(vc)
    check("score", qh.hip_attn_score(sc.ptr, dq.ptr, dk.ptr, seq, hd, kvd, off, C.c_float(0.125)))
    check("softmax", qh.hip_softmax_sink(sc.ptr, seq, C.c_float(0.7)))
    check("values", qh.hip_attn_values(out.ptr, sc.ptr, dv.ptr, seq, hd, kvd, off))
    sync(qh)
    p = g.softmax_sink(kc[:, off:off + hd].astype(np.float64) @ q * 0.125, 0.7)
    assert cf.rel_l2(down(sc, seq), p) < 1e-5
    assert cf.rel_l2(down(out, hd), p @ vc[:, off:off + hd]) < 1e-5


@pytest.mark.parametrize("oai", [0, 1])
def test_swiglu(qh, oai):
    rng = np.random.default_rng(oai)
    n = 14336
    gt, u = (rng.standard_normal(n) * 4).astype(np.float32), (rng.standard_normal(n) * 4).astype(np.float32)
    out = GpuBuf.alloc_f32(n)
    fn = qh.hip_swiglu_oai if oai else qh.hip_swiglu
    dg, du = up(gt), up(u)
    check("swiglu", fn(out.ptr, dg.ptr, du.ptr, n))
    sync(qh)
    ref = (g.swiglu_oai if oai else g.swiglu)(gt, u)
    assert cf.rel_l2(down(out, n), ref) < 1e-5


@pytest.mark.parametrize("t", sorted(GGML_TYPES))
def test_embed_lookup_bit_exact(qh, oracle, t):
    qk = GGML_TYPES[t][1]
    vocab, dim = 7, 4096 if qk > 1 else 100
    data = synth.weights(t, vocab, dim, seed=31 + t)
    dd = GpuBuf.upload(data)
    out = GpuBuf.alloc_f32(dim)
    check("embed", qh.hip_embed_lookup(out.ptr, dd.ptr, t, 5, dim))
    sync(qh)
    ref = oracle.dequant(t, data, vocab * dim).reshape(vocab, dim)[5]
    assert np.array_equal(out.download(np.uint32)[:dim], ref.view(np.uint32))


@pytest.mark.parametrize("n", [1, 5, 70])
@pytest.mark.parametrize("t", [12, 14, 8, 21])
def test_embed_lookup_batched_bit_exact(qh, oracle, t, n):
    """hip_embed_lookup_batched_async: n rows (repeats included; 70 takes two
    launches of at most 64) at a row stride past embed_dim, each bit-exact to
    the oracle's dequantised row; the gap between rows is left untouched."""
    qk = GGML_TYPES[t][1]
    vocab, dim, stride = 40, 4096 if qk > 1 else 100, 4096 + 64 if qk > 1 else 128
    data = synth.weights(t, vocab, dim, seed=57 + t)
    dd = GpuBuf.upload(data)
    rng = np.random.default_rng(n + t)
    toks = rng.integers(0, vocab, n).astype(np.int32)
    out = GpuBuf.upload_f32(np.full(n * stride, 7.0, np.float32))
    check("embed_batched", qh.hip_embed_lookup_batched_async(out.ptr, stride, dd.ptr, t, (C.c_int * n)(*toks.tolist()),
                                                             n, dim, None))
    sync(qh)
    ref = oracle.dequant(t, data, vocab * dim).reshape(vocab, dim)
    got = out.download(np.uint32)[:n * stride].reshape(n, stride)
    for i in range(n):
        assert np.array_equal(got[i, :dim], ref[toks[i]].view(np.uint32)), i
        assert np.all(got[i, dim:].view(np.float32) == 7.0), i


@pytest.mark.parametrize("t", [12, 14])
def test_embed_lookup_odd_stride_bit_exact(qh, oracle, t):
    """Rows at an odd float stride (not 16-byte aligned): the 16-values-per-thread
    decode stores them one float at a time, still bit-exact."""
    vocab, dim, stride, n = 9, 1024, 1027, 3
    data = synth.weights(t, vocab, dim, seed=5 + t)
    dd = GpuBuf.upload(data)
    toks = [4, 0, 8]
    out = GpuBuf.upload_f32(np.full(n * stride, 7.0, np.float32))
    check("embed_batched", qh.hip_embed_lookup_batched_async(out.ptr, stride, dd.ptr, t, (C.c_int * n)(*toks), n,
                                                             dim, None))
    sync(qh)
    ref = oracle.dequant(t, data, vocab * dim).reshape(vocab, dim)
    got = out.download(np.uint32)[:n * stride].reshape(n, stride)
    for i in range(n):
        assert np.array_equal(got[i, :dim], ref[toks[i]].view(np.uint32)), i
        assert np.all(got[i, dim:].view(np.float32) == 7.0), i


def test_embed_lookup_batched_rejects(qh):
    """Negative tokens and a row stride below embed_dim are rejected before any
    launch."""
    out = GpuBuf.alloc_f32(2 * 256)
    dd = GpuBuf.upload(synth.weights(12, 4, 256, seed=1))
    assert qh.hip_embed_lookup_batched_async(out.ptr, 256, dd.ptr, 12, (C.c_int * 2)(1, -1), 2, 256, None) != 0
    assert qh.hip_embed_lookup_batched_async(out.ptr, 128, dd.ptr, 12, (C.c_int * 2)(1, 2), 2, 256, None) != 0
    assert qh.hip_embed_lookup_batched_async(out.ptr, 256, dd.ptr, 12, (C.c_int * 2)(1, 2), 0, 256, None) == 0


@pytest.mark.parametrize("heads", [(32, 8), (4, 2), (8, 8), (6, 4), (16, 1), (8, 2, 64), (4, 4, 96)], ids=str)
@pytest.mark.parametrize("pos", [0, 5, 31, 32, 33, 100, 1000, 2047, 5000])
def test_attention_step(qh, heads, pos):
    """hip_attention_step (RoPE q/k + K/V append at pos + attention over pos + 1
    rows, split over 32-row slices and merged by the last workgroup per kv head)
    against the oracle's rope_yarn + kv_append + attention: 1e-5 relative L2 on
    the output (2e-4 at pos >= 1000, the f32 RoPE angle's rounding), the
    appended k row at the same bar and the v row bit-exact; rows before pos are
    left untouched."""
    nh, nkv = heads[:2]
    hd, theta = (heads[2] if len(heads) > 2 else 128), 500000.0  # head_dim below the kernel's 128 too
    kvd = nkv * hd
    neox = pos % 2
    rng = np.random.default_rng(pos * 7 + nh)
    q = rng.standard_normal(nh * hd).astype(np.float32)
    k = rng.standard_normal(kvd).astype(np.float32)
    v = rng.standard_normal(kvd).astype(np.float32)
    max_seq = pos + 3
    kc = rng.standard_normal((max_seq, kvd)).astype(np.float32)
    vc = rng.standard_normal((max_seq, kvd)).astype(np.float32)
    sinks = rng.standard_normal(nh).astype(np.float32) if pos % 3 == 0 else None
    dq, dk, dv, dkc, dvc, do = up(q), up(k), up(v), up(kc), up(vc), GpuBuf.alloc_f32(nh * hd)
    ds = up(sinks) if sinks is not None else None
    scale = 1.0 / np.sqrt(hd)
    check("attention_step", qh.hip_attention_step_async(do.ptr, dq.ptr, dk.ptr, dv.ptr, dkc.ptr, dvc.ptr,
                                                        ds.ptr if ds else None, nh, nkv, hd, kvd, pos, theta, 1.0, 0,
                                                        neox, scale, None))
    sync(qh)
    qr = g.rope_yarn(q, nh, hd, pos, theta, neox=bool(neox))
    kr = g.rope_yarn(k, nkv, hd, pos, theta, neox=bool(neox))
    kc64, vc64 = kc.astype(np.float64), vc.astype(np.float64)
    kc64[pos], vc64[pos] = kr, v
    _, ref = g.attention(qr, kc64, vc64, nh, nkv, pos + 1, hd, kvd, scale, sinks)
    tol = 1e-5 if pos < 1000 else 2e-4
    assert cf.rel_l2(down(do, nh * hd), ref) < tol
    kc_got = dkc.download(np.float32).reshape(max_seq, kvd)
    vc_got = dvc.download(np.float32).reshape(max_seq, kvd)
    assert cf.rel_l2(kc_got[pos], kr) < tol
    assert np.array_equal(vc_got[pos], v)
    assert np.array_equal(kc_got[:pos], kc[:pos]) and np.array_equal(vc_got[:pos], vc[:pos])
    assert np.array_equal(kc_got[pos + 1:], kc[pos + 1:])


def test_attention_step_repeat(qh):
    """Two launches in a row (the per-kv-head arrival counters are back at zero
    after each) give the same output."""
    nh, nkv, hd, pos = 8, 2, 128, 700
    rng = np.random.default_rng(3)
    bufs = [up(rng.standard_normal(n).astype(np.float32)) for n in (nh * hd, nkv * hd, nkv * hd)]
    kc, vc = up(rng.standard_normal((pos + 1) * nkv * hd)), up(rng.standard_normal((pos + 1) * nkv * hd))
    outs = []
    for _ in range(2):
        o = GpuBuf.alloc_f32(nh * hd)
        check("attention_step", qh.hip_attention_step_async(o.ptr, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, kc.ptr,
                                                            vc.ptr, None, nh, nkv, hd, nkv * hd, pos, 10000.0, 1.0, 0,
                                                            0, 0.088, None))
        sync(qh)
        outs.append(down(o, nh * hd))
    assert np.array_equal(outs[0], outs[1])


@pytest.mark.parametrize("n_seq, pos", [(1, 40), (4, 0), (4, 77), (16, 300), (32, 511), (3, 2100)])
def test_attention_step_batched(qh, n_seq, pos):
    """hip_attention_step_batched: each sequence against its own single-sequence
    oracle (own q/k/v rows and own cache), 1e-5 relative L2 (2e-4 past 1000
    cached rows, as the single-sequence test: the output is a near-cancelling
    f32 sum over that many value rows)."""
    nh, nkv, hd = 8, 2, 128
    kvd = nkv * hd
    max_seq = pos + 2
    rng = np.random.default_rng(n_seq * 1000 + pos)
    q = rng.standard_normal((n_seq, nh * hd)).astype(np.float32)
    k = rng.standard_normal((n_seq, kvd)).astype(np.float32)
    v = rng.standard_normal((n_seq, kvd)).astype(np.float32)
    kc = rng.standard_normal((n_seq, max_seq, kvd)).astype(np.float32)
    vc = rng.standard_normal((n_seq, max_seq, kvd)).astype(np.float32)
    dq, dk, dv, dkc, dvc = up(q), up(k), up(v), up(kc), up(vc)
    do = GpuBuf.alloc_f32(n_seq * nh * hd)
    check("batched", qh.hip_attention_step_batched_async(do.ptr, dq.ptr, dk.ptr, dv.ptr, dkc.ptr, dvc.ptr, None,
                                                         n_seq, max_seq * kvd, nh, nkv, hd, kvd, pos, 10000.0, 1.0,
                                                         0, 0, 0.09, None))
    sync(qh)
    got = down(do, n_seq * nh * hd).reshape(n_seq, nh * hd)
    for z in range(n_seq):
        qr = g.rope_yarn(q[z], nh, hd, pos, 10000.0)
        kr = g.rope_yarn(k[z], nkv, hd, pos, 10000.0)
        kc64, vc64 = kc[z].astype(np.float64), vc[z].astype(np.float64)
        kc64[pos], vc64[pos] = kr, v[z]
        _, ref = g.attention(qr, kc64, vc64, nh, nkv, pos + 1, hd, kvd, 0.09)
        assert cf.rel_l2(got[z], ref) < (1e-5 if pos < 1000 else 2e-4), z


def test_rms_norm_rows(qh):
    rng = np.random.default_rng(5)
    x, w = rng.standard_normal((7, 4096)) * 2, rng.standard_normal(4096)
    dx, dw, do = up(x), up(w), GpuBuf.alloc_f32(7 * 4096)
    check("rows", qh.hip_rms_norm_rows_async(do.ptr, dx.ptr, dw.ptr, 7, 4096, None))
    sync(qh)
    got = down(do, 7 * 4096).reshape(7, 4096)
    for r in range(7):
        assert cf.rel_l2(got[r], g.rms_norm(x[r].astype(np.float32), w.astype(np.float32))) < 1e-5
