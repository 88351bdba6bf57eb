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
