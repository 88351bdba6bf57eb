"""hip_gemv_fused: GEMVs with the RMS norm before them and/or the residual add
after them fused in, against the oracle's GEMV of the float64-normed x (1e-3
relative L2, the GEMV bar), for the fused matrix-core types and for types and
shapes that take the separate-kernel fallback through the scratch buffer."""
import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf, gemv_fused_async

pytestmark = pytest.mark.gpu


def rms(x, w):
    x = x.astype(np.float64)
    return x / np.sqrt(np.mean(x * x) + 1e-5) * w.astype(np.float64)


@pytest.mark.parametrize("t", [12, 13, 14, 8, 6])
@pytest.mark.parametrize("dims, in_dim", [((4096, 1024), 4096), ((300,), 512), ((37, 1000, 5), 1024),
                                          ((700,), 4352), ((4096,), 14336)], ids=str)
@pytest.mark.parametrize("norm, acc", [(True, False), (False, True), (True, True)])
def test_gemv_fused(qh, oracle, t, dims, in_dim, norm, acc):
    rng = np.random.default_rng(in_dim + len(dims) + t)
    x = (rng.standard_normal(in_dim) * 2.5).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=30 + k) for k, o in enumerate(dims)]
    y0 = [rng.standard_normal(o).astype(np.float32) for o in dims]
    ws = [GpuBuf.upload(d) for d in datas]
    ys = [GpuBuf.upload_f32(a) for a in y0]
    dx, dn = GpuBuf.upload_f32(x), GpuBuf.upload_f32(nw)
    scratch = GpuBuf.alloc_f32(in_dim + max(dims))
    gemv_fused_async(qh, t, [w.ptr for w in ws], [y.ptr for y in ys], list(dims), dx.ptr, in_dim, None,
                     norm_ptr=dn.ptr if norm else None, accumulate=acc, scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    xin = rms(x, nw) if norm else x.astype(np.float64)
    for k, o in enumerate(dims):
        w = oracle.dequant(t, datas[k], o * in_dim).astype(np.float64).reshape(o, in_dim)
        ref = w @ xin + (y0[k] if acc else 0.0)
        got = ys[k].download(np.float32)[:o]
        assert np.all(np.isfinite(got))
        assert cf.rel_l2(got, ref) < 1e-3, (k, cf.rel_l2(got, ref))


def test_gemv_fused_needs_scratch_only_on_fallback(qh):
    """Q2_K and Q5_0 have no fused kernel: without scratch the call reports
    QH_ERR_NULL (-3) instead of writing anywhere; Q4_K, Q8_0 and Q5_1 at in_dim
    4096 need none."""
    x = GpuBuf.upload_f32(np.ones(4096, np.float32))
    n = GpuBuf.upload_f32(np.ones(4096, np.float32))
    y = GpuBuf.alloc_f32(64)
    import ctypes as C
    for t, want in ((10, -3), (6, -3), (12, 0), (8, 0), (7, 0)):
        w = GpuBuf.upload(synth.weights(t, 64, 4096, seed=1))
        rc = qh.hip_gemv_fused_async(t, 1, (C.c_void_p * 1)(w.ptr), (C.c_void_p * 1)(y.ptr), (C.c_int * 1)(64),
                                     x.ptr, n.ptr, 0, 4096, None, None)
        assert rc == want
    check("hip_sync", qh.hip_sync())


def silu(g):
    return g / (1.0 + np.exp(-g))


@pytest.mark.parametrize("t", [12, 13, 14, 8])
@pytest.mark.parametrize("ffn, in_dim", [(1024, 512), (14336, 4096), (999, 1024), (40000, 512), (300, 4352)],
                         ids=str)
@pytest.mark.parametrize("norm", [True, False])
def test_gemv_swiglu(qh, oracle, t, ffn, in_dim, norm):
    """hip_gemv_swiglu: silu(W_gate x') * (W_up x') in one launch (gate and up
    tiles paired per workgroup; 40000 rows exercises many pairs per workgroup)
    or through the separate kernels (Q8_0, in_dim past one workgroup's chunk)."""
    if ffn * in_dim > 14336 * 4096 and t != 12:
        pytest.skip("large shape only for Q4_K")
    from test_gpu_decode_step import realistic_scale
    rng = np.random.default_rng(ffn + in_dim + t)
    x = (rng.standard_normal(in_dim) * 1.5).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(in_dim)).astype(np.float32)
    wg, wu = synth.weights(t, ffn, in_dim, seed=11), synth.weights(t, ffn, in_dim, seed=12)
    if t in (12, 13, 14):
        # the K-quant blocks' O(1) weights give gate values in the thousands, where
        # silu is linear or zero and the oracle's exp overflows: a checkpoint's
        # weight size (scales / 64) keeps |gate| below 40
        wg, wu = realistic_scale(wg, t), realistic_scale(wu, t)
    dg, du = GpuBuf.upload(wg), GpuBuf.upload(wu)
    dx, dn, act = GpuBuf.upload_f32(x), GpuBuf.upload_f32(nw), GpuBuf.alloc_f32(ffn)
    scratch = GpuBuf.alloc_f32(in_dim + 2 * ffn)
    check("hip_gemv_swiglu_async", qh.hip_gemv_swiglu_async(t, dg.ptr, du.ptr, act.ptr, ffn, dx.ptr,
                                                            dn.ptr if norm else None, in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xin = rms(x, nw) if norm else x.astype(np.float64)
    g = oracle.dequant(t, wg, ffn * in_dim).astype(np.float64).reshape(ffn, in_dim) @ xin
    u = oracle.dequant(t, wu, ffn * in_dim).astype(np.float64).reshape(ffn, in_dim) @ xin
    ref = silu(g) * u
    got = act.download(np.float32)[:ffn]
    assert np.all(np.isfinite(got))
    assert cf.rel_l2(got, ref) < 1e-3, cf.rel_l2(got, ref)


@pytest.mark.parametrize("types, dims", [((12, 12, 14), (4096, 1024, 1024)), ((14, 12), (300, 700)),
                                         ((13, 14), (1000, 37)), ((12, 13), (64, 4096)), ((12, 8), (500, 500)),
                                         ((12, 14, 13), (100, 200, 300))], ids=str)
@pytest.mark.parametrize("in_dim", [4096, 1024, 14336])
@pytest.mark.parametrize("norm, acc", [(True, False), (False, True), (False, False)])
def test_gemv_group(qh, oracle, types, dims, in_dim, norm, acc):
    """hip_gemv_group: per-matrix types sharing x; two matrix-core types run as
    one split launch, other mixes per type.  Each y against the oracle."""
    from saient_quartz_amd.host import gemv_group_async
    if norm and in_dim > 4096:
        pytest.skip("covered by the fused tests")
    rng = np.random.default_rng(in_dim + sum(dims))
    x = (rng.standard_normal(in_dim) * 2).astype(np.float32)
    nw = (1 + 0.2 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=70 + k) for k, (t, o) in enumerate(zip(types, dims))]
    y0 = [rng.standard_normal(o).astype(np.float32) for o in dims]
    ws = [GpuBuf.upload(d) for d in datas]
    ys = [GpuBuf.upload_f32(a) for a in y0]
    dx, dn = GpuBuf.upload_f32(x), GpuBuf.upload_f32(nw)
    scratch = GpuBuf.alloc_f32(in_dim + max(dims))
    gemv_group_async(qh, list(types), [w.ptr for w in ws], [y.ptr for y in ys], list(dims), dx.ptr, in_dim, None,
                     norm_ptr=dn.ptr if norm else None, accumulate=acc, scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    xin = rms(x, nw) if norm else x.astype(np.float64)
    for k, (t, o) in enumerate(zip(types, dims)):
        w = oracle.dequant(t, datas[k], o * in_dim).astype(np.float64).reshape(o, in_dim)
        ref = w @ xin + (y0[k] if acc else 0.0)
        got = ys[k].download(np.float32)[:o]
        assert cf.rel_l2(got, ref) < 1e-3, (k, t, cf.rel_l2(got, ref))


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("out_dim, in_dim", [(14336, 4096), (40000, 1024), (4097, 14336)], ids=str)
def test_residual_gemv_many_tiles(qh, oracle, t, out_dim, in_dim):
    """y += W x with several row tiles per workgroup: a workgroup's first tile
    takes the y values its threads loaded at the start, the later tiles read y
    at the end; every row against the oracle."""
    rng = np.random.default_rng(out_dim + t)
    x = rng.standard_normal(in_dim).astype(np.float32)
    data = synth.weights(t, out_dim, in_dim, seed=44 + t)
    y0 = (10 * rng.standard_normal(out_dim)).astype(np.float32)
    w, y, dx = GpuBuf.upload(data), GpuBuf.upload_f32(y0), GpuBuf.upload_f32(x)
    scratch = GpuBuf.alloc_f32(in_dim + out_dim)
    gemv_fused_async(qh, t, [w.ptr], [y.ptr], [out_dim], dx.ptr, in_dim, None, norm_ptr=None, accumulate=True,
                     scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    ref = oracle.gemv(t, x, data, in_dim, out_dim).astype(np.float64) + y0
    got = y.download(np.float32)[:out_dim]
    assert cf.rel_l2(got, ref) < 1e-3, cf.rel_l2(got, ref)
    # row by row: a lost or doubled residual shows as an error of |y0| on its row
    assert np.max(np.abs(got - ref)) < 1e-2 * np.max(np.abs(ref))
