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


@pytest.mark.parametrize("t", [12, 13, 14, 8])
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
    """Q8_0 has no fused kernel: without scratch the call reports QH_ERR_NULL (-3)
    instead of writing anywhere; Q4_K at in_dim 4096 needs none."""
    x = GpuBuf.upload_f32(np.ones(4096, np.float32))
    n = GpuBuf.upload_f32(np.ones(4096, np.float32))
    y = GpuBuf.alloc_f32(64)
    import ctypes as C
    for t, want in ((8, -3), (12, 0)):
        w = GpuBuf.upload(synth.weights(t, 64, 4096, seed=1))
        rc = qh.hip_gemv_fused_async(t, 1, (C.c_void_p * 1)(w.ptr), (C.c_void_p * 1)(y.ptr), (C.c_int * 1)(64),
                                     x.ptr, n.ptr, 0, 4096, None, None)
        assert rc == want
    check("hip_sync", qh.hip_sync())
