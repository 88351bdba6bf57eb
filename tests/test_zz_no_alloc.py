"""hip_gemm_grouped_norm_static_async, the entry point that allocates nothing
(the normalised rows in the library's static device array), against
hip_gemm_grouped_norm_async with a caller workspace: bit-identical outputs on
two calls in a row, the second with fewer tokens and a shorter in_dim (the
static array keeps the first call's contents), and the size limit."""
import ctypes as C

import numpy as np
import pytest

from saient_quartz_amd import synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf

pytestmark = pytest.mark.gpu

QH_ERR_RANGE = -5


def _call(qh, fn, t, dws, dx, dn, dys, n, outs, in_dim, scratch=None):
    k = len(dws)
    args = [t, k, (C.c_void_p * k)(*[b.ptr for b in dws]), dx.ptr, dn.ptr, (C.c_void_p * k)(*[b.ptr for b in dys]), n,
            (C.c_int * k)(*outs), in_dim]
    if fn == "hip_gemm_grouped_norm_async":
        args.append(scratch.ptr)
    args.append(None)
    return getattr(qh, fn)(*args)


@pytest.mark.parametrize("t", [12, 14, 8])
def test_static_norm_gemm_matches_workspace_form(qh, t):
    rng = np.random.default_rng(t)
    for n, in_dim, outs in ((12, 4096, (300, 77)), (6, 2048, (64, 200))):
        print(f"type {t} n {n} in_dim {in_dim}", flush=True)
        x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.5, 4, (n, 1))).astype(np.float32)
        w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
        dws = [GpuBuf.upload(synth.weights(t, o, in_dim, seed=o + t)) for o in outs]
        dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
        ya = [GpuBuf.alloc_f32(n * o) for o in outs]
        yb = [GpuBuf.alloc_f32(n * o) for o in outs]
        scratch = GpuBuf.alloc_f32(n * in_dim)
        check("static", _call(qh, "hip_gemm_grouped_norm_static_async", t, dws, dx, dn, ya, n, outs, in_dim))
        check("workspace", _call(qh, "hip_gemm_grouped_norm_async", t, dws, dx, dn, yb, n, outs, in_dim, scratch))
        check("hip_sync", qh.hip_sync())
        for a, b, o in zip(ya, yb, outs):
            ga, gb = a.download(np.float32), b.download(np.float32)
            assert np.all(np.isfinite(ga))
            assert np.array_equal(ga.view(np.uint32), gb.view(np.uint32)), (n, o)


def test_static_norm_gemm_rejects_oversize(qh):
    n, in_dim = 65, 16384  # 1064960 floats > the 1048576-float array
    dw = GpuBuf.alloc(16)
    dx, dn, dy = GpuBuf.alloc_f32(1), GpuBuf.alloc_f32(1), GpuBuf.alloc_f32(1)
    rc = _call(qh, "hip_gemm_grouped_norm_static_async", 12, [dw], dx, dn, [dy], n, [1], in_dim)
    assert rc == QH_ERR_RANGE
    assert b"static scratch" in qh.hip_last_error()
