"""GPU parity of the grouped batched entry points (hip_gemm_grouped, hip_gemm_moe)
against the CPU oracle's gemm (src/dequant.rs:143-200), per matrix and token.

Bar: 1e-3 relative L2 per token row, as for hip_gemm.
"""
import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES, synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf, gemm_grouped_async, gemm_moe_async

pytestmark = pytest.mark.gpu

TOL = 1e-3


def _nbytes(t, out_dim, in_dim):
    _, qk, bs = GGML_TYPES[t]
    return out_dim * in_dim // qk * bs


def _check_rows(got, ref, what):
    for k in range(ref.shape[0]):
        e = cf.rel_l2(got[k], ref[k])
        assert e < TOL, (what, k, e)


def _run_grouped(qh, oracle, t, in_dim, mats):
    """mats: list of (out_dim, n, x_key); matrices with the same x_key share one
    device x buffer (and so one digitisation).  Returns (got, ref) lists."""
    xs, dxs = {}, {}
    for out_dim, n, key in mats:
        if key not in xs:
            nmax = max(m[1] for m in mats if m[2] == key)
            xs[key] = synth.activations(max(nmax, 1), in_dim, seed=11 + 7 * key)
            xs[key] *= (10.0 ** np.linspace(-2, 2, xs[key].shape[0], dtype=np.float32))[:, None].astype(np.float32)
            dxs[key] = GpuBuf.upload_f32(xs[key].reshape(-1))
    ws, dws, dys = [], [], []
    for i, (out_dim, n, key) in enumerate(mats):
        w = synth.weights(t, out_dim, in_dim, seed=500 + 13 * i + t)
        ws.append(w)
        dws.append(GpuBuf.upload(w))
        dys.append(GpuBuf.alloc_f32(max(n * out_dim, 1)))
    gemm_grouped_async(qh, t, [d.ptr for d in dws], [dxs[m[2]].ptr for m in mats], [d.ptr for d in dys],
                       [m[1] for m in mats], [m[0] for m in mats], in_dim, None)
    check("hip_sync", qh.hip_sync())
    out = []
    for i, (out_dim, n, key) in enumerate(mats):
        if n == 0 or out_dim == 0:
            continue
        got = dys[i].download(np.float32)[:n * out_dim].reshape(n, out_dim)
        ref = oracle.gemm(t, xs[key][:n], ws[i], in_dim, out_dim, n)
        out.append((i, got, ref))
    return out


@pytest.mark.parametrize("t", [12, 13, 14, 21, 16])
def test_grouped_mixed_shapes(qh, oracle, t):
    """Different row counts and token counts in one call, two matrices sharing x,
    an empty matrix, a single-token matrix and one past 16 tokens."""
    mats = [(40, 3, 0), (300, 16, 1), (64, 16, 1), (0, 5, 2), (33, 1, 3), (130, 7, 4), (17, 20, 5)]
    for i, got, ref in _run_grouped(qh, oracle, t, 4096, mats):
        _check_rows(got, ref, (t, i))


@pytest.mark.parametrize("t", [12, 21])
def test_grouped_more_than_one_launch(qh, oracle, t):
    """20 matrices (more than one launch holds) with 12 distinct x blocks."""
    mats = [(24 + 8 * (i % 5), 2 + i % 15, i % 12) for i in range(20)]
    for i, got, ref in _run_grouped(qh, oracle, t, 1024, mats):
        _check_rows(got, ref, (t, i))


def test_grouped_scratch_slots_limit(qh, oracle):
    """in_dim 65536: only a few x images fit the scratch at once, so the call
    goes out in several launches."""
    mats = [(8, 2 + i, i) for i in range(6)]
    for i, got, ref in _run_grouped(qh, oracle, 12, 65536, mats):
        _check_rows(got, ref, i)


@pytest.mark.parametrize("t", [8, 2, 17])
def test_grouped_types_without_batched_kernel(qh, oracle, t):
    """Types with no matrix-core batched kernel go matrix by matrix."""
    mats = [(40, 3, 0), (24, 5, 0), (9, 1, 1)]
    for i, got, ref in _run_grouped(qh, oracle, t, 1024, mats):
        _check_rows(got, ref, (t, i))


def test_grouped_single_matches_gemm_bitwise(qh):
    """One matrix through hip_gemm_grouped is hip_gemm: the same launches."""
    t, out_dim, in_dim, n = 12, 200, 4096, 9
    w = synth.weights(t, out_dim, in_dim, seed=77)
    x = synth.activations(n, in_dim, seed=78)
    dw, dx = GpuBuf.upload(w), GpuBuf.upload_f32(x.reshape(-1))
    y1, y2 = GpuBuf.alloc_f32(n * out_dim), GpuBuf.alloc_f32(n * out_dim)
    check("hip_gemm", qh.hip_gemm(t, dw.ptr, dx.ptr, y1.ptr, in_dim, out_dim, n))
    gemm_grouped_async(qh, t, [dw.ptr], [dx.ptr], [y2.ptr], [n], [out_dim], in_dim, None)
    check("hip_sync", qh.hip_sync())
    assert np.array_equal(y1.download(np.uint32), y2.download(np.uint32))


@pytest.mark.parametrize("t", [21, 16, 12])
def test_gemm_moe(qh, oracle, t):
    """Stacked experts (base + e * type_size, src/cuda.rs:250-258), gathered
    tokens per selected expert, including an expert chosen twice, one with no
    tokens, one with a single token and one past 16."""
    n_exp, in_dim, out_dim = 8, 1024, 96
    per = _nbytes(t, out_dim, in_dim)
    experts = [synth.weights(t, out_dim, in_dim, seed=60 + e) for e in range(n_exp)]
    base = GpuBuf.upload(np.concatenate(experts))
    ids = [3, 0, 7, 3, 5, 1]
    counts = [4, 16, 0, 1, 18, 6]
    off = np.concatenate([[0], np.cumsum(counts)]).astype(int).tolist()
    x = synth.activations(off[-1], in_dim, seed=61)
    dx = GpuBuf.upload_f32(x.reshape(-1))
    dy = GpuBuf.alloc_f32(off[-1] * out_dim)
    gemm_moe_async(qh, t, base.ptr, ids, off, dx.ptr, dy.ptr, in_dim, out_dim, None)
    check("hip_sync", qh.hip_sync())
    y = dy.download(np.float32).reshape(off[-1], out_dim)
    for i, e in enumerate(ids):
        a, b = off[i], off[i + 1]
        if a == b:
            continue
        ref = oracle.gemm(t, x[a:b], experts[e], in_dim, out_dim, b - a)
        _check_rows(y[a:b], ref, (t, i, e))
    assert per == len(experts[0])

