"""GPU parity: the HIP library (through its C ABI) against the CPU oracle.

Bars: dequant bit-exact; GEMV/GEMM within 1e-3 relative L2 of the oracle
(f32 accumulate; observed ~1e-6); --verify-gemv criterion
max|cpu-gpu| / max|cpu| < 1e-3 (src/main.rs:2653-2662).
"""
import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES, synth
from saient_quartz_amd.host import GpuBuf, GpuScratch, gpu_expert_slice, verify_gemv_hip
from saient_quartz_amd.api import check

pytestmark = pytest.mark.gpu

TOL = 1e-3
ALL_TYPES = sorted(GGML_TYPES)


def gpu_gemv(qh, t, x, data, in_dim, out_dim):
    return verify_gemv_hip(x, data, t, in_dim, out_dim)


def gpu_gemm(qh, t, x, data, in_dim, out_dim, n):
    w = GpuBuf.upload(data)
    dx = GpuBuf.upload_f32(x.reshape(-1))
    dy = GpuBuf.alloc_f32(n * out_dim)
    check("hip_gemm", qh.hip_gemm(t, w.ptr, dx.ptr, dy.ptr, in_dim, out_dim, n))
    return dy.download(np.float32).reshape(n, out_dim)


@pytest.mark.parametrize("t", ALL_TYPES)
def test_dequant_bit_exact(qh, oracle, t):
    _, qk, _ = GGML_TYPES[t]
    out_dim, in_dim = 37, 1024
    data = synth.weights(t, out_dim, in_dim, seed=100 + t)
    n = out_dim * in_dim
    w = GpuBuf.upload(data)
    out = GpuBuf.alloc_f32(n)
    check("hip_dequant", qh.hip_dequant(t, w.ptr, out.ptr, n))
    got = out.download(np.float32)
    ref = oracle.dequant(t, data, n)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


def test_dequant_f16_all_patterns(qh, oracle):
    bits = np.arange(65536, dtype=np.uint16).view(np.uint8)
    w = GpuBuf.upload(bits)
    out = GpuBuf.alloc_f32(65536)
    check("hip_dequant", qh.hip_dequant(1, w.ptr, out.ptr, 65536))
    assert np.array_equal(out.download(np.uint32), oracle.dequant(1, bits, 65536).view(np.uint32))


# (21, 768) and (9, 3840): an odd number of 256-weight groups, so with 2-byte
# aligned blocks (Q6_K: 210 bytes) both rows and groups alternate their 4-byte
# alignment within one K chunk
SHAPES = [(64, 4096), (37, 4096), (5, 256), (130, 512), (21, 768), (9, 3840), (19, 14336), (3, 8192), (2, 12288),
          (1, 28672)]


@pytest.mark.parametrize("t", ALL_TYPES)
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_vs_oracle(qh, oracle, t, shape):
    out_dim, in_dim = shape
    data = synth.weights(t, out_dim, in_dim, seed=7 * t + in_dim)
    x = synth.activations(1, in_dim, seed=11 + in_dim)[0]
    got = gpu_gemv(qh, t, x, data, in_dim, out_dim)
    ref = oracle.gemv(t, x, data, in_dim, out_dim)
    bad = np.nonzero(~np.isclose(got, ref, rtol=1e-3, atol=1e-3 * np.abs(ref).max()))[0]
    assert cf.rel_l2(got, ref) < TOL, (t, shape, cf.rel_l2(got, ref), bad[:16])


@pytest.mark.parametrize("t", [2, 3, 6, 7, 8, 20, 0, 1, 30])
@pytest.mark.parametrize("in_dim", [32, 96, 4064])
def test_gemv_fallback_shapes(qh, oracle, t, in_dim):
    """in_dim % 64 != 0 takes the generic kernel (32-element formats, floats)."""
    out_dim = 9
    data = synth.weights(t, out_dim, in_dim, seed=5 + in_dim)
    x = synth.activations(1, in_dim, seed=6)[0]
    got = gpu_gemv(qh, t, x, data, in_dim, out_dim)
    assert cf.rel_l2(got, oracle.gemv(t, x, data, in_dim, out_dim)) < TOL


# Shapes that give the persistent matrix-core kernel several row tiles per
# workgroup (14336 rows), the tiles-per-workgroup cap (200000 rows), a partial
# last tile, multi-chunk K (14336) and the 16-row tiles chosen for 4096 rows.
BIG_SHAPES = [(14336, 4096), (4101, 14336), (200003, 256), (4096, 4096), (4096, 14336)]


@pytest.mark.parametrize("t", [12, 13, 14])
@pytest.mark.parametrize("shape", BIG_SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_gemv_many_tiles(qh, oracle, t, shape):
    out_dim, in_dim = shape
    data = synth.weights(t, out_dim, in_dim, seed=31 * t + out_dim)
    x = synth.activations(1, in_dim, seed=5 + in_dim)[0]
    got = gpu_gemv(qh, t, x, data, in_dim, out_dim)
    ref = oracle.gemv(t, x, data, in_dim, out_dim)
    assert cf.rel_l2(got, ref) < TOL, (t, shape, cf.rel_l2(got, ref))
    # every row is written (no stale rows from a missed tile)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - ref)) <= 1e-3 * np.max(np.abs(ref)) + 1e-6


@pytest.mark.parametrize("t", [12, 13, 14, 8, 21])
@pytest.mark.parametrize("dims", [(4096, 1024), (14336, 14336), (37, 300, 5, 1000)], ids=str)
def test_gemv_multi_matches_single(qh, t, dims):
    """hip_gemv_multi (one launch for up to 4 matrices sharing x) gives each
    matrix exactly the hip_gemv result (same kernel arithmetic; types without a
    fused kernel fall back to one launch per matrix)."""
    from saient_quartz_amd.host import gemv_multi_async
    in_dim = 4096
    datas = [synth.weights(t, o, in_dim, seed=50 + k) for k, o in enumerate(dims)]
    x = synth.activations(1, in_dim, seed=9)[0]
    ws = [GpuBuf.upload(d) for d in datas]
    dx = GpuBuf.upload_f32(x)
    ys = [GpuBuf.alloc_f32(o) for o in dims]
    gemv_multi_async(qh, t, [w.ptr for w in ws], [y.ptr for y in ys], list(dims), dx.ptr, in_dim, None)
    check("hip_sync", qh.hip_sync())
    for k, o in enumerate(dims):
        single = GpuBuf.alloc_f32(o)
        check("hip_gemv", qh.hip_gemv(t, ws[k].ptr, dx.ptr, single.ptr, in_dim, o))
        assert np.array_equal(ys[k].download(np.float32).view(np.uint32), single.download(np.float32).view(np.uint32))


def test_gemv_launch_variant_8x2(qh):
    """The tuning override QUARTZ_HIP_MMV16=2 (8 waves x 2 groups) selects a
    launch shape the defaults do not use; it must give the same results.  Runs in
    a child process because the override is read once per process."""
    import os
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    code = (
        "import sys, numpy as np; sys.path.insert(0, %r); sys.path.insert(0, %r)\n"
        "from saient_quartz_amd import synth\n"
        "from saient_quartz_amd.host import verify_gemv_hip\n"
        "from oracle_lib import Oracle\n"
        "import closed_form as cf\n"
        "o = Oracle.load()\n"
        "for t, (od, idim) in [(12, (3000, 4096)), (14, (2000, 14336)), (13, (1000, 2048))]:\n"
        "    d = synth.weights(t, od, idim, seed=t); x = synth.activations(1, idim, seed=2)[0]\n"
        "    e = cf.rel_l2(verify_gemv_hip(x, d, t, idim, od), o.gemv(t, x, d, idim, od))\n"
        "    assert e < 1e-3, (t, e)\n"
        "print('ok')\n" % (str(root), str(root / "tests")))
    env = dict(os.environ, QUARTZ_HIP_MMV16="2")
    r = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, timeout=110)
    assert r.returncode == 0 and "ok" in r.stdout, r.stdout + r.stderr


@pytest.mark.parametrize("t", ALL_TYPES)
def test_verify_gemv_criterion(qh, oracle, t):
    """Quartz's --verify-gemv check with its deterministic x (src/main.rs:2640-2662)."""
    out_dim, in_dim = 96, 4096
    data = synth.weights(t, out_dim, in_dim, seed=300 + t)
    x = synth.verify_x(in_dim)
    cpu = oracle.gemv(t, x, data, in_dim, out_dim)
    gpu = gpu_gemv(qh, t, x, data, in_dim, out_dim)
    maxdiff = float(np.max(np.abs(cpu - gpu)))
    maxmag = max(float(np.max(np.abs(cpu))), 1e-6)
    assert maxdiff / maxmag < 1e-3


@pytest.mark.parametrize("t", ALL_TYPES)
@pytest.mark.parametrize("n", [2, 4, 16])
def test_gemm_vs_oracle(qh, oracle, t, n):
    out_dim, in_dim = 40, 4096 if GGML_TYPES[t][1] > 1 else 1024
    data = synth.weights(t, out_dim, in_dim, seed=900 + t)
    x = synth.activations(n, in_dim, seed=901 + n)
    got = gpu_gemm(qh, t, x, data, in_dim, out_dim, n)
    ref = oracle.gemm(t, x, data, in_dim, out_dim, n)
    assert cf.rel_l2(got, ref) < TOL


# The matrix-core batched path (Q4_K, Q5_K, Q6_K, IQ3_S, IQ2_XXS): token counts that use each
# token-tile size (2, 4, 8, 16) and the chunking past 16; shapes with several K
# chunks, a partial last row tile and more tiles than one workgroup keeps.
# The last two reach the kernel's other x-image modes: 40000 x 1024 (157 row
# blocks sharing x, one split of 4 groups: images from the prologue launch,
# resident) and 9000 x 16384 (7 splits of 9-10 groups: images streamed).
MMQ_CASES = [(40, 4096, 2), (40, 4096, 3), (77, 4096, 5), (300, 14336, 8), (100, 4096, 11), (130, 2048, 16),
             (64, 4096, 17), (33, 1024, 33), (9000, 256, 16), (4100, 512, 4), (40000, 1024, 16), (9000, 16384, 16),
             (300, 4096, 24), (9000, 1024, 32), (130, 2048, 40), (64, 14336, 20)]


@pytest.mark.parametrize("t", [12, 13, 14, 21, 16])
@pytest.mark.parametrize("case", MMQ_CASES, ids=lambda c: f"{c[0]}x{c[1]}n{c[2]}")
def test_gemm_matrix_core(qh, oracle, t, case):
    out_dim, in_dim, n = case
    data = synth.weights(t, out_dim, in_dim, seed=17 * t + out_dim + n)
    x = synth.activations(n, in_dim, seed=3 + n + in_dim)
    # tokens of very different magnitudes: each has its own digit exponent
    x = x * (10.0 ** np.linspace(-3, 3, n, dtype=np.float32))[:, None].astype(np.float32)
    got = gpu_gemm(qh, t, x, data, in_dim, out_dim, n)
    ref = oracle.gemm(t, x, data, in_dim, out_dim, n)
    for k in range(n):
        assert cf.rel_l2(got[k], ref[k]) < TOL, (t, case, k, cf.rel_l2(got[k], ref[k]))


def test_expert_slices_and_moe4(qh, oracle):
    """Stacked experts addressed as base + e * type_size (src/cuda.rs:250-258)."""
    t, in_dim, out_dim, n_exp = 21, 1024, 64, 4
    per = out_dim * in_dim
    data = np.concatenate([synth.weights(t, out_dim, in_dim, seed=40 + e) for e in range(n_exp)])
    buf = GpuBuf.upload(data)
    xs = synth.activations(n_exp, in_dim, seed=41)
    sc = GpuScratch(in_dim, out_dim)
    nbytes = per * GGML_TYPES[t][2] // GGML_TYPES[t][1]
    for e in range(n_exp):
        sl = gpu_expert_slice(buf, t, e, per)
        got = sc.gemv_slice(xs[e], sl, in_dim, out_dim)
        ref = oracle.gemv(t, xs[e], data[e * nbytes:(e + 1) * nbytes], in_dim, out_dim)
        assert cf.rel_l2(got, ref) < TOL
    dx = [GpuBuf.upload_f32(xs[e]) for e in range(n_exp)]
    dy = [GpuBuf.alloc_f32(out_dim) for _ in range(n_exp)]
    ws = [gpu_expert_slice(buf, t, e, per).ptr for e in range(n_exp)]
    check("hip_gemv_moe4", qh.hip_gemv_moe4(t, *ws, *[b.ptr for b in dx], *[b.ptr for b in dy], 3, in_dim, out_dim))
    check("hip_sync", qh.hip_sync())
    for e in range(3):
        ref = oracle.gemv(t, xs[e], data[e * nbytes:(e + 1) * nbytes], in_dim, out_dim)
        assert cf.rel_l2(dy[e].download(np.float32), ref) < TOL


def test_unknown_type_zero_fills(qh):
    y = GpuBuf.upload_f32(np.full(16, 7.0, np.float32))
    w = GpuBuf.alloc(64)
    x = GpuBuf.alloc_f32(256)
    assert qh.hip_gemv(5, w.ptr, x.ptr, y.ptr, 256, 16) == -1
    check("hip_sync", qh.hip_sync())
    assert np.all(y.download(np.float32) == 0.0)


def test_iq_grid_upload_roundtrip(qh, oracle):
    """hip_set_*_grid with the standard tables leaves results unchanged."""
    # keep every host table referenced while the library copies it
    t2xxs = np.ascontiguousarray(cf.GRIDS["IQ2XXS"][0], dtype=np.uint64)
    t2xs = np.ascontiguousarray(cf.GRIDS["IQ2XS"][0], dtype=np.uint64)
    t2s = np.ascontiguousarray(cf.GRIDS["IQ2S"][0], dtype=np.uint64)
    t3s = np.ascontiguousarray(cf.GRIDS["IQ3S"][0], dtype=np.uint32)
    check("set", qh.hip_set_iq2xxs_grid(t2xxs.ctypes.data))
    check("set", qh.hip_set_iq2xs_grid(t2xs.ctypes.data))
    check("set", qh.hip_set_iq2s_grid(t2s.ctypes.data))
    check("set", qh.hip_set_iq3s_grid(t3s.ctypes.data))
    for t in (16, 17, 21, 22):
        data = synth.weights(t, 8, 512, seed=t)
        x = synth.activations(1, 512, seed=1)[0]
        assert cf.rel_l2(gpu_gemv(qh, t, x, data, 512, 8), oracle.gemv(t, x, data, 512, 8)) < TOL


def test_mem_info(qh):
    import ctypes as C
    f, tot = C.c_size_t(), C.c_size_t()
    check("hip_mem_info", qh.hip_mem_info(C.byref(f), C.byref(tot)))
    assert 0 < f.value <= tot.value


@pytest.mark.parametrize("t", [12, 14, 13, 8])
@pytest.mark.parametrize("n", [1, 4, 16, 27])
@pytest.mark.parametrize("swiglu, acc", [(True, True), (True, False), (False, True)])
def test_gemm_grouped_ex(qh, oracle, t, n, swiglu, acc):
    """hip_gemm_grouped_ex: y (+)= W (silu(gate) * up) or W x for n tokens, two
    matrices in one call, against the oracle (1e-3 relative L2 per token; the
    n = 1 and Q8_0 cases take the separate-kernel path)."""
    from saient_quartz_amd.host import gemm_grouped_ex_async
    in_dim, dims = 1024, (300, 64)
    rng = np.random.default_rng(n + 10 * t)
    xg = rng.standard_normal((n, in_dim)).astype(np.float32)
    xu = rng.standard_normal((n, in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=90 + k) for k, o in enumerate(dims)]
    y0 = [rng.standard_normal((n, o)).astype(np.float32) for o in dims]
    ws = [GpuBuf.upload(d) for d in datas]
    ys = [GpuBuf.upload_f32(a.reshape(-1)) for a in y0]
    dg, du = GpuBuf.upload_f32(xg.reshape(-1)), GpuBuf.upload_f32(xu.reshape(-1))
    scratch = GpuBuf.alloc_f32(n * in_dim + n * max(dims))
    gemm_grouped_ex_async(qh, t, [w.ptr for w in ws], [dg.ptr] * 2, [y.ptr for y in ys], [n] * 2, list(dims), in_dim,
                          None, up_ptrs=[du.ptr] * 2 if swiglu else None, accumulate=acc, scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    xin = xg.astype(np.float64)
    if swiglu:
        xin = xin / (1.0 + np.exp(-xin)) * xu.astype(np.float64)
    for k, o in enumerate(dims):
        w = oracle.dequant(t, datas[k], o * in_dim).astype(np.float64).reshape(o, in_dim)
        got = ys[k].download(np.float32)[:n * o].reshape(n, o)
        for i in range(n):
            ref = w @ xin[i] + (y0[k][i] if acc else 0.0)
            assert cf.rel_l2(got[i], ref) < TOL, (k, i, cf.rel_l2(got[i], ref))


@pytest.mark.parametrize("in_dim, out_dim, n, off", [(4096, 8, 64, 0), (1001, 257, 3, 0), (2880, 32, 5, 1),
                                                     (64, 128, 300, 0)])
def test_gemm_f32_router(qh, oracle, in_dim, out_dim, n, off):
    """F32 weights over a batch (MoE routers) take one launch; off = 1 shifts x
    by one float so the float4 path is not used."""
    import torch
    rng = np.random.default_rng(in_dim + n)
    w = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    x = rng.standard_normal((n, in_dim)).astype(np.float32)
    W = torch.from_numpy(w).cuda()
    X = torch.from_numpy(np.concatenate([np.zeros(off, np.float32), x.reshape(-1)])).cuda()
    Y = torch.empty(n, out_dim, device="cuda")
    check("hip_gemm", qh.hip_gemm(0, W.data_ptr(), X.data_ptr() + 4 * off, Y.data_ptr(), in_dim, out_dim, n))
    torch.cuda.synchronize()
    ref = oracle.gemm(0, x, w.view(np.uint8).reshape(-1), in_dim, out_dim, n)
    assert cf.rel_l2(Y.cpu().numpy(), ref) < 1e-5  # two f32 summation orders over up to 4096 terms


@pytest.mark.parametrize("t", [12, 13, 14, 8, 21, 16])
@pytest.mark.parametrize("n", [2, 3, 4])
@pytest.mark.parametrize("out_dim, in_dim", [(300, 4096), (77, 14336), (4100, 512)])
def test_gemm_few_tokens_equal_gemv(qh, oracle, t, n, out_dim, in_dim):
    """2-4 tokens run through the GEMV kernel with shared weight loads: each
    token's row is the one-token GEMV of that token, bit for bit, and within
    the GEMV bar of the oracle (x 16-byte aligned, so both take the matrix-core
    kernels)."""
    data = synth.weights(t, out_dim, in_dim, seed=40 + t + n)
    x = synth.activations(n, in_dim, seed=41 + n)
    x[n - 1] *= 1e-4  # tokens of very different magnitudes keep their own exponents
    got = gpu_gemm(qh, t, x, data, in_dim, out_dim, n)
    w = GpuBuf.upload(data)
    for k in range(n):
        dx = GpuBuf.upload_f32(np.ascontiguousarray(x[k]))
        dy = GpuBuf.alloc_f32(out_dim)
        check("hip_gemv", qh.hip_gemv(t, w.ptr, dx.ptr, dy.ptr, in_dim, out_dim))
        one = dy.download(np.float32)[:out_dim]
        assert np.array_equal(got[k].view(np.uint32), one.view(np.uint32)), (k, np.argwhere(got[k] != one)[:4])
    ref = oracle.gemm(t, x, data, in_dim, out_dim, n)
    for k in range(n):
        assert cf.rel_l2(got[k], ref[k]) < TOL


@pytest.mark.parametrize("t", [12, 14, 13, 21])
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 16, 20])
@pytest.mark.parametrize("in_dim", [2048, 768])
def test_gemm_grouped_norm(qh, oracle, t, n, in_dim):
    """y[k] = W[k] (rms_norm(x) * w) with the norm fused into the GEMMs (the
    one-token GEMV, the 2-4 token GEMV, the batched kernel's x prologue) against
    the oracle on the normalised rows, computed in float64."""
    import ctypes as C
    outs = [300, 77]
    rng = np.random.default_rng(n + t)
    x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + n) for o in outs]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    k = len(outs)
    check("hip_gemm_grouped_norm_async", qh.hip_gemm_grouped_norm_async(
        t, k, (C.c_void_p * k)(*[b.ptr for b in dw]), dx.ptr, dn.ptr, (C.c_void_p * k)(*[b.ptr for b in dy]), n,
        (C.c_int * k)(*outs), in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xd = x.astype(np.float64)
    xn = (xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w).astype(np.float32)
    for b, d, o in zip(dy, datas, outs):
        got = b.download(np.float32)[:n * o].reshape(n, o)
        ref = oracle.gemm(t, xn, d, in_dim, o, n)
        for r in range(n):
            assert cf.rel_l2(got[r], ref[r]) < TOL, (r, cf.rel_l2(got[r], ref[r]))


@pytest.mark.gpu
@pytest.mark.parametrize("types", [(12, 12, 14), (13, 14, 13), (12, 21), (12, 12), (14,), (16, 16)], ids=str)
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 16, 17, 20, 32])
@pytest.mark.parametrize("in_dim", [4096, 2048, 5120])
def test_gemm_group_norm_mixed(qh, oracle, types, n, in_dim):
    """hip_gemm_group_norm_async (mixed types: a Q4_K_M layer's q, k (Q4_K) and v
    (Q6_K)): bit-identical to one hip_gemm_grouped_norm_async per type (the
    two-format GEMV launch for 2-4 tokens, the per-type calls otherwise), and
    within the GEMV bar of the oracle on the normalised rows (float64 norm).
    Q4_K + Q6_K at 5-16 tokens runs the two-format batched launch, whose K
    splits may differ from the per-type calls': there the bar is 1e-5 relative
    against them.  5120 is past the one-workgroup norm; IQ3_S + Q4_K has no
    two-format kernel.  One type at 5-16 tokens, and any types at 17-32 tokens
    (in_dim <= 4096), take the norm fused into the batched kernel's x images
    (two image halves past 16 tokens): its images are the per-type call's
    digitised normalised rows, so it is bit-identical too."""
    import ctypes as C
    outs = [300, 77, 64][:len(types)]
    rng = np.random.default_rng(n + in_dim + sum(types))
    x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + n + t) for t, o in zip(types, outs)]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    k = len(outs)
    check("hip_gemm_group_norm_async", qh.hip_gemm_group_norm_async(
        k, (C.c_uint32 * k)(*types), (C.c_void_p * k)(*[b.ptr for b in dw]), dx.ptr, dn.ptr,
        (C.c_void_p * k)(*[b.ptr for b in dy]), n, (C.c_int * k)(*outs), in_dim, scratch.ptr, None))
    # the per-type reference calls
    ey = [GpuBuf.alloc_f32(n * o) for o in outs]
    for t in sorted(set(types)):
        ks = [i for i, tt in enumerate(types) if tt == t]
        m = len(ks)
        check("hip_gemm_grouped_norm_async", qh.hip_gemm_grouped_norm_async(
            t, m, (C.c_void_p * m)(*[dw[i].ptr for i in ks]), dx.ptr, dn.ptr, (C.c_void_p * m)(*[ey[i].ptr for i in ks]),
            n, (C.c_int * m)(*[outs[i] for i in ks]), in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xd = x.astype(np.float64)
    xn = (xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w).astype(np.float32)
    for b, e, d, o, t in zip(dy, ey, datas, outs, types):
        got = b.download(np.float32)[:n * o].reshape(n, o)
        exp = e.download(np.float32)[:n * o].reshape(n, o)
        if n >= 5 and set(types) == {12, 14}:
            for r in range(n):
                assert cf.rel_l2(got[r], exp[r]) < 1e-5, (t, o, r)
        else:
            assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (t, o)
        ref = oracle.gemm(t, xn, d, in_dim, o, n)
        for r in range(n):
            assert cf.rel_l2(got[r], ref[r]) < TOL, (r, cf.rel_l2(got[r], ref[r]))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [3, 4])
def test_gemm_group_norm_fused_images_few_tokens(qh, oracle, n):
    """3-4 tokens over more than 16 MB of one type (a batch of 3-4 sequences'
    gate and up) take the norm fused into the batched kernel's x images:
    bit-identical to the per-type normalise-then-GEMM call, and within the bar
    of the oracle on the float64-normalised rows."""
    import ctypes as C
    t, in_dim, outs = 12, 4096, [4096, 4096]
    rng = np.random.default_rng(7 + n)
    x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + n + k) for k, o in enumerate(outs)]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    ey = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    k = len(outs)
    check("hip_gemm_group_norm_async", qh.hip_gemm_group_norm_async(
        k, (C.c_uint32 * k)(*([t] * k)), (C.c_void_p * k)(*[b.ptr for b in dw]), dx.ptr, dn.ptr,
        (C.c_void_p * k)(*[b.ptr for b in dy]), n, (C.c_int * k)(*outs), in_dim, scratch.ptr, None))
    check("hip_gemm_grouped_norm_async", qh.hip_gemm_grouped_norm_async(
        t, k, (C.c_void_p * k)(*[b.ptr for b in dw]), dx.ptr, dn.ptr, (C.c_void_p * k)(*[b.ptr for b in ey]),
        n, (C.c_int * k)(*outs), in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xd = x.astype(np.float64)
    xn = (xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w).astype(np.float32)
    for b, e, d, o in zip(dy, ey, datas, outs):
        got = b.download(np.float32)[:n * o].reshape(n, o)
        exp = e.download(np.float32)[:n * o].reshape(n, o)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), o
        ref = oracle.gemm(t, xn, d, in_dim, o, n)
        for r in range(n):
            assert cf.rel_l2(got[r], ref[r]) < TOL, (r, cf.rel_l2(got[r], ref[r]))


@pytest.mark.gpu
@pytest.mark.parametrize("n", [8, 27])
@pytest.mark.parametrize("types", [(12, 12), (12, 12, 14)], ids=str)
def test_gemm_group_norm_non_finite_token(qh, types, n):
    """A token whose row holds an Inf through the fused norm images (5-32
    tokens): every output of that token is NaN (its norm is NaN), the other
    tokens equal the per-type call bit for bit."""
    import ctypes as C
    in_dim, outs = 2048, [300, 77, 64][:len(types)]
    rng = np.random.default_rng(3)
    x = rng.standard_normal((n, in_dim)).astype(np.float32)
    x[5, 700] = np.inf
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + t) for t, o in zip(types, outs)]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    k = len(outs)
    check("hip_gemm_group_norm_async", qh.hip_gemm_group_norm_async(
        k, (C.c_uint32 * k)(*types), (C.c_void_p * k)(*[b.ptr for b in dw]), dx.ptr, dn.ptr,
        (C.c_void_p * k)(*[b.ptr for b in dy]), n, (C.c_int * k)(*outs), in_dim, scratch.ptr, None))
    x2 = x.copy()
    x2[5] = 1.0  # the clean rows alone, through the per-type calls
    dx2 = GpuBuf.upload_f32(x2.reshape(-1))
    ey = [GpuBuf.alloc_f32(n * o) for o in outs]
    for t in sorted(set(types)):
        ks = [i for i, tt in enumerate(types) if tt == t]
        m = len(ks)
        check("hip_gemm_grouped_norm_async", qh.hip_gemm_grouped_norm_async(
            t, m, (C.c_void_p * m)(*[dw[i].ptr for i in ks]), dx2.ptr, dn.ptr,
            (C.c_void_p * m)(*[ey[i].ptr for i in ks]), n, (C.c_int * m)(*[outs[i] for i in ks]), in_dim,
            scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    for b, e, o, t in zip(dy, ey, outs, types):
        got = b.download(np.float32)[:n * o].reshape(n, o)
        exp = e.download(np.float32)[:n * o].reshape(n, o)
        assert np.isnan(got[5]).all(), (t, o)
        for r in range(n):
            if r == 5:
                continue
            if set(types) == {12, 14}:
                assert cf.rel_l2(got[r], exp[r]) < 1e-5, (t, o, r)
            else:
                assert np.array_equal(got[r].view(np.uint32), exp[r].view(np.uint32)), (t, o, r)


@pytest.mark.parametrize("t", [12, 14, 8, 21])
@pytest.mark.parametrize("n", [1, 3, 16])
def test_non_finite_x_flags_rows(qh, oracle, t, n):
    """An Inf in x (one element of one token): every output row of that token
    that the reference makes non-finite (+-Inf where the row's weight there is
    nonzero, NaN where it is zero) is non-finite here too (this build returns
    NaN for them, not the reference's signed Inf), and the other tokens' rows
    keep the 1e-3 bar."""
    out_dim, in_dim = 70, 4096
    data = synth.weights(t, out_dim, in_dim, seed=1200 + t)
    x = synth.activations(n, in_dim, seed=1201 + n)
    x[0, 777] = np.inf
    got = gpu_gemv(qh, t, x[0], data, in_dim, out_dim)[None] if n == 1 else gpu_gemm(qh, t, x, data, in_dim,
                                                                                     out_dim, n)
    ref = oracle.gemv(t, x[0], data, in_dim, out_dim)[None] if n == 1 else oracle.gemm(t, x, data, in_dim, out_dim, n)
    assert not np.isfinite(ref[0]).any()  # random weights: no zero weight at column 777
    assert np.array_equal(np.isfinite(got[0]), np.isfinite(ref[0]))
    for k in range(1, n):
        assert cf.rel_l2(got[k], ref[k]) < TOL


@pytest.mark.parametrize("t", [12, 14])
@pytest.mark.parametrize("n", [2, 3, 4])
def test_gemm_residual_tokens_many_tiles(qh, oracle, t, n):
    """y += W x for 2-4 tokens through the GEMV kernel with several row tiles per
    workgroup (9000 rows): each token's rows against the oracle, so a residual
    value taken from the wrong token or tile would show."""
    from saient_quartz_amd.host import gemm_grouped_ex_async
    in_dim, o = 1024, 9000
    rng = np.random.default_rng(7 * n + t)
    x = rng.standard_normal((n, in_dim)).astype(np.float32)
    data = synth.weights(t, o, in_dim, seed=300 + t)
    y0 = (10 * rng.standard_normal((n, o))).astype(np.float32)
    w, y, dx = GpuBuf.upload(data), GpuBuf.upload_f32(y0.reshape(-1)), GpuBuf.upload_f32(x.reshape(-1))
    scratch = GpuBuf.alloc_f32(n * in_dim + n * o)
    gemm_grouped_ex_async(qh, t, [w.ptr], [dx.ptr], [y.ptr], [n], [o], in_dim, None, accumulate=True,
                          scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    got = y.download(np.float32)[:n * o].reshape(n, o)
    wd = oracle.dequant(t, data, o * in_dim).astype(np.float64).reshape(o, in_dim)
    for i in range(n):
        ref = wd @ x[i].astype(np.float64) + y0[i]
        assert cf.rel_l2(got[i], ref) < TOL, (i, cf.rel_l2(got[i], ref))
        assert np.max(np.abs(got[i] - ref)) < 1e-2 * np.max(np.abs(ref)), i
