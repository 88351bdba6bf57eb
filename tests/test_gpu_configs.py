"""GPU parity at the benchmark configurations' full shapes (BASELINE.json
configs[2], [3], [4]), through the C ABI, against the CPU oracle.

  * the Q6_K 128256x4096 output head, as hip_gemv (cuda_gemv's
    launch at src/cuda.rs:834-836) and as the fused final-norm + head launch
    (hip_gemv_fused_async with norm_w, the cuda_rms_norm + cuda_gemv pair of
    src/cuda.rs:824-836).
  * the Mixtral-shaped expert GEMMs (gate/up 14336x4096, down
    4096x14336, IQ3_S and IQ2_XXS, 16 gathered tokens per expert), through
    hip_gemm_moe (the per-expert loop of src/cuda.rs:667-798) and
    hip_gemm_grouped, against oracle.gemm (dequant::gemm, src/dequant.rs:143).
  * one ForwardStep layer (N = 1) and one BatchStep layer (N = 4,
    16, 32) at the Llama-3-8B dimensions (hidden 4096, 32 q / 8 kv heads, FFN
    14336, vocab 128256) against glue_ref.forward_step per sequence, with the
    logits checked through oracle.gemv of the float64-normed hidden state; and
    the batched kernels at those shapes on their own: hip_gemm (Q4_K 14336x4096,
    Q6_K 4096x14336, Q4_K 4096x4096), the q/k/v launch with the norm fused
    (hip_gemm_group_norm_async), and the down projection with SwiGLU and the
    residual (hip_gemm_grouped_ex_async), at N = 4 .. 32.
Bar: 1e-3 relative L2 (per token for GEMMs), the north_star's GEMV tolerance."""
import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import synth
from saient_quartz_amd.api import check
from saient_quartz_amd.host import GpuBuf, gemm_grouped_async, gemm_moe_async, gemv_fused_async

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import glue_ref as g  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3
Q4_K, Q6_K, IQ2_XXS, IQ3_S = 12, 14, 16, 21
VOCAB, HIDDEN, FFN = 128256, 4096, 14336


@pytest.fixture(scope="module")
def head():
    """configs[2]'s seeded Q6_K head (431 MB) on the host and the device."""
    data = synth.weights(Q6_K, VOCAB, HIDDEN, seed=synth.SEED_BASE + 2)
    return data, GpuBuf.upload(data)


def test_head_gemv_configs2(qh, oracle, head):
    data, dw = head
    x = synth.activations(1, HIDDEN, seed=synth.SEED_BASE + 12)[0]
    print(f"hip_gemv Q6_K {VOCAB}x{HIDDEN}", flush=True)
    dx, dy = GpuBuf.upload_f32(x), GpuBuf.alloc_f32(VOCAB)
    check("hip_gemv", qh.hip_gemv(Q6_K, dw.ptr, dx.ptr, dy.ptr, HIDDEN, VOCAB))
    check("hip_sync", qh.hip_sync())
    got = dy.download(np.float32)
    ref = oracle.gemv(Q6_K, x, data, HIDDEN, VOCAB)
    err = cf.rel_l2(got, ref)
    print(f"rel_l2 {err:.2e}", flush=True)
    assert err < TOL
    # the reference's --verify-gemv criterion (src/main.rs:2653-2662) as well
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-3


def test_head_fused_norm_configs2(qh, oracle, head):
    """The final RMS norm fused into the head launch (the decode step's last
    GEMV), against oracle.gemv of the float64-normed x."""
    data, dw = head
    rng = np.random.default_rng(5)
    x = (3.0 * rng.standard_normal(HIDDEN)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(HIDDEN)).astype(np.float32)
    print(f"hip_gemv_fused (norm) Q6_K {VOCAB}x{HIDDEN}", flush=True)
    dx, dn, dy = GpuBuf.upload_f32(x), GpuBuf.upload_f32(w), GpuBuf.alloc_f32(VOCAB)
    gemv_fused_async(qh, Q6_K, [dw.ptr], [dy.ptr], [VOCAB], dx.ptr, HIDDEN, None, norm_ptr=dn.ptr)
    check("hip_sync", qh.hip_sync())
    got = dy.download(np.float32)
    xn = g.rms_norm(x.astype(np.float64), w.astype(np.float64)).astype(np.float32)
    ref = oracle.gemv(Q6_K, xn, data, HIDDEN, VOCAB)
    err = cf.rel_l2(got, ref)
    print(f"rel_l2 {err:.2e}", flush=True)
    assert err < TOL


@pytest.mark.parametrize("t", [IQ3_S, IQ2_XXS])
@pytest.mark.parametrize("shape", [(FFN, HIDDEN), (HIDDEN, FFN)], ids=["gate_up", "down"])
def test_expert_gemms_configs4(qh, oracle, t, shape):
    """8 experts at the Mixtral shape, 16 gathered tokens each, in one
    hip_gemm_moe call (expert order 3, 0, 7, ...: the device order follows
    the host array, not the expert index), every token against oracle.gemm."""
    out_dim, in_dim = shape
    n_exp, ntok = 8, 16
    per = synth.weights(t, out_dim, in_dim, seed=0).nbytes
    datas = [synth.weights(t, out_dim, in_dim, seed=synth.SEED_BASE + 40 + e) for e in range(n_exp)]
    dw = GpuBuf.upload(np.concatenate(datas))
    assert dw.bytes == n_exp * per
    ids = [3, 0, 7, 1, 6, 2, 5, 4]
    tok_off = [ntok * i for i in range(n_exp + 1)]
    rng = np.random.default_rng(t + out_dim)
    x = rng.standard_normal((n_exp * ntok, in_dim)).astype(np.float32)
    dx, dy = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.alloc_f32(n_exp * ntok * out_dim)
    print(f"hip_gemm_moe type {t} {out_dim}x{in_dim} x {n_exp} experts x {ntok} tokens", flush=True)
    gemm_moe_async(qh, t, dw.ptr, ids, tok_off, dx.ptr, dy.ptr, in_dim, out_dim, None)
    check("hip_sync", qh.hip_sync())
    got = dy.download(np.float32).reshape(n_exp * ntok, out_dim)
    worst = 0.0
    for i, e in enumerate(ids):
        sl = slice(tok_off[i], tok_off[i + 1])
        ref = oracle.gemm(t, x[sl], datas[e], in_dim, out_dim, ntok)
        for r in range(ntok):
            err = cf.rel_l2(got[sl][r], ref[r])
            worst = max(worst, err)
            assert err < TOL, (e, r, err)
    print(f"worst rel_l2 {worst:.2e}", flush=True)
    # hip_gemm_grouped on two of the experts (distinct x blocks) agrees with the oracle too
    ys = [GpuBuf.alloc_f32(ntok * out_dim) for _ in range(2)]
    xs = [GpuBuf.upload_f32(x[:ntok].reshape(-1)), GpuBuf.upload_f32(x[ntok:2 * ntok].reshape(-1))]
    ws = [GpuBuf.upload(datas[1]), GpuBuf.upload(datas[6])]
    gemm_grouped_async(qh, t, [w.ptr for w in ws], [b.ptr for b in xs], [y.ptr for y in ys], [ntok] * 2,
                       [out_dim] * 2, in_dim, None)
    check("hip_sync", qh.hip_sync())
    for y, d, xx in zip(ys, (datas[1], datas[6]), (x[:ntok], x[ntok:2 * ntok])):
        got = y.download(np.float32).reshape(ntok, out_dim)
        ref = oracle.gemm(t, xx, d, in_dim, out_dim, ntok)
        for r in range(ntok):
            assert cf.rel_l2(got[r], ref[r]) < TOL, r


LLAMA_Q4KM = (("q", Q4_K), ("k", Q4_K), ("v", Q6_K), ("o", Q4_K), ("gate", Q4_K), ("up", Q4_K),
              ("down", Q6_K), ("head", Q6_K), ("embed", Q4_K))


@pytest.fixture(scope="module")
def llama_layer(oracle):
    """One Llama-3-8B-dimension layer, Q4_K_M types (q, k, o, gate, up Q4_K;
    v, down Q6_K; Q6_K head, Q4_K embedding), weights at a real checkpoint's
    scale: the config, the host bytes and norms, the device weights, and the
    oracle's float64 layer (dequantized bit-exactly)."""
    from saient_quartz_amd.decode import ModelConfig
    from test_gpu_decode_step import device_weights, host_model

    cfg = ModelConfig(hidden=HIDDEN, n_heads=32, n_kv=8, head_dim=128, ffn=FFN, vocab=VOCAB, layers=1, max_seq=8,
                      types=LLAMA_Q4KM)
    print("building the 8B-dimension layer", flush=True)
    raw, norms = host_model(cfg, seed=101, realistic=True)
    deq = lambda n, a, o, i: oracle.dequant(cfg.type_of(n), a, o * i).astype(np.float64).reshape(o, i)
    L = {n: deq(n, raw[n][0], o, i) for n, o, i in cfg.mats()}
    L["attn_norm"], L["ffn_norm"] = norms["attn_norm"][0], norms["ffn_norm"][0]
    return cfg, raw, norms, device_weights(raw, norms), L


def _layer_reference(oracle, cfg, raw, norms, L, token, pos, kv):
    """glue_ref.forward_step over the one layer for `token` at `pos` (kv updated
    in place), and the logits as oracle.gemv of the float64 final norm."""
    ocfg = dict(n_heads=cfg.n_heads, n_kv=cfg.n_kv, head_dim=cfg.head_dim, theta=cfg.theta, neox=bool(cfg.neox))
    row_bytes = HIDDEN // 256 * 144
    emb = oracle.dequant(Q4_K, raw["embed"][token * row_bytes:(token + 1) * row_bytes], HIDDEN).astype(np.float64)
    _, hidden = g.forward_step(emb, pos, [L], np.zeros((1, HIDDEN)), norms["out_norm"], kv, ocfg)
    xn = g.rms_norm(hidden, norms["out_norm"].astype(np.float64)).astype(np.float32)
    return oracle.gemv(Q6_K, xn, raw["head"], HIDDEN, VOCAB), hidden


def test_forward_step_full_8b_dims(qh, oracle, llama_layer):
    """One ForwardStep layer at the Llama-3-8B dimensions, three consecutive
    positions.  Hidden state against glue_ref.forward_step (float64 on the
    oracle's dequantized weights); logits against oracle.gemv of the float64
    final norm of the reference hidden state."""
    import torch

    from saient_quartz_amd.decode import ForwardStep

    cfg, raw, norms, dw, L = llama_layer
    step = ForwardStep(cfg, dw)
    kvd = cfg.n_kv * cfg.head_dim
    kv = [[np.zeros((cfg.max_seq, kvd)), np.zeros((cfg.max_seq, kvd))]]
    for pos, token in enumerate([11, VOCAB - 1, 4242]):
        print(f"8B layer pos {pos} token {token}", flush=True)
        step.issue(token, pos)
        torch.cuda.synchronize()
        ref_logits, ref_hidden = _layer_reference(oracle, cfg, raw, norms, L, token, pos, kv)
        got = step.logits.cpu().numpy()
        eh, el = cf.rel_l2(step.hidden.cpu().numpy(), ref_hidden), cf.rel_l2(got, ref_logits)
        print(f"  hidden rel_l2 {eh:.2e} logits rel_l2 {el:.2e}", flush=True)
        assert np.all(np.isfinite(got))
        assert eh < TOL and el < TOL, (pos, eh, el)


@pytest.mark.parametrize("n", [4, 16, 32])
def test_batch_step_full_8b_dims(qh, oracle, llama_layer, n):
    """configs[3] at N = 4, 16 and 32: one BatchStep layer at the Llama-3-8B
    dimensions (the batched GEMMs at their real shapes: q/k/v with the norm in
    one two-format launch, o + residual, gate/up with the norm, down with the
    SwiGLU and the residual), three positions, every sequence against
    glue_ref.forward_step with its own K/V cache, logits through oracle.gemv."""
    import torch

    from saient_quartz_amd.decode import BatchStep

    cfg, raw, norms, dw, L = llama_layer
    step = BatchStep(cfg, dw, n)
    kvd = cfg.n_kv * cfg.head_dim
    kvs = [[[np.zeros((cfg.max_seq, kvd)), np.zeros((cfg.max_seq, kvd))]] for _ in range(n)]
    rng = np.random.default_rng(n)
    worst = 0.0
    for pos in range(3):
        tokens = rng.integers(0, VOCAB, n)
        print(f"8B batch n={n} pos {pos}", flush=True)
        step.issue(tokens, pos)
        torch.cuda.synchronize()
        got_l, got_h = step.logits.cpu().numpy(), step.hidden.cpu().numpy()
        for i in range(n):
            ref_logits, ref_hidden = _layer_reference(oracle, cfg, raw, norms, L, int(tokens[i]), pos, kvs[i])
            eh, el = cf.rel_l2(got_h[i], ref_hidden), cf.rel_l2(got_l[i], ref_logits)
            worst = max(worst, eh, el)
            assert np.all(np.isfinite(got_l[i]))
            assert eh < TOL and el < TOL, (pos, i, eh, el)
    print(f"worst rel_l2 {worst:.2e}", flush=True)


@pytest.mark.parametrize("n", [4, 16, 32])
@pytest.mark.parametrize("t, out_dim, in_dim", [(Q4_K, FFN, HIDDEN), (Q6_K, HIDDEN, FFN), (Q4_K, HIDDEN, HIDDEN)],
                         ids=["q4k_gate_up", "q6k_down", "q4k_o"])
def test_gemm_8b_shapes(qh, oracle, t, out_dim, in_dim, n):
    """hip_gemm (dequant::gemm, src/dequant.rs:143-200) at configs[3]'s
    batched shapes, with token magnitudes spread over six decades and one
    activation outlier per token, every token against oracle.gemm."""
    data = synth.weights(t, out_dim, in_dim, seed=synth.SEED_BASE + 300 + n)
    rng = np.random.default_rng(n + out_dim)
    x = rng.standard_normal((n, in_dim)).astype(np.float32)
    x[np.arange(n), rng.integers(0, in_dim, n)] *= 200.0
    x *= (10.0 ** np.linspace(-3, 3, n))[:, None].astype(np.float32)
    w, dx, dy = GpuBuf.upload(data), GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.alloc_f32(n * out_dim)
    print(f"hip_gemm type {t} {out_dim}x{in_dim} n={n}", flush=True)
    check("hip_gemm", qh.hip_gemm(t, w.ptr, dx.ptr, dy.ptr, in_dim, out_dim, n))
    got = dy.download(np.float32).reshape(n, out_dim)
    ref = oracle.gemm(t, x, data, in_dim, out_dim, n)
    errs = [cf.rel_l2(got[k], ref[k]) for k in range(n)]
    print(f"worst rel_l2 {max(errs):.2e}", flush=True)
    assert max(errs) < TOL, int(np.argmax(errs))


def _rows_norm(x, w):
    xd = x.astype(np.float64)
    return (xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w).astype(np.float32)


@pytest.mark.parametrize("n", [4, 8, 16, 24, 32])
def test_group_norm_qkv_8b(qh, oracle, n):
    """hip_gemm_group_norm_async on a layer's q, k (Q4_K 4096 and 1024 rows) and
    v (Q6_K 1024 rows) over 4096 with the RMS norm fused, at the token counts
    of configs[3] (the NT GEMV kernel at 4, the norm-image launch and one
    two-format batched launch at 8-32), against oracle.gemm of the float64-
    normed rows."""
    types, outs, in_dim = (Q4_K, Q4_K, Q6_K), (HIDDEN, 1024, 1024), HIDDEN
    rng = np.random.default_rng(100 + n)
    x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + n + k) for k, (t, o) in enumerate(zip(types, outs))]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    print(f"hip_gemm_group_norm q/k/v n={n}", flush=True)
    check("hip_gemm_group_norm_async", qh.hip_gemm_group_norm_async(
        3, (C.c_uint32 * 3)(*types), (C.c_void_p * 3)(*[b.ptr for b in dw]), dx.ptr, dn.ptr,
        (C.c_void_p * 3)(*[b.ptr for b in dy]), n, (C.c_int * 3)(*outs), in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xn = _rows_norm(x, w)
    for b, d, o, t in zip(dy, datas, outs, types):
        got = b.download(np.float32).reshape(n, o)
        ref = oracle.gemm(t, xn, d, in_dim, o, n)
        for r in range(n):
            assert cf.rel_l2(got[r], ref[r]) < TOL, (t, o, r, cf.rel_l2(got[r], ref[r]))


@pytest.mark.parametrize("n", [4, 16, 32])
def test_gemm_ex_down_swiglu_residual_8b(qh, oracle, n):
    """hip_gemm_grouped_ex as BatchStep's down projection: hidden += W_down
    (silu(gate) * up), Q6_K 4096x14336, the SwiGLU in the x digitisation and
    the residual in the epilogue; against oracle.gemm of the f32 SwiGLU rows
    plus the old hidden state."""
    from saient_quartz_amd.host import gemm_grouped_ex_async
    from test_gpu_decode_step import realistic_scale
    data = realistic_scale(synth.weights(Q6_K, HIDDEN, FFN, seed=synth.SEED_BASE + 400 + n), Q6_K)
    rng = np.random.default_rng(200 + n)
    gate = (rng.standard_normal((n, FFN)) * 3).astype(np.float32)
    up = rng.standard_normal((n, FFN)).astype(np.float32)
    h0 = rng.standard_normal((n, HIDDEN)).astype(np.float32)
    w, dg, du = GpuBuf.upload(data), GpuBuf.upload_f32(gate.reshape(-1)), GpuBuf.upload_f32(up.reshape(-1))
    dh = GpuBuf.upload_f32(h0.reshape(-1))
    scratch = GpuBuf.alloc_f32(2 * n * FFN)
    print(f"hip_gemm_grouped_ex down n={n}", flush=True)
    gemm_grouped_ex_async(qh, Q6_K, [w.ptr], [dg.ptr], [dh.ptr], [n], [HIDDEN], FFN, None, up_ptrs=[du.ptr],
                          accumulate=True, scratch_ptr=scratch.ptr)
    check("hip_sync", qh.hip_sync())
    got = dh.download(np.float32).reshape(n, HIDDEN)
    act = g.swiglu(gate, up).astype(np.float32)
    ref = oracle.gemm(Q6_K, act, data, FFN, HIDDEN, n).astype(np.float64) + h0
    for r in range(n):
        assert cf.rel_l2(got[r], ref[r]) < TOL, (r, cf.rel_l2(got[r], ref[r]))


@pytest.mark.parametrize("n", [3, 4])
def test_group_norm_mixed_above_16mb(qh, oracle, n):
    """hip_gemm_group_norm_async at 3-4 tokens with more than 16 MB of weights
    per type (Q4_K 8192x4096, Q6_K 5120x4096): bit-identical to the per-type
    hip_gemm_grouped_norm_async calls, and within the bar of the oracle."""
    types, outs, in_dim = (Q4_K, Q6_K), (8192, 5120), HIDDEN
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((n, in_dim)) * rng.uniform(0.1, 10, (n, 1))).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(in_dim)).astype(np.float32)
    datas = [synth.weights(t, o, in_dim, seed=o + n) for t, o in zip(types, outs)]
    dw = [GpuBuf.upload(d) for d in datas]
    dx, dn = GpuBuf.upload_f32(x.reshape(-1)), GpuBuf.upload_f32(w)
    dy = [GpuBuf.alloc_f32(n * o) for o in outs]
    ey = [GpuBuf.alloc_f32(n * o) for o in outs]
    scratch = GpuBuf.alloc_f32(n * in_dim)
    check("hip_gemm_group_norm_async", qh.hip_gemm_group_norm_async(
        2, (C.c_uint32 * 2)(*types), (C.c_void_p * 2)(*[b.ptr for b in dw]), dx.ptr, dn.ptr,
        (C.c_void_p * 2)(*[b.ptr for b in dy]), n, (C.c_int * 2)(*outs), in_dim, scratch.ptr, None))
    for i, t in enumerate(types):
        check("hip_gemm_grouped_norm_async", qh.hip_gemm_grouped_norm_async(
            t, 1, (C.c_void_p * 1)(dw[i].ptr), dx.ptr, dn.ptr, (C.c_void_p * 1)(ey[i].ptr), n,
            (C.c_int * 1)(outs[i]), in_dim, scratch.ptr, None))
    check("hip_sync", qh.hip_sync())
    xd = x.astype(np.float64)
    xn = (xd / np.sqrt(np.mean(xd * xd, axis=1, keepdims=True) + 1e-5) * w).astype(np.float32)
    for b, e, d, o, t in zip(dy, ey, datas, outs, types):
        got = b.download(np.float32).reshape(n, o)
        exp = e.download(np.float32).reshape(n, o)
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), (t, o)
        ref = oracle.gemm(t, xn, d, in_dim, o, n)
        for r in range(n):
            assert cf.rel_l2(got[r], ref[r]) < TOL, (r, cf.rel_l2(got[r], ref[r]))
