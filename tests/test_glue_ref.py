"""Closed-form pins of oracle/glue_ref.py (the checker of the glue kernels):
properties the reference formulas fix, chosen so a dropped term, a swapped
pair index or a wrong sign fails one of them.  CPU only."""
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import glue_ref as g  # noqa: E402


def test_rope_identity_at_pos0_and_norm_preserving():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(4 * 64)
    for neox in (False, True):
        assert np.allclose(g.rope_yarn(x, 4, 64, 0, 10000.0, neox=neox), x)
        y = g.rope_yarn(x, 4, 64, 37, 10000.0, neox=neox).reshape(4, 64)
        xr = x.reshape(4, 64)
        if neox:
            pn = lambda a: a[:, :32] ** 2 + a[:, 32:] ** 2
        else:
            pn = lambda a: a[:, 0::2] ** 2 + a[:, 1::2] ** 2
        assert np.allclose(pn(y), pn(xr))


def test_rope_pairing_and_angle():
    # one head, head_dim 4: pair 0 has inv_freq 1, pair 1 has theta^-0.5
    x = np.array([1.0, 0.0, 0.0, 0.0])
    y = g.rope_yarn(x, 1, 4, 2, 100.0, neox=False)  # NORM: pair (0, 1), angle 2
    assert np.allclose(y, [np.cos(2), np.sin(2), 0, 0])
    y = g.rope_yarn(x, 1, 4, 2, 100.0, neox=True)  # NEOX: pair (0, 2)
    assert np.allclose(y, [np.cos(2), 0, np.sin(2), 0])
    x = np.array([0.0, 1.0, 0.0, 0.0])
    y = g.rope_yarn(x, 1, 4, 3, 100.0, neox=True)  # pair 1: (1, 3), inv_freq 0.1
    assert np.allclose(y, [0, np.cos(0.3), 0, np.sin(0.3)])


def test_yarn_ramp_limits():
    # wavelengths far below hfw keep inv_freq; far above lfw divide by the scale
    x = np.zeros(2 * 64)
    x[0] = 1.0
    x[62] = 1.0  # the last (longest) pair of head 0 in NORM pairing
    a = g.rope_yarn(x, 2, 64, 5, 1e6, yarn_scale=4.0, yarn_orig_ctx=4096)
    b = g.rope_yarn(x, 2, 64, 5, 1e6)
    assert np.allclose(a[:2], b[:2])  # pair 0: wavelen 2*pi < hfw = 128 -> unchanged
    inv_last = 1e6 ** (-62 / 64)
    assert np.allclose(a[62:64], [np.cos(5 * inv_last / 4), np.sin(5 * inv_last / 4)])


def test_rms_norm_constant_and_scale():
    w = np.linspace(0.5, 2.0, 16)
    y = g.rms_norm(np.full(16, -3.0), w)
    assert np.allclose(y, -w * 3.0 / np.sqrt(9.0 + 1e-5))
    x = np.random.default_rng(2).standard_normal(16)
    assert np.allclose(g.rms_norm(2 * x, w), g.rms_norm(x, w), rtol=1e-5)


def test_softmax_sink():
    x = np.array([1.0, 2.0, -1.0])
    p = g.softmax_sink(x)
    assert np.isclose(p.sum(), 1.0) and np.allclose(p, np.exp(x) / np.exp(x).sum())
    q = g.softmax_sink(x, 0.5)
    assert np.isclose(q.sum(), 1.0 - np.exp(0.5) / (np.exp(x).sum() + np.exp(0.5)))
    assert np.allclose(g.softmax_sink(x, -1e30), p)


def test_attention_one_token_and_gqa_mapping():
    rng = np.random.default_rng(3)
    hd, nh, nkv = 8, 4, 2
    kc = rng.standard_normal((5, nkv * hd))
    vc = rng.standard_normal((5, nkv * hd))
    q = rng.standard_normal(nh * hd)
    _, out = g.attention(q, kc, vc, nh, nkv, 1, hd, nkv * hd, 0.3)
    for h in range(nh):
        kvh = h * nkv // nh
        assert np.allclose(out[h * hd:(h + 1) * hd], vc[0, kvh * hd:(kvh + 1) * hd])
    probs, out = g.attention(q, kc, vc, nh, nkv, 5, hd, nkv * hd, 0.3)
    h = 3  # kv head 1
    s = kc[:, hd:] @ q[3 * hd:] * 0.3
    p = np.exp(s - s.max()) / np.exp(s - s.max()).sum()
    assert np.allclose(probs[h], p) and np.allclose(out[3 * hd:], p @ vc[:, hd:])


def test_swiglu_forms():
    gg = np.array([-3.0, 0.0, 2.0, 9.0])
    assert np.allclose(g.swiglu(gg, np.ones(4)), gg / (1 + np.exp(-gg)))
    assert np.allclose(g.swiglu(np.zeros(4), gg), 0.0)
    o = g.swiglu_oai(gg, np.array([0.0, 1.0, 8.0, -9.0]))
    assert np.isclose(o[3], 7 / (1 + np.exp(-1.702 * 7)) * (-7 + 1))
    assert np.isclose(o[2], 2 / (1 + np.exp(-3.404)) * 8.0)


def test_moe_route_order():
    rng = np.random.default_rng(3)
    v = rng.standard_normal(37).astype(np.float32)
    for k in (1, 4, 37):
        ids, _ = g.moe_route(v, k)
        assert list(ids) == list(np.argsort(-v.astype(np.float64), kind="stable")[:k])
    # total order: +0 above -0; +NaN above +inf, -NaN below -inf; ties: lower index first
    nan, neg_nan = np.float32(np.nan), -np.float32(np.nan)
    v = np.array([-0.0, 0.0, 1.0, 1.0, -np.inf, np.inf, neg_nan, nan, -5.0], np.float32)
    ids, _ = g.moe_route(v, 9)
    assert list(ids) == [7, 5, 2, 3, 1, 0, 8, 4, 6]
    # the router bias is added before the sort
    ids, _ = g.moe_route([0.0, 1.0, 2.0], 1, bias=[5.0, 0.0, 0.0])
    assert list(ids) == [0]


def test_greedy_next():
    rng = np.random.default_rng(6)
    for n in (1, 7, 1000):
        v = rng.standard_normal(n).astype(np.float32)
        assert g.greedy_next(v) == int(np.argmax(v))  # distinct values: the one maximum
    # equal maxima: the last one (max_by keeps the later of equal elements)
    assert g.greedy_next(np.array([1, 3, 2, 3, 0], np.float32)) == 3
    assert g.greedy_next(np.zeros(9, np.float32)) == 8
    # +0 above -0; +inf above every finite value; +NaN above +inf; -NaN below -inf
    nan = np.float32(np.nan)
    assert g.greedy_next(np.array([0.0, -0.0], np.float32)) == 0
    assert g.greedy_next(np.array([5.0, np.inf, 1e38], np.float32)) == 1
    assert g.greedy_next(np.array([np.inf, nan, 1.0], np.float32)) == 1
    assert g.greedy_next(np.array([-np.inf, -nan, -1.0], np.float32)) == 2
    assert g.greedy_next(np.array([-nan, -np.inf], np.float32)) == 1


def test_moe_route_weights():
    rng = np.random.default_rng(4)
    v = (rng.standard_normal(16) * 3).astype(np.float32)
    # renorm: softmax over the chosen k; with k = all, they sum to 1
    _, w = g.moe_route(v, 16, renorm=True)
    assert abs(float(np.sum(w.astype(np.float64))) - 1.0) < 1e-6
    ids, w = g.moe_route(v, 3, renorm=True)
    top = v[ids].astype(np.float64)
    ref = np.exp(top - top.max()) / np.exp(top - top.max()).sum()
    assert np.allclose(w, ref, rtol=1e-6)
    # OLMoE: the chosen entries of a softmax over all experts (not renormalised)
    ids, w = g.moe_route(v, 3, renorm=False)
    full = np.exp(v.astype(np.float64) - v.max()) / np.exp(v.astype(np.float64) - v.max()).sum()
    assert np.allclose(w, full[ids], rtol=1e-6)
    assert float(np.sum(w)) < 1.0


def test_moe_ffn_single_expert_is_dense_ffn():
    rng = np.random.default_rng(5)
    d, f, E = 8, 12, 3
    gate = [rng.standard_normal((f, d)) for _ in range(E)]
    up = [rng.standard_normal((f, d)) for _ in range(E)]
    down = [rng.standard_normal((d, f)) for _ in range(E)]
    x = rng.standard_normal(d)
    dense = down[1] @ (gate[1] @ x / (1 + np.exp(-(gate[1] @ x))) * (up[1] @ x))
    assert np.allclose(g.moe_ffn(x, [1], [1.0], gate, up, down), dense)
    # linear in the weights, biases added where the reference adds them
    bd = rng.standard_normal((E, d))
    two = g.moe_ffn(x, [1, 2], [0.25, 0.5], gate, up, down, down_b=bd)
    one1 = g.moe_ffn(x, [1], [1.0], gate, up, down, down_b=bd)
    one2 = g.moe_ffn(x, [2], [1.0], gate, up, down, down_b=bd)
    assert np.allclose(two, 0.25 * one1 + 0.5 * one2)
    assert np.allclose(one1, dense + bd[1])
