"""Pins of the oracle's forward_step (oracle/glue_ref.py) as a composition: closed
forms and structural properties of the dense decode step (src/cuda.rs:556-837),
each chosen so that a plausible wiring mistake fails one of them:

  * at position 0 attention over the one cached row returns that row's v, so the
    layer's output does not depend on the q/k weights and equals
    x + O [v of kv head h * n_kv / n_heads for each q head h] (a wrong GQA
    mapping, or q/k leaking into the result, fails);
  * zero o and down weights leave the hidden state unchanged and the logits are
    head @ (x / rms(x) * out_norm) (a lost residual or final norm fails);
  * with o zero the layer adds down @ (silu(gate xn) * up xn) with xn normed by
    ffn_norm (swapped gate/up or the attention norm fails);
  * at position 1 the attention of each head is the closed-form two-row softmax
    (a wrong score scale or cache row fails);
  * the K/V cache gets rope(k) and v at row pos and nothing else;
  * two layers are the first layer followed by the second (layer order).
The expected values are built from numpy products and explicit formulas, not from
forward_step's own helpers beyond rms_norm / rope_yarn, which are pinned in
tests/test_glue_ref.py.
"""
import sys
from pathlib import Path

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import glue_ref as g  # noqa: E402

CFG = {"n_heads": 8, "n_kv": 2, "head_dim": 8, "theta": 10000.0, "neox": False}
D, F, V = 64, 96, 50
KVD = CFG["n_kv"] * CFG["head_dim"]


def _layer(rng, **zero):
    L = {"q": rng.standard_normal((D, D)) / 8, "k": rng.standard_normal((KVD, D)) / 8,
         "v": rng.standard_normal((KVD, D)) / 8, "o": rng.standard_normal((D, D)) / 8,
         "gate": rng.standard_normal((F, D)) / 8, "up": rng.standard_normal((F, D)) / 8,
         "down": rng.standard_normal((D, F)) / 8,
         "attn_norm": rng.uniform(0.5, 1.5, D), "ffn_norm": rng.uniform(0.5, 1.5, D)}
    for name in zero:
        L[name] = np.zeros_like(L[name])
    return L


def _kv(n_layers, rng, max_seq=4):
    return [[rng.standard_normal((max_seq, KVD)), rng.standard_normal((max_seq, KVD))] for _ in range(n_layers)]


def _rms(x, w):
    return x / np.sqrt(np.mean(x * x) + 1e-5) * w


def _silu(z):
    return z / (1.0 + np.exp(-z))


def _rel(a, b):
    return np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300)


def test_pos0_attention_is_v_and_ignores_qk():
    rng = np.random.default_rng(1)
    x = rng.standard_normal(D)
    L = _layer(rng, gate=1, up=1, down=1)
    head, on = rng.standard_normal((V, D)), rng.uniform(0.5, 1.5, D)
    _, got = g.forward_step(x, 0, [L], head, on, _kv(1, rng), CFG)
    v = L["v"] @ _rms(x, L["attn_norm"])
    hd, nh, nkv = CFG["head_dim"], CFG["n_heads"], CFG["n_kv"]
    att = np.concatenate([v[(h * nkv // nh) * hd:(h * nkv // nh + 1) * hd] for h in range(nh)])
    assert _rel(got, x + L["o"] @ att) < 1e-12
    L2 = dict(L, q=rng.standard_normal((D, D)), k=rng.standard_normal((KVD, D)))
    _, got2 = g.forward_step(x, 0, [L2], head, on, _kv(1, rng), CFG)
    assert _rel(got2, got) < 1e-12


def test_zero_blocks_keep_hidden_and_head_norm():
    rng = np.random.default_rng(2)
    x = rng.standard_normal(D)
    L = _layer(rng, o=1, down=1)
    head, on = rng.standard_normal((V, D)), rng.uniform(0.5, 1.5, D)
    logits, hid = g.forward_step(x, 2, [L], head, on, _kv(1, rng), CFG)
    assert np.array_equal(hid, x)
    assert _rel(logits, head @ _rms(x, on)) < 1e-12


def test_ffn_block_uses_ffn_norm_and_silu_gate():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(D)
    L = _layer(rng, o=1)
    head, on = rng.standard_normal((V, D)), rng.uniform(0.5, 1.5, D)
    _, got = g.forward_step(x, 1, [L], head, on, _kv(1, rng), CFG)
    xn = _rms(x, L["ffn_norm"])
    assert _rel(got, x + L["down"] @ (_silu(L["gate"] @ xn) * (L["up"] @ xn))) < 1e-12
    # the plausible miswirings give a different result
    assert _rel(got, x + L["down"] @ (_silu(L["up"] @ xn) * (L["gate"] @ xn))) > 1e-3
    xa = _rms(x, L["attn_norm"])
    assert _rel(got, x + L["down"] @ (_silu(L["gate"] @ xa) * (L["up"] @ xa))) > 1e-3


def test_pos1_two_row_softmax_and_cache_rows():
    rng = np.random.default_rng(4)
    x = rng.standard_normal(D)
    L = _layer(rng, gate=1, up=1, down=1)
    head, on = rng.standard_normal((V, D)), rng.uniform(0.5, 1.5, D)
    kv = _kv(1, rng)
    k0, v0 = kv[0][0][0].copy(), kv[0][1][0].copy()
    rest = [kv[0][0][2:].copy(), kv[0][1][2:].copy()]
    _, got = g.forward_step(x, 1, [L], head, on, kv, CFG)
    hd, nh, nkv = CFG["head_dim"], CFG["n_heads"], CFG["n_kv"]
    xn = _rms(x, L["attn_norm"])
    q = g.rope_yarn(L["q"] @ xn, nh, hd, 1, CFG["theta"])
    k1 = g.rope_yarn(L["k"] @ xn, nkv, hd, 1, CFG["theta"])
    v1 = L["v"] @ xn
    assert _rel(kv[0][0][1], k1) < 1e-15 and np.array_equal(kv[0][1][1], v1)
    assert np.array_equal(kv[0][0][0], k0) and np.array_equal(kv[0][1][0], v0)
    assert np.array_equal(kv[0][0][2:], rest[0]) and np.array_equal(kv[0][1][2:], rest[1])
    att = []
    for h in range(nh):
        kh = h * nkv // nh
        sl = slice(kh * hd, (kh + 1) * hd)
        qh = q[h * hd:(h + 1) * hd]
        s0, s1 = qh @ k0[sl] / np.sqrt(hd), qh @ k1[sl] / np.sqrt(hd)
        p1 = 1.0 / (1.0 + np.exp(s0 - s1))  # two-row softmax
        att.append((1.0 - p1) * v0[sl] + p1 * v1[sl])
    assert _rel(got, x + L["o"] @ np.concatenate(att)) < 1e-12


def test_two_layers_compose_in_order():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(D)
    L1, L2 = _layer(rng), _layer(rng)
    head, on = rng.standard_normal((V, D)), rng.uniform(0.5, 1.5, D)
    kv = _kv(2, rng)
    kv_a = [[a.copy() for a in kv[0]]]
    kv_b = [[a.copy() for a in kv[1]]]
    logits, got = g.forward_step(x, 1, [L1, L2], head, on, kv, CFG)
    _, h1 = g.forward_step(x, 1, [L1], head, on, kv_a, CFG)
    l2, h2 = g.forward_step(h1, 1, [L2], head, on, kv_b, CFG)
    assert np.array_equal(got, h2) and np.array_equal(logits, l2)
    _, swapped = g.forward_step(x, 1, [L2, L1], head, on, [[a.copy() for a in kv[1]], [a.copy() for a in kv[0]]], CFG)
    assert _rel(swapped, got) > 1e-6
