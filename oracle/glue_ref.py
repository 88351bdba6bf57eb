"""float64 restatement of Quartz's decode-step glue kernels and of the dense
(LLaMA) path of forward_gpu_step.

TEST INFRASTRUCTURE ONLY: the checker for saient_quartz_amd/csrc/qh_glue.hip and
the step built on it; only tests/ import it.

  rms_norm        src/cuda_kernels.cu:563-575   x * rsqrt(mean(x^2) + 1e-5) * w
  rope_yarn       src/cuda_kernels.cu:577-605   NORM (2i, 2i+1) / NEOX (i, i+d/2) pairs,
                                                YaRN ramp beta_fast 32, beta_slow 1
  kv_append       src/cuda_kernels.cu:609-619
  attention       src/cuda_kernels.cu:1199-1266 scores * scale, softmax with sink in
                                                the normaliser only, value sums;
                                                kv_head = head * n_kv / n_heads
  swiglu(_oai)    src/cuda_kernels.cu:660-676
  forward_step    src/cuda.rs:556-837 (dense FFN, no biases / QK-norm / sliding
                                       window): the sequence of the above around
                                       the seven GEMVs and the head.
  moe_route       src/main.rs:964-993 (= src/cuda.rs:684-701): router logits
                                       (+ bias), sort by total_cmp descending,
                                       top k, softmax over the k (renorm) or over
                                       all experts (OLMoE); weights in f32 as
                                       the reference computes them.
  greedy_next     src/main.rs:1684-1692: the temperature <= 0 arm, max_by over
                                       total_cmp (the last of equal maxima).
  moe_ffn         src/main.rs:995-1040: per chosen expert gate/up (+ biases),
                                       SwiGLU (plain or OAI), down (+ bias),
                                       output += w * down, in float64.

Pinned by tests/test_glue_ref.py with closed forms: rope at pos 0 is the
identity and preserves each pair's norm at any pos; rms_norm of a constant
vector is sign(x) * w (up to the eps term); softmax rows sum to 1 without a sink
and to 1 - p_sink with one; attention over one cached token returns that
token's value; swiglu(0, .) = 0 and swiglu(g, 1) = silu(g); the OAI form
clamps at 7; moe_route's order against numpy's stable argsort on distinct
values, -0 < +0 and NaN placement by sign, k = n_exp weights summing to 1, and
the OLMoE weights against a float64 softmax; greedy_next against numpy's
argmax on distinct finite values, with ties, +-0, +-inf and NaNs by hand; moe_ffn with one expert of weight
1 against the dense FFN.  forward_step as a composition is pinned by
tests/test_forward_step_ref.py: at pos 0 the output ignores q/k and attention
returns each group's v; zero o/down weights keep the hidden state and leave
logits = head @ rms_norm; the FFN block uses ffn_norm and silu(gate) * up; the
pos 1 attention is the closed-form two-row softmax; K/V rows land at pos only;
two layers compose in order.
"""
import struct

import numpy as np


def rms_norm(x, w):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + 1e-5) * np.asarray(w, np.float64)


def rope_yarn(x, n_heads, head_dim, pos, theta, yarn_scale=1.0, yarn_orig_ctx=0, neox=False):
    x = np.array(x, np.float64).reshape(n_heads, head_dim)
    half = head_dim // 2
    i = np.arange(half, dtype=np.float64)
    std_inv = 1.0 / np.power(theta, 2.0 * i / head_dim)
    eff = std_inv
    if yarn_scale > 1.0 and yarn_orig_ctx > 0:
        hfw, lfw = yarn_orig_ctx / 32.0, yarn_orig_ctx / 1.0
        wavelen = 2.0 * np.pi / std_inv
        ramp = np.clip((lfw - wavelen) / (lfw - hfw), 0.0, 1.0)
        eff = ramp * std_inv + (1.0 - ramp) * (std_inv / yarn_scale)
    ang = pos * eff
    c, s = np.cos(ang), np.sin(ang)
    i0 = i.astype(int) if neox else 2 * i.astype(int)
    i1 = i0 + half if neox else i0 + 1
    x0, x1 = x[:, i0].copy(), x[:, i1].copy()
    x[:, i0] = x0 * c - x1 * s
    x[:, i1] = x0 * s + x1 * c
    return x.reshape(-1)


def softmax_sink(x, sink=None):
    x = np.asarray(x, np.float64)
    m = x.max() if x.size else -1e30
    if sink is not None and sink > -1e29:
        m = max(m, sink)
    e = np.exp(x - m)
    tot = e.sum() + (np.exp(sink - m) if sink is not None and sink > -1e29 else 0.0)
    return e / tot


def attention(q, k_cache, v_cache, n_heads, n_kv, seq, head_dim, kv_dim, scale, sinks=None):
    """-> (scores [n_heads, seq] after softmax, out [n_heads * head_dim])."""
    q = np.asarray(q, np.float64).reshape(n_heads, head_dim)
    kc = np.asarray(k_cache, np.float64).reshape(-1, kv_dim)[:seq]
    vc = np.asarray(v_cache, np.float64).reshape(-1, kv_dim)[:seq]
    probs = np.zeros((n_heads, seq))
    out = np.zeros((n_heads, head_dim))
    for h in range(n_heads):
        kvh = h * n_kv // n_heads
        k = kc[:, kvh * head_dim:(kvh + 1) * head_dim]
        v = vc[:, kvh * head_dim:(kvh + 1) * head_dim]
        probs[h] = softmax_sink(k @ q[h] * scale, None if sinks is None else float(sinks[h]))
        out[h] = probs[h] @ v
    return probs, out.reshape(-1)


def swiglu(g, u):
    g = np.asarray(g, np.float64)
    return g / (1.0 + np.exp(-g)) * np.asarray(u, np.float64)


def swiglu_oai(g, u):
    x = np.minimum(np.asarray(g, np.float64), 7.0)
    y = np.clip(np.asarray(u, np.float64), -7.0, 7.0)
    return x / (1.0 + np.exp(-1.702 * x)) * (y + 1.0)


def forward_step(hidden, pos, layers, head_w, out_norm, kv, cfg):
    """One dense decode step in float64.  hidden: the token's embedding row;
    layers: list of dicts with dequantized f64 matrices q, k, v, o, gate, up,
    down ([out, in]) and norms attn_norm, ffn_norm; kv: list of [k_cache,
    v_cache] f64 arrays [max_seq, kv_dim], updated in place; cfg: dict with
    n_heads, n_kv, head_dim, theta, neox.  Returns (logits, hidden)."""
    h, nkv, hd = cfg["n_heads"], cfg["n_kv"], cfg["head_dim"]
    kvd = nkv * hd
    x = np.array(hidden, np.float64)
    for l, L in enumerate(layers):
        xn = rms_norm(x, L["attn_norm"])
        q = L["q"] @ xn
        k = L["k"] @ xn
        v = L["v"] @ xn
        q = rope_yarn(q, h, hd, pos, cfg["theta"], neox=cfg["neox"])
        k = rope_yarn(k, nkv, hd, pos, cfg["theta"], neox=cfg["neox"])
        kv[l][0][pos] = k
        kv[l][1][pos] = v
        _, att = attention(q, kv[l][0], kv[l][1], h, nkv, pos + 1, hd, kvd, 1.0 / np.sqrt(hd))
        x = x + L["o"] @ att
        xn = rms_norm(x, L["ffn_norm"])
        x = x + L["down"] @ swiglu(L["gate"] @ xn, L["up"] @ xn)
    return head_w @ rms_norm(x, out_norm), x


def total_order_key(v):
    """f32::total_cmp as an integer key (Rust's core::f32::total_cmp: flip the
    magnitude bits of negative values, then compare as signed 32-bit)."""
    b = struct.unpack("<i", struct.pack("<f", float(np.float32(v))))[0]
    return b ^ ((b >> 31) & 0x7FFFFFFF)


def greedy_next(logits):
    """Greedy token (src/main.rs:1684-1692): Iterator::max_by with total_cmp,
    which keeps the later element when two compare equal, so among equal
    maxima the last index wins; NaN with the sign bit clear orders above +inf."""
    best, best_key = 0, None
    for i, v in enumerate(np.asarray(logits, np.float32)):
        k = total_order_key(v)
        if best_key is None or k >= best_key:
            best, best_key = i, k
    return best


def moe_route(logits, k, renorm=True, bias=None):
    """Top-k experts and weights of one token (src/main.rs:964-993), f32
    arithmetic as the reference.  Ties keep the lower index first (the
    reference's sort_unstable_by leaves them unspecified).  Returns (ids, w)."""
    v = np.asarray(logits, np.float32).copy()
    if bias is not None:
        v = (v + np.asarray(bias, np.float32)).astype(np.float32)
    order = sorted(range(len(v)), key=lambda i: (-total_order_key(v[i]), i))
    top = order[:k]
    tv = v[top]
    with np.errstate(over="ignore", invalid="ignore"):
        if renorm:
            mx = np.float32(-np.inf)
            for t in tv:
                mx = t if np.isnan(mx) else (mx if np.isnan(t) else max(mx, t))
            e = np.exp((tv - mx).astype(np.float32)).astype(np.float32)
            s = np.float32(0)
            for x in e:
                s = np.float32(s + x)
        else:
            mx = np.float32(-np.inf)
            for t in v:
                mx = t if np.isnan(mx) else (mx if np.isnan(t) else max(mx, t))
            s = np.float32(0)
            for x in v:
                s = np.float32(s + np.float32(np.exp(np.float32(x - mx))))
            e = np.exp((tv - mx).astype(np.float32)).astype(np.float32)
        w = (e / s).astype(np.float32)
    return np.array(top, np.int64), w


def moe_ffn(x, ids, w, gate, up, down, gate_b=None, up_b=None, down_b=None, oai=False):
    """One token's MoE output in float64 (src/main.rs:995-1040): gate/up/down are
    per-expert dequantized f64 matrices ([E] lists of [f, d] / [d, f]); biases
    [E][f] / [E][d] or None."""
    x = np.asarray(x, np.float64)
    out = np.zeros(down[0].shape[0])
    for e, rw in zip(ids, w):
        g = gate[e] @ x + (gate_b[e] if gate_b is not None else 0.0)
        u = up[e] @ x + (up_b[e] if up_b is not None else 0.0)
        h = swiglu_oai(g, u) if oai else swiglu(g, u)
        o = down[e] @ h + (down_b[e] if down_b is not None else 0.0)
        out += float(rw) * o
    return out
