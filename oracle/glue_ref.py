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

Pinned by tests/test_glue_ref.py with closed forms: rope at pos 0 is the
identity and preserves each pair's norm at any pos; rms_norm of a constant
vector is sign(x) * w (up to the eps term); softmax rows sum to 1 without a sink
and to 1 - p_sink with one; attention over one cached token returns that
token's value; swiglu(0, .) = 0 and swiglu(g, 1) = silu(g); the OAI form
clamps at 7.
"""
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
