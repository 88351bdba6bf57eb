"""Decode-step drivers over the C ABI, with random-init weights generated on the
device (seeded).

  DecodeStep   the weight GEMVs/GEMMs of a Llama-3-8B Q4_K_M step alone
               (activations fixed): weight streaming, >99% of a step's bytes.
  MoeLayer     a Mixtral-shaped expert layer's GEMMs over fixed gathered tokens.
  MoeStep      a full MoE FFN for a batch of tokens: router GEMM, device-side
               top-k routing, gather, expert GEMMs, SwiGLU, weighted combine
               (moe_ffn, src/main.rs:952-1043; src/cuda.rs:667-798).
  ForwardStep  forward_gpu_step (src/cuda.rs:507-851, dense path) end to end for
               one token: embedding, 32 layers of fused GEMVs, attention and
               glue, the head.
  BatchStep    the same for N sequences in lockstep on batched GEMMs.

Layer shapes (forward_gpu_step's order, src/cuda.rs:556-562, :647, :773-788):
  q 4096x4096 Q4_K, k 1024x4096 Q4_K, v 1024x4096 Q6_K, o 4096x4096 Q4_K,
  gate 14336x4096 Q4_K, up 14336x4096 Q4_K, down 4096x14336 Q6_K;
then the output head 128256x4096 Q6_K.  32 layers: 4,875,853,824 weight bytes.
"""
import ctypes as C
from dataclasses import dataclass

import torch

from . import synth_device
from .api import check, lib
from .host import (gemm_group_norm_async, gemm_grouped_async, gemm_grouped_ex_async, gemm_moe_async, gemm_moe_dev_async,
                   gemv_group_async, gemv_multi_async)

Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_S = 12, 13, 14, 16, 21


def _write_state(L, state, values, stream):
    """hip_h2d_async of int32 values into a step's device state, ordered on the
    stream (a pageable source: the call returns once it is read)."""
    buf = (C.c_int * len(values))(*[int(v) for v in values])
    check("hip_h2d_async", L.hip_h2d_async(state.data_ptr(), buf, 4 * len(values), _stream_ptr(stream)))
    return buf


def _stream_ptr(stream):
    """A torch stream, a raw hipStream_t (int, e.g. from hip_stream_create) or
    None (torch's current stream) -> the raw handle the C ABI takes."""
    if isinstance(stream, int):
        return stream
    return (stream or torch.cuda.current_stream()).cuda_stream


@dataclass(frozen=True)
class Shape:
    hidden: int = 4096
    kv_dim: int = 1024  # 8 kv heads x 128
    ffn: int = 14336
    vocab: int = 128256
    layers: int = 32

    def layer_mats(self):
        """(name, ggml_type, out_dim, in_dim) in call order."""
        h, kv, f = self.hidden, self.kv_dim, self.ffn
        return [("q", Q4_K, h, h), ("k", Q4_K, kv, h), ("v", Q6_K, kv, h), ("o", Q4_K, h, h),
                ("gate", Q4_K, f, h), ("up", Q4_K, f, h), ("down", Q6_K, h, f)]

    def weight_bytes(self) -> int:
        from . import type_size
        per_layer = sum(type_size(t, o * i) for _, t, o, i in self.layer_mats())
        return per_layer * self.layers + type_size(Q6_K, self.vocab * self.hidden)


class DecodeStep:
    def __init__(self, shape: Shape = Shape(), n_max: int = 16, seed: int = 20261204):
        self.shape = shape
        self.L = lib()
        s = shape
        self.layers = []
        for l in range(s.layers):
            mats = []
            for j, (name, t, o, i) in enumerate(s.layer_mats()):
                mats.append((t, synth_device.weights(t, o, i, seed + 16 * l + j), o, i))
            self.layers.append(mats)
        self.head = (Q6_K, synth_device.weights(Q6_K, s.vocab, s.hidden, seed - 1), s.vocab, s.hidden)
        g = torch.Generator(device="cuda")
        g.manual_seed(seed + 7)
        # token-major activations: x[n][hidden] for every GEMV but down, xf[n][ffn] for down
        self.x = torch.randn(n_max, s.hidden, device="cuda", generator=g)
        self.xf = torch.randn(n_max, s.ffn, device="cuda", generator=g)
        self.y = {name: torch.empty(n_max, o, device="cuda") for name, _, o, _ in s.layer_mats()}
        self.logits = torch.empty(n_max, s.vocab, device="cuda")
        self.n_max = n_max

    def _mm(self, t, w, out, o, i, n, sp):
        x = self.x if i == self.shape.hidden else self.xf
        if n == 1:
            check("hip_gemv_async", self.L.hip_gemv_async(t, w.data_ptr(), x.data_ptr(), out.data_ptr(),
                                                          i, o, sp))
        else:
            check("hip_gemm_async", self.L.hip_gemm_async(t, w.data_ptr(), x.data_ptr(), out.data_ptr(),
                                                          i, o, n, sp))

    def issue(self, n: int = 1, stream=None, fuse: bool = True):
        """Enqueue one decode step's GEMVs for n tokens on `stream` (torch stream).
        With `fuse`, the projections that share x and type go out as one call
        each: q+k (Q4_K) and gate+up (Q4_K), through hip_gemv_multi at n = 1 and
        hip_gemm_grouped (one x digitisation, one weight launch) at n > 1."""
        assert 1 <= n <= self.n_max
        sp = _stream_ptr(stream)
        names = [m[0] for m in self.shape.layer_mats()]
        for mats in self.layers:
            by = dict(zip(names, mats))
            if fuse:
                for group in (("q", "k"), ("v",), ("o",), ("gate", "up"), ("down",)):
                    if len(group) == 1:
                        t, w, o, i = by[group[0]]
                        self._mm(t, w, self.y[group[0]], o, i, n, sp)
                        continue
                    t, _, _, i = by[group[0]]
                    x = self.x if i == self.shape.hidden else self.xf
                    if n == 1:
                        gemv_multi_async(self.L, t, [by[g][1].data_ptr() for g in group],
                                         [self.y[g].data_ptr() for g in group], [by[g][2] for g in group],
                                         x.data_ptr(), i, sp)
                    else:
                        gemm_grouped_async(self.L, t, [by[g][1].data_ptr() for g in group],
                                           [x.data_ptr()] * len(group), [self.y[g].data_ptr() for g in group],
                                           [n] * len(group), [by[g][2] for g in group], i, sp)
                continue
            for name, (t, w, o, i) in zip(names, mats):
                self._mm(t, w, self.y[name], o, i, n, sp)
        t, w, o, i = self.head
        self._mm(t, w, self.logits, o, i, n, sp)


class MoeLayer:
    """Mixtral-8x7B-shaped MoE expert layer: 8 experts,
    each gate/up 14336x4096 and down 4096x14336 in one IQ type, 16 tokens
    gathered per expert (top-2 routing of 64 tokens).  Each projection's experts
    are stacked in one buffer (expert e at base + e * slice bytes, as
    src/cuda.rs:250-258 addresses them).  A step runs every expert's three GEMMs:
    grouped (default), gate and up of all experts in one hip_gemm_grouped call
    (each expert's x digitised once for both) and down in one hip_gemm_moe call;
    or per expert, three hip_gemm calls each, as the reference's loop does
    (src/cuda.rs:667-798).  The router, the gather/scatter and swiglu are glue
    outside this library: the gathered activations are fixed buffers."""

    def __init__(self, ggml_type: int, experts: int = 8, tokens: int = 16, hidden: int = 4096, ffn: int = 14336,
                 seed: int = 20261205):
        from . import type_size
        self.t, self.E, self.n, self.h, self.f = ggml_type, experts, tokens, hidden, ffn
        self.L = lib()
        self.slice = type_size(ggml_type, ffn * hidden)
        self.wg = torch.cat([synth_device.weights(ggml_type, ffn, hidden, seed + 3 * e) for e in range(experts)])
        self.wu = torch.cat([synth_device.weights(ggml_type, ffn, hidden, seed + 3 * e + 1) for e in range(experts)])
        self.wd = torch.cat([synth_device.weights(ggml_type, hidden, ffn, seed + 3 * e + 2) for e in range(experts)])
        g = torch.Generator(device="cuda")
        g.manual_seed(seed - 1)
        self.x = torch.randn(experts, tokens, hidden, device="cuda", generator=g)
        self.hbuf = torch.randn(experts, tokens, ffn, device="cuda", generator=g)
        self.gate = torch.empty(experts, tokens, ffn, device="cuda")
        self.up = torch.empty(experts, tokens, ffn, device="cuda")
        self.down = torch.empty(experts, tokens, hidden, device="cuda")

    def weight_bytes(self) -> int:
        return 3 * self.E * self.slice

    def expert(self, w, e):
        return w.data_ptr() + e * self.slice

    def issue(self, stream=None, grouped: bool = True):
        sp = _stream_ptr(stream)
        t, n, h, f, E = self.t, self.n, self.h, self.f, self.E
        if grouped:
            xs = [self.x[e].data_ptr() for e in range(E)]
            gemm_grouped_async(self.L, t, [self.expert(self.wg, e) for e in range(E)] +
                               [self.expert(self.wu, e) for e in range(E)], xs + xs,
                               [self.gate[e].data_ptr() for e in range(E)] + [self.up[e].data_ptr() for e in range(E)],
                               [n] * (2 * E), [f] * (2 * E), h, sp)
            gemm_moe_async(self.L, t, self.wd.data_ptr(), list(range(E)), [n * e for e in range(E + 1)],
                           self.hbuf.data_ptr(), self.down.data_ptr(), f, h, sp)
            return
        for e in range(E):
            check("hip_gemm_async", self.L.hip_gemm_async(t, self.expert(self.wg, e), self.x[e].data_ptr(),
                                                          self.gate[e].data_ptr(), h, f, n, sp))
            check("hip_gemm_async", self.L.hip_gemm_async(t, self.expert(self.wu, e), self.x[e].data_ptr(),
                                                          self.up[e].data_ptr(), h, f, n, sp))
            check("hip_gemm_async", self.L.hip_gemm_async(t, self.expert(self.wd, e), self.hbuf[e].data_ptr(),
                                                          self.down[e].data_ptr(), f, h, n, sp))


class MoeStep:
    """One MoE FFN for n tokens, all on the device: moe_ffn (src/main.rs:952-1043)
    and its GPU twin (src/cuda.rs:667-798) for any expert count, top-k and types.

      logits = router_w x (+ router_b)       hip_gemm (F32)
      ids, w = top-k + softmax               hip_moe_route (renorm or OLMoE form)
      slots  = expert-ordered (token, j)     hip_moe_plan
      xg     = x[slot_tok]                   hip_moe_gather
      g, u   = gate/up of each slot's expert hip_gemm_moe_dev (token ranges read on
                                             the device; other types: tok_off copied
                                             back, hip_gemm_grouped / hip_gemm_moe)
      act    = swiglu(g + bg, u + bu)        hip_moe_swiglu (plain or OAI clamp; the plain
                                             form without biases is folded into the
                                             device-driven down GEMM)
      yg     = down act                      hip_gemm_moe_dev / hip_gemm_moe
      out    = (out +) sum_j w * (yg + bd)   hip_moe_combine

    Weights: wg, wu [E][f][d] and wd [E][d][f] stacked GGUF bytes (expert e at
    e * slice, src/cuda.rs:250-258); router_w [E][d] f32; biases optional
    [E][f] / [E][d] / [E].  For the matrix-core types there is no host round
    trip (the step can be captured in a HIP graph); for the others tok_off (E + 1
    ints) comes back at the point where the reference copies the router logits
    back."""

    def __init__(self, types, wg, wu, wd, router_w, E, k, d, f, n_max, renorm=True, oai=False, router_b=None,
                 gate_b=None, up_b=None, down_b=None):
        from . import type_size
        self.L = lib()
        self.tg, self.tu, self.td = types
        self.wg, self.wu, self.wd, self.rw = wg, wu, wd, router_w
        self.E, self.k, self.d, self.f, self.n_max = E, k, d, f, n_max
        self.renorm, self.oai = int(renorm), int(oai)
        self.rb, self.gb, self.ub, self.db = router_b, gate_b, up_b, down_b
        self.sg, self.su = type_size(self.tg, f * d), type_size(self.tu, f * d)
        dev, S = "cuda", n_max * k
        self.logits = torch.empty(n_max, E, device=dev)
        self.ids = torch.empty(n_max, k, dtype=torch.int32, device=dev)
        self.wts = torch.empty(n_max, k, device=dev)
        self.tok_off = torch.empty(E + 1, dtype=torch.int32, device=dev)
        self.slot_of = torch.empty(n_max, k, dtype=torch.int32, device=dev)
        self.slot_tok = torch.empty(S, dtype=torch.int32, device=dev)
        self.slot_exp = torch.empty(S, dtype=torch.int32, device=dev)
        self.xg = torch.empty(S, d, device=dev)
        self.g = torch.empty(S, f, device=dev)
        self.u = torch.empty(S, f, device=dev)
        self.act = torch.empty(S, f, device=dev)
        self.yg = torch.empty(S, d, device=dev)
        self.tok_off_host = torch.empty(E + 1, dtype=torch.int32, pin_memory=True)
        # the expert GEMMs read the token ranges on the device (matrix-core types);
        # otherwise tok_off comes back to the host to build them
        mc = (Q4_K, Q5_K, Q6_K, IQ3_S, IQ2_XXS)
        self.device_driven = (all(t in mc for t in types) and d % 256 == 0 and f % 256 == 0)

    @staticmethod
    def _p(t):
        return t.data_ptr() if t is not None else None

    def issue(self, x, out, n, accumulate=False, stream=None):
        """x: device f32 [n][d] (normed activations), out: device f32 [n][d]."""
        assert 0 < n <= self.n_max
        st = stream or torch.cuda.current_stream()
        sp = st.cuda_stream
        L, E, k, d, f = self.L, self.E, self.k, self.d, self.f
        xp = x.data_ptr()
        check("hip_gemm_async", L.hip_gemm_async(0, self.rw.data_ptr(), xp, self.logits.data_ptr(), d, E, n, sp))
        check("hip_moe_route_async",
              L.hip_moe_route_async(self.logits.data_ptr(), self._p(self.rb), n, E, k, self.renorm,
                                    self.ids.data_ptr(), self.wts.data_ptr(), sp))
        check("hip_moe_plan_async",
              L.hip_moe_plan_async(self.ids.data_ptr(), n, k, E, self.tok_off.data_ptr(), self.slot_of.data_ptr(),
                                   self.slot_tok.data_ptr(), self.slot_exp.data_ptr(), sp))
        S = n * k  # every token takes k slots
        check("hip_moe_gather_async", L.hip_moe_gather_async(self.xg.data_ptr(), xp, self.slot_tok.data_ptr(), S, d,
                                                             sp))
        if self.device_driven:
            # token ranges read on the device: no host round trip (graph-capturable)
            if self.tg == self.tu:
                gemm_moe_dev_async(L, self.tg, [self.wg.data_ptr(), self.wu.data_ptr()],
                                   [self.g.data_ptr(), self.u.data_ptr()], E, self.tok_off.data_ptr(), n,
                                   self.xg.data_ptr(), d, f, sp)
            else:
                for t, w_, y_ in ((self.tg, self.wg, self.g), (self.tu, self.wu, self.u)):
                    gemm_moe_dev_async(L, t, [w_.data_ptr()], [y_.data_ptr()], E, self.tok_off.data_ptr(), n,
                                       self.xg.data_ptr(), d, f, sp)
            if self.gb is None and self.ub is None and not self.oai:
                # plain SwiGLU folded into the down GEMM's x digitisation
                gemm_moe_dev_async(L, self.td, [self.wd.data_ptr()], [self.yg.data_ptr()], E, self.tok_off.data_ptr(),
                                   n, self.g.data_ptr(), f, d, sp, x_up_ptr=self.u.data_ptr())
            else:
                check("hip_moe_swiglu_async",
                      L.hip_moe_swiglu_async(self.act.data_ptr(), self.g.data_ptr(), self.u.data_ptr(),
                                             self._p(self.gb), self._p(self.ub), self.slot_exp.data_ptr(), S, f,
                                             self.oai, sp))
                gemm_moe_dev_async(L, self.td, [self.wd.data_ptr()], [self.yg.data_ptr()], E, self.tok_off.data_ptr(),
                                   n, self.act.data_ptr(), f, d, sp)
            check("hip_moe_combine_async",
                  L.hip_moe_combine_async(out.data_ptr(), self.yg.data_ptr(), self.slot_of.data_ptr(),
                                          self.wts.data_ptr(), self.ids.data_ptr(), self._p(self.db), n, k, d,
                                          int(accumulate), sp))
            return
        self.tok_off_host.copy_(self.tok_off, non_blocking=True)
        st.synchronize()
        off = self.tok_off_host.tolist()
        sel = [e for e in range(E) if off[e + 1] > off[e]]
        s_off = [off[e] for e in sel] + [off[E]]
        if self.tg == self.tu and 2 * len(sel) <= 16:
            # gate and up of every selected expert in one grouped launch (x digitised once per expert)
            xs = [self.xg.data_ptr() + 4 * d * off[e] for e in sel]
            gemm_grouped_async(L, self.tg, [self.wg.data_ptr() + e * self.sg for e in sel] +
                               [self.wu.data_ptr() + e * self.su for e in sel], xs + xs,
                               [self.g.data_ptr() + 4 * f * off[e] for e in sel] +
                               [self.u.data_ptr() + 4 * f * off[e] for e in sel],
                               [off[e + 1] - off[e] for e in sel] * 2, [f] * (2 * len(sel)), d, sp)
        else:
            gemm_moe_async(L, self.tg, self.wg.data_ptr(), sel, s_off, self.xg.data_ptr(), self.g.data_ptr(), d, f, sp)
            gemm_moe_async(L, self.tu, self.wu.data_ptr(), sel, s_off, self.xg.data_ptr(), self.u.data_ptr(), d, f, sp)
        check("hip_moe_swiglu_async",
              L.hip_moe_swiglu_async(self.act.data_ptr(), self.g.data_ptr(), self.u.data_ptr(), self._p(self.gb),
                                     self._p(self.ub), self.slot_exp.data_ptr(), S, f, self.oai, sp))
        gemm_moe_async(L, self.td, self.wd.data_ptr(), sel, s_off, self.act.data_ptr(), self.yg.data_ptr(), f, d, sp)
        check("hip_moe_combine_async",
              L.hip_moe_combine_async(out.data_ptr(), self.yg.data_ptr(), self.slot_of.data_ptr(),
                                      self.wts.data_ptr(), self.ids.data_ptr(), self._p(self.db), n, k, d,
                                      int(accumulate), sp))


@dataclass(frozen=True)
class ModelConfig:
    """Dense LLaMA-family shape of forward_gpu_step (src/cuda.rs:507-851).  The
    default is Llama-3-8B Q4_K_M: q/k/o/gate/up and the embedding in Q4_K, v,
    down and the output head in Q6_K; RoPE NORM pairing (rope_neox false),
    theta 500000, no YaRN, no biases, no QK-norm, no sliding window."""
    hidden: int = 4096
    n_heads: int = 32
    n_kv: int = 8
    head_dim: int = 128
    ffn: int = 14336
    vocab: int = 128256
    layers: int = 32
    theta: float = 500000.0
    neox: int = 0
    max_seq: int = 1024
    types: tuple = (("q", Q4_K), ("k", Q4_K), ("v", Q6_K), ("o", Q4_K), ("gate", Q4_K), ("up", Q4_K),
                    ("down", Q6_K), ("head", Q6_K), ("embed", Q4_K))

    def type_of(self, name):
        return dict(self.types)[name]

    def mats(self):
        """(name, out_dim, in_dim) of one layer's matrices."""
        h, q, kv, f = self.hidden, self.n_heads * self.head_dim, self.n_kv * self.head_dim, self.ffn
        return [("q", q, h), ("k", kv, h), ("v", kv, h), ("o", h, q), ("gate", f, h), ("up", f, h), ("down", h, f)]

    def weight_bytes(self) -> int:
        from . import type_size
        per_layer = sum(type_size(self.type_of(n), o * i) for n, o, i in self.mats())
        return per_layer * self.layers + type_size(self.type_of("head"), self.vocab * self.hidden)


class ForwardStep:
    """One token of forward_gpu_step (src/cuda.rs:507-851, dense path) on the
    device, through the C ABI, in 5 launches per layer instead of the
    reference's 18:

      hip_gemv_group  q,k,v (Q4_K + Q6_K in one launch)  rms_norm(hidden) fused in
      hip_attention_step   RoPE q/k + K/V append + attention over pos + 1 rows
      hip_gemv_group  o    hidden += W_o att (residual fused in)
      hip_gemv_swiglu gate,up   rms_norm(hidden) and silu(gate) * up fused in
      hip_gemv_group  down hidden += W_down act

    then the final norm fused into the head GEMV.  The embedding row comes from
    hip_embed_lookup (the reference dequantizes it on the CPU and uploads it).
    Weights: `w[name][layer]` uint8 device tensors in GGUF layout; norms f32."""

    def __init__(self, cfg: ModelConfig, weights: dict):
        import math
        self.cfg, self.L, self.w = cfg, lib(), weights
        c = cfg
        qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
        f32 = dict(device="cuda", dtype=torch.float32)
        self.hidden = torch.zeros(c.hidden, **f32)
        self.q = torch.zeros(qd, **f32)
        self.k = torch.zeros(kvd, **f32)
        self.v = torch.zeros(kvd, **f32)
        self.att = torch.zeros(qd, **f32)
        self.gate = torch.zeros(c.ffn, **f32)
        self.up = torch.zeros(c.ffn, **f32)
        self.act = torch.zeros(c.ffn, **f32)
        self.logits = torch.zeros(c.vocab, **f32)
        # fallback scratch of hip_gemv_fused (in_dim + max out_dim floats)
        big = max(c.hidden, c.ffn, qd)
        self.scratch = torch.zeros(big + max(2 * big, c.vocab), **f32)
        self.kc = [torch.zeros(c.max_seq * kvd, **f32) for _ in range(c.layers)]
        self.vc = [torch.zeros(c.max_seq * kvd, **f32) for _ in range(c.layers)]
        self.scale = 1.0 / math.sqrt(c.head_dim)
        # device-side step state [token, pos] read by issue(dev=True)
        self.state = torch.zeros(2, dtype=torch.int32, device="cuda")

    def set_state(self, token: int, pos: int, stream=None):
        """Write the token and position a dev=True step reads (outside any graph)."""
        self._state_src = _write_state(self.L, self.state, [token, pos], stream)  # kept alive until the next write

    def embed_rows(self) -> int:
        from . import type_size
        return self.w["embed"].numel() // type_size(self.cfg.type_of("embed"), self.cfg.hidden)

    @staticmethod
    def random_weights(cfg: ModelConfig, seed: int = 20261204) -> dict:
        """Random-init weights generated on the device (synth_device)."""
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        w = {n: [] for n, _, _ in cfg.mats()}
        for l in range(cfg.layers):
            for j, (n, o, i) in enumerate(cfg.mats()):
                w[n].append(synth_device.weights(cfg.type_of(n), o, i, seed + 16 * l + j))
        w["head"] = synth_device.weights(cfg.type_of("head"), cfg.vocab, cfg.hidden, seed - 1)
        w["embed"] = synth_device.weights(cfg.type_of("embed"), cfg.vocab, cfg.hidden, seed - 2)
        norm = lambda: (1.0 + 0.1 * torch.randn(cfg.hidden, device="cuda", generator=g))
        w["attn_norm"] = [norm() for _ in range(cfg.layers)]
        w["ffn_norm"] = [norm() for _ in range(cfg.layers)]
        w["out_norm"] = norm()
        return w

    def _fused(self, names, layer, x, ys, in_dim, norm, accumulate, sp):
        """hip_gemv_group over the matrices `names` (any mix of weight types)."""
        ws = [(self.w[n][layer] if layer is not None else self.w[n]).data_ptr() for n in names]
        gemv_group_async(self.L, [self.cfg.type_of(n) for n in names], ws, [y.data_ptr() for y in ys],
                         [y.numel() for y in ys], x.data_ptr(), in_dim, sp,
                         norm_ptr=None if norm is None else norm.data_ptr(), accumulate=accumulate,
                         scratch_ptr=self.scratch.data_ptr())

    def issue(self, token: int = 0, pos: int = 0, stream=None, logits: bool = True, dev: bool = False,
              greedy: bool = False):
        """Enqueue one decode step (token at position pos) on `stream`.
        dev: read the token and position from self.state when the kernels run
        (set_state, or the previous step's greedy pick), so a captured step
        replays at consecutive positions.  greedy (with logits): end with
        hip_greedy_next, which writes the argmax token to state[0] and
        advances state[1]."""
        c, L = self.cfg, self.L
        assert dev or 0 <= pos < c.max_seq
        assert logits or not greedy
        sp = _stream_ptr(stream)
        kvd = c.n_kv * c.head_dim
        tok_p, pos_p = self.state.data_ptr(), self.state.data_ptr() + 4
        if dev:
            check("hip_embed_lookup_dev_async", L.hip_embed_lookup_dev_async(
                self.hidden.data_ptr(), c.hidden, self.w["embed"].data_ptr(), c.type_of("embed"), tok_p, 1,
                self.embed_rows(), c.hidden, sp))
        else:
            check("hip_embed_lookup_async", L.hip_embed_lookup_async(
                self.hidden.data_ptr(), self.w["embed"].data_ptr(), c.type_of("embed"), token, c.hidden, sp))
        for l in range(c.layers):
            self._fused(("q", "k", "v"), l, self.hidden, (self.q, self.k, self.v), c.hidden,
                        self.w["attn_norm"][l], False, sp)
            if dev:
                check("hip_attention_step_dev_async", L.hip_attention_step_dev_async(
                    self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                    self.kc[l].data_ptr(), self.vc[l].data_ptr(), None, 1, 0, c.n_heads, c.n_kv, c.head_dim, kvd,
                    pos_p, c.max_seq - 1, c.theta, 1.0, 0, c.neox, self.scale, sp))
            else:
                check("hip_attention_step_async", L.hip_attention_step_async(
                    self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                    self.kc[l].data_ptr(), self.vc[l].data_ptr(), None, c.n_heads, c.n_kv, c.head_dim, kvd, pos,
                    c.theta, 1.0, 0, c.neox, self.scale, sp))
            self._fused(("o",), l, self.att, (self.hidden,), c.n_heads * c.head_dim, None, True, sp)
            if c.type_of("gate") == c.type_of("up"):
                check("hip_gemv_swiglu_async", L.hip_gemv_swiglu_async(
                    c.type_of("gate"), self.w["gate"][l].data_ptr(), self.w["up"][l].data_ptr(), self.act.data_ptr(),
                    c.ffn, self.hidden.data_ptr(), self.w["ffn_norm"][l].data_ptr(), c.hidden,
                    self.scratch.data_ptr(), sp))
            else:
                self._fused(("gate", "up"), l, self.hidden, (self.gate, self.up), c.hidden, self.w["ffn_norm"][l],
                            False, sp)
                check("hip_swiglu_async", L.hip_swiglu_async(self.act.data_ptr(), self.gate.data_ptr(),
                                                             self.up.data_ptr(), c.ffn, sp))
            self._fused(("down",), l, self.act, (self.hidden,), c.ffn, None, True, sp)
        if logits:
            self._fused(("head",), None, self.hidden, (self.logits,), c.hidden, self.w["out_norm"], False, sp)
        if greedy:
            check("hip_greedy_next_async", L.hip_greedy_next_async(self.logits.data_ptr(), c.vocab, 1, c.vocab, tok_p,
                                                                   pos_p, sp))


class BatchStep:
    """forward_gpu_step for n sequences decoding in lockstep (token batch N of
    BatchConfig configs[3]): every sequence has its own token, hidden state and
    K/V cache, all at the same position.  The weight products are batched GEMMs
    (hip_gemm_grouped: one weight pass per 32 tokens on the matrix cores; q/k
    share one launch, v another, since they differ in type); the residual adds
    and the SwiGLU before the down projection are fused into the GEMMs
    (hip_gemm_grouped_ex); the norms and the attention are one launch each for
    all sequences (hip_rms_norm_rows, hip_attention_step_batched).
    Weights: the dict ForwardStep takes."""

    def __init__(self, cfg: ModelConfig, weights: dict, n: int):
        import math
        self.cfg, self.L, self.w, self.n = cfg, lib(), weights, n
        c = cfg
        qd, kvd = c.n_heads * c.head_dim, c.n_kv * c.head_dim
        f32 = dict(device="cuda", dtype=torch.float32)
        z = lambda d: torch.zeros(n, d, **f32)
        self.hidden, self.xn = z(c.hidden), z(c.hidden)
        self.q, self.k, self.v, self.att = z(qd), z(kvd), z(kvd), z(qd)
        self.gate, self.up, self.act = z(c.ffn), z(c.ffn), z(c.ffn)
        self.logits = z(c.vocab)
        self.tokens = torch.zeros(n, dtype=torch.int32)
        self.cache_stride = c.max_seq * kvd
        self.kc = [torch.zeros(n * self.cache_stride, **f32) for _ in range(c.layers)]
        self.vc = [torch.zeros(n * self.cache_stride, **f32) for _ in range(c.layers)]
        self.scale = 1.0 / math.sqrt(c.head_dim)
        big = max(c.hidden, c.ffn, qd)
        self.scratch = torch.zeros(2 * n * big, **f32)  # fallback of hip_gemm_grouped_ex
        # device-side step state [tokens[0..n), pos] read by issue(dev=True)
        self.state = torch.zeros(n + 1, dtype=torch.int32, device="cuda")

    def set_state(self, tokens, pos: int, stream=None):
        """Write the tokens and position a dev=True step reads (outside any graph)."""
        self._state_src = _write_state(self.L, self.state, list(tokens) + [pos], stream)

    def _gemm_res(self, name, layer, x, in_dim, sp, up=None):
        """hidden += W x (or W (silu(x) * up)) in one hip_gemm_grouped_ex call."""
        c = self.cfg
        gemm_grouped_ex_async(self.L, c.type_of(name), [self.w[name][layer].data_ptr()], [x.data_ptr()],
                              [self.hidden.data_ptr()], [self.n], [c.hidden], in_dim, sp,
                              up_ptrs=[up.data_ptr()] if up is not None else None, accumulate=True,
                              scratch_ptr=self.scratch.data_ptr())

    def _gemm(self, names, layer, x, ys, in_dim, sp):
        """Batched GEMMs of the matrices `names` sharing x, one call per weight type."""
        by_type = {}
        for nm, y in zip(names, ys):
            by_type.setdefault(self.cfg.type_of(nm), []).append((nm, y))
        for t, group in by_type.items():
            ws = [(self.w[nm][layer] if layer is not None else self.w[nm]).data_ptr() for nm, _ in group]
            gemm_grouped_async(self.L, t, ws, [x.data_ptr()] * len(group), [y.data_ptr() for _, y in group],
                               [self.n] * len(group), [y.shape[1] for _, y in group], in_dim, sp)

    def _gemm_norm(self, names, layer, norm, ys, sp):
        """y = W rms_norm(hidden) * norm for the matrices `names`, one
        hip_gemm_group_norm call.  Up to 4 tokens: the norm fused into the GEMMs
        (q/k (Q4_K) and v (Q6_K) in one launch); 5-16: the norm fused into the
        batched kernel's x images (one launch), then the GEMMs on those images
        (both types in one launch); 17-32: the same images in two halves, then
        one launch for Q4_K + Q6_K or one per type.  More than 32 tokens of one
        type: one
        hip_rms_norm_rows, then the type's grouped GEMMs."""
        if self.n > 32 and len({self.cfg.type_of(nm) for nm in names}) == 1:
            check("hip_rms_norm_rows_async", self.L.hip_rms_norm_rows_async(
                self.xn.data_ptr(), self.hidden.data_ptr(), norm.data_ptr(), self.n, self.cfg.hidden, sp))
            self._gemm(names, layer, self.xn, ys, self.cfg.hidden, sp)
            return
        ws = [(self.w[nm][layer] if layer is not None else self.w[nm]).data_ptr() for nm in names]
        gemm_group_norm_async(self.L, [self.cfg.type_of(nm) for nm in names], ws, self.hidden.data_ptr(),
                              norm.data_ptr(), [y.data_ptr() for y in ys], self.n, [y.shape[1] for y in ys],
                              self.cfg.hidden, sp, self.scratch.data_ptr())

    def issue(self, tokens=None, pos: int = 0, stream=None, logits: bool = True, dev: bool = False,
              greedy: bool = False):
        """Enqueue one lockstep decode step: sequence i takes tokens[i] at `pos`.
        dev / greedy: as ForwardStep.issue, with the n tokens and the shared
        position in self.state."""
        c, L, n = self.cfg, self.L, self.n
        assert dev or (len(tokens) == n and 0 <= pos < c.max_seq)
        assert logits or not greedy
        sp = _stream_ptr(stream)
        kvd = c.n_kv * c.head_dim
        row = self.hidden.stride(0)
        tok_p, pos_p = self.state.data_ptr(), self.state.data_ptr() + 4 * n
        if dev:
            from . import type_size
            rows = self.w["embed"].numel() // type_size(c.type_of("embed"), c.hidden)
            check("hip_embed_lookup_dev_async", L.hip_embed_lookup_dev_async(
                self.hidden.data_ptr(), row, self.w["embed"].data_ptr(), c.type_of("embed"), tok_p, n, rows,
                c.hidden, sp))
        else:
            toks = (C.c_int * n)(*[int(t) for t in tokens])
            check("hip_embed_lookup_batched_async", L.hip_embed_lookup_batched_async(
                self.hidden.data_ptr(), row, self.w["embed"].data_ptr(), c.type_of("embed"), toks, n, c.hidden, sp))
        for l in range(c.layers):
            self._gemm_norm(("q", "k", "v"), l, self.w["attn_norm"][l], (self.q, self.k, self.v), sp)
            if dev:
                check("hip_attention_step_dev_async", L.hip_attention_step_dev_async(
                    self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                    self.kc[l].data_ptr(), self.vc[l].data_ptr(), None, n, self.cache_stride, c.n_heads, c.n_kv,
                    c.head_dim, kvd, pos_p, c.max_seq - 1, c.theta, 1.0, 0, c.neox, self.scale, sp))
            else:
                check("hip_attention_step_batched_async", L.hip_attention_step_batched_async(
                    self.att.data_ptr(), self.q.data_ptr(), self.k.data_ptr(), self.v.data_ptr(),
                    self.kc[l].data_ptr(), self.vc[l].data_ptr(), None, n, self.cache_stride, c.n_heads, c.n_kv,
                    c.head_dim, kvd, pos, c.theta, 1.0, 0, c.neox, self.scale, sp))
            self._gemm_res("o", l, self.att, c.n_heads * c.head_dim, sp)
            self._gemm_norm(("gate", "up"), l, self.w["ffn_norm"][l], (self.gate, self.up), sp)
            self._gemm_res("down", l, self.gate, c.ffn, sp, up=self.up)
        if logits:
            self._gemm_norm(("head",), None, self.w["out_norm"], (self.logits,), sp)
        if greedy:
            check("hip_greedy_next_async", L.hip_greedy_next_async(self.logits.data_ptr(), c.vocab, n, c.vocab, tok_p,
                                                                   pos_p, sp))
