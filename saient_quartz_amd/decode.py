"""Llama-3-8B-shaped Q4_K_M decode step: the weight GEMVs of one token.

Per layer, in the order of forward_gpu_step (src/cuda.rs:556-562, :647, :773-788):
  q 4096x4096 Q4_K, k 1024x4096 Q4_K, v 1024x4096 Q6_K, o 4096x4096 Q4_K,
  gate 14336x4096 Q4_K, up 14336x4096 Q4_K, down 4096x14336 Q6_K;
then the output head 128256x4096 Q6_K.  32 layers: 4,875,853,824 weight bytes.

`DecodeStep` holds random-init weights (seeded, generated on the device) and
issues the step's GEMVs (n tokens: hip_gemm, n = 1: hip_gemv) through the C ABI
on a caller stream.  The glue between GEMVs (rms_norm, rope, attention, swiglu,
residual adds) is not part of this library yet: activations are fixed buffers,
so a step measures weight streaming, which is >99% of the bytes of a decode step
at short context.
"""
from dataclasses import dataclass

import torch

from . import synth_device
from .api import check, lib
from .host import gemm_grouped_async, gemm_moe_async, gemv_multi_async

Q4_K, Q6_K = 12, 14


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
        sp = (stream or torch.cuda.current_stream()).cuda_stream
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
        sp = (stream or torch.cuda.current_stream()).cuda_stream
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
