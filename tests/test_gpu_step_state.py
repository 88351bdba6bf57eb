"""GPU parity of the decode step driven from device-side state: one captured
step replayed at consecutive positions (forward_gpu_step(token, pos, ...) once
per token, src/cuda.rs:507, caller src/main.rs:481), the greedy pick of the
next token on the device (src/main.rs:1684-1692), and the C-ABI route a host
without torch uses to capture and replay a step.

Bars: the _dev entries equal the host-argument entries bit for bit (same
kernels, same split of the sequence); hip_greedy_next equals
oracle/glue_ref.greedy_next exactly; a replayed step equals the eager step
issued with host arguments bit for bit, at every position."""
import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from saient_quartz_amd.api import check, lib
from saient_quartz_amd.decode import BatchStep, ForwardStep, ModelConfig

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import glue_ref as g  # noqa: E402
from test_gpu_decode_step import LLAMA_TYPES, device_weights, host_model  # noqa: E402

pytestmark = pytest.mark.gpu


def _f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def test_greedy_next_vs_oracle(qh):
    L = lib()
    rng = np.random.default_rng(1)
    nan = np.float32(np.nan)
    rows = [rng.standard_normal(128256).astype(np.float32),
            np.zeros(128256, np.float32),                                    # all equal: the last index
            np.array([1, 3, 2, 3, 0], np.float32),
            np.array([0.0, -0.0], np.float32),
            np.array([-np.inf, -nan, -1.0], np.float32),
            np.array([5.0, np.inf, nan, 1e38], np.float32),
            rng.integers(-3, 4, 5000).astype(np.float32),                    # many ties
            np.full(3, -np.inf, np.float32)]
    for r in rows:
        x = _f32(r)
        out = torch.full((2,), -7, dtype=torch.int32, device="cuda")
        check("hip_greedy_next_async", L.hip_greedy_next_async(x.data_ptr(), r.size, 1, r.size, out.data_ptr(),
                                                               None, None))
        torch.cuda.synchronize()
        assert int(out[0]) == g.greedy_next(r), r[:8]
        assert int(out[1]) == -7
    # a row starting off a 16-byte boundary (scalar head, vector body, scalar tail)
    r = rng.integers(-20, 20, 1003).astype(np.float32)
    buf = _f32(np.concatenate([[0.0], r]))
    out = torch.zeros(1, dtype=torch.int32, device="cuda")
    check("hip_greedy_next_async", L.hip_greedy_next_async(buf.data_ptr() + 4, r.size, 1, r.size, out.data_ptr(),
                                                           None, None))
    torch.cuda.synchronize()
    assert int(out[0]) == g.greedy_next(r)
    # several rows at a stride, and the position advance (once per launch)
    n, stride, rows_n = 1000, 1024, 5
    x = rng.integers(-50, 50, (rows_n, stride)).astype(np.float32)
    state = torch.tensor([0] * rows_n + [41], dtype=torch.int32, device="cuda")
    dx = _f32(x)
    check("hip_greedy_next_async", L.hip_greedy_next_async(dx.data_ptr(), stride, rows_n, n, state.data_ptr(),
                                                           state.data_ptr() + 4 * rows_n, None))
    torch.cuda.synchronize()
    got = state.cpu().numpy()
    assert list(got[:rows_n]) == [g.greedy_next(x[r, :n]) for r in range(rows_n)]
    assert got[rows_n] == 42


def test_embed_lookup_dev_matches_host(qh):
    L = lib()
    from saient_quartz_amd import synth
    vocab, dim, t = 300, 512, 12
    data = torch.from_numpy(synth.weights(t, vocab, dim, seed=3)).cuda()
    toks = [0, 299, 17, 300, -1, 5]  # 300 and -1 lie outside the table: zero rows
    dtok = torch.tensor(toks, dtype=torch.int32, device="cuda")
    got = torch.full((len(toks), dim), 9.0, device="cuda")
    check("hip_embed_lookup_dev_async", L.hip_embed_lookup_dev_async(got.data_ptr(), dim, data.data_ptr(), t,
                                                                     dtok.data_ptr(), len(toks), vocab, dim, None))
    for i, tk in enumerate(toks):
        ref = torch.full((dim,), 9.0, device="cuda")
        if 0 <= tk < vocab:
            check("hip_embed_lookup_async", L.hip_embed_lookup_async(ref.data_ptr(), data.data_ptr(), t, tk, dim,
                                                                     None))
            torch.cuda.synchronize()
            assert torch.equal(got[i], ref), i
        else:
            torch.cuda.synchronize()
            assert torch.all(got[i] == 0), i


@pytest.mark.parametrize("n_seq", [1, 3])
def test_attention_step_dev_matches_host(qh, n_seq):
    """hip_attention_step_dev_async at positions whose split of the sequence
    differs (1 .. 23 slices of 32 rows; one workgroup per slice up to 16, two
    past that), and one past max_pos (clamped): bit-equal outputs and caches to
    the host-position call."""
    L = lib()
    nh, nkv, hd, max_seq = 8, 2, 128, 736
    kvd = nkv * hd
    rng = np.random.default_rng(n_seq)
    stride = max_seq * kvd
    kc0 = rng.standard_normal(n_seq * stride).astype(np.float32)
    vc0 = rng.standard_normal(n_seq * stride).astype(np.float32)
    kc = [_f32(kc0), _f32(kc0)]
    vc = [_f32(vc0), _f32(vc0)]
    pos_d = torch.zeros(1, dtype=torch.int32, device="cuda")
    for pos in (0, 1, 31, 32, 95, 511, 512, 600, max_seq - 1, max_seq + 4):
        q = _f32(rng.standard_normal(n_seq * nh * hd))
        k = _f32(rng.standard_normal(n_seq * kvd))
        v = _f32(rng.standard_normal(n_seq * kvd))
        outs = [torch.zeros(n_seq * nh * hd, device="cuda") for _ in range(2)]
        hp = min(pos, max_seq - 1)
        check("host", L.hip_attention_step_batched_async(
            outs[0].data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), kc[0].data_ptr(), vc[0].data_ptr(), None,
            n_seq, stride, nh, nkv, hd, kvd, hp, 500000.0, 1.0, 0, 0, 0.088388, None))
        pos_d.fill_(pos)
        check("dev", L.hip_attention_step_dev_async(
            outs[1].data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), kc[1].data_ptr(), vc[1].data_ptr(), None,
            n_seq, stride, nh, nkv, hd, kvd, pos_d.data_ptr(), max_seq - 1, 500000.0, 1.0, 0, 0, 0.088388, None))
        torch.cuda.synchronize()
        print(f"attention dev n_seq {n_seq} pos {pos}", flush=True)
        assert torch.equal(outs[0], outs[1]), pos
        assert torch.equal(kc[0], kc[1]) and torch.equal(vc[0], vc[1]), pos


def _small_cfg(**kw):
    base = dict(hidden=512, n_heads=4, n_kv=2, head_dim=128, ffn=1024, vocab=300, layers=2, max_seq=40,
                types=LLAMA_TYPES)
    base.update(kw)
    return ModelConfig(**base)


def test_forward_step_graph_advances_positions(qh):
    """One step captured with dev=True, replayed at positions 0..7 with a new
    token written before each replay: logits and hidden state equal an eager
    twin's host-argument steps bit for bit at every position."""
    cfg = _small_cfg()
    raw, norms = host_model(cfg, seed=21, realistic=True)
    w = device_weights(raw, norms)
    eager, replay = ForwardStep(cfg, w), ForwardStep(cfg, w)
    graph = torch.cuda.CUDAGraph()
    replay.set_state(0, 0)
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        replay.issue(dev=True)
    # capture recorded the work without running it: the caches are untouched
    for c in replay.kc:
        c.zero_()
    for c in replay.vc:
        c.zero_()
    tokens = [5, 299, 0, 17, 17, 123, 8, 250]
    for pos, tok in enumerate(tokens):
        eager.issue(tok, pos)
        replay.set_state(tok, pos)
        graph.replay()
        torch.cuda.synchronize()
        print(f"graph step pos {pos}", flush=True)
        assert torch.equal(replay.logits, eager.logits), pos
        assert torch.equal(replay.hidden, eager.hidden), pos


def test_forward_step_greedy_generation(qh):
    """Greedy generation on the device: a step captured with dev=True and
    greedy=True replayed 10 times from (token 7, pos 0) produces the tokens an
    eager host loop produces (glue_ref.greedy_next on each step's logits), and
    the same final logits."""
    cfg = _small_cfg()
    raw, norms = host_model(cfg, seed=22, realistic=True)
    w = device_weights(raw, norms)
    eager, replay = ForwardStep(cfg, w), ForwardStep(cfg, w)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        replay.issue(dev=True, greedy=True)
    for c in replay.kc + replay.vc:
        c.zero_()
    replay.set_state(7, 0)
    tok, want = 7, []
    for pos in range(10):
        eager.issue(tok, pos)
        torch.cuda.synchronize()
        tok = g.greedy_next(eager.logits.cpu().numpy())
        want.append(tok)
    got = []
    for pos in range(10):
        graph.replay()
        st = replay.state.cpu().numpy()
        got.append(int(st[0]))
        assert int(st[1]) == pos + 1
    print("greedy tokens", got, flush=True)
    assert got == want
    assert torch.equal(replay.logits, eager.logits)


def test_c_abi_graph_route(qh):
    """The route a host without torch takes: hip_stream_create,
    hip_graph_begin / hip_graph_end around one dev=True step, then per token
    hip_h2d_async of (token, pos) and hip_graph_launch; equal to eager steps
    bit for bit."""
    L = lib()
    cfg = _small_cfg(layers=1)
    raw, norms = host_model(cfg, seed=23, realistic=True)
    w = device_weights(raw, norms)
    eager, replay = ForwardStep(cfg, w), ForwardStep(cfg, w)
    torch.cuda.synchronize()
    st = C.c_void_p()
    check("hip_stream_create", L.hip_stream_create(C.byref(st)))
    exe = C.c_void_p()
    try:
        check("hip_graph_begin", L.hip_graph_begin(st))
        replay.issue(dev=True, stream=st.value)
        check("hip_graph_end", L.hip_graph_end(st, C.byref(exe)))
        for pos, tok in enumerate([3, 1, 4, 1, 5]):
            eager.issue(tok, pos)
            torch.cuda.synchronize()  # the two streams share the library's attention scratch
            replay.set_state(tok, pos, stream=st.value)
            check("hip_graph_launch", L.hip_graph_launch(exe, st))
            check("hip_stream_sync", L.hip_stream_sync(st))
            torch.cuda.synchronize()
            assert torch.equal(replay.logits, eager.logits), pos
    finally:
        L.hip_graph_destroy(exe)
        L.hip_stream_destroy(st)


@pytest.mark.parametrize("n", [4, 16])
def test_batch_step_greedy_generation(qh, n):
    """BatchStep with the n tokens and the position on the device: one graph
    (dev=True, greedy=True) replayed 6 times equals an eager host loop over
    hip_embed_lookup_batched / the host-position attention, token for token and
    in the final logits bit for bit."""
    cfg = _small_cfg()
    raw, norms = host_model(cfg, seed=24, realistic=True)
    w = device_weights(raw, norms)
    eager, replay = BatchStep(cfg, w, n), BatchStep(cfg, w, n)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        replay.issue(dev=True, greedy=True)
    for c in replay.kc + replay.vc:
        c.zero_()
    start = list(np.random.default_rng(n).integers(0, cfg.vocab, n))
    replay.set_state(start, 0)
    toks = start
    for pos in range(6):
        eager.issue(toks, pos)
        torch.cuda.synchronize()
        lg = eager.logits.cpu().numpy()
        toks = [g.greedy_next(lg[i]) for i in range(n)]
        graph.replay()
        st = replay.state.cpu().numpy()
        print(f"batch n={n} pos {pos} tokens {toks[:4]}", flush=True)
        assert list(st[:n]) == toks, pos
        assert int(st[n]) == pos + 1
        assert torch.equal(replay.logits, eager.logits), pos
