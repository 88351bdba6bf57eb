"""The C-ABI library loads and exports every symbol include/quartz_hip.h declares;
argument validation that never reaches the GPU.  No GPU needed."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

import closed_form as cf
from saient_quartz_amd import GGML_TYPES, lib

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    txt = (ROOT / "include" / "quartz_hip.h").read_text()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(hip_\w+)\s*\(", txt)))


def test_header_declares_reference_twins():
    syms = declared_symbols()
    for ref in ("gemv", "gemv_moe4", "alloc", "drop", "h2d", "d2h", "sync", "mem_info",
                "set_iq3s_grid", "set_iq2s_grid", "set_iq2xxs_grid", "set_iq2xs_grid", "set_ksigns"):
        assert "hip_" + ref in syms  # every cuda_* symbol of the GEMV surface has a twin


def test_library_exports_all_symbols():
    L = lib()
    for s in declared_symbols():
        assert hasattr(L, s), f"missing export {s}"


@pytest.mark.parametrize("t", sorted(GGML_TYPES))
def test_type_size_abi(t):
    _, qk, bb = GGML_TYPES[t]
    for n in (qk, 4096 * 14336):
        assert lib().hip_type_size(t, n) == (n // qk) * bb
    assert lib().hip_type_size(99, 256) == 0
    assert lib().hip_type_size(4, 256) == 0  # Q4_2 was removed from GGUF


def test_argument_errors_before_any_gpu_call():
    L = lib()
    nul = None
    assert L.hip_gemv(12, nul, nul, nul, 200, 10) == -2        # in_dim not a multiple of 256
    assert L.hip_gemv(12, nul, nul, nul, 0, 10) == -2
    assert L.hip_gemv(12, nul, nul, nul, 256, -1) == -2
    assert L.hip_gemv(12, nul, nul, nul, 256, 10) == -3        # null pointers
    assert L.hip_gemv(12, nul, nul, nul, 256, 0) == 0          # empty output: no-op
    assert L.hip_gemv(99, nul, nul, nul, 256, 0) == -1         # unknown type (nothing to zero)
    assert L.hip_gemm(14, nul, nul, nul, 256, 4, -1) == -2
    assert L.hip_gemm(14, nul, nul, nul, 256, 4, 0) == 0
    assert L.hip_gemm(8, nul, nul, nul, 48, 4, 2) == -2
    assert L.hip_gemv_moe4(12, *([nul] * 12), 5, 256, 4) == -5
    assert L.hip_dequant(12, nul, nul, 300) == -2
    assert L.hip_dequant(12, nul, nul, 256) == -3
    assert L.hip_dequant(12, nul, nul, 0) == 0
    assert L.hip_dequant(5, nul, nul, 32) == -1
    assert L.hip_gemm_grouped(12, -1, nul, nul, nul, nul, nul, 256) == -5
    assert L.hip_gemm_grouped(12, 0, nul, nul, nul, nul, nul, 256) == 0
    assert L.hip_gemm_grouped(12, 1, nul, nul, nul, nul, nul, 256) == -3
    assert L.hip_gemm_moe(12, nul, -1, nul, nul, nul, nul, 256, 8) == -5
    assert L.hip_gemm_moe(12, nul, 0, nul, nul, nul, nul, 256, 8) == 0
    assert L.hip_gemm_moe(12, nul, 2, nul, nul, nul, nul, 256, 8) == -3
    assert L.hip_gemm_moe(12, nul, 1, (C.c_int * 1)(-1), (C.c_int * 2)(0, 1), nul, nul, 256, 8) == -5
    assert L.hip_status_string(-2).decode().startswith("bad dimensions")


def test_set_ksigns_checks_closed_form():
    L = lib()
    ks = cf.ksigns()
    assert L.hip_set_ksigns(ks.ctypes.data) == 0
    bad = ks.copy()
    bad[5] ^= 0x80
    assert L.hip_set_ksigns(bad.ctypes.data) == -5
    assert L.hip_set_ksigns(None) == -3


def test_device_state_and_graph_argument_errors():
    """The device-state, graph and stream entry points reject bad arguments
    before touching the GPU (this runs without one)."""
    L = lib()
    nul = None
    # hip_greedy_next_async(logits, row_stride, rows, n, d_tokens, d_pos, stream)
    assert L.hip_greedy_next_async(nul, 0, 1, 10, nul, nul, nul) == -3
    assert L.hip_greedy_next_async(nul, 5, 2, 10, nul, nul, nul) == -2   # rows overlap
    assert L.hip_greedy_next_async(nul, 0, -1, 10, nul, nul, nul) == -2
    assert L.hip_greedy_next_async(nul, 0, 1, -1, nul, nul, nul) == -2
    assert L.hip_greedy_next_async(nul, 0, 0, 10, nul, nul, nul) == 0   # nothing to pick
    assert L.hip_greedy_next_async(nul, 0, 1, 0, nul, nul, nul) == 0
    # hip_embed_lookup_dev_async(out, out_stride, data, type, d_tokens, n_tok, n_vocab, embed_dim, stream)
    assert L.hip_embed_lookup_dev_async(nul, 0, nul, 99, nul, 1, 100, 4096, nul) == -1
    assert L.hip_embed_lookup_dev_async(nul, 0, nul, 12, nul, 1, 100, 100, nul) == -2   # not whole blocks
    assert L.hip_embed_lookup_dev_async(nul, 10, nul, 12, nul, 2, 100, 256, nul) == -2  # rows overlap
    assert L.hip_embed_lookup_dev_async(nul, 0, nul, 12, nul, 0, 100, 256, nul) == 0
    assert L.hip_embed_lookup_dev_async(nul, 0, nul, 12, nul, 1, 100, 256, nul) == -3
    # hip_attention_step_dev_async: the position pointer is required
    args = [nul] * 7 + [1, 0, 32, 8, 128, 1024, nul, 0, 5e5, 1.0, 0, 0, 0.088, nul]
    assert L.hip_attention_step_dev_async(*args) == -3
    # graphs and streams
    assert L.hip_graph_begin(nul) == -3          # the null stream cannot be captured
    assert L.hip_graph_end(nul, nul) == -3
    assert L.hip_graph_launch(nul, nul) == -3
    assert L.hip_stream_create(nul) == -3
    assert L.hip_timestamp_async(nul, nul) == -3
    L.hip_graph_destroy(nul)                     # no-ops
    L.hip_stream_destroy(nul)
