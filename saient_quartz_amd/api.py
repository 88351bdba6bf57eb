"""ctypes binding of libquartz_hip.so (see include/quartz_hip.h)."""
import ctypes as C
from pathlib import Path

_PKG = Path(__file__).resolve().parent
_LIB = None

QH_OK = 0
STATUS = {0: "ok", -1: "unsupported ggml_type", -2: "bad dimensions", -3: "null pointer",
          -4: "HIP runtime error", -5: "argument out of range", -6: "malformed GGUF file", -7: "file I/O error"}

# ggml type id -> (name, elements per block, bytes per block); src/gguf.rs:172-191
GGML_TYPES = {
    0: ("F32", 1, 4), 1: ("F16", 1, 2), 2: ("Q4_0", 32, 18), 3: ("Q4_1", 32, 20),
    6: ("Q5_0", 32, 22), 7: ("Q5_1", 32, 24), 8: ("Q8_0", 32, 34), 10: ("Q2_K", 256, 84),
    12: ("Q4_K", 256, 144), 13: ("Q5_K", 256, 176), 14: ("Q6_K", 256, 210),
    16: ("IQ2_XXS", 256, 66), 17: ("IQ2_XS", 256, 74), 20: ("IQ4_NL", 32, 18),
    21: ("IQ3_S", 256, 110), 22: ("IQ2_S", 256, 82), 30: ("BF16", 1, 2),
}
TYPE_IDS = {v[0]: k for k, v in GGML_TYPES.items()}


class QuartzHipError(RuntimeError):
    def __init__(self, fn, status):
        msg = f"{fn} -> {status} ({STATUS.get(status, '?')})"
        if status in (-4, -6, -7) and _LIB is not None:
            msg += ": " + _LIB.hip_last_error().decode()
        super().__init__(msg)
        self.status = status


def block_elems(t: int) -> int:
    return GGML_TYPES[t][1]


def type_size(t: int, n: int) -> int:
    _, qk, b = GGML_TYPES[t]
    return (n // qk) * b


def lib_path() -> Path:
    return _PKG / "libquartz_hip.so"


_SIGS = {
    "hip_gemv": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    "hip_gemv_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hip_gemv_multi": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]),
    "hip_gemv_multi_async": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int,
                                       C.c_void_p]),
    "hip_gemv_fused_async": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_gemv_group_async": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_rms_norm_rows_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hip_attention_step_batched_async": (C.c_int, [C.c_void_p] * 7 + [C.c_int, C.c_size_t] + [C.c_int] * 5 +
                                         [C.c_float, C.c_float, C.c_int, C.c_int, C.c_float, C.c_void_p]),
    "hip_gemv_swiglu_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p,
                                        C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_attention_step_async": (C.c_int, [C.c_void_p] * 7 + [C.c_int] * 5 + [C.c_float, C.c_float, C.c_int, C.c_int,
                                                                           C.c_float, C.c_void_p]),
    "hip_gemm": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int]),
    "hip_gemm_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                 C.c_void_p]),
    "hip_gemm_grouped": (C.c_int, [C.c_uint32, C.c_int] + [C.c_void_p] * 5 + [C.c_int]),
    "hip_gemm_grouped_async": (C.c_int, [C.c_uint32, C.c_int] + [C.c_void_p] * 5 + [C.c_int, C.c_void_p]),
    "hip_gemm_grouped_ex_async": (C.c_int, [C.c_uint32, C.c_int] + [C.c_void_p] * 6 + [C.c_int, C.c_int, C.c_void_p,
                                                                                     C.c_void_p]),
    "hip_moe_route_async": (C.c_int, [C.c_void_p, C.c_void_p] + [C.c_int] * 4 + [C.c_void_p] * 3),
    "hip_moe_plan_async": (C.c_int, [C.c_void_p] + [C.c_int] * 3 + [C.c_void_p] * 5),
    "hip_moe_gather_async": (C.c_int, [C.c_void_p] * 3 + [C.c_int] * 2 + [C.c_void_p]),
    "hip_moe_swiglu_async": (C.c_int, [C.c_void_p] * 6 + [C.c_int] * 3 + [C.c_void_p]),
    "hip_moe_combine_async": (C.c_int, [C.c_void_p] * 6 + [C.c_int] * 4 + [C.c_void_p]),
    "hip_gemm_grouped_norm_async": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                             C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_gemm_grouped_norm_static_async": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p,
                                                    C.c_void_p, C.c_int, C.c_void_p, C.c_int, C.c_void_p]),
    "hip_gemm_group_norm_async": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                           C.c_int, C.c_void_p, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_gemm_q8_1_mmq": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_int] * 5),
    "hip_gemm_q8_1_mmq_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p] + [C.c_int] * 5 +
                                [C.c_void_p]),
    "hip_gemm_moe": (C.c_int, [C.c_uint32, C.c_void_p, C.c_int] + [C.c_void_p] * 4 + [C.c_int, C.c_int]),
    "hip_gemm_moe_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_int] + [C.c_void_p] * 4 + [C.c_int, C.c_int,
                                                                                          C.c_void_p]),
    "hip_gemm_moe_dev_async": (C.c_int, [C.c_uint32, C.c_int, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p, C.c_int,
                                         C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hip_gguf_open": (C.c_int, [C.c_char_p, C.c_void_p]),
    "hip_gguf_close": (None, [C.c_void_p]),
    "hip_gguf_version": (C.c_uint32, [C.c_void_p]),
    "hip_gguf_data_offset": (C.c_uint64, [C.c_void_p]),
    "hip_gguf_alignment": (C.c_uint64, [C.c_void_p]),
    "hip_gguf_kv_count": (C.c_int64, [C.c_void_p]),
    "hip_gguf_kv_key": (C.c_char_p, [C.c_void_p, C.c_int64]),
    "hip_gguf_kv_type": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p]),
    "hip_gguf_get_u32": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_u64": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_i64": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_f32": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_f64": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_str": (C.c_void_p, [C.c_void_p, C.c_char_p, C.c_void_p]),
    "hip_gguf_get_array": (C.c_void_p, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p]),
    "hip_gguf_get_array_str": (C.c_void_p, [C.c_void_p, C.c_char_p, C.c_uint64, C.c_void_p]),
    "hip_gguf_tensor_count": (C.c_int64, [C.c_void_p]),
    "hip_gguf_find_tensor": (C.c_int64, [C.c_void_p, C.c_char_p]),
    "hip_gguf_tensor_info": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "hip_gguf_tensor_data": (C.c_void_p, [C.c_void_p, C.c_int64, C.c_void_p]),
    "hip_gguf_upload": (C.c_int, [C.c_void_p, C.c_int64, C.c_void_p, C.c_void_p]),
    "hip_gguf_writer_new": (C.c_void_p, []),
    "hip_gguf_writer_free": (None, [C.c_void_p]),
    "hip_gguf_writer_kv_scalar": (C.c_int, [C.c_void_p, C.c_char_p, C.c_uint32, C.c_void_p]),
    "hip_gguf_writer_kv_str": (C.c_int, [C.c_void_p, C.c_char_p, C.c_char_p, C.c_uint64]),
    "hip_gguf_writer_kv_array": (C.c_int, [C.c_void_p, C.c_char_p, C.c_uint32, C.c_void_p, C.c_uint64]),
    "hip_gguf_writer_kv_array_str": (C.c_int, [C.c_void_p, C.c_char_p, C.c_void_p, C.c_void_p, C.c_uint64]),
    "hip_gguf_writer_tensor": (C.c_int, [C.c_void_p, C.c_char_p, C.c_uint32, C.c_void_p, C.c_uint32, C.c_void_p]),
    "hip_gguf_writer_write": (C.c_int, [C.c_void_p, C.c_char_p]),
    "hip_vec_add": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int]),
    "hip_vec_add_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "hip_vec_scale_add": (C.c_int, [C.c_void_p, C.c_void_p, C.c_float, C.c_int]),
    "hip_vec_scale_add_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_float, C.c_int, C.c_void_p]),
    "hip_vec_zero": (C.c_int, [C.c_void_p, C.c_int]),
    "hip_vec_zero_async": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
    "hip_rms_norm": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]),
    "hip_rms_norm_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "hip_rope_yarn": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int]),
    "hip_rope_yarn_async": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int, C.c_void_p]),
    "hip_kv_append": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int]),
    "hip_kv_append_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "hip_attn_score_all": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    "hip_attn_score_all_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_void_p]),
    "hip_softmax_sink_all": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hip_softmax_sink_all_async": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "hip_attn_values_all": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "hip_attn_values_all_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "hip_attention_decode": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    "hip_attention_decode_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float, C.c_void_p]),
    "hip_swiglu": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]),
    "hip_swiglu_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "hip_swiglu_oai": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int]),
    "hip_swiglu_oai_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "hip_embed_lookup": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_int, C.c_int]),
    "hip_embed_lookup_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_int, C.c_int, C.c_void_p]),
    "hip_embed_lookup_batched_async": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_uint32, C.c_void_p, C.c_int,
                                                 C.c_int, C.c_void_p]),
    "hip_embed_lookup_dev_async": (C.c_int, [C.c_void_p, C.c_size_t, C.c_void_p, C.c_uint32, C.c_void_p, C.c_int,
                                             C.c_int, C.c_int, C.c_void_p]),
    "hip_attention_step_dev_async": (C.c_int, [C.c_void_p] * 7 + [C.c_int, C.c_size_t] + [C.c_int] * 4 +
                                     [C.c_void_p, C.c_int, C.c_float, C.c_float, C.c_int, C.c_int, C.c_float,
                                      C.c_void_p]),
    "hip_greedy_next_async": (C.c_int, [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_void_p, C.c_void_p,
                                        C.c_void_p]),
    "hip_h2d_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "hip_d2h_async": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "hip_stream_create": (C.c_int, [C.c_void_p]),
    "hip_stream_sync": (C.c_int, [C.c_void_p]),
    "hip_stream_destroy": (None, [C.c_void_p]),
    "hip_graph_begin": (C.c_int, [C.c_void_p]),
    "hip_graph_end": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hip_graph_launch": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hip_graph_destroy": (None, [C.c_void_p]),
    "hip_attn_score": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_float]),
    "hip_softmax_sink": (C.c_int, [C.c_void_p, C.c_int, C.c_float]),
    "hip_attn_values": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_int]),
    "hip_gemv_moe4": (C.c_int, [C.c_uint32] + [C.c_void_p] * 12 + [C.c_int, C.c_int, C.c_int]),
    "hip_dequant": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_size_t]),
    "hip_dequant_async": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]),
    "hip_type_size": (C.c_size_t, [C.c_uint32, C.c_size_t]),
    "hip_alloc": (C.c_void_p, [C.c_size_t]),
    "hip_drop": (None, [C.c_void_p]),
    "hip_h2d": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "hip_d2h": (C.c_int, [C.c_void_p, C.c_void_p, C.c_size_t]),
    "hip_sync": (C.c_int, []),
    "hip_timestamp_async": (C.c_int, [C.c_void_p, C.c_void_p]),
    "hip_wallclock_khz": (C.c_int, []),
    "hip_mem_info": (C.c_int, [C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]),
    "hip_set_iq3s_grid": (C.c_int, [C.c_void_p]),
    "hip_set_iq2s_grid": (C.c_int, [C.c_void_p]),
    "hip_set_iq2xxs_grid": (C.c_int, [C.c_void_p]),
    "hip_set_iq2xs_grid": (C.c_int, [C.c_void_p]),
    "hip_set_ksigns": (C.c_int, [C.c_void_p]),
    "hip_status_string": (C.c_char_p, [C.c_int]),
    "hip_last_error": (C.c_char_p, []),
}


def lib() -> C.CDLL:
    """Load libquartz_hip.so; raises if it is missing (build it with __graft_entry__.build())."""
    global _LIB
    if _LIB is None:
        p = lib_path()
        if not p.exists():
            raise RuntimeError(f"{p} is not built: the HIP path is required, there is no fallback")
        L = C.CDLL(str(p))
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _LIB = L
    return _LIB


def check(fn: str, status: int):
    if status != QH_OK:
        raise QuartzHipError(fn, status)
