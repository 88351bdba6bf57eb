"""Host-side wrappers over the C ABI, mirroring Quartz's Rust FFI wrapper
(src/cuda.rs:59-150, 250-281): GpuBuf (RAII device buffer), GpuScratch (reusable
x/y buffers + gemv), gpu_expert_slice, ensure_iq_grids and verify_gemv_hip.
Same names and argument meaning; failures raise instead of panicking.
"""
import ctypes as C

import numpy as np

from .api import check, lib, type_size


class GpuBuf:
    """Owned device buffer (src/cuda.rs:59-90).  Freed with hip_drop."""

    def __init__(self, ptr: int, nbytes: int):
        self.ptr = ptr
        self.bytes = nbytes

    @classmethod
    def alloc(cls, nbytes: int) -> "GpuBuf":
        p = lib().hip_alloc(max(nbytes, 1))
        if not p:
            raise MemoryError(f"hipMalloc failed for {nbytes} bytes")
        return cls(p, nbytes)

    @classmethod
    def upload(cls, data: np.ndarray) -> "GpuBuf":
        data = np.ascontiguousarray(data)
        b = cls.alloc(data.nbytes)
        check("hip_h2d", lib().hip_h2d(b.ptr, data.ctypes.data, data.nbytes))
        return b

    @classmethod
    def alloc_f32(cls, n: int) -> "GpuBuf":
        return cls.alloc(4 * n)

    @classmethod
    def upload_f32(cls, data) -> "GpuBuf":
        return cls.upload(np.asarray(data, dtype=np.float32))

    def download(self, dtype=np.uint8, count=None) -> np.ndarray:
        dtype = np.dtype(dtype)
        count = self.bytes // dtype.itemsize if count is None else count
        out = np.empty(count, dtype=dtype)
        check("hip_d2h", lib().hip_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def drop(self):
        if self.ptr:
            lib().hip_drop(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.drop()
        except Exception:
            pass


class GpuSlice:
    """View into an uploaded stacked-expert tensor (src/cuda.rs:244-258)."""

    def __init__(self, ptr: int, ggml_type: int):
        self.ptr = ptr
        self.ggml_type = ggml_type


def gpu_expert_slice(buf: GpuBuf, ggml_type: int, expert: int, n_elems_per_expert: int) -> GpuSlice:
    return GpuSlice(buf.ptr + expert * type_size(ggml_type, n_elems_per_expert), ggml_type)


class GpuScratch:
    """Reusable x / y device buffers (src/cuda.rs:94-128, 261-281)."""

    def __init__(self, max_in: int, max_out: int):
        self.d_x = GpuBuf.alloc_f32(max_in)
        self.d_y = GpuBuf.alloc_f32(max_out)

    def _run(self, x, ptr, ggml_type, in_dim, out_dim):
        x = np.ascontiguousarray(x, dtype=np.float32)
        L = lib()
        check("hip_h2d", L.hip_h2d(self.d_x.ptr, x.ctypes.data, x.nbytes))
        check("hip_gemv", L.hip_gemv(ggml_type, ptr, self.d_x.ptr, self.d_y.ptr, in_dim, out_dim))
        out = np.empty(out_dim, dtype=np.float32)
        check("hip_d2h", L.hip_d2h(out.ctypes.data, self.d_y.ptr, out.nbytes))
        check("hip_sync", L.hip_sync())
        return out

    def gemv(self, x, data: GpuBuf, ggml_type: int, in_dim: int, out_dim: int) -> np.ndarray:
        return self._run(x, data.ptr, ggml_type, in_dim, out_dim)

    def gemv_slice(self, x, sl: GpuSlice, in_dim: int, out_dim: int) -> np.ndarray:
        return self._run(x, sl.ptr, sl.ggml_type, in_dim, out_dim)


def ensure_iq_grids():
    """src/cuda.rs:131-140.  The codebooks are resident from load time; nothing to do."""
    return None


def verify_gemv_hip(x, data: np.ndarray, ggml_type: int, in_dim: int, out_dim: int) -> np.ndarray:
    """src/cuda.rs:144-150: upload the raw tensor fresh, run one GEMV, return y."""
    ensure_iq_grids()
    buf = GpuBuf.upload(data)
    sc = GpuScratch(in_dim, out_dim)
    return sc.gemv(x, buf, ggml_type, in_dim, out_dim)


def gemv_multi_async(L, ggml_type, w_ptrs, y_ptrs, out_dims, x_ptr, in_dim, stream_ptr):
    """hip_gemv_multi_async with host arrays built from Python ints (device pointers)."""
    import ctypes as C
    k = len(w_ptrs)
    wa = (C.c_void_p * k)(*w_ptrs)
    ya = (C.c_void_p * k)(*y_ptrs)
    oa = (C.c_int * k)(*out_dims)
    check("hip_gemv_multi_async", L.hip_gemv_multi_async(ggml_type, k, wa, ya, oa, x_ptr, in_dim, stream_ptr))


def gemv_fused_async(L, ggml_type, w_ptrs, y_ptrs, out_dims, x_ptr, in_dim, stream_ptr, norm_ptr=None,
                     accumulate=False, scratch_ptr=None):
    """hip_gemv_fused_async: y_k (+)= W_k . rms_norm(x) * norm (norm optional), host
    arrays built from Python ints (device pointers)."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemv_fused_async",
          L.hip_gemv_fused_async(ggml_type, k, (C.c_void_p * k)(*w_ptrs), (C.c_void_p * k)(*y_ptrs),
                                 (C.c_int * k)(*out_dims), x_ptr, norm_ptr, 1 if accumulate else 0, in_dim,
                                 scratch_ptr, stream_ptr))


def gemv_group_async(L, types, w_ptrs, y_ptrs, out_dims, x_ptr, in_dim, stream_ptr, norm_ptr=None,
                     accumulate=False, scratch_ptr=None):
    """hip_gemv_group_async: GEMVs of per-matrix types sharing x (fused norm /
    residual optional), host arrays built from Python ints."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemv_group_async",
          L.hip_gemv_group_async(k, (C.c_uint32 * k)(*types), (C.c_void_p * k)(*w_ptrs), (C.c_void_p * k)(*y_ptrs),
                                 (C.c_int * k)(*out_dims), x_ptr, norm_ptr, 1 if accumulate else 0, in_dim,
                                 scratch_ptr, stream_ptr))


def gemm_grouped_async(L, ggml_type, w_ptrs, x_ptrs, y_ptrs, ns, out_dims, in_dim, stream_ptr):
    """hip_gemm_grouped_async with host arrays built from Python ints (device pointers)."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemm_grouped_async",
          L.hip_gemm_grouped_async(ggml_type, k, (C.c_void_p * k)(*w_ptrs), (C.c_void_p * k)(*x_ptrs),
                                   (C.c_void_p * k)(*y_ptrs), (C.c_int * k)(*ns), (C.c_int * k)(*out_dims),
                                   in_dim, stream_ptr))


def gemm_grouped_ex_async(L, ggml_type, w_ptrs, x_ptrs, y_ptrs, ns, out_dims, in_dim, stream_ptr, up_ptrs=None,
                          accumulate=False, scratch_ptr=None):
    """hip_gemm_grouped_ex_async: batched GEMMs with SwiGLU of (x, up) as input
    and/or the residual add fused in."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemm_grouped_ex_async",
          L.hip_gemm_grouped_ex_async(ggml_type, k, (C.c_void_p * k)(*w_ptrs), (C.c_void_p * k)(*x_ptrs),
                                      (C.c_void_p * k)(*up_ptrs) if up_ptrs else None, (C.c_void_p * k)(*y_ptrs),
                                      (C.c_int * k)(*ns), (C.c_int * k)(*out_dims), in_dim, 1 if accumulate else 0,
                                      scratch_ptr, stream_ptr))


def gemm_grouped_norm_async(L, ggml_type, w_ptrs, x_ptr, norm_w_ptr, y_ptrs, n, out_dims, in_dim, stream_ptr,
                            scratch_ptr=None):
    """hip_gemm_grouped_norm_async: y[k] = W[k] (rms_norm(x) * norm_w) for the n token rows of x."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemm_grouped_norm_async",
          L.hip_gemm_grouped_norm_async(ggml_type, k, (C.c_void_p * k)(*w_ptrs), x_ptr, norm_w_ptr,
                                        (C.c_void_p * k)(*y_ptrs), n, (C.c_int * k)(*out_dims), in_dim, scratch_ptr,
                                        stream_ptr))


def gemm_group_norm_async(L, types, w_ptrs, x_ptr, norm_w_ptr, y_ptrs, n, out_dims, in_dim, stream_ptr,
                          scratch_ptr=None):
    """hip_gemm_group_norm_async: gemm_grouped_norm_async over matrices of mixed types."""
    import ctypes as C
    k = len(w_ptrs)
    check("hip_gemm_group_norm_async",
          L.hip_gemm_group_norm_async(k, (C.c_uint32 * k)(*types), (C.c_void_p * k)(*w_ptrs), x_ptr, norm_w_ptr,
                                      (C.c_void_p * k)(*y_ptrs), n, (C.c_int * k)(*out_dims), in_dim, scratch_ptr,
                                      stream_ptr))


def gemm_moe_async(L, ggml_type, experts_ptr, expert_ids, tok_off, x_ptr, y_ptr, in_dim, out_dim, stream_ptr):
    """hip_gemm_moe_async: expert_ids[i] takes gathered tokens tok_off[i] .. tok_off[i+1]-1."""
    import ctypes as C
    k = len(expert_ids)
    assert len(tok_off) == k + 1
    check("hip_gemm_moe_async",
          L.hip_gemm_moe_async(ggml_type, experts_ptr, k, (C.c_int * k)(*expert_ids), (C.c_int * (k + 1))(*tok_off),
                               x_ptr, y_ptr, in_dim, out_dim, stream_ptr))


def gemm_moe_dev_async(L, ggml_type, experts_ptrs, y_ptrs, n_exp, tok_off_ptr, max_tokens, x_ptr, in_dim, out_dim,
                       stream_ptr, x_up_ptr=None, accumulate=False):
    """hip_gemm_moe_dev_async: token ranges read on the device from tok_off_ptr
    (n_exp + 1 ints); experts_ptrs / y_ptrs: one or two weight sets sharing x."""
    import ctypes as C
    k = len(experts_ptrs)
    assert len(y_ptrs) == k
    check("hip_gemm_moe_dev_async",
          L.hip_gemm_moe_dev_async(ggml_type, k, (C.c_void_p * k)(*experts_ptrs), (C.c_void_p * k)(*y_ptrs), n_exp,
                                   tok_off_ptr, max_tokens, x_ptr, x_up_ptr, in_dim, out_dim, int(accumulate),
                                   stream_ptr))
