"""ctypes binding of the CPU oracle (oracle/liboracle.so).  Test infrastructure."""
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
SO = ROOT / "oracle" / "liboracle.so"


class Oracle:
    _inst = None

    @classmethod
    def load(cls):
        if cls._inst is None:
            if not SO.exists():
                subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True)
            cls._inst = cls(C.CDLL(str(SO)))
        return cls._inst

    def __init__(self, L):
        self.L = L
        L.o_f16_to_f32.restype = C.c_float
        L.o_f16_to_f32.argtypes = [C.c_uint16]
        L.o_type_size.restype = C.c_size_t
        L.o_type_size.argtypes = [C.c_uint32, C.c_size_t]
        L.o_block_elems.restype = C.c_int
        L.o_block_elems.argtypes = [C.c_uint32]
        L.o_dequant.restype = C.c_int
        L.o_dequant.argtypes = [C.c_uint32, C.c_void_p, C.c_size_t, C.c_void_p]
        L.o_gemv.restype = C.c_int
        L.o_gemv.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p]
        L.o_gemv_dequant_matmul.restype = C.c_int
        L.o_gemv_dequant_matmul.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_void_p,
                                            C.c_void_p]
        L.o_gemm.restype = C.c_int
        L.o_gemm.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]
        L.o_set_threads.argtypes = [C.c_int]
        L.o_get_threads.restype = C.c_int
        L.o_grid_sha256.restype = C.c_char_p
        L.o_grid_sha256.argtypes = [C.c_int]
        L.o_f32_to_f16_rne.restype = C.c_uint16
        L.o_f32_to_f16_rne.argtypes = [C.c_float]
        L.o_quantize_q8_1_mmq.argtypes = [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        L.o_stream_k_cut.restype = C.c_int
        L.o_stream_k_cut.argtypes = [C.c_int] * 6
        L.o_gemm_q8_1_mmq.restype = C.c_int
        L.o_gemm_q8_1_mmq.argtypes = [C.c_uint32, C.c_void_p, C.c_void_p] + [C.c_int] * 5 + [C.c_void_p]

    def f16(self, bits: int) -> float:
        return self.L.o_f16_to_f32(bits)

    def type_size(self, t, n):
        return self.L.o_type_size(t, n)

    def dequant(self, t, data: np.ndarray, n: int) -> np.ndarray:
        data = np.ascontiguousarray(data, dtype=np.uint8)
        out = np.empty(n, dtype=np.float32)
        rc = self.L.o_dequant(t, data.ctypes.data, n, out.ctypes.data)
        if rc:
            raise ValueError(f"o_dequant rc={rc}")
        return out

    def gemv(self, t, x: np.ndarray, data: np.ndarray, in_dim: int, out_dim: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        y = np.empty(out_dim, dtype=np.float32)
        rc = self.L.o_gemv(t, x.ctypes.data, data.ctypes.data, in_dim, out_dim, y.ctypes.data)
        if rc:
            raise ValueError(f"o_gemv rc={rc}")
        return y

    def gemv_dequant_matmul(self, t, x: np.ndarray, data: np.ndarray, in_dim: int, out_dim: int,
                            w_scratch: np.ndarray = None) -> np.ndarray:
        """The `_` arm as the reference runs it: the whole matrix dequantized
        into w_scratch (out_dim * in_dim f32), then the row-parallel matmul."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        if w_scratch is None:
            w_scratch = np.empty(out_dim * in_dim, dtype=np.float32)
        assert w_scratch.dtype == np.float32 and w_scratch.size >= out_dim * in_dim
        y = np.empty(out_dim, dtype=np.float32)
        rc = self.L.o_gemv_dequant_matmul(t, x.ctypes.data, data.ctypes.data, in_dim, out_dim, w_scratch.ctypes.data,
                                          y.ctypes.data)
        if rc:
            raise ValueError(f"o_gemv_dequant_matmul rc={rc}")
        return y

    def gemm(self, t, x: np.ndarray, data: np.ndarray, in_dim: int, out_dim: int, n: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        y = np.empty((n, out_dim), dtype=np.float32)
        rc = self.L.o_gemm(t, x.ctypes.data, data.ctypes.data, in_dim, out_dim, n, y.ctypes.data)
        if rc:
            raise ValueError(f"o_gemm rc={rc}")
        return y

    def f32_to_f16_rne(self, v: float) -> int:
        return self.L.o_f32_to_f16_rne(v)

    def quantize_q8_1(self, x: np.ndarray, in_dim: int, rows: int, d4: bool):
        x = np.ascontiguousarray(x, dtype=np.float32)
        q = np.empty(rows * in_dim, dtype=np.int8)
        sc = np.empty(rows * in_dim // 32, dtype=np.float32)
        sm = np.empty(rows * in_dim // 32, dtype=np.float32)
        self.L.o_quantize_q8_1_mmq(x.ctypes.data, in_dim, rows, 1 if d4 else 0, q.ctypes.data, sc.ctypes.data,
                                   sm.ctypes.data)
        return q.reshape(rows, in_dim), sc.reshape(rows, -1), sm.reshape(rows, -1)

    def stream_k_cut(self, row, column, in_dim, out_dim, reference_rows, mps) -> int:
        return self.L.o_stream_k_cut(row, column, in_dim, out_dim, reference_rows, mps)

    def gemm_q8_1_mmq(self, t, x, data, in_dim, out_dim, rows, reference_rows=0, mps=0) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        data = np.ascontiguousarray(data, dtype=np.uint8)
        y = np.empty((rows, out_dim), dtype=np.float32)
        rc = self.L.o_gemm_q8_1_mmq(t, x.ctypes.data, data.ctypes.data, in_dim, out_dim, rows, reference_rows, mps,
                                    y.ctypes.data)
        if rc:
            raise ValueError(f"o_gemm_q8_1_mmq rc={rc}")
        return y

    def set_threads(self, n):
        self.L.o_set_threads(n)

    def threads(self):
        return self.L.o_get_threads()
