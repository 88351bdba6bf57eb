"""GGUF container access through the library's native reader / writer
(include/quartz_hip.h, hip_gguf_*), mirroring Quartz's GgufFile
(src/gguf.rs:52-169): the same fields (version, metadata, tensors, data_offset)
and accessors (tensor_data, tensor_map, architecture, meta_u32, meta_u64,
arch_u32, arch_u32_any, arch_f32, arch_f32_any), plus `upload` (a tensor to a
GpuBuf, as GpuWeights::from_weights does, src/cuda.rs:170-172) and GgufWriter,
which writes what make_test_model.py writes, for any type.
"""
import ctypes as C
from dataclasses import dataclass

import numpy as np

from .api import QuartzHipError, check, lib

# GGUF metadata value types (src/gguf.rs:224-243)
U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_NP = {U8: np.uint8, I8: np.int8, U16: np.uint16, I16: np.int16, U32: np.uint32, I32: np.int32,
       F32: np.float32, BOOL: np.uint8, U64: np.uint64, I64: np.int64, F64: np.float64}


class GgufError(QuartzHipError):
    pass


@dataclass
class TensorInfo:
    """src/gguf.rs:37-50.  dims[0] is the fastest-varying dimension."""
    name: str
    n_dims: int
    dims: list
    ggml_type: int
    offset: int
    index: int = -1

    def n_elems(self) -> int:
        n = 1
        for d in self.dims:
            n *= d
        return n


@dataclass
class Value:
    """A metadata value: `type` is the GGUF value type, `elem` the element type
    of an array; `value` is a Python scalar / str / list (string arrays) or a
    numpy array (other arrays)."""
    type: int
    value: object
    elem: int = 0

    def as_u32(self):
        return self.value & 0xFFFFFFFF if self.type in (U32, I32) else None

    def as_u64(self):
        return self.value if self.type in (U64, U32) else None

    def as_str(self):
        return self.value if self.type == STRING else None


class GgufFile:
    def __init__(self, path):
        self.L = lib()
        h = C.c_void_p()
        rc = self.L.hip_gguf_open(str(path).encode(), C.byref(h))
        if rc:
            raise GgufError("hip_gguf_open", rc)
        self._h = h
        L = self.L
        self.version = L.hip_gguf_version(h)
        self.data_offset = L.hip_gguf_data_offset(h)
        self.alignment = L.hip_gguf_alignment(h)
        self.metadata = {}
        for i in range(L.hip_gguf_kv_count(h)):
            key = L.hip_gguf_kv_key(h, i)
            self.metadata[key.decode("utf-8", "replace")] = self._value(key)
        self.tensors = []
        name = C.c_char_p()
        nd = C.c_uint32()
        dims = (C.c_uint64 * 8)()
        t = C.c_uint32()
        off = C.c_uint64()
        for i in range(L.hip_gguf_tensor_count(h)):
            check("hip_gguf_tensor_info", L.hip_gguf_tensor_info(h, i, C.byref(name), C.byref(nd), dims, C.byref(t),
                                                                 C.byref(off)))
            n = nd.value
            if n > 8:
                raise GgufError("hip_gguf_tensor_info", -5)
            self.tensors.append(TensorInfo(name.value.decode("utf-8", "replace"), n, list(dims[:n]), t.value,
                                           off.value, i))

    def _value(self, key: bytes) -> Value:
        L, h = self.L, self._h
        elem, count = C.c_uint32(), C.c_uint64()
        t = L.hip_gguf_kv_type(h, key, C.byref(elem), C.byref(count))
        if t == STRING:
            n = C.c_uint64()
            p = L.hip_gguf_get_str(h, key, C.byref(n))
            return Value(t, C.string_at(p, n.value).decode("utf-8", "replace"))
        if t == ARRAY:
            if elem.value == STRING:
                out = []
                for i in range(count.value):
                    n = C.c_uint64()
                    p = L.hip_gguf_get_array_str(h, key, i, C.byref(n))
                    out.append(C.string_at(p, n.value).decode("utf-8", "replace"))
                return Value(t, out, elem.value)
            e, c = C.c_uint32(), C.c_uint64()
            p = L.hip_gguf_get_array(h, key, C.byref(e), C.byref(c))
            dt = np.dtype(_NP[e.value])
            raw = C.string_at(p, c.value * dt.itemsize) if c.value else b""
            return Value(t, np.frombuffer(raw, dtype=dt).copy(), e.value)
        if t == F32:
            v = C.c_float()
            check("hip_gguf_get_f32", L.hip_gguf_get_f32(h, key, C.byref(v)))
            return Value(t, v.value)
        if t == F64:
            v = C.c_double()
            check("hip_gguf_get_f64", L.hip_gguf_get_f64(h, key, C.byref(v)))
            return Value(t, v.value)
        v = C.c_int64()
        check("hip_gguf_get_i64", L.hip_gguf_get_i64(h, key, C.byref(v)))
        x = v.value
        if t in (U8, U16, U32, U64, BOOL):
            x &= (1 << (8 * _NP[t]().itemsize)) - 1
        return Value(t, bool(x) if t == BOOL else x)

    def close(self):
        if getattr(self, "_h", None):
            self.L.hip_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    # ---- GgufFile accessors (src/gguf.rs:116-169)
    def tensor_data(self, info: TensorInfo) -> np.ndarray:
        """The tensor's bytes (a copy of the mapped range)."""
        n = C.c_size_t()
        p = self.L.hip_gguf_tensor_data(self._h, info.index, C.byref(n))
        if not p:
            raise GgufError("hip_gguf_tensor_data", -6)
        return np.frombuffer(C.string_at(p, n.value), dtype=np.uint8).copy()

    def tensor_map(self) -> dict:
        return {t.name: t for t in self.tensors}

    def architecture(self):
        v = self.metadata.get("general.architecture")
        return v.as_str() if v else None

    def meta_u32(self, key):
        v = self.metadata.get(key)
        return v.as_u32() if v else None

    def meta_u64(self, key):
        v = self.metadata.get(key)
        return v.as_u64() if v else None

    def arch_u32(self, suffix):
        return self.meta_u32(f"{self.architecture() or 'llama'}.{suffix}")

    def arch_u32_any(self, suffixes):
        for s in suffixes:
            v = self.arch_u32(s)
            if v is not None:
                return v
        return None

    def arch_f32(self, suffix):
        v = self.metadata.get(f"{self.architecture() or 'llama'}.{suffix}")
        return v.value if v is not None and v.type == F32 else None

    def arch_f32_any(self, suffixes):
        for s in suffixes:
            v = self.arch_f32(s)
            if v is not None:
                return v
        return None

    def upload(self, info: TensorInfo):
        """The tensor in a new device buffer (GpuBuf, freed with hip_drop)."""
        from .host import GpuBuf
        p, n = C.c_void_p(), C.c_size_t()
        check("hip_gguf_upload", self.L.hip_gguf_upload(self._h, info.index, C.byref(p), C.byref(n)))
        return GpuBuf(p.value, n.value)


class GgufWriter:
    """Builds a GGUF v3 file (make_test_model.py's layout) through the native writer."""

    def __init__(self):
        self.L = lib()
        self._w = self.L.hip_gguf_writer_new()
        self._keep = []  # host buffers the writer points at until write()

    def add(self, key: str, vtype: int, value):
        k = key.encode()
        if vtype == STRING:
            b = value.encode()
            check("kv_str", self.L.hip_gguf_writer_kv_str(self._w, k, b, len(b)))
        elif vtype == ARRAY:
            elem, items = value
            if elem == STRING:
                bs = [s.encode() for s in items]
                ptrs = (C.c_char_p * max(len(bs), 1))(*bs)
                lens = (C.c_uint64 * max(len(bs), 1))(*[len(b) for b in bs])
                check("kv_array_str", self.L.hip_gguf_writer_kv_array_str(self._w, k, ptrs, lens, len(bs)))
            else:
                a = np.ascontiguousarray(np.asarray(items, dtype=_NP[elem]))
                check("kv_array", self.L.hip_gguf_writer_kv_array(self._w, k, elem, a.ctypes.data, a.size))
        else:
            a = np.zeros(1, dtype=np.uint64)
            a.view(_NP[vtype])[0] = value
            check("kv_scalar", self.L.hip_gguf_writer_kv_scalar(self._w, k, vtype, a.ctypes.data))
        return self

    def add_tensor(self, name: str, data: np.ndarray, dims, ggml_type: int):
        """dims[0] fastest-varying (for a [rows][cols] matrix: [cols, rows]); data
        holds the tensor's bytes (any dtype, C order)."""
        data = np.ascontiguousarray(data)
        self._keep.append(data)
        d = (C.c_uint64 * max(len(dims), 1))(*dims)
        check("hip_gguf_writer_tensor",
              self.L.hip_gguf_writer_tensor(self._w, name.encode(), len(dims), d, ggml_type, data.ctypes.data))
        return self

    def write(self, path):
        check("hip_gguf_writer_write", self.L.hip_gguf_writer_write(self._w, str(path).encode()))

    def __del__(self):
        try:
            if self._w:
                self.L.hip_gguf_writer_free(self._w)
                self._w = None
        except Exception:
            pass
