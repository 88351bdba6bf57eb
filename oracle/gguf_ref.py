"""Pure-Python restatement of Quartz's GGUF reader (src/gguf.rs).

TEST INFRASTRUCTURE ONLY: the checker for the library's native GGUF reader
(saient_quartz_amd/csrc/qh_gguf.hip); only tests/ import it.

  parse            src/gguf.rs:68-113   header, metadata, tensor infos, data offset
  read_value       src/gguf.rs:224-244  typed values; arrays of one element type
  read_value_typed src/gguf.rs:246-262  array elements (no nested arrays)
  read_string      src/gguf.rs:216-222  u64 length + bytes (lossy utf-8)
  tensor_data      src/gguf.rs:116-121  ggml_type_size(type, n_elems) bytes at
                                        data_offset + offset
  ggml_type_size   src/gguf.rs:172-191

Errors raise GgufRefError with the reference's bail! message.  Pinned by
tests/test_gguf.py against files laid out as make_test_model.py writes them
(the reference's own writer) and hand-built v1/v2 files.
"""
import struct


class GgufRefError(Exception):
    pass


_SIZES = {0: ("<B", 1), 1: ("<b", 1), 2: ("<H", 2), 3: ("<h", 2), 4: ("<I", 4), 5: ("<i", 4),
          6: ("<f", 4), 7: ("<B", 1), 10: ("<Q", 8), 11: ("<q", 8), 12: ("<d", 8)}

# ggml type -> (elements per block, bytes per block); src/gguf.rs:172-191
TYPE_SIZE = {0: (1, 4), 1: (1, 2), 6: (32, 22), 7: (32, 24), 8: (32, 34), 10: (256, 84), 12: (256, 144),
             13: (256, 176), 14: (256, 210), 20: (32, 18), 30: (1, 2), 16: (256, 66), 17: (256, 74),
             22: (256, 82), 21: (256, 110)}


def ggml_type_size(t, n):
    if t not in TYPE_SIZE:
        raise GgufRefError(f"unsupported ggml_type: {t}")
    qk, b = TYPE_SIZE[t]
    return n // qk * b


class _R:
    def __init__(self, data):
        self.d, self.p = data, 0

    def take(self, n, what):
        if self.p + n > len(self.d):
            raise GgufRefError(f"EOF {what}")
        b = self.d[self.p:self.p + n]
        self.p += n
        return b

    def fmt(self, f, n, what):
        return struct.unpack(f, self.take(n, what))[0]

    def u32(self):
        return self.fmt("<I", 4, "u32")

    def u64(self):
        return self.fmt("<Q", 8, "u64")

    def string(self):
        n = self.u64()
        if self.p + n > len(self.d):
            raise GgufRefError(f"EOF reading string len={n}")
        return self.take(n, "string").decode("utf-8", "replace")

    def typed(self, t):
        if t == 8:
            return self.string()
        if t not in _SIZES:
            raise GgufRefError(f"Unknown array elem type: {t}")
        f, n = _SIZES[t]
        v = self.fmt(f, n, "value")
        return bool(v) if t == 7 else v

    def value(self, version):
        t = self.u32()
        if t == 9:
            et = self.u32()
            count = self.u32() if version == 1 else self.u64()
            return (9, [self.typed(et) for _ in range(count)], et)
        if t not in _SIZES and t != 8:
            raise GgufRefError(f"Unknown GGUF value type: {t}")
        return (t, self.typed(t), 0)


def parse(data: bytes):
    """-> dict(version, metadata {key: (type, value, elem_type)}, tensors [(name, dims,
    type, offset)], data_offset)."""
    r = _R(data)
    magic = r.u32()
    if magic != 0x46554747:
        raise GgufRefError(f"Not a GGUF file (magic 0x{magic:08X})")
    version = r.u32()
    if not 1 <= version <= 3:
        raise GgufRefError(f"Unsupported GGUF version {version}")
    nt = r.u32() if version == 1 else r.u64()
    nkv = r.u32() if version == 1 else r.u64()
    meta = {}
    for _ in range(nkv):
        k = r.string()
        meta[k] = r.value(version)
    tensors = []
    for _ in range(nt):
        name = r.string()
        nd = r.u32()
        dims = [r.u32() if version == 1 else r.u64() for _ in range(nd)]
        t = r.u32()
        off = r.u64()
        tensors.append((name, dims, t, off))
    a = meta.get("general.alignment")
    align = a[1] & 0xFFFFFFFF if a is not None and a[0] in (4, 5) else 32
    pos = r.p
    if pos % align:
        pos += align - pos % align
    return {"version": version, "metadata": meta, "tensors": tensors, "data_offset": pos}


def tensor_data(data: bytes, parsed, i):
    name, dims, t, off = parsed["tensors"][i]
    n = 1
    for d in dims:
        n *= d
    start = parsed["data_offset"] + off
    return data[start:start + ggml_type_size(t, n)]
