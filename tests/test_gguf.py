"""The native GGUF reader / writer (hip_gguf_*) against the reference's format:
files laid out as make_test_model.py writes them (the reference's own writer,
restated below from its documented packing), the restated reader
oracle/gguf_ref.py (src/gguf.rs), hand-built v1/v2 files, and the reference's
error messages.  CPU only: nothing here touches the GPU except the last test.
"""
import struct
import sys
from pathlib import Path

import numpy as np
import pytest

from saient_quartz_amd import synth
from saient_quartz_amd.gguf import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64,
                                    GgufError, GgufFile, GgufWriter)

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "oracle"))
import gguf_ref  # noqa: E402


# ---- make_test_model.py's container layout (vocab 64, embed 32, 4 heads, 2 kv heads,
# 1 layer, ffn 128, seed 42, F32 tensors, alignment 32), restated from the script.
def _pack_str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def tiny_model_tensors():
    rng = np.random.default_rng(42)
    V, E, H, KV, FF = 64, 32, 4, 2, 128
    hd = E // H
    t = {"token_embd.weight": rng.standard_normal((V, E)).astype(np.float32) * 0.02}
    t["blk.0.attn_norm.weight"] = np.ones(E, np.float32)
    t["blk.0.attn_q.weight"] = rng.standard_normal((H * hd, E)).astype(np.float32) * 0.02
    t["blk.0.attn_k.weight"] = rng.standard_normal((KV * hd, E)).astype(np.float32) * 0.02
    t["blk.0.attn_v.weight"] = rng.standard_normal((KV * hd, E)).astype(np.float32) * 0.02
    t["blk.0.attn_output.weight"] = rng.standard_normal((E, E)).astype(np.float32) * 0.02
    t["blk.0.ffn_norm.weight"] = np.ones(E, np.float32)
    t["blk.0.ffn_gate.weight"] = rng.standard_normal((FF, E)).astype(np.float32) * 0.02
    t["blk.0.ffn_up.weight"] = rng.standard_normal((FF, E)).astype(np.float32) * 0.02
    t["blk.0.ffn_down.weight"] = rng.standard_normal((E, FF)).astype(np.float32) * 0.02
    t["output_norm.weight"] = np.ones(E, np.float32)
    t["output.weight"] = rng.standard_normal((V, E)).astype(np.float32) * 0.02
    kv = [("general.architecture", STRING, "llama"), ("general.name", STRING, "quartz-test"),
          ("general.file_type", U32, 0), ("llama.embedding_length", U32, E), ("llama.head_count", U32, H),
          ("llama.head_count_kv", U32, KV), ("llama.block_count", U32, 1), ("llama.feed_forward_length", U32, FF),
          ("llama.vocab_size", U32, V), ("general.alignment", U32, 32)]
    return t, kv


def tiny_model_bytes():
    tensors, kv = tiny_model_tensors()
    kvb = b""
    for k, t, v in kv:
        kvb += _pack_str(k) + (struct.pack("<I", 8) + _pack_str(v) if t == STRING else struct.pack("<II", 4, v))
    parts, offs, cur = [], [], 0
    for a in tensors.values():
        offs.append(cur)
        d = a.flatten().astype(np.float32).tobytes()
        parts.append(d)
        cur += (len(d) + 31) & ~31
    info = b""
    for (name, a), off in zip(tensors.items(), offs):
        info += _pack_str(name) + struct.pack("<I", a.ndim)
        for s in a.shape[::-1]:
            info += struct.pack("<Q", s)
        info += struct.pack("<I", 0) + struct.pack("<Q", off)
    h = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(kv)) + kvb + info
    h += b"\x00" * ((32 - len(h) % 32) % 32)
    body = b"".join(d + b"\x00" * ((32 - len(d) % 32) % 32) for d in parts)
    return h + body


@pytest.fixture
def tiny(tmp_path):
    p = tmp_path / "tiny_model.gguf"
    p.write_bytes(tiny_model_bytes())
    return p


def test_reads_reference_tiny_model(tiny):
    tensors, kv = tiny_model_tensors()
    raw = tiny.read_bytes()
    ref = gguf_ref.parse(raw)
    with GgufFile(tiny) as f:
        assert f.version == 3 == ref["version"]
        assert f.data_offset == ref["data_offset"] and f.data_offset % 32 == 0
        assert list(f.metadata) == [k for k, _, _ in kv]
        for k, t, v in kv:
            assert f.metadata[k].type == t and f.metadata[k].value == v == ref["metadata"][k][1]
        assert f.architecture() == "llama"
        assert f.arch_u32("head_count_kv") == 2 and f.arch_u32_any(["missing", "block_count"]) == 1
        assert f.meta_u64("llama.vocab_size") == 64  # Uint32 reads as u64 (as_u64)
        assert [t.name for t in f.tensors] == list(tensors)
        for i, (t, (name, a)) in enumerate(zip(f.tensors, tensors.items())):
            assert t.dims == list(a.shape[::-1]) == ref["tensors"][i][1]
            assert t.ggml_type == 0 and t.offset == ref["tensors"][i][3]
            got = f.tensor_data(t)
            assert got.tobytes() == a.astype(np.float32).tobytes() == gguf_ref.tensor_data(raw, ref, i)
        assert f.tensor_map()["output.weight"].dims == [32, 64]


def test_writer_reproduces_reference_layout_bytewise(tmp_path):
    """The native writer, fed make_test_model.py's tensors and keys, writes the
    same bytes as the reference's script does."""
    tensors, kv = tiny_model_tensors()
    w = GgufWriter()
    for k, t, v in kv:
        w.add(k, t, v)
    for name, a in tensors.items():
        w.add_tensor(name, a.astype(np.float32), list(a.shape[::-1]), 0)
    p = tmp_path / "w.gguf"
    w.write(p)
    assert p.read_bytes() == tiny_model_bytes()


def test_every_value_type_round_trips(tmp_path):
    vals = [("a.u8", U8, 250), ("a.i8", I8, -7), ("a.u16", U16, 65000), ("a.i16", I16, -30000),
            ("a.u32", U32, 4000000000), ("a.i32", I32, -2000000000), ("a.f32", F32, 1.5), ("a.bool", BOOL, True),
            ("a.str", STRING, "héllo"), ("a.u64", U64, 2 ** 63 + 5), ("a.i64", I64, -(2 ** 62)), ("a.f64", F64, -2.25)]
    arrs = [("b.u8", U8, [1, 2, 255]), ("b.i16", I16, [-1, 7]), ("b.f32", F32, [0.5, -3.0, 2.0 ** 100]),
            ("b.u64", U64, [1, 2 ** 40]), ("b.f64", F64, [1.25]), ("b.bool", BOOL, [1, 0, 1]), ("b.empty", I32, []),
            ("b.strs", STRING, ["", "tok", "two words"])]
    w = GgufWriter()
    for k, t, v in vals:
        w.add(k, t, v)
    for k, e, v in arrs:
        w.add(k, ARRAY, (e, v))
    p = tmp_path / "v.gguf"
    w.write(p)
    ref = gguf_ref.parse(p.read_bytes())
    with GgufFile(p) as f:
        for k, t, v in vals:
            assert f.metadata[k].type == t
            assert f.metadata[k].value == pytest.approx(v) if t in (F32, F64) else f.metadata[k].value == v
            assert ref["metadata"][k][0] == t
        for k, e, v in arrs:
            m = f.metadata[k]
            assert m.type == ARRAY and m.elem == e
            assert list(m.value) == list(v) == [int(x) if e == BOOL else x for x in ref["metadata"][k][1]]
        assert f.meta_u32("a.i32") == (-2000000000) & 0xFFFFFFFF  # as_u32 of an Int32
        assert f.meta_u32("a.u64") is None and f.meta_u64("a.u32") == 4000000000
        assert f.tensors == [] and f.data_offset % 32 == 0


def _v1_or_v2(version, align=None):
    cnt = (lambda n: struct.pack("<I", n)) if version == 1 else (lambda n: struct.pack("<Q", n))
    kvs = [_pack_str("general.architecture") + struct.pack("<I", 8) + _pack_str("llama"),
           _pack_str("x.arr") + struct.pack("<II", 9, 5) + cnt(3) + struct.pack("<iii", -1, 0, 9)]
    if align:
        kvs.append(_pack_str("general.alignment") + struct.pack("<II", 5, align))
    data = np.arange(64, dtype=np.float32)
    info = _pack_str("w") + struct.pack("<I", 2) + cnt(16) + cnt(4) + struct.pack("<I", 0) + struct.pack("<Q", 0)
    h = struct.pack("<II", 0x46554747, version) + cnt(1) + cnt(len(kvs)) + b"".join(kvs) + info
    a = align or 32
    h += b"\x00" * ((a - len(h) % a) % a)
    return h + data.tobytes(), data


@pytest.mark.parametrize("version", [1, 2])
@pytest.mark.parametrize("align", [None, 64])
def test_older_versions_and_alignment(tmp_path, version, align):
    raw, data = _v1_or_v2(version, align)
    p = tmp_path / "o.gguf"
    p.write_bytes(raw)
    ref = gguf_ref.parse(raw)
    with GgufFile(p) as f:
        assert f.version == version
        assert f.alignment == (align or 32) and f.data_offset == ref["data_offset"]
        assert list(f.metadata["x.arr"].value) == [-1, 0, 9]
        assert f.tensors[0].dims == [16, 4]
        assert np.array_equal(f.tensor_data(f.tensors[0]).view(np.float32), data)


def test_quantized_tensor_bytes(tmp_path):
    w = synth.weights(12, 8, 512, seed=5)
    g = GgufWriter().add("general.alignment", U32, 32)
    g.add_tensor("blk.0.ffn_gate.weight", w, [512, 8], 12)
    g.add_tensor("odd", np.arange(3, dtype=np.float32), [3], 0)
    g.add_tensor("after", synth.weights(14, 2, 256, seed=6), [256, 2], 14)
    p = tmp_path / "q.gguf"
    g.write(p)
    with GgufFile(p) as f:
        assert f.tensor_data(f.tensors[0]).tobytes() == w.tobytes()
        assert f.tensors[1].offset % 32 == 0 and f.tensors[2].offset % 32 == 0
        assert len(f.tensor_data(f.tensors[2])) == 2 * 210


def test_duplicates_keep_the_last(tmp_path):
    g = GgufWriter().add("k", U32, 1).add("k", U32, 2)
    g.add_tensor("t", np.zeros(4, np.float32), [4], 0).add_tensor("t", np.ones(8, np.float32), [8], 0)
    p = tmp_path / "d.gguf"
    g.write(p)
    with GgufFile(p) as f:
        assert f.metadata["k"].value == 2  # HashMap::insert
        assert f.tensor_map()["t"].dims == [8] and len(f.tensors) == 2
        assert f.L.hip_gguf_find_tensor(f._h, b"t") == 1


@pytest.mark.parametrize("raw, msg", [
    (b"GGML" + b"\x00" * 20, "Not a GGUF file (magic 0x4C4D4747)"),
    (struct.pack("<II", 0x46554747, 4) + b"\x00" * 16, "Unsupported GGUF version 4"),
    (struct.pack("<II", 0x46554747, 0) + b"\x00" * 16, "Unsupported GGUF version 0"),
    (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _pack_str("k") + struct.pack("<I", 13), "Unknown GGUF value type: 13"),
    (struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + _pack_str("k") + struct.pack("<IIQ", 9, 9, 1),
     "Unknown array elem type: 9"),
])
def test_reference_error_messages(tmp_path, raw, msg):
    p = tmp_path / "bad.gguf"
    p.write_bytes(raw)
    with pytest.raises(gguf_ref.GgufRefError, match=msg.replace("(", r"\(").replace(")", r"\)")):
        gguf_ref.parse(raw)
    with pytest.raises(GgufError) as e:
        GgufFile(p)
    assert e.value.status == -6 and msg in str(e.value)


def test_every_truncation_is_an_error(tmp_path, tiny):
    """Every prefix of a valid file that cuts the header short fails cleanly
    (EOF), as the reference's bounds-checked readers do; prefixes that keep the
    header parse, and tensor_data refuses ranges past the end."""
    raw = tiny.read_bytes()
    hdr = gguf_ref.parse(raw)["data_offset"]
    p = tmp_path / "cut.gguf"
    for n in list(range(0, 64)) + list(range(64, hdr, 7)):
        p.write_bytes(raw[:n])
        try:
            gguf_ref.parse(raw[:n])
            ok_ref = True
        except gguf_ref.GgufRefError:
            ok_ref = False
        try:
            GgufFile(p).close()
            ok = True
        except GgufError as e:
            ok = False
            assert e.status == -6
        assert ok == ok_ref, n
    p.write_bytes(raw[:hdr + 100])
    with GgufFile(p) as f:
        with pytest.raises(GgufError):
            f.tensor_data(f.tensors[-1])


def test_missing_file_and_unsupported_type(tmp_path):
    with pytest.raises(GgufError) as e:
        GgufFile(tmp_path / "nope.gguf")
    assert e.value.status == -7
    raw = bytearray(tiny_model_bytes())
    # retag the first tensor (token_embd) as ggml type 4 (absent from ggml_type_size)
    ref = gguf_ref.parse(bytes(raw))
    i = bytes(raw).index(_pack_str("token_embd.weight")) + len(_pack_str("token_embd.weight")) + 4 + 16
    raw[i:i + 4] = struct.pack("<I", 4)
    p = tmp_path / "t4.gguf"
    p.write_bytes(bytes(raw))
    with GgufFile(p) as f:
        assert f.tensors[0].ggml_type == 4
        with pytest.raises(GgufError):
            f.tensor_data(f.tensors[0])
    with pytest.raises(gguf_ref.GgufRefError):
        gguf_ref.tensor_data(bytes(raw), gguf_ref.parse(bytes(raw)), 0)
    assert ref["tensors"][0][2] == 0


@pytest.mark.gpu
def test_upload_and_gemv_from_gguf(tmp_path, oracle):
    """A Q4_K tensor read from a GGUF file, uploaded (GpuWeights::from_weights)
    and multiplied: same result as the oracle on the written bytes."""
    import closed_form as cf
    from saient_quartz_amd.host import GpuScratch
    out_dim, in_dim = 300, 4096
    w = synth.weights(12, out_dim, in_dim, seed=9)
    g = GgufWriter().add("general.architecture", STRING, "llama")
    g.add_tensor("blk.0.attn_q.weight", w, [in_dim, out_dim], 12)
    p = tmp_path / "m.gguf"
    g.write(p)
    x = synth.activations(1, in_dim, seed=10)[0]
    with GgufFile(p) as f:
        t = f.tensor_map()["blk.0.attn_q.weight"]
        buf = f.upload(t)
        got = GpuScratch(in_dim, out_dim).gemv(x, buf, t.ggml_type, in_dim, out_dim)
    assert cf.rel_l2(got, oracle.gemv(12, x, w, in_dim, out_dim)) < 1e-3
