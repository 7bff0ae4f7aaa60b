"""GGUF reader (flatrun_amd.gguf) on the CPU.

The first group restates the reference's own reader tests
(src/flatrun/tests/test_gguf.py:104-284): the same synthetic file -- three
F32 4x4 tensors named blk.0.attn_{q,k,v}.weight, qwen2 metadata, 32-byte
alignment -- built here by an independent byte-level writer that follows the
GGUF layout (not the package's write_gguf), and the same expectations
(translated names, metadata values, shape, dtype, byte size, payloads, error
messages). The rest covers what those tests leave open: block-quantized
tensors of every format the kernels serve, ne[] reversal of non-square
matrices, a non-default alignment, version 2, every metadata value type,
and malformed files.
"""

from __future__ import annotations

import struct

import numpy as np
import pytest

from flatrun_amd import gguf, synth


# ----------------------------------------------------------- independent writer
def _s(text: str) -> bytes:
    b = (text + "\x00").encode()          # NUL-terminated, as the reference's test writer does
    return struct.pack("<Q", len(b)) + b


def _kv(key: str, vtype: int, body: bytes) -> bytes:
    return _s(key) + struct.pack("<I", vtype) + body


def build(tensors, kvs, *, version=3, align=32):
    """tensors: (name, ne list (fastest first), type id, payload); kvs: encoded KV entries."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)) + b"".join(kvs)
    rel, cur = [], 0
    for _, _, _, payload in tensors:
        rel.append(cur)
        cur += (len(payload) + align - 1) // align * align
    for (name, ne, tid, _), off in zip(tensors, rel):
        head += _s(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        head += struct.pack("<IQ", tid, off)
    out = head + b"\0" * ((-len(head)) % align)
    for _, _, _, payload in tensors:
        out += payload + b"\0" * ((-len(payload)) % align)
    return out


@pytest.fixture()
def tiny(tmp_path):
    """The reference test's fixture (test_gguf.py:170-186)."""
    kvs = [
        _kv("general.architecture", 8, _s("qwen2")),
        _kv("general.alignment", 10, struct.pack("<q", 32)),
        _kv("qwen2.embedding_length", 10, struct.pack("<q", 16)),
        _kv("qwen2.block_count", 10, struct.pack("<q", 2)),
    ]
    tensors = [
        ("blk.0.attn_q.weight", [4, 4], 0, np.zeros(16, np.float32).tobytes()),
        ("blk.0.attn_k.weight", [4, 4], 0, np.arange(16, dtype=np.float32).tobytes()),
        ("blk.0.attn_v.weight", [4, 4], 0, np.full(16, 7.0, np.float32).tobytes()),
    ]
    p = tmp_path / "tiny.gguf"
    p.write_bytes(build(tensors, kvs))
    return p


# ------------------------------------------------ the reference's expectations
def test_translate_blk_prefix():
    assert gguf.translate_gguf_name("blk.0.attn_q.weight", "qwen2") == "model.layers.0.self_attn.q_proj.weight"


def test_translate_unlayered():
    assert gguf.translate_gguf_name("token_embd.weight", "qwen2") == "model.embed_tokens.weight"


def test_translate_passthrough_non_qwen():
    assert gguf.translate_gguf_name("blk.0.attn_q.weight", "llama") == "blk.0.attn_q.weight"


def test_open_lists_and_translates(tiny):
    with gguf.GGUFFile(tiny) as f:
        names = set(f.names())
    assert {"model.layers.0.self_attn.q_proj.weight", "model.layers.0.self_attn.k_proj.weight",
            "model.layers.0.self_attn.v_proj.weight"} <= names


def test_metadata_kv(tiny):
    with gguf.GGUFFile(tiny) as f:
        assert f.metadata["general.architecture"] == "qwen2"
        assert f.metadata["qwen2.embedding_length"] == 16
        assert f.metadata["qwen2.block_count"] == 2


def test_metadata_shape_dtype_size(tiny):
    with gguf.GGUFFile(tiny) as f:
        m = f.info("model.layers.0.self_attn.q_proj.weight")
        assert m.shape == (4, 4)
        assert m.quantization is None and m.dtype == "float32"
        assert m.nbytes == 4 * 4 * 4
        assert m.offset < tiny.stat().st_size


def test_missing_tensor(tiny):
    with gguf.GGUFFile(tiny) as f:
        with pytest.raises(gguf.TensorNotFound):
            f.info("does.not.exist")
        with pytest.raises(KeyError):
            f.raw("does.not.exist")


def test_payloads(tiny):
    with gguf.GGUFFile(tiny) as f:
        np.testing.assert_array_equal(f.raw("model.layers.0.self_attn.q_proj.weight"), np.zeros((4, 4), np.float32))
        np.testing.assert_array_equal(f.raw("model.layers.0.self_attn.k_proj.weight"),
                                      np.arange(16, dtype=np.float32).reshape(4, 4))
        np.testing.assert_array_equal(f.raw("model.layers.0.self_attn.v_proj.weight"), np.full((4, 4), 7.0, np.float32))


def test_bad_magic(tmp_path):
    p = tmp_path / "bad.gguf"
    p.write_bytes(b"XXXX" + b"\x00" * 64)
    with pytest.raises(gguf.GGUFError, match="Bad GGUF magic"):
        gguf.GGUFFile(p)


def test_unsupported_version(tmp_path):
    p = tmp_path / "v1.gguf"
    p.write_bytes(b"GGUF" + struct.pack("<I", 1) + struct.pack("<QQ", 0, 0))
    with pytest.raises(gguf.GGUFError, match="Unsupported GGUF version"):
        gguf.GGUFFile(p)


# ------------------------------------------------------------ beyond those
QUANT = [("Q4_K", 3, 512), ("Q6_K", 5, 768), ("Q8_0", 7, 96), ("Q5_K", 2, 256), ("Q1_0", 4, 384),
         ("Q4_0", 3, 64), ("Q5_0", 2, 96), ("Q5_1", 5, 32)]


def test_quantized_tensors_zero_copy(tmp_path):
    tensors, raws = [], {}
    for i, (q, n, k) in enumerate(QUANT):
        raw = synth.make_blocks(q, n, k, seed=i)
        raws[q] = raw
        tensors.append((f"blk.{i}.ffn_up.weight", [k, n], gguf.TYPE_IDS[q], raw.tobytes()))
    p = tmp_path / "q.gguf"
    p.write_bytes(build(tensors, [_kv("general.architecture", 8, _s("llama"))]))
    with gguf.GGUFFile(p) as f:
        for i, (q, n, k) in enumerate(QUANT):
            t = f.info(f"model.layers.{i}.mlp.up_proj.weight")      # translated although arch = llama
            assert t.gguf_name == f"blk.{i}.ffn_up.weight"
            assert t.shape == (n, k) and t.matrix == (n, k)         # ne = [k, n] reversed
            assert t.type_name == q and t.quantization == q and t.dtype == "uint8"
            assert t.nbytes == synth.nbytes(q, n, k) == raws[q].nbytes
            assert t.offset % 32 == 0
            v = f.raw(t.name)
            assert v.dtype == np.uint8 and v.shape == (t.nbytes,) and not v.flags.writeable
            assert np.array_equal(v, raws[q])


def test_translate_off_and_f16(tmp_path):
    h = (np.arange(24, dtype=np.float16) - 5).reshape(2, 12)
    p = tmp_path / "f16.gguf"
    p.write_bytes(build([("output_norm.weight", [12, 2], 1, h.tobytes())], []))
    with gguf.GGUFFile(p, translate_names=False) as f:
        assert f.names() == ["output_norm.weight"]
        a = f.raw("output_norm.weight")
        assert a.dtype == np.float16 and a.shape == (2, 12) and np.array_equal(a, h)
    with gguf.GGUFFile(p) as f:
        assert f.names() == ["model.norm.weight"]


def test_alignment_64_and_version_2(tmp_path):
    raw = synth.make_blocks("Q8_0", 3, 64, seed=5)               # 204 bytes: not a multiple of 64
    tensors = [("a.weight", [64, 3], 8, raw.tobytes()), ("b.weight", [64, 3], 8, raw[::-1].tobytes())]
    p = tmp_path / "a64.gguf"
    p.write_bytes(build(tensors, [_kv("general.alignment", 4, struct.pack("<I", 64))], version=2, align=64))
    with gguf.GGUFFile(p) as f:
        assert f.version == 2 and f.alignment == 64 and f.data_offset % 64 == 0
        assert f.info("a.weight").offset % 64 == 0 and f.info("b.weight").offset % 64 == 0
        assert np.array_equal(f.raw("b.weight"), raw[::-1])


def test_every_metadata_value_type(tmp_path):
    kvs = [
        _kv("u8", 0, struct.pack("<B", 200)), _kv("i8", 1, struct.pack("<b", -3)),
        _kv("u16", 2, struct.pack("<H", 60000)), _kv("i16", 3, struct.pack("<h", -300)),
        _kv("u32", 4, struct.pack("<I", 4000000000)), _kv("i32", 5, struct.pack("<i", -70000)),
        _kv("f32", 6, struct.pack("<f", 0.5)), _kv("bool", 7, struct.pack("<?", True)),
        _kv("str", 8, _s("héllo")),
        _kv("u64", 10, struct.pack("<Q", 2 ** 63 + 5)), _kv("i64", 11, struct.pack("<q", -(2 ** 40))),
        _kv("f64", 12, struct.pack("<d", 1e300)),
        _kv("arr_i32", 9, struct.pack("<IQ", 5, 3) + struct.pack("<3i", 1, -2, 3)),
        _kv("arr_str", 9, struct.pack("<IQ", 8, 2) + _s("a") + _s("bc")),
        _kv("arr_arr", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 0, 2) + bytes([1, 2])
            + struct.pack("<IQ", 0, 1) + bytes([3])),
        _kv("arr_bool", 9, struct.pack("<IQ", 7, 2) + bytes([1, 0])),
    ]
    p = tmp_path / "kv.gguf"
    p.write_bytes(build([], kvs))
    with gguf.GGUFFile(p) as f:
        m = f.metadata
    assert (m["u8"], m["i8"], m["u16"], m["i16"], m["u32"], m["i32"]) == (200, -3, 60000, -300, 4000000000, -70000)
    assert m["f32"] == 0.5 and m["bool"] is True and m["str"] == "héllo"
    assert m["u64"] == 2 ** 63 + 5 and m["i64"] == -(2 ** 40) and m["f64"] == 1e300
    assert m["arr_i32"] == [1, -2, 3] and m["arr_str"] == ["a", "bc"] and m["arr_arr"] == [[1, 2], [3]]
    assert m["arr_bool"] == [True, False]


def test_malformed_files(tmp_path):
    good = build([("w.weight", [32, 2], 8, synth.make_blocks("Q8_0", 2, 32, seed=1).tobytes())],
                 [_kv("general.architecture", 8, _s("qwen2"))])
    cases = {
        "short": b"GGUF\x03\x00",
        "truncated_header": good[:40],
        "tensor_past_eof": good[:-40],
        "bad_kv_type": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + _kv("k", 99, b"\0" * 8),
        "huge_string": b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", 1 << 40) + b"\0" * 16,
    }
    for name, data in cases.items():
        p = tmp_path / f"{name}.gguf"
        p.write_bytes(data)
        with pytest.raises(gguf.GGUFError):
            gguf.GGUFFile(p)
    with pytest.raises(gguf.GGUFError, match="not found"):
        gguf.GGUFFile(tmp_path / "absent.gguf")


def test_package_writer_round_trip(tmp_path):
    """write_gguf (the package's writer, used for synthetic model files) reads back
    through both the reader and the independent byte layout above."""
    raw = synth.make_blocks("Q4_K", 6, 512, seed=9)
    meta = {"general.architecture": "llama", "llama.block_count": 32, "neg": -7, "eps": 1e-5,
            "toks": ["a", "b"], "flag": False}
    p = tmp_path / "w.gguf"
    gguf.write_gguf(p, [("blk.3.attn_q.weight", (6, 512), "Q4_K", raw.tobytes()),
                        ("blk.3.attn_norm.weight", (512,), "F32", np.ones(512, np.float32).tobytes())],
                    meta, alignment=128)
    expect = build([("blk.3.attn_q.weight", [512, 6], 12, raw.tobytes()),
                    ("blk.3.attn_norm.weight", [512], 0, np.ones(512, np.float32).tobytes())], [], align=128)
    with gguf.GGUFFile(p) as f:
        assert f.alignment == 128
        assert f.metadata["llama.block_count"] == 32 and f.metadata["neg"] == -7
        assert abs(f.metadata["eps"] - 1e-5) < 1e-12 and f.metadata["toks"] == ["a", "b"] and f.metadata["flag"] is False
        q = f.info("model.layers.3.self_attn.q_proj.weight")
        assert q.shape == (6, 512) and np.array_equal(f.raw(q.name), raw)
        nrm = f.raw("model.layers.3.input_layernorm.weight")
        assert nrm.shape == (512,) and np.all(nrm == 1.0)
    # same tensor data section as the independent layout (metadata differs)
    data = p.read_bytes()
    with gguf.GGUFFile(p) as f:
        start = f.data_offset
    tail = expect[len(expect) - (len(data) - start):]
    assert data[start:] == tail
