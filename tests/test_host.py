"""The host library (libgq_host.so): GGUF parsing and loading, on the CPU.

Cases follow the reference's own parser and loader tests
(src/parser.rs:198-303, src/loader.rs:104-119) plus every metadata kind,
tensor data read from a file and from a split set, and the error kinds
(src/error.rs:4-42).  Fixtures are written by tests/gguf_write.py.
"""
import os
import struct

import numpy as np
import pytest

import gguf_write as gw
import gq


def _gguf(data):
    return gq.GgufFile(data=data)


def _code(exc_info):
    return exc_info.value.code


def test_parse_minimal_v2():
    f = _gguf(gw.header(2, 0, 0))
    assert f.version == 2 and f.tensor_count == 0 and f.metadata_count == 0 and f.tensors == []
    assert f.data_offset == 32  # the 24-byte header rounded up


def test_invalid_magic():
    with pytest.raises(gq.GgufError) as e:
        _gguf(bytes(24))
    assert _code(e) == -101 and "magic" in str(e.value)


@pytest.mark.parametrize("version", [1, 4])
def test_unsupported_version(version):
    with pytest.raises(gq.GgufError) as e:
        _gguf(gw.header(version, 0, 0))
    assert _code(e) == -102 and f"version: {version}" in str(e.value)


def test_v3_string_and_u32_metadata():
    data, _ = gw.build_file([("general.architecture", gw.STRING, "llama"), ("test.value", gw.U32, 42)])
    f = _gguf(data)
    assert f.version == 3 and f.architecture() == "llama" and f.get_u64("test.value") == 42
    with pytest.raises(gq.GgufError) as e:
        f.get_string("test.value")
    assert _code(e) == -108
    assert f.get_u64("absent.key") is None


def test_tensor_info():
    data, _ = gw.build_file(tensors=[("output.weight", [4096, 4096], 8, b"")])
    f = _gguf(data)
    t = f.tensors[0]
    assert (t.name, t.dims, t.ggml_type, t.byte_offset) == ("output.weight", [4096, 4096], 8, 0)
    assert t.nbytes == 4096 * 4096 // 32 * 34


def test_array_metadata():
    data, _ = gw.build_file([("tokenizer.ggml.bos_token_id", gw.ARRAY, (gw.U32, [1]))])
    f = _gguf(data)
    assert f.get_i64_array("tokenizer.ggml.bos_token_id") == [1]


def test_unexpected_eof():
    with pytest.raises(gq.GgufError) as e:
        _gguf(gw.header(3, 0, 1))
    assert _code(e) == -103 and "byte 24" in str(e.value)


def test_every_metadata_kind():
    meta = [("u8", gw.U8, 200), ("i8", gw.I8, -100), ("u16", gw.U16, 60000), ("i16", gw.I16, -30000),
            ("u32", gw.U32, 4000000000), ("i32", gw.I32, -2000000000), ("f32", gw.F32, 1.5),
            ("t", gw.BOOL, True), ("f", gw.BOOL, False), ("s", gw.STRING, "héllo"),
            ("u64", gw.U64, 2 ** 63 + 5), ("i64", gw.I64, -(2 ** 62)), ("f64", gw.F64, -2.25),
            ("ai", gw.ARRAY, (gw.I32, [-1, 2, -3])), ("as", gw.ARRAY, (gw.STRING, ["a", "bc", ""])),
            ("empty", gw.ARRAY, (gw.U8, []))]
    f = _gguf(gw.build_file(meta)[0])
    assert f.metadata_count == len(meta)
    assert f.get("u8") == 200 and f.get("i8") == -100 and f.get("u16") == 60000
    assert f.get("i16") == -30000 and f.get("u32") == 4000000000 and f.get("i32") == -2000000000
    assert f.get("f32") == 1.5 and f.get("t") is True and f.get("f") is False
    assert f.get("s") == "héllo" and f.get("u64") == 2 ** 63 + 5 and f.get("i64") == -(2 ** 62)
    assert f.get("f64") == -2.25
    assert f.get("ai") == [-1, 2, -3] and f.get("as") == ["a", "bc", ""] and f.get("empty") == []
    # as_u64 covers only unsigned kinds; as_i64 every integer kind
    with pytest.raises(gq.GgufError):
        f.get_u64("i8")
    assert f.get_i64("u16") == 60000
    assert [f.meta_type(k) for k in ("u8", "f64", "ai")] == [0, 12, 9]


def test_bad_string_and_unknown_types():
    bad = gw.header(3, 0, 1) + struct.pack("<Q", 3) + b"k\xff\xfe" + struct.pack("<I", gw.U8) + b"\0"
    with pytest.raises(gq.GgufError) as e:
        _gguf(bad)
    assert _code(e) == -106
    unk = gw.header(3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<I", 13)
    with pytest.raises(gq.GgufError) as e:
        _gguf(unk)
    assert _code(e) == -104 and "13" in str(e.value)
    arr_of_arr = gw.header(3, 0, 1) + struct.pack("<Q", 1) + b"k" + struct.pack("<IIQ", 9, 9, 0)
    with pytest.raises(gq.GgufError) as e:
        _gguf(arr_of_arr)
    assert _code(e) == -104
    tens = gw.header(3, 1, 0) + struct.pack("<Q", 1) + b"t" + struct.pack("<IQIQ", 1, 32, 4, 0)
    with pytest.raises(gq.GgufError) as e:  # ggml type 4 does not exist
        _gguf(tens)
    assert _code(e) == -105


def test_truncated_everywhere():
    """Every prefix that stops inside the header or the tensor infos fails
    with UnexpectedEof, never worse; from the end of the tensor infos on
    (the padding to the data section is not needed to parse) it parses."""
    data, _ = gw.build_file([("a", gw.STRING, "xyz"), ("b", gw.ARRAY, (gw.U16, [1, 2]))],
                            [("w", [256, 2], 12, bytes(288))])
    header_len = len(data) - 288  # header, metadata, tensor infos, padding
    ok = []
    for n in range(header_len + 1):
        try:
            f = _gguf(data[:n])
            ok.append(n)
            assert f.data_offset == header_len
        except gq.GgufError as e:
            assert e.code == -103, n
    assert ok == list(range(ok[0], header_len + 1)) and header_len - 32 < ok[0]


@pytest.mark.parametrize("name,want", [("MiniMax-M2.7-UD-IQ4_XS-00001-of-00004.gguf", (1, 4)),
                                       ("model-00003-of-00005.gguf", (3, 5)),
                                       ("single.gguf", None), ("x-1-of-2.bin", None)])
def test_parse_split_index(name, want):
    assert gq.parse_split_index(name) == want


def _blocks(seed, nbytes):
    return np.random.default_rng(seed).integers(0, 256, nbytes, dtype=np.uint8).tobytes()


def test_load_file_tensor_bytes(tmp_path):
    a, b = _blocks(1, 144 * 2 * 3), _blocks(2, 210 * 4)
    path = tmp_path / "m.gguf"
    offs = gw.write(path, [("general.architecture", gw.STRING, "qwen2")],
                    [("blk.0.attn_q.weight", [512, 3], 12, a), ("output.weight", [256, 4], 14, b)])
    f = gq.GgufFile(path=str(path))
    assert [t.name for t in f.tensors] == ["blk.0.attn_q.weight", "output.weight"]
    assert f.tensors[1].byte_offset == offs[1] and offs[1] % 32 == 0
    assert f.tensor_bytes("blk.0.attn_q.weight").tobytes() == a
    assert f.tensor_bytes("output.weight").tobytes() == b
    assert f.data_offset % 32 == 0
    assert f.data_offset + offs[1] + (len(b) + 31) // 32 * 32 == os.path.getsize(path)
    with pytest.raises(gq.GgufError) as e:
        f.tensor_bytes("nope")
    assert _code(e) == -107
    f.close()


def test_load_missing_file(tmp_path):
    with pytest.raises(gq.GgufError) as e:
        gq.GgufFile(path=str(tmp_path / "absent.gguf"))
    assert _code(e) == -111


def test_tensor_past_end_of_file(tmp_path):
    data, _ = gw.build_file(tensors=[("w", [256, 2], 12, bytes(288))])
    path = tmp_path / "cut.gguf"
    path.write_bytes(data[:-10])
    f = gq.GgufFile(path=str(path))
    with pytest.raises(gq.GgufError) as e:
        f.tensor_bytes("w")
    assert _code(e) == -103


def test_split_files(tmp_path):
    """Part 1 holds the header and the first tensor; the second tensor's
    offset runs on into part 2 (MultiFileMmap::slice)."""
    a, b = _blocks(3, 144 * 2), _blocks(4, 144 * 3)
    data, offs = gw.build_file([("split.count", gw.U16, 2)],
                               [("first", [256, 2], 12, a), ("second", [256, 3], 12, b)])
    f0 = gq.GgufFile(data=data)
    cut = f0.data_offset + offs[1]  # part 2 starts exactly at the second tensor
    (tmp_path / "m-00001-of-00002.gguf").write_bytes(data[:cut])
    (tmp_path / "m-00002-of-00002.gguf").write_bytes(data[cut:])
    f = gq.GgufFile(path=str(tmp_path / "m-00001-of-00002.gguf"))
    assert f.tensor_bytes("first").tobytes() == a and f.tensor_bytes("second").tobytes() == b
    (tmp_path / "m-00002-of-00002.gguf").unlink()
    with pytest.raises(gq.GgufError) as e:
        gq.GgufFile(path=str(tmp_path / "m-00001-of-00002.gguf"))
    assert _code(e) == -111


# ---- gqh_model_load: what is refused before any device work -------------

def _decoder_file(tmp_path, extra_meta=(), extra_tensors=(), drop=()):
    H, V = 64, 10
    md = gw.decoder_metadata(dict(n_layers=1, hidden=H, ffn=128, n_heads=2, n_kv_heads=1,
                                  theta=1e6, eps=1e-6), extra=extra_meta)
    z32 = np.zeros(H, np.float32).tobytes()
    q4 = lambda rows, cols: bytes(rows * (cols // 256 + (cols % 256 > 0)) * 144)
    ts = [("token_embd.weight", [H, V], 0, np.zeros((V, H), np.float32).tobytes()),
          ("blk.0.attn_norm.weight", [H], 0, z32), ("blk.0.ffn_norm.weight", [H], 0, z32),
          ("blk.0.attn_q.weight", [H, H], 12, b""), ("output_norm.weight", [H], 0, z32)]
    ts = [t for t in ts if t[0] not in drop] + list(extra_tensors)
    path = str(tmp_path / "m.gguf")
    gw.write(path, md, ts)
    return gq.GgufFile(path)


@pytest.mark.parametrize("extra,what", [
    ([("blk.0.shortconv.conv.weight", [3, 64], 0, bytes(768))], "ShortConv"),
    ([("blk.0.ssm_alpha.weight", [64, 2], 0, bytes(512))], "GatedDeltaNet"),
    ([("blk.0.attn_q_norm.weight", [32], 0, bytes(128))], "QK-norm"),
])
def test_model_load_refuses_uncovered_mixers(tmp_path, extra, what):
    f = _decoder_file(tmp_path, extra_tensors=extra)
    with pytest.raises(gq.GgufError) as e:
        f.load_model()
    assert _code(e) == -112 and what in str(e.value)


def test_model_load_refuses_gated_attention(tmp_path):
    f = _decoder_file(tmp_path, drop=("blk.0.attn_q.weight",),
                      extra_tensors=[("blk.0.attn_q.weight", [64, 128], 12, b"")])
    with pytest.raises(gq.GgufError) as e:
        f.load_model()
    assert _code(e) == -112 and "GatedAttention" in str(e.value)


def test_model_load_refuses_rope_scaling(tmp_path):
    f = _decoder_file(tmp_path, extra_meta=[("qwen2.rope.scaling.type", gw.STRING, "yarn")])
    with pytest.raises(gq.GgufError) as e:
        f.load_model()
    assert _code(e) == -112 and "yarn" in str(e.value)


@pytest.mark.parametrize("drop,what", [("token_embd.weight", "token_embd.weight"),
                                       ("blk.0.attn_q.weight", "blk.0.attn_q.weight")])
def test_model_load_missing_tensors(tmp_path, drop, what):
    f = _decoder_file(tmp_path, drop=(drop,))
    with pytest.raises(gq.GgufError) as e:
        f.load_model()
    assert _code(e) == -107 and what in str(e.value)


def test_model_load_missing_head_count(tmp_path):
    f = _decoder_file(tmp_path)
    data = open(f"{tmp_path}/m.gguf", "rb").read()
    f.close()
    g = gq.GgufFile(data=data.replace(b"qwen2.attention.head_count\x04",
                                      b"qwen2.attention.head_xxxxx\x04"))
    with pytest.raises(gq.GgufError) as e:
        g.load_model()
    assert _code(e) == -107 and "attention.head_count" in str(e.value)


def test_tensor_dims_overflow_rejected():
    """A tensor whose element count overflows 64 bits cannot be backed by
    the file: parse fails (UnexpectedEof) instead of wrapping the count."""
    data, _ = gw.build_file(tensors=[("w", [1 << 33, 1 << 33], 12, b"")])
    with pytest.raises(gq.GgufError, match="overflows"):
        _gguf(data)
    # the largest product that fits is parsed (its data is checked on access)
    data, _ = gw.build_file(tensors=[("w", [1 << 31, 1 << 32], 12, b"")])
    assert _gguf(data).tensors[0].dims == [1 << 31, 1 << 32]
