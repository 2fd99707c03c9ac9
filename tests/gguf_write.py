"""A small GGUF writer for test fixtures (version 2/3 container format).

Writes the layout the reference's parser reads (src/parser.rs:9-66): magic,
version, tensor count, metadata count, typed metadata, tensor infos, then the
tensor data from the next 32-byte boundary, each tensor at an offset aligned
to 32.  Test infrastructure only.
"""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
        U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def _value(t, v):
    if t == STRING:
        return _str(v)
    if t == ARRAY:
        et, items = v
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_FMT[t], v)


def header(version=3, n_tensors=0, n_kv=0):
    return b"GGUF" + struct.pack("<IQQ", version, n_tensors, n_kv)


def write(path, metadata=(), tensors=(), version=3):
    data, offsets = build_file(metadata, tensors, version)
    with open(path, "wb") as f:
        f.write(data)
    return offsets


def build_file(metadata=(), tensors=(), version=3, align=32):
    """metadata: [(key, type, value)] (arrays: (elem_type, [items]));
    tensors: [(name, dims, ggml_type, bytes)].  Returns the file image and
    the tensor data offsets (relative to the data section)."""
    meta = bytearray(header(version, len(tensors), len(metadata)))
    for key, t, v in metadata:
        meta += _str(key) + struct.pack("<I", t) + _value(t, v)
    offsets, off = [], 0
    for name, dims, gt, data in tensors:
        offsets.append(off)
        meta += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        meta += struct.pack("<IQ", gt, off)
        off += (len(data) + align - 1) // align * align
    meta += b"\0" * ((-len(meta)) % align)
    body = bytearray(off)
    for (_, _, _, data), o in zip(tensors, offsets):
        body[o:o + len(data)] = bytes(data)
    return bytes(meta) + bytes(body), offsets


GGML_F32, GGML_F16 = 0, 1
_NAMES = dict(wq="attn_q", wk="attn_k", wv="attn_v", wo="attn_output", wgate="ffn_gate",
              wup="ffn_up", wdown="ffn_down")
ORDER = ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown")


def decoder_tensors(cfg, w, layer_types, embd=None, head_type=None, norm_f16=False):
    """The tensors of a dense decoder in GGUF naming (blk.N.attn_q.weight ...,
    dims [in_dim, out_dim]).  w as gq_synth.make_decoder; layer_types
    [n_layers][7] per-tensor types in ORDER; embd = (ggml_type, bytes) of
    token_embd.weight ((GGML_F32, f32 table) if None); head_type None ties
    lm_head to token_embd (no output.weight)."""
    import numpy as np
    H, F, V = cfg["hidden"], cfg["ffn"], cfg["vocab"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    dims = dict(wq=[H, qd], wk=[H, kvd], wv=[H, kvd], wo=[qd, H], wgate=[H, F], wup=[H, F],
                wdown=[F, H])

    def norm(a):
        a = np.asarray(a, np.float32)
        return (GGML_F16, a.astype(np.float16).tobytes()) if norm_f16 else (GGML_F32, a.tobytes())

    et, eb = embd if embd is not None else (GGML_F32, np.asarray(w["embd"], np.float32).tobytes())
    out = [("token_embd.weight", [H, V], et, eb)]
    for l in range(cfg["n_layers"]):
        b = f"blk.{l}."
        nt, nb = norm(w["attn_norm"][l])
        out.append((b + "attn_norm.weight", [H], nt, nb))
        for k, t in zip(ORDER, layer_types[l]):
            out.append((b + _NAMES[k] + ".weight", dims[k], t, bytes(w[k][l])))
        nt, nb = norm(w["ffn_norm"][l])
        out.append((b + "ffn_norm.weight", [H], nt, nb))
    nt, nb = norm(w["output_norm"])
    out.append(("output_norm.weight", [H], nt, nb))
    if head_type is not None:
        out.append(("output.weight", [H, V], head_type, bytes(w["lm_head"])))
    return out


def decoder_metadata(cfg, arch="qwen2", context_length=None, extra=()):
    md = [("general.architecture", STRING, arch), ("general.name", STRING, "synthetic"),
          (f"{arch}.block_count", U32, cfg["n_layers"]),
          (f"{arch}.embedding_length", U32, cfg["hidden"]),
          (f"{arch}.feed_forward_length", U32, cfg["ffn"]),
          (f"{arch}.attention.head_count", U32, cfg["n_heads"]),
          (f"{arch}.attention.head_count_kv", U32, cfg["n_kv_heads"]),
          (f"{arch}.rope.freq_base", F32, cfg["theta"]),
          (f"{arch}.attention.layer_norm_rms_epsilon", F32, cfg["eps"])]
    if context_length is not None:
        md.append((f"{arch}.context_length", U32, context_length))
    return md + list(extra)
