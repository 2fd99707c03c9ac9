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
