"""GGUF files written by the tests, in the layout ggufindex reads
(ggufindex/index.go:236-414): "GGUF", version, tensor and metadata counts,
metadata key/type/value entries, the tensor directory (name, dimensions,
shape, type, offset from the data base), then the tensor data from the
first multiple of the alignment after the directory.  Little-endian; strings
are a u64 length and the bytes."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)


def gstr(s):
    b = s.encode() if isinstance(s, str) else bytes(s)
    return struct.pack("<Q", len(b)) + b


def array(elem_type, count, payload=b""):
    """An array value: element type, count, then the encoded elements."""
    return struct.pack("<IQ", elem_type, count) + payload


def u32(v):
    return struct.pack("<I", v)


def u64(v):
    return struct.pack("<Q", v)


def align_up(n, a):
    return (n + a - 1) // a * a


def build(metadata=(), tensors=(), version=3, alignment=32, tensor_count=None, metadata_count=None):
    """File bytes and the absolute data range of each tensor.

    metadata: (key, type, encoded value) triples, written in order.
    tensors: (name, ggml type, shape, data bytes) -- data at the next
    multiple of `alignment` after the previous tensor (the data base is the
    directory's end rounded up the same way, as the reader computes it);
    a tensor given as (name, type, shape, data, offset) is placed at that
    offset from the base instead."""
    head = b"GGUF" + u32(version)
    head += u64(len(tensors) if tensor_count is None else tensor_count)
    head += u64(len(metadata) if metadata_count is None else metadata_count)
    for key, typ, value in metadata:
        head += gstr(key) + u32(typ) + value
    directory, place, off = b"", [], 0
    for t in tensors:
        name, typ, shape, data = t[:4]
        o = t[4] if len(t) > 4 else align_up(off, alignment)
        directory += gstr(name) + u32(len(shape)) + b"".join(u64(d) for d in shape) + u32(typ) + u64(o)
        place.append((o, bytes(data)))
        off = o + len(data)
    body = head + directory
    base = align_up(len(body), alignment)
    out = bytearray(body + b"\0" * (base - len(body)))
    ranges = []
    for o, data in place:
        end = base + o + len(data)
        if len(out) < end:
            out += b"\0" * (end - len(out))
        out[base + o:end] = data
        ranges.append((base + o, end))
    return bytes(out), ranges


def write(path, metadata=(), tensors=(), **kw):
    data, ranges = build(metadata, tensors, **kw)
    with open(path, "wb") as f:
        f.write(data)
    return data, ranges
