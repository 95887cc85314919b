"""CPU tests of the GGUF tensor directory (spt_gguf_open / _tensor_at /
_find / _layer_span / _metadata), the index the residency loader uploads
from.  The metadata cases replay the reference's
tests/index_optimization_test.go:52-175 (TestIndexOptimizationFixedArrays,
VariableArrays, RejectsMalformedArrays, NestingLimit) on files written the
same way; the directory, size-table, split-file and layer cases check the
rules of ggufindex.Open / readFile / tensorSize (ggufindex/index.go:60-574)
on files whose ranges the writer knows."""
import struct

import pytest

import spt
from gguf_file import (ARRAY, BOOL, F32, F64, I8, I16, I32, I64, STRING, U8, U16, U32, U64, array, build, gstr,
                       u32, u64, write)

WIDTHS = {U8: 1, I8: 1, U16: 2, I16: 2, U32: 4, I32: 4, F32: 4, BOOL: 1, U64: 8, I64: 8, F64: 8}


def _opt_fixture(tmp_path, *entries):
    """indexOptimizationFixture: version 3, no tensors, general.alignment = 1
    (u32) first, then the entries."""
    meta = [("general.alignment", U32, u32(1))] + list(entries)
    data, _ = build(meta, (), alignment=1)
    path = tmp_path / "index.gguf"
    path.write_bytes(data)
    return str(path), data


def _open_err(paths):
    with pytest.raises(spt.SptError) as e:
        spt.Gguf(paths)
    return e.value


@pytest.mark.parametrize("typ,width", sorted(WIDTHS.items()))
@pytest.mark.parametrize("count", [0, 3])
@pytest.mark.parametrize("trailing", [False, True])
def test_fixed_arrays(tmp_path, typ, width, count, trailing):
    value = array(typ, count, b"\x01" * (count * width))
    entries = [("array", ARRAY, value)]
    if trailing:
        entries.append(("sentinel", STRING, gstr("after")))
    path, data = _opt_fixture(tmp_path, *entries)
    with spt.Gguf(path) as g:
        t, f, a, b = g.metadata("array")
        assert t == ARRAY and f == 0 and b - a == len(value) and data[a:b] == value
        if not trailing:
            assert b == len(data), "array does not end at EOF"
        else:
            st, _, sa, sb = g.metadata("sentinel")
            assert st == STRING and data[sa:sb] == gstr("after") and sb == len(data)


def test_variable_arrays(tmp_path):
    strings = array(STRING, 3, gstr("") + gstr("hello") + gstr("ä"))
    fixed = array(U16, 2, b"\x01\x00\x02\x00")
    nested = array(ARRAY, 3, strings + fixed + array(ARRAY, 0))
    for value in (strings, nested):
        path, data = _opt_fixture(tmp_path, ("array", ARRAY, value))
        with spt.Gguf(path) as g:
            _, _, a, b = g.metadata("array")
            assert b == len(data) and b - a == len(value) and data[a:b] == value


MALFORMED = [
    ("unknown-empty", array(13, 0), "unknown metadata type"),
    ("unknown", array(0xFFFFFFFF, 1), "unknown metadata type"),
    ("count-limit", array(U8, 100_000_001), "array is too large"),
    ("uint64-overflow", array(U64, 2**64 - 1), "array is too large"),
    ("int64-overflow", array(U64, (2**63 - 1) // 8 + 1), "array is too large"),
    ("missing-type", b"", "EOF"),
    ("missing-count", b"\x00\x00\x00\x00\x01", "EOF"),
    ("string-truncated", array(STRING, 1, u64(2) + b"x"), "EOF"),
    ("string-too-long", array(STRING, 1, u64((1 << 20) + 1)), "too long"),
    ("nested-truncated", array(ARRAY, 1, array(U64, 1, b"\x01")), "EOF"),
    ("nested-unknown-empty", array(ARRAY, 1, array(13, 0)), "unknown metadata type"),
] + [(f"type{t}-short-by-one", array(t, 2, b"\x00" * (2 * w - 1)), "EOF") for t, w in sorted(WIDTHS.items())]


@pytest.mark.parametrize("name,value,error", MALFORMED, ids=[m[0] for m in MALFORMED])
def test_rejects_malformed_arrays(tmp_path, name, value, error):
    path, _ = _opt_fixture(tmp_path, ("array", ARRAY, value))
    e = _open_err(path)
    assert e.code == spt.ERR_INVALID and error in e.message, e.message
    assert path in e.message and '"array"' in e.message


@pytest.mark.parametrize("empty", [False, True])
@pytest.mark.parametrize("wrappers", [7, 8, 9])
def test_nesting_limit(tmp_path, empty, wrappers):
    value = array(U8, 0) if empty else array(U8, 1, b"\x01")
    for _ in range(wrappers):
        value = array(ARRAY, 1, value)
    path, _ = _opt_fixture(tmp_path, ("array", ARRAY, value))
    valid = wrappers < 8 or (empty and wrappers == 8)
    if valid:
        spt.Gguf(path).close()
    else:
        assert "nesting is too deep" in _open_err(path).message


# tensorSize (index.go:535-574): elements per block, bytes per block
SIZES = {0: (1, 4), 1: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 8: (32, 34), 9: (32, 40),
         28: (1, 2), 39: (32, 17)}


def _model(tmp_path, alignment=None, version=3):
    """Two layers and two shared tensors, one of every type, names given
    out of order."""
    meta = [("general.architecture", STRING, gstr("gpt-oss")), ("gpt_oss.block_count", U32, u32(2))]
    if alignment is not None:
        meta.append(("general.alignment", U32, u32(alignment)))
    tens = []
    for i, (typ, (per, nb)) in enumerate(sorted(SIZES.items())):
        shape = [64, 3] if per == 32 else [5, 3]
        n = shape[0] * shape[1] // per * nb
        layer = ["blk.1.", "blk.0.", "shared."][i % 3]
        tens.append((f"{layer}t{9 - i}.weight", typ, shape, bytes((i * 7 + j) % 251 for j in range(n))))
    data, ranges = build(meta, tens, version=version, alignment=alignment or 32)
    path = tmp_path / "model.gguf"
    path.write_bytes(data)
    return str(path), data, tens, ranges


@pytest.mark.parametrize("alignment", [None, 1, 64, 4096])
@pytest.mark.parametrize("version", [2, 3])
def test_tensor_directory(tmp_path, alignment, version):
    path, data, tens, ranges = _model(tmp_path, alignment, version)
    with spt.Gguf(path) as g:
        layers, n, al = g.info()
        assert (layers, n, al) == (2, len(tens), alignment or 32)
        got = g.tensors()
        names = [t.name.decode() for t in got]
        # Layers in order, names sorted within each, then the shared ones sorted
        want = (sorted(t[0] for t in tens if t[0].startswith("blk.0.")) +
                sorted(t[0] for t in tens if t[0].startswith("blk.1.")) +
                sorted(t[0] for t in tens if not t[0].startswith("blk.")))
        assert names == want
        by = {t[0]: (t, r) for t, r in zip(tens, ranges)}
        for t in got:
            (name, typ, shape, blob), (a, b) = by[t.name.decode()]
            assert (t.type, t.dims, t.file, t.start, t.end) == (typ, shape, 0, a, b)
            assert data[t.start:t.end] == blob
            assert t.layer == (int(name[4]) if name.startswith("blk.") else -1)
            per, nb = SIZES[typ]
            assert t.end - t.start == shape[0] * shape[1] // per * nb
            assert t.start % (alignment or 32) == 0
            f = g.find(name)
            assert f is not None and (f.start, f.end, f.type) == (t.start, t.end, t.type)
        assert g.find("missing.weight") is None
        for layer in (0, 1):
            mine = [t for t in got if t.layer == layer]
            assert g.layer_spans(layer) == [(0, min(t.start for t in mine), max(t.end for t in mine))]
        assert g.layer_spans(2) == []
        t, f, a, b = g.metadata("general.architecture")
        assert t == STRING and data[a:b] == gstr("gpt-oss")
        assert g.metadata("general.name") is None


@pytest.mark.parametrize("typ", sorted(SIZES))
def test_tensor_sizes(tmp_path, typ):
    per, nb = SIZES[typ]
    for shape in ([32], [96, 2], [64, 3, 5]):
        n = 1
        for d in shape:
            n *= d
        blob = bytes(n // per * nb)
        path = tmp_path / f"t{typ}.gguf"
        _, ranges = write(path, [], [("w", typ, shape, blob)])
        with spt.Gguf(str(path)) as g:
            t = g.find("w")
            assert (t.start, t.end) == ranges[0]


@pytest.mark.parametrize("typ,shape,error", [
    (30, [32], "unsupported GGML tensor type 30"),
    (12, [256], "unsupported GGML tensor type 12"),
    (2, [48], "invalid block size or tensor is too large"),
    (39, [0, 32], "invalid tensor shape"),
    (0, [2**32, 2**32], "invalid tensor shape"),
    (0, [2**62, 32], "invalid tensor shape"),
    (8, [2**59 - 1, 32], "invalid block size or tensor is too large"),
])
def test_tensor_size_errors(tmp_path, typ, shape, error):
    path = tmp_path / "bad.gguf"
    write(path, [], [("w", typ, shape, b"")])
    e = _open_err(str(path))
    assert e.code == spt.ERR_INVALID and f'tensor "w": {error}' in e.message, e.message


def _header(version=3, tensors=0, meta=0):
    return b"GGUF" + u32(version) + u64(tensors) + u64(meta)


@pytest.mark.parametrize("case,blob,error", [
    ("short", b"GGUF" + u32(3) + b"\x00" * 8, "file is too small"),
    ("magic", b"GGUX" + _header()[4:], "not a GGUF file"),
    ("version1", _header(1), "unsupported GGUF version 1"),
    ("version4", _header(4), "unsupported GGUF version 4"),
    ("tensors", _header(3, 10_000_001, 0), "implausible header count"),
    ("meta", _header(3, 0, 1_000_001), "implausible header count"),
    ("key-eof", _header(3, 0, 1), "EOF"),
    ("key-long", _header(3, 0, 1) + u64((1 << 20) + 1), "GGUF string is too long"),
    ("dup-key", _header(3, 0, 2) + (gstr("k") + u32(U8) + b"\x01") * 2, 'duplicate metadata key "k"'),
    ("unknown-type", _header(3, 0, 1) + gstr("k") + u32(13) + b"\x00" * 8, 'metadata "k": unknown metadata type 13'),
    ("dims0", _header(3, 1, 0) + gstr("w") + u32(0) + b"\x00" * 12, 'tensor "w": invalid dimension count'),
    ("dims9", _header(3, 1, 0) + gstr("w") + u32(9) + b"\x00" * 84, 'tensor "w": invalid dimension count'),
    ("beyond", _header(3, 1, 0) + gstr("w") + u32(1) + u64(32) + u32(0) + u64(0), "tensor data starts beyond"),
])
def test_header_errors(tmp_path, case, blob, error):
    path = tmp_path / f"{case}.gguf"
    path.write_bytes(blob)
    e = _open_err(str(path))
    assert e.code == spt.ERR_INVALID and error in e.message and str(path) in e.message, e.message


def test_range_and_alignment_errors(tmp_path):
    # a tensor past the end of the file
    data, _ = build([], [("w", 0, [8], bytes(32))])
    path = tmp_path / "trunc.gguf"
    path.write_bytes(data[:-4])
    assert 'tensor "w": byte range extends beyond the file' in _open_err(str(path)).message
    # an offset past the end
    path2 = tmp_path / "off.gguf"
    data, _ = build([], [("w", 0, [8], bytes(32))])
    entry = gstr("w") + u32(1) + u64(8) + u32(0) + u64(0)
    path2.write_bytes(data.replace(entry, entry[:-8] + u64(64)))
    assert 'tensor "w": byte range extends beyond the file' in _open_err(str(path2)).message
    # alignments that are not a power of two, or too large; a signed value
    # is not numeric for the reader and leaves the default of 32
    for al, msg in ((3, "invalid alignment 3"), (1 << 21, "invalid alignment 2097152")):
        p = tmp_path / f"al{al}.gguf"
        p.write_bytes(build([("general.alignment", U32, u32(al))], [], alignment=1)[0] + bytes(8))
        assert msg in _open_err(str(p)).message
    p = tmp_path / "signed.gguf"
    write(p, [("general.alignment", I32, struct.pack("<i", 64))], [("w", 0, [8], bytes(32))], alignment=32)
    with spt.Gguf(str(p)) as g:
        assert g.info()[2] == 32


def _split(tmp_path, n, numbers=True, count=True, extra=None, tensors=None):
    paths = []
    for i in range(n):
        meta = [("general.architecture", STRING, gstr("gpt-oss")), ("gpt_oss.block_count", U32, u32(2))]
        if count:
            meta.append(("split.count", U16, struct.pack("<H", n)))
        if numbers:
            meta.append(("split.no", U16, struct.pack("<H", i)))
        if extra:
            meta += extra(i)
        tens = tensors(i) if tensors else [(f"blk.{i % 2}.w{i}", 0, [4], struct.pack("<4f", i, i, i, i)),
                                           (f"blk.{(i + 1) % 2}.v{i}", 0, [4], bytes(16))]
        p = tmp_path / f"m-{i:05d}-of-{n:05d}.gguf"
        write(p, meta, tens)
        paths.append(str(p))
    return paths


def test_split_files(tmp_path):
    paths = _split(tmp_path, 2)
    with spt.Gguf(list(reversed(paths))) as g:   # any order
        layers, n, _ = g.info()
        assert (layers, n) == (2, 4)
        ts = g.tensors()
        assert [t.name.decode() for t in ts] == ["blk.0.v1", "blk.0.w0", "blk.1.v0", "blk.1.w1"]
        # file indices refer to the order the paths were given in
        assert [t.file for t in ts] == [0, 1, 1, 0]
        for layer in (0, 1):
            spans = g.layer_spans(layer)
            files = sorted(set(t.file for t in ts if t.layer == layer), key=lambda f: list(reversed(paths))[f])
            assert [s[0] for s in spans] == files and len(spans) == 2


@pytest.mark.parametrize("case,error", [
    ("incomplete", "incomplete model: 1 of 2 splits provided"),
    ("no-number", "a file is missing its split number"),
    ("dup-number", "duplicate split 0"),
    ("missing-number", "split 1 is missing"),
    ("inconsistent", 'inconsistent metadata "general.architecture"'),
    ("dup-tensor", 'duplicate tensor "blk.0.w"'),
    ("dup-file", "duplicate file"),
    # differing split counts or layer counts are caught first as differing
    # metadata (the metadata merge precedes those checks, index.go:95-133)
    ("count", 'inconsistent metadata "split.count"'),
    ("layers", 'inconsistent metadata "gpt_oss.block_count"'),
])
def test_split_errors(tmp_path, case, error):
    if case == "incomplete":
        paths = _split(tmp_path, 2)[:1]
    elif case == "no-number":
        paths = _split(tmp_path, 2, numbers=False, extra=lambda i: [("split.no", U16, struct.pack("<H", 0))] if i == 0 else [])
    elif case == "dup-number":
        paths = _split(tmp_path, 2, numbers=False, extra=lambda i: [("split.no", U16, struct.pack("<H", 0))])
    elif case == "missing-number":
        paths = _split(tmp_path, 2, numbers=False, extra=lambda i: [("split.no", U16, struct.pack("<H", 2 * i))])
    elif case == "inconsistent":
        paths = []
        for i in range(2):
            p = tmp_path / f"x{i}.gguf"
            write(p, [("general.architecture", STRING, gstr("gpt-oss" if i == 0 else "gpt-os2"))],
                  [(f"blk.0.w{i}", 0, [4], bytes(16))])
            paths.append(str(p))
    elif case == "dup-tensor":
        paths = _split(tmp_path, 2, tensors=lambda i: [("blk.0.w", 0, [4], bytes(16)), (f"blk.1.v{i}", 0, [4], bytes(16))])
    elif case == "dup-file":
        p = _split(tmp_path, 1)[0]
        paths = [p, p]
    elif case == "count":
        paths = _split(tmp_path, 2, count=False, extra=lambda i: [("split.count", U16, struct.pack("<H", 2 + i))])
    else:
        paths = []
        for i in range(2):
            p = tmp_path / f"l{i}.gguf"
            write(p, [("gpt_oss.block_count", U32, u32(1 + i))], [(f"blk.{i}.w", 0, [4], bytes(16))])
            paths.append(str(p))
    e = _open_err(paths)
    assert error in e.message, e.message


def test_layer_errors(tmp_path):
    p = tmp_path / "a.gguf"
    write(p, [("gpt_oss.block_count", U32, u32(3))], [("blk.0.w", 0, [4], bytes(16)), ("blk.1.w", 0, [4], bytes(16))])
    assert "expected 3 layers, found 2" in _open_err(str(p)).message
    write(p, [("gpt_oss.block_count", U32, u32(2))], [("blk.0.w", 0, [4], bytes(16)), ("blk.2.w", 0, [4], bytes(16))])
    assert "layer 1 is missing" in _open_err(str(p)).message
    write(p, [], [("blk.0.w", 0, [4], bytes(16)), ("blk.5.w", 0, [4], bytes(16))])
    assert "layer 1 is missing" in _open_err(str(p)).message
    write(p, [], [("blk.99999999999999999999.w", 0, [4], bytes(16))])
    assert 'invalid layer number in "blk.99999999999999999999.w"' in _open_err(str(p)).message
    # names that do not match ^blk\.([0-9]+)\. are shared tensors
    write(p, [], [("blk.x.w", 0, [4], bytes(16)), ("blk.1", 0, [4], bytes(16)), ("blk..w", 0, [4], bytes(16))])
    with spt.Gguf(str(p)) as g:
        assert g.info()[0] == 0 and all(t.layer == -1 for t in g.tensors())
    # no block count: the number of layers found
    write(p, [], [("blk.1.w", 0, [4], bytes(16)), ("blk.0.w", 0, [4], bytes(16))])
    with spt.Gguf(str(p)) as g:
        assert g.info()[0] == 2


def test_open_errors(tmp_path):
    e = _open_err([])
    assert e.code == spt.ERR_INVALID and "no GGUF files provided" in e.message
    e = _open_err(str(tmp_path / "absent.gguf"))
    assert e.code == spt.ERR_IO and "absent.gguf" in e.message
