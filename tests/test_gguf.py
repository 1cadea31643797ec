"""The GGUF reader (grx_gguf_*, host code, no GPU) against the reference's
own tests of internal/gguf: TestParse (gguf_test.go:51-113), the crafted
files of TestHostileFiles (hostile_test.go:34-77), TestArrayCountAllocates
Nothing (:81-105), TestReadMeta (:127-149) and TestOpenOwnMemory (:154-205),
plus every value type, the alignment key and File.Weight's shape rule."""
import math
import resource
import struct

import numpy as np
import pytest

from gorelaxor_amd import GrxError
from gorelaxor_amd import gguf
from tests import _gguf as G


def _parse_kvs():
    return [G.kv("general.architecture", G.T_STR, "parakeet"), G.kv("n", G.T_U32, 7),
            G.kv("toks", G.T_ARR, ["a", "▁b"], G.T_STR)]


def _parse_file():
    f32 = struct.pack("<6f", *[i + 0.5 for i in range(6)])
    f16 = G.f16_bytes(np.arange(32))
    q8 = G.q8_block(0.25, [i - 16 for i in range(32)])
    return G.build(_parse_kvs(), [("a", [3, 2], G.F32, f32), ("pw", [1, 4, 8], G.F16, f16),
                                   ("q", [32, 1], G.Q8_0, q8)])


def test_parse():
    """TestParse: settings, string arrays, Weight shapes (a 1x1 convolution
    kernel [1,4,8] is 8 rows of 4), Float32 of F32 and Q8_0, a cut file."""
    b = _parse_file()
    f = gguf.Parse(b)
    assert f.Version == 3
    assert f.String("general.architecture", "") == "parakeet" and f.Int("n", 0) == 7
    assert f.Strings("toks") == ["a", "▁b"]
    assert f.WeightShape("a") == (2, 3)
    assert f.Float32("a")[4] == 4.5
    assert f.WeightShape("pw") == (8, 4)
    assert np.array_equal(f.Float32("pw"), np.arange(32, dtype=np.float32))
    q = f.Float32("q")
    assert q[0] == -4 and q[31] == 3.75
    assert f.Names() == ["a", "pw", "q"] and f.Keys() == ["general.architecture", "n", "toks"]
    assert f.Tensors["pw"].Dims == [1, 4, 8] and f.Tensors["q"].Type == G.Q8_0
    with pytest.raises(GrxError, match="cut short|past the end"):
        gguf.Parse(b[:-40])


def _align(v, typ):
    k = struct.pack("<Q", 17) + b"general.alignment" + struct.pack("<I", typ)
    return k + (struct.pack("<I", v) if typ == 4 else struct.pack("<Q", v))


_B0 = G.one(b"", 0, [2], G.F32, 0, 64)
_BASE = len(_B0) - 64
HOSTILE = {
    "a dimension that reads as negative": G.one(b"", 0, [2**64 - 1], G.F32, 8, 64),
    "an offset that wraps": G.one(b"", 0, [2], G.F32, 2**64 - 1 - 3, 64),
    "an offset that wraps onto the header": G.one(b"", 0, [2], G.F32, -_BASE - 4, 64),
    "dimensions whose product overflows": G.one(b"", 0, [1 << 32, 1 << 31], G.F16, 0, 0),
    "a dimension past the file": G.one(b"", 0, [(1 << 62) + 1], G.F32, 0, 32),
    "two negative dimensions": G.one(b"", 0, [2**64 - 2, 2**64 - 3], G.F32, 0, 64),
    "negative Q8_0 dimensions": G.one(b"", 0, [2**64 - 32, 2**64 - 32], G.Q8_0, 0, 40000),
    "a zero dimension": G.one(b"", 0, [0, 4], G.F32, 0, 64),
    "an alignment near the largest integer": G.one(_align(2**63 - 1 - 5, 10), 1, [4], G.F32, 0, 0),
    "an alignment that isn't a power of two": G.one(_align(48, 4), 1, [4], G.F32, 0, 64),
}


@pytest.mark.parametrize("case", list(HOSTILE))
def test_hostile_files(case):
    """TestHostileFiles: each crafted file gives an error, no crash."""
    with pytest.raises(GrxError, match="gguf: "):
        gguf.Parse(HOSTILE[case])


def test_hostile_seed_files_parse():
    """FuzzParse's seeds are valid files whose tensors read back."""
    for b in (G.one(b"", 0, [4, 2], G.F32, 0, 64), G.one(b"", 0, [32, 2], G.Q8_0, 0, 96)):
        f = gguf.Parse(b)
        for n in f.Names():
            f.Float32(n)
            f.WeightShape(n)


def test_array_count_allocates_nothing():
    """TestArrayCountAllocatesNothing: a count past the bytes left is refused
    before anything is reserved for it."""
    big = 8 << 20
    kvb = struct.pack("<Q", 1) + b"a" + struct.pack("<IIQ", 9, 0, big)
    b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + kvb
    b = b + bytes(big - len(b))
    rss0 = resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    with pytest.raises(GrxError, match="array too long"):
        gguf.Parse(b)
    assert (resource.getrusage(resource.RUSAGE_SELF).ru_maxrss - rss0) >> 10 <= 4


def test_read_meta(tmp_path):
    """TestReadMeta: the settings of a file without its weights; a cut-off
    or foreign file gives an error."""
    kvb = G.kv("general.architecture", G.T_STR, "parakeet")
    b = G.one(kvb, 1, [2], G.F32, 0, 8)
    p = tmp_path / "m.gguf"
    p.write_bytes(b)
    assert gguf.ReadMeta(p).String("general.architecture", "") == "parakeet"
    p.write_bytes(b[:30])
    with pytest.raises(GrxError):
        gguf.ReadMeta(p)
    p.write_bytes(b"ggml not gguf")
    with pytest.raises(GrxError, match="not a GGUF file"):
        gguf.ReadMeta(p)


def test_open_long_header_and_overlap(tmp_path):
    """TestOpenOwnMemory: Open reads a header longer than its first 1 MB
    read and gives the bytes Parse sees; two tensors at the same offset, each
    most of the file, parse but Open refuses them."""
    data = bytes(i & 255 for i in range(4096))
    pad = G.gstr("pad") + struct.pack("<I", G.T_STR) + G.gstr(bytes(2 << 20))
    b = G.build([pad], [("a", [1024], G.F32, data), ("b", [16], G.F32, data[:64])])
    p = tmp_path / "m.gguf"
    p.write_bytes(b)
    f, ref = gguf.Open(p), gguf.Parse(b)
    for n in ("a", "b"):
        assert np.array_equal(f.Float32(n).view(np.uint32), ref.Float32(n).view(np.uint32))
    assert np.array_equal(f.Float32("b"), np.frombuffer(data[:64], np.float32))
    two = b"GGUF" + struct.pack("<IQQ", 3, 2, 0)
    for name in (b"x", b"y"):
        two += struct.pack("<Q", 1) + name + struct.pack("<IQIQ", 1, 1024, G.F32, 0)
    two += bytes((32 - len(two) % 32) % 32) + data
    p.write_bytes(two)
    gguf.Parse(two)
    with pytest.raises(GrxError, match="overlap"):
        gguf.Open(p)


def test_value_types_and_accessors():
    """Every value type (gguf.go:167-210) and File.Int/Float/Bool/String and
    the array forms, with the reference's conversions (Int of a bool, Float
    of an int, Floats of float64 narrowed to float32)."""
    kvs = [G.kv("u8", G.T_U8, 200), G.kv("i8", G.T_I8, -5), G.kv("u16", G.T_U16, 60000),
           G.kv("i16", G.T_I16, -300), G.kv("u32", G.T_U32, 4000000000), G.kv("i32", G.T_I32, -7),
           G.kv("f32", G.T_F32, 0.1), G.kv("t", G.T_BOOL, True), G.kv("s", G.T_STR, "x y"),
           G.kv("u64", G.T_U64, 2**64 - 1), G.kv("i64", G.T_I64, -2**40), G.kv("f64", G.T_F64, 0.1),
           G.kv("ints", G.T_ARR, [1, -2, 3], G.T_I32), G.kv("fl", G.T_ARR, [0.1, 2.5], G.T_F64)]
    # an array of arrays (element type 9, each element an array of u8)
    nest = G.gstr("nest") + struct.pack("<IIQ", G.T_ARR, G.T_ARR, 2)
    nest += struct.pack("<IQ", G.T_U8, 1) + bytes([1]) + struct.pack("<IQ", G.T_U8, 2) + bytes([2, 3])
    kvs.append(nest)
    f = gguf.Parse(G.build(kvs, []))
    assert f.Int("u8", 0) == 200 and f.Int("i8", 0) == -5 and f.Int("u16", 0) == 60000
    assert f.Int("i16", 0) == -300 and f.Int("u32", 0) == 4000000000 and f.Int("i32", 0) == -7
    assert f.Int("u64", 0) == -1 and f.Int("i64", 0) == -2**40  # Go's int(uint64) wraps
    assert f.Int("t", 0) == 1 and f.Int("f32", 9) == 9 and f.Int("s", 9) == 9 and f.Int("missing", 4) == 4
    assert f.Float("f32", 0) == float(np.float32(0.1)) and f.Float("f64", 0) == 0.1 and f.Float("i32", 0) == -7
    assert f.Bool("t", False) and f.Bool("u8", False) and not f.Bool("missing", False) and f.Bool("s", True)
    assert f.String("s", "") == "x y" and f.String("u8", "d") == "d"
    assert f.Ints("ints") == [1, -2, 3] and f.Strings("ints") == ["", "", ""]
    assert f.Floats("fl").tolist() == [float(np.float32(0.1)), 2.5]
    assert f.Floats("ints").tolist() == [1, -2, 3] and f.Ints("missing") == []
    assert f.Strings("nest") == ["", ""]


@pytest.mark.parametrize("case, msg", [
    ("magic", "not a GGUF file"), ("version", "version 4 is not supported"),
    ("counts", "header counts out of range"), ("deep", "arrays nested too deep"),
    ("vtype", "unknown value type 13"), ("dims", "has 5 dimensions"),
    ("ttype", "has type 2, which this reader doesn't handle"), ("q8rows", "rows are not a multiple of 32"),
    ("past", "runs past the end of the file"), ("long", "string too long"),
])
def test_header_errors(case, msg):
    """The reference's error for each malformed header (gguf.go:123-370)."""
    good = G.build([], [("w", [32, 2], G.F32, bytes(256))])
    if case == "magic":
        b = b"GGUG" + good[4:]
    elif case == "version":
        b = good[:4] + struct.pack("<I", 4) + good[8:]
    elif case == "counts":
        b = b"GGUF" + struct.pack("<IQQ", 3, (1 << 20) + 1, 0)
    elif case == "deep":
        v = struct.pack("<IQ", G.T_ARR, 1) * 3 + struct.pack("<IQ", G.T_U8, 1) + b"\0"
        b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + G.gstr("d") + struct.pack("<I", G.T_ARR) + v
    elif case == "vtype":
        b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + G.gstr("k") + struct.pack("<I", 13) + bytes(16)
    elif case == "dims":
        b = b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + G.gstr("w") + struct.pack("<I", 5) + bytes(64)
    elif case == "ttype":
        b = G.build([], [("w", [32, 2], 2, bytes(256))])
    elif case == "q8rows":
        b = G.build([], [("w", [16, 2], G.Q8_0, bytes(68))])
    elif case == "past":
        b = good[:-32]
    elif case == "long":
        b = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + struct.pack("<Q", (1 << 30) + 1)
    with pytest.raises(GrxError, match=msg):
        gguf.Parse(b)


def test_alignment_key():
    """general.alignment moves the data start; a tensor read back from it."""
    data = struct.pack("<4f", 1, 2, 3, 4)
    for align in (8, 64, 4096):
        b = G.build([G.kv("general.alignment", G.T_U32, align)], [("v", [4], G.F32, data)], align=align)
        assert gguf.Parse(b).Float32("v").tolist() == [1, 2, 3, 4]
    with pytest.raises(GrxError, match="general.alignment"):
        gguf.Parse(G.build([G.kv("general.alignment", G.T_U64, 64)], [("v", [4], G.F32, data)], align=64))


def test_float32_widening():
    """Float32 of F16 (subnormals, infinities), BF16 (the top half of the
    float32 bits) and Q8_0 with a subnormal scale: exact values."""
    h = np.array([0x0001, 0x03FF, 0x7BFF, 0xFC00, 0x8000, 0x3C00], np.uint16)
    bf = np.array([0x3F80, 0xC2F7, 0x0001, 0x7F80], np.uint16)
    q8 = struct.pack("<H", 0x0003) + np.arange(-16, 16, dtype=np.int8).tobytes()
    b = G.build([], [("h", [6], G.F16, h.tobytes()), ("bf", [4], G.BF16, bf.tobytes()), ("q", [32], G.Q8_0, q8)])
    f = gguf.Parse(b)
    assert f.Float32("h").tolist() == [2.0**-24, 1023 * 2.0**-24, 65504.0, -math.inf, -0.0, 1.0]
    assert np.array_equal(f.Float32("bf").view(np.uint32), bf.astype(np.uint32) << 16)
    assert f.Float32("q").tolist() == [3 * 2.0**-24 * k for k in range(-16, 16)]
    # a Q8_0 tensor whose first dimension is 1 is refused at parse time
    # (byteSize), so File.Weight's leading-unit check never sees one
    with pytest.raises(GrxError, match="rows are not a multiple of 32"):
        gguf.Parse(G.build([], [("q", [1, 32], G.Q8_0, q8)]))
    with pytest.raises(GrxError, match="no tensor zz"):
        f.Float32("zz")
