"""CPU tests of the native GGUF header reader (glm-ssd_amd/csrc/gguf.cpp) through its C ABI.
The cases restate the reference reader's own tests (crates/gguf/src/lib.rs:467-608: a minimal
valid file, hostile counts, dimensions, sizes, offsets, alignment, nesting, string lengths,
shard-name patterns) against our implementation, plus metadata getters and split models."""
import os
import struct

import pytest

from glmssd.gguf import Gguf, GgufError, STR, U32, ARR, U8
from gguf_writer import Writer

MAX_COUNT, MAX_ARR = 1 << 20, 1 << 24


def _open(tmp_path, b, name="m.gguf", mode="all"):
    p = tmp_path / name
    p.write_bytes(b)
    return Gguf(p, mode)


def _err(tmp_path, b, mode="all"):
    with pytest.raises(GgufError) as e:
        _open(tmp_path, b, mode=mode)
    return str(e.value)


def test_valid_minimal_file(tmp_path):
    b = Writer().kv_u32("general.alignment", 32).tensor("a", [64, 2], 0, 0).tensor("q", [256, 3], 8, 512) \
        .build(512 + 3 * 272)
    g = _open(tmp_path, b)
    assert g.u64("general.alignment") == 32
    assert len(g.tensors) == 2
    a, q = g.tensors
    assert a.n_bytes == 64 * 2 * 4
    assert q.n_bytes == 3 * 8 * 34 and q.row_bytes == 8 * 34
    assert q.offset == a.offset + 512
    assert a.offset % 32 == 0 and a.dims == (64, 2) and q.ty == 8
    # one byte short: rejected when sizes are checked, accepted header-only
    assert "past the end" in _err(tmp_path, b[:-1])
    assert len(_open(tmp_path, b[:-1], mode="headers").tensors) == 2


def test_huge_counts_rejected(tmp_path):
    assert "implausible" in _err(tmp_path, Writer().build(0, n_t=(1 << 64) - 1, n_kv=0))
    _err(tmp_path, Writer().build(0, n_t=MAX_COUNT + 1, n_kv=0))
    _err(tmp_path, Writer().build(0, n_t=0, n_kv=(1 << 63) - 1))
    # a plausible count with nothing behind it: an end-of-file error, not a huge allocation
    _err(tmp_path, Writer().build(0, n_t=MAX_COUNT, n_kv=0))


@pytest.mark.parametrize("dims", [[], [1, 1, 1, 1, 1]])
def test_dimension_count_rejected(tmp_path, dims):
    assert "dimensions" in _err(tmp_path, Writer().tensor("t", dims, 0, 0).build(64))


def test_zero_dimension_rejected(tmp_path):
    assert "zero dimension" in _err(tmp_path, Writer().tensor("t", [32, 0], 0, 0).build(64))


def test_bad_shapes_rejected(tmp_path):
    assert "bad shape" in _err(tmp_path, Writer().tensor("t", [1 << 32, 1 << 32, 4], 0, 0).build(64))
    assert "bad shape" in _err(tmp_path, Writer().tensor("t", [((1 << 64) - 1) // 32 * 32], 8, 0).build(64))
    assert "bad shape" in _err(tmp_path, Writer().tensor("t", [33], 8, 0).build(64))   # not whole blocks
    assert "unsupported ggml type" in _err(tmp_path, Writer().tensor("t", [32], 4, 0).build(64))


def test_offset_overflow_rejected(tmp_path):
    b = Writer().tensor("t", [64], 0, (1 << 64) - 9).build(64)
    assert "overflows" in _err(tmp_path, b)
    _err(tmp_path, b, mode="headers")                                     # arithmetic checked header-only too
    _err(tmp_path, Writer().tensor("t", [1 << 40, 1 << 20], 0, 0).build(64))   # wrapped end
    assert "past the end" in _err(tmp_path, Writer().tensor("t", [64], 0, 1 << 20).build(64))


@pytest.mark.parametrize("a", [0, 3, 1 << 21])
def test_bad_alignment_rejected(tmp_path, a):
    assert "alignment" in _err(tmp_path, Writer().kv_u32("general.alignment", a).tensor("t", [8], 0, 0).build(64))


def test_alignment_64(tmp_path):
    b = Writer().kv_u32("general.alignment", 64).tensor("t", [8], 0, 0).build(128, align=64)
    g = _open(tmp_path, b)
    assert g.tensors[0].offset % 64 == 0


def test_array_nesting_and_lengths(tmp_path):
    # array of arrays of arrays of u8: one level too deep
    b = Writer().kv_raw("deep", 9, struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 0, 1)
                        + b"\x07").build(0)
    assert "nested" in _err(tmp_path, b)
    ok = struct.pack("<IQ", 9, 1) + struct.pack("<IQ", 0, 2) + b"\x01\x02"       # array of arrays: fine
    g = _open(tmp_path, Writer().kv_raw("aa", 9, ok).build(0))
    assert g.arr("aa") == (ARR, 1)
    assert "too long" in _err(tmp_path, Writer().kv_raw("long", 9, struct.pack("<IQ", 0, 1 << 40)).build(0))
    body = struct.pack("<IQ", 0, MAX_ARR + 1) + b"\0" * (MAX_ARR + 1)          # over the cap, bytes present
    assert "too long" in _err(tmp_path, Writer().kv_raw("long", 9, body).build(0))


def test_oversized_strings_rejected(tmp_path):
    assert "too long" in _err(tmp_path, Writer().kv_raw("s", 8, struct.pack("<Q", 1 << 29) + b"abc").build(0))
    _err(tmp_path, Writer().kv_raw("s", 8, struct.pack("<Q", (1 << 64) - 1)).build(0))


def test_metadata_getters(tmp_path):
    w = Writer().kv_str("general.architecture", "glm4moe").kv_u32("glm4moe.expert_count", 288)
    w.kv_f32("glm4moe.rope_theta", 10000.0).kv_raw("neg", 5, struct.pack("<i", -3))
    w.kv_raw("toks", 9, struct.pack("<IQ", 8, 2) + struct.pack("<Q", 1) + b"a" + struct.pack("<Q", 2) + b"bc")
    g = _open(tmp_path, w.build(0))
    assert g.arch() == "glm4moe"
    assert g.u64("glm4moe.expert_count") == 288 and g.kv_type("glm4moe.expert_count") == U32
    assert g.f64("glm4moe.rope_theta") == 10000.0 and g.f64("glm4moe.expert_count") == 288.0
    assert g.kv_type("general.architecture") == STR and g.kv_type("missing") is None
    assert g.arr("toks") == (STR, 2)
    with pytest.raises(GgufError):
        g.u64("neg")                          # negative integer is not a u64 (lib.rs:52-58)
    with pytest.raises(GgufError):
        g.u64("missing")


def test_slice_range(tmp_path):
    # 3-D expert tensor [in = 256, out = 4, experts = 3], Q8_0: each expert slice is 4 rows of 272 B
    b = Writer().tensor("ffn_gate_exps", [256, 4, 3], 8, 0).build(3 * 4 * 272)
    g = _open(tmp_path, b)
    t = g.tensors[0]
    assert t.n_bytes == 3 * 4 * 272
    assert t.slice_range(0) == (t.offset, 4 * 272)
    assert t.slice_range(2) == (t.offset + 2 * 4 * 272, 4 * 272)
    big = t.slice_range((1 << 64) - 1)[0]      # saturating, no wrap
    assert big == (1 << 64) - 1


def _shard(tmp_path, name, tensors, kv=None, data=None):
    w = Writer()
    for k, v in (kv or {}).items():
        w.kv_u32(k, v)
    size = 0
    for tname, dims, ty, off, n in tensors:
        w.tensor(tname, dims, ty, off)
        size = max(size, off + n)
    (tmp_path / name).write_bytes(w.build(size if data is None else data))


def test_split_model(tmp_path):
    _shard(tmp_path, "m-00001-of-00002.gguf", [("a", [32, 2], 0, 0, 256)], {"split.tensors.count": 2})
    _shard(tmp_path, "m-00002-of-00002.gguf", [("b", [256, 1], 8, 0, 34 * 8)])
    for name in ("m-00001-of-00002.gguf", "m-00002-of-00002.gguf"):   # any shard opens the whole model
        g = Gguf.open(tmp_path / name)
        assert [os.path.basename(s) for s in g.shards] == ["m-00001-of-00002.gguf", "m-00002-of-00002.gguf"]
        assert [(t.name, t.shard) for t in g.tensors] == [("a", 0), ("b", 1)]
    g = Gguf.open_shard(tmp_path / "m-00002-of-00002.gguf")
    assert len(g.shards) == 1 and g.tensors[0].name == "b"
    # the count must match
    _shard(tmp_path, "n-00001-of-00002.gguf", [("a", [32, 2], 0, 0, 256)], {"split.tensors.count": 3})
    _shard(tmp_path, "n-00002-of-00002.gguf", [("b", [32, 1], 0, 0, 128)])
    with pytest.raises(GgufError, match="split.tensors.count"):
        Gguf.open(tmp_path / "n-00001-of-00002.gguf")
    with pytest.raises(GgufError, match="missing shard"):
        _shard(tmp_path, "k-00001-of-00003.gguf", [("a", [32], 0, 0, 128)])
        Gguf.open(tmp_path / "k-00001-of-00003.gguf")


@pytest.mark.parametrize("stem", ["m-00001-of-00000", "m-00000-of-00002", "m-00003-of-00002", "m-00001-of-10000"])
def test_bad_shard_patterns_rejected(tmp_path, stem):
    _shard(tmp_path, stem + ".gguf", [("a", [32], 0, 0, 128)])
    with pytest.raises(GgufError):
        Gguf.open(tmp_path / (stem + ".gguf"))


@pytest.mark.parametrize("stem", ["modèle-0001-of-00002", "ééééééééééééééééé", "x€€€€€-of-€€€€€", "a-00001-of-0000é"])
def test_non_ascii_names_are_single_files(tmp_path, stem):
    _shard(tmp_path, stem + ".gguf", [("a", [32], 0, 0, 128)])
    g = Gguf.open(tmp_path / (stem + ".gguf"))
    assert len(g.shards) == 1


def test_read_tensor_bytes(tmp_path):
    data = bytes(range(256)) * 2
    (tmp_path / "r.gguf").write_bytes(Writer().tensor("t", [128], 0, 0).build(data))
    g = Gguf.open(tmp_path / "r.gguf")
    t = g.tensors[0]
    assert bytes(g.read(t)) == data
    assert bytes(g.read(t, 4, 8)) == data[4:12]
    with pytest.raises(GgufError):
        g.read(t, 500, 100)
