"""The `.gturbo` resident-index reader behind turbo_lmhead_create_from_bundle (CPU: host code
only). Pinned by the reference's header codec test (tests/test_format.cpp:120-129), the entry
layout and validation rules of ResidentIndexCodec (src/resident_index.cpp:42-104) and the
geometry the reference derives from an entry (src/cpu_reference.cpp:229-247)."""
import struct

import numpy as np
import pytest

import bundle_util as BU
import synth
import turbo_decode_tail as T


def test_header_codec_known_answer():
    # tests/test_format.cpp:121-128: {index_size 81920, resident_size 1361346560, entries 597}
    raw = struct.pack("<QQQ", 81920, 1361346560, 597)
    assert raw[:8] == bytes.fromhex("0040010000000000")  # little-endian, low byte first
    assert T.bundle_decode_header(raw) == (81920, 1361346560, 597)
    with pytest.raises(T.TurboError, match="resident.header: truncated header"):
        T.bundle_decode_header(raw[:23])


@pytest.fixture(scope="module")
def small_head():
    V, D = 256, 128
    W, S, B, g = synth.make_head(V, D, 7)
    return W, S, B, g


def test_find_tensor_fields_and_geometry(tmp_path, small_head):
    W, S, B, g = small_head
    V, D = W.shape[0], 2 * W.shape[1]
    p = tmp_path / "resident.bin"
    index_size, total = BU.write_resident(p, BU.head_tensors(W, S, B, g))
    assert index_size % BU.ALIGN == 0
    e = T.bundle_find_tensor(p, "model.embed_tokens.weight")
    assert (e.dtype, e.quantized, e.rows, e.in_dim, e.bits) == (0, 1, V, D, 4)
    assert list(e.shape) == [V, D // 8, 0, 0]
    assert e.size_bytes == W.nbytes and e.scale_size == S.nbytes and e.bias_size == B.nbytes
    for off in (e.file_offset, e.scale_offset, e.bias_offset):
        assert off % BU.ALIGN == 0 and off >= index_size
    raw = p.read_bytes()
    assert raw[e.file_offset:e.file_offset + e.size_bytes] == W.tobytes()
    assert raw[e.scale_offset:e.scale_offset + e.scale_size] == S.tobytes()
    n = T.bundle_find_tensor(p, "model.norm.weight")
    assert (n.dtype, n.quantized, n.rows, n.in_dim, n.bits) == (1, 0, D, D, 16)
    r = T.bundle_find_tensor(p, "model.layers.0.router.proj.weight")  # shape[1] * 4 == in_dim
    assert (r.quantized, r.rows, r.in_dim, r.bits) == (1, 128, D, 8)
    f = T.bundle_find_tensor(p, "model.layers.0.layer_scalar")
    assert (f.dtype, f.size_bytes, f.rows) == (3, 4, 1)
    with pytest.raises(T.TurboError, match="resident index has no tensor 'model.lm_head.weight'"):
        T.bundle_find_tensor(p, "model.lm_head.weight")


@pytest.mark.parametrize("kind,msg", [
    ("unaligned", "resident.index: truncated or unaligned index"),
    ("too_big", "resident.indexSize: exceeds max cap"),
    ("table", "resident.entryTable: outside index range"),
    ("reserved", "resident.entry: reserved byte must be zero"),
    ("name_in_table", "resident.entry.name: range outside string table"),
    ("name_past_index", "resident.entry.name: range outside string table"),
    ("region", "region outside resident.bin"),
])
def test_malformed_index_is_rejected(tmp_path, small_head, kind, msg):
    W, S, B, g = small_head
    p = tmp_path / "resident.bin"

    def corrupt(ix, table_end):
        if kind == "unaligned":
            struct.pack_into("<Q", ix, 0, len(ix) - 8)
        elif kind == "too_big":
            struct.pack_into("<Q", ix, 0, (16 << 20) + BU.ALIGN)
        elif kind == "table":
            struct.pack_into("<Q", ix, 16, (len(ix) - 24) // 72 + 1)
        elif kind == "reserved":
            ix[24 + 7] = 1
        elif kind == "name_in_table":
            struct.pack_into("<I", ix, 24, table_end - 4)
        elif kind == "name_past_index":
            struct.pack_into("<I", ix, 24, len(ix) - 2)
        elif kind == "region":
            # the first entry's data region runs past the end of the file
            struct.pack_into("<Q", ix, 24 + 16, 1 << 40)

    BU.write_resident(p, BU.head_tensors(W, S, B, g), corrupt=corrupt)
    name = "model.layers.0.router.proj.weight" if kind == "region" else "model.norm.weight"
    with pytest.raises(T.TurboError, match=msg):
        T.bundle_find_tensor(p, name)
