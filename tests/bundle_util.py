"""Writes small `.gturbo` resident.bin files for the loader tests.

Layout (docs/GTURBO_FORMAT.md:26-58, src/resident_index.cpp:106-131): a 24-byte header
(index_size, resident_size, entry_count as little-endian u64), 72-byte entries (name_offset u32,
name_len u16, dtype u8, reserved u8, file_offset u64, size_bytes u64, shape 4 x u32,
scale_offset, scale_size, bias_offset, bias_size u64), the names after the entry table, the
index padded to a 16 KB multiple, then every region on a 16 KB boundary."""
import struct

ALIGN = 16384
DT_U32, DT_BF16, DT_FP16, DT_FP32 = 0, 1, 2, 3


def _pad(n, a=ALIGN):
    return (n + a - 1) // a * a


def entry_bytes(name_offset, name_len, dtype, file_offset, size, shape, scale_offset=0, scale_size=0,
                bias_offset=0, bias_size=0, reserved=0):
    sh = list(shape) + [0] * (4 - len(shape))
    return struct.pack("<IHBBQQIIIIQQQQ", name_offset, name_len, dtype, reserved, file_offset, size,
                       *sh, scale_offset, scale_size, bias_offset, bias_size)


def write_resident(path, tensors, *, corrupt=None):
    """tensors: list of dicts {name, dtype, shape, data: bytes, scales: bytes | None,
    biases: bytes | None}. corrupt: optional callable(index_bytearray, table_end) applied to the
    index before writing."""
    names = [t["name"].encode() for t in tensors]
    table_end = 24 + 72 * len(tensors)
    index_size = _pad(table_end + sum(len(n) for n in names))
    # regions after the index, each 16 KB aligned
    off = index_size
    layout = []
    for t in tensors:
        regs = []
        for key in ("data", "scales", "biases"):
            blob = t.get(key)
            if blob is None:
                regs.append((0, 0))
                continue
            regs.append((off, len(blob)))
            off = _pad(off + len(blob))
        layout.append(regs)
    total = off
    index = bytearray(index_size)
    struct.pack_into("<QQQ", index, 0, index_size, total, len(tensors))
    name_off = table_end
    for i, (t, regs) in enumerate(zip(tensors, layout)):
        (fo, fs), (so, ss), (bo, bs) = regs
        index[24 + 72 * i: 24 + 72 * (i + 1)] = entry_bytes(name_off, len(names[i]), t["dtype"], fo, fs,
                                                            t["shape"], so, ss, bo, bs)
        index[name_off:name_off + len(names[i])] = names[i]
        name_off += len(names[i])
    if corrupt:
        corrupt(index, table_end)
    with open(path, "wb") as f:
        f.write(index)
        for t, regs in zip(tensors, layout):
            for key, (o, n) in zip(("data", "scales", "biases"), regs):
                if n:
                    f.seek(o)
                    f.write(t[key])
        f.truncate(total)
    return index_size, total


def head_tensors(W, S, B, g, extra=True):
    """The tied table (4-bit: shape [V, D/8] u32 words per row) and the final norm, plus a few
    other tensors of the kinds a bundle holds."""
    V, half = W.shape
    D = 2 * half
    ts = [{"name": "model.embed_tokens.weight", "dtype": DT_U32, "shape": [V, D // 8],
           "data": W.tobytes(), "scales": S.tobytes(), "biases": B.tobytes()},
          {"name": "model.norm.weight", "dtype": DT_BF16, "shape": [D], "data": g.tobytes()}]
    if extra:
        # an 8-bit quantised router (shape[1] counts u32 words: 4 values each) and an fp32 vector
        ts.insert(0, {"name": "model.layers.0.router.proj.weight", "dtype": DT_U32, "shape": [128, D // 4],
                      "data": bytes(128 * D), "scales": bytes(128 * (D // 64) * 2),
                      "biases": bytes(128 * (D // 64) * 2)})
        ts.append({"name": "model.layers.0.layer_scalar", "dtype": DT_FP32, "shape": [1],
                   "data": struct.pack("<f", 0.5)})
    return ts
