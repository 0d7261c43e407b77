"""Reading and rewriting the metadata table of a .qlm file -- TEST INFRASTRUCTURE.

Format (reference src/qlm_file.h:1-9): "QLMF" | u32 version | u32 n_kv | u32 n_tensors | u64 data_offset,
then n_kv entries {u32 key_len, key, u32 type (0 u32, 1 f32, 2 str, 3 u32 array), value}, the tensor
table, zero padding, and the tensor data at data_offset (tensor offsets are relative to it)."""
import struct

import numpy as np

U32, F32, STR, ARR = 0, 1, 2, 3


def read_qlm(path):
    """(version, kv entries [(key, type, raw value bytes)], n_tensors, tensor table bytes, data bytes)."""
    b = open(path, "rb").read()
    assert b[:4] == b"QLMF"
    ver, n_kv, n_t, data_off = struct.unpack_from("<IIIQ", b, 4)
    off = 24
    kv = []
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<I", b, off)
        key = b[off + 4:off + 4 + kl].decode()
        off += 4 + kl
        (ty,) = struct.unpack_from("<I", b, off)
        off += 4
        if ty in (U32, F32):
            val = b[off:off + 4]
            off += 4
        elif ty == STR:
            (n,) = struct.unpack_from("<I", b, off)
            val = b[off:off + 4 + n]
            off += 4 + n
        else:
            (n,) = struct.unpack_from("<I", b, off)
            val = b[off:off + 4 + 4 * n]
            off += 4 + 4 * n
        kv.append((key, ty, val))
    t0 = off
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<I", b, off)
        off += 4 + nl
        _, nd = struct.unpack_from("<II", b, off)
        off += 8 + 8 * nd + 8
    return ver, kv, n_t, b[t0:off], b[data_off:]


def write_qlm(path, ver, kv, n_t, table, data):
    head = bytearray(b"QLMF" + struct.pack("<IIIQ", ver, len(kv), n_t, 0))
    for key, ty, val in kv:
        kb = key.encode()
        head += struct.pack("<I", len(kb)) + kb + struct.pack("<I", ty) + val
    head += table
    data_off = (len(head) + 63) // 64 * 64
    struct.pack_into("<Q", head, 16, data_off)
    with open(path, "wb") as f:
        f.write(bytes(head) + bytes(data_off - len(head)) + data)


def u32(v):
    return struct.pack("<I", v)


def f32(v):
    return struct.pack("<f", v)


def add_byte_pair_merges(src, dst, n_merges, seed=1):
    """A copy of src with a tokenizer.merges table of n_merges merges of two byte tokens each (ids
    2..257, so every merged token is a 2-byte text; reference src/tokenizer.c:27-60), so that every
    id of the vocabulary decodes to text."""
    rs = np.random.default_rng(seed)
    pairs = rs.integers(2, 258, size=(n_merges, 2)).astype("<u4")
    ver, kv, n_t, table, data = read_qlm(src)
    kv = [e for e in kv if e[0] != "tokenizer.merges"]
    kv.append(("tokenizer.merges", ARR, struct.pack("<I", 2 * n_merges) + pairs.tobytes()))
    write_qlm(dst, ver, kv, n_t, table, data)
