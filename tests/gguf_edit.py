"""Edits of a GGUF blob's tensor table for tests (no reference code).

set_tensor_dims rewrites the dimensions of one tensor record in place (same
rank), leaving every offset as it was: a way to make one tensor shorter than
the model's configured shape."""
import struct

STRING, ARRAY = 8, 9
_SCALAR = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 6: 4, 7: 1, 10: 8, 11: 8, 12: 8}


def _skip_value(raw, pos, vt):
    if vt == STRING:
        (n,) = struct.unpack_from("<Q", raw, pos)
        return pos + 8 + n
    if vt == ARRAY:
        et, n = struct.unpack_from("<IQ", raw, pos)
        pos += 12
        for _ in range(n):
            pos = _skip_value(raw, pos, et)
        return pos
    return pos + _SCALAR[vt]


def tensor_records(raw):
    """[(name, dims offset in the blob, rank)] of every tensor record."""
    raw = bytes(raw)
    n_t, n_kv = struct.unpack_from("<QQ", raw, 8)
    pos = 24
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<Q", raw, pos)
        pos += 8 + kl
        (vt,) = struct.unpack_from("<I", raw, pos)
        pos = _skip_value(raw, pos + 4, vt)
    out = []
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<Q", raw, pos)
        name = raw[pos + 8:pos + 8 + nl].decode()
        pos += 8 + nl
        (nd,) = struct.unpack_from("<I", raw, pos)
        out.append((name, pos + 4, nd))
        pos += 4 + 8 * nd + 4 + 8
    return out


def set_tensor_dims(blob, name, dims):
    b = bytearray(bytes(blob))
    for n, off, nd in tensor_records(b):
        if n == name:
            assert len(dims) == nd
            struct.pack_into("<" + "Q" * nd, b, off, *dims)
            return bytes(b)
    raise KeyError(name)


# bytes per block and elements per block of the tensor types the tests use
_TYPE_BLOCK = {0: (4, 1), 2: (18, 32), 6: (22, 32), 8: (34, 32), 12: (144, 256), 14: (210, 256)}


def tensor_table(raw):
    """{name: (dims, ggml type, byte offset in the blob, byte size)} of every
    tensor: the data section starts at the first multiple of
    general.alignment (default 32) after the tensor records."""
    raw = bytes(raw)
    n_t, n_kv = struct.unpack_from("<QQ", raw, 8)
    pos = 24
    align = 32
    for _ in range(n_kv):
        (kl,) = struct.unpack_from("<Q", raw, pos)
        key = raw[pos + 8:pos + 8 + kl].decode()
        pos += 8 + kl
        (vt,) = struct.unpack_from("<I", raw, pos)
        if key == "general.alignment" and vt == 4:
            (align,) = struct.unpack_from("<I", raw, pos + 4)
        pos = _skip_value(raw, pos + 4, vt)
    recs = []
    for _ in range(n_t):
        (nl,) = struct.unpack_from("<Q", raw, pos)
        name = raw[pos + 8:pos + 8 + nl].decode()
        pos += 8 + nl
        (nd,) = struct.unpack_from("<I", raw, pos)
        dims = struct.unpack_from("<" + "Q" * nd, raw, pos + 4)
        t, off = struct.unpack_from("<IQ", raw, pos + 4 + 8 * nd)
        pos += 4 + 8 * nd + 4 + 8
        recs.append((name, dims, t, off))
    base = (pos + align - 1) // align * align
    out = {}
    for name, dims, t, off in recs:
        n = 1
        for d in dims:
            n *= d
        bb, be = _TYPE_BLOCK[t]
        out[name] = (dims, t, base + off, n // be * bb)
    return out


def zero_tensors(blob, names):
    """The blob with the data of every named tensor set to zero bytes (a
    k-quant block of zeros decodes to all-zero weights: d = dmin = 0)."""
    b = bytearray(bytes(blob))
    table = tensor_table(b)
    for name in names:
        _, _, off, size = table[name]
        b[off:off + size] = bytes(size)
    return bytes(b)
