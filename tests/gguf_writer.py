"""Writes small GGUF v3 files for the loader tests (test infrastructure).

Layout per the public GGUF format: magic, version, tensor and metadata
counts, metadata key/value pairs, tensor descriptors (name, n_dims, dims,
GGML type, offset relative to the data start), then the data from the next
multiple of the alignment.
"""
import struct

VT = {"u8": 0, "i8": 1, "u16": 2, "i16": 3, "u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9,
      "u64": 10, "i64": 11, "f64": 12}
FMT = {"u8": "<B", "i8": "<b", "u16": "<H", "i16": "<h", "u32": "<I", "i32": "<i", "f32": "<f", "bool": "<B",
       "u64": "<Q", "i64": "<q", "f64": "<d"}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vt, v):
    if vt == "str":
        return _str(v)
    if vt == "arr":
        et, items = v
        out = struct.pack("<IQ", VT[et], len(items))
        return out + b"".join(_value(et, x) for x in items)
    return struct.pack(FMT[vt], v)


def write(path, tensors, meta=(), alignment=32, version=3, magic=b"GGUF", n_tensors=None, n_meta=None,
          raw_header_tail=b""):
    """tensors: [(name, dims, ggml_type, data bytes)]; meta: [(key, vtype, value)], vtype a
    name from VT or an int type code written with the raw bytes `value`.
    The declared alignment must match a "general.alignment" entry if one is given."""
    hdr = magic + struct.pack("<IQQ", version, len(tensors) if n_tensors is None else n_tensors,
                              len(meta) if n_meta is None else n_meta)
    for k, vt, v in meta:
        if isinstance(vt, int):           # a raw type code and payload (malformed-file tests)
            hdr += _str(k) + struct.pack("<I", vt) + v
        else:
            hdr += _str(k) + struct.pack("<I", VT[vt]) + _value(vt, v)
    offs, off = [], 0
    for name, dims, gt, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, gt, data), o in zip(tensors, offs):
        hdr += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        hdr += struct.pack("<IQ", gt, o)
    hdr += raw_header_tail
    start = (len(hdr) + alignment - 1) // alignment * alignment
    body = bytearray(hdr + b"\0" * (start - len(hdr)))
    for (name, dims, gt, data), o in zip(tensors, offs):
        need = start + o + len(data)
        if len(body) < need:
            body += b"\0" * (need - len(body))
        body[start + o:start + o + len(data)] = data
    with open(path, "wb") as f:
        f.write(bytes(body))
    return start, offs
