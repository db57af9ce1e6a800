"""A small GGUF v3 writer for the ingest tests (the public file format:
header, metadata key/values, tensor directory, aligned data section)."""
import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
T_F32, T_F16, T_Q8_0, T_Q5_K, T_Q6_K, T_BF16, T_MXFP4 = 0, 1, 8, 13, 14, 30, 39
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<?",
           U64: "<Q", I64: "<q", F64: "<d"}


def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def _value(vtype, v):
    if vtype == STR:
        return _str(v)
    if vtype == ARR:
        et, items = v
        out = struct.pack("<IQ", et, len(items))
        return out + b"".join(_str(x) if et == STR else struct.pack(_SCALAR[et], x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def write(path, kvs, tensors, alignment=32, version=3):
    """kvs: [(key, vtype, value)]; tensors: [(name, dims (innermost first),
    ggml_type, bytes)].  Tensor data is laid out in order, each start
    aligned to `alignment`; a general.alignment key is the caller's."""
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs))
    for k, t, v in kvs:
        head += _str(k) + struct.pack("<I", t) + _value(t, v)
    offs, off = [], 0
    for name, dims, ty, data in tensors:
        offs.append(off)
        off += len(data)
        off = (off + alignment - 1) // alignment * alignment
    for (name, dims, ty, data), o in zip(tensors, offs):
        head += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", ty, o)
    pad = (-len(head)) % alignment
    with open(path, "wb") as f:
        f.write(head + b"\0" * pad)
        for (name, dims, ty, data), o in zip(tensors, offs):
            f.write(bytes(data))
            f.write(b"\0" * ((-len(data)) % alignment))
    return len(head) + pad


def bf16_bytes(a):
    """RNE bf16 of an f32 array, as bytes."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r.tobytes()
