"""A minimal GGUF v3 writer for tests (the reference's tests build their files the same way,
quintrit-format/tests/gguf_decoder_tests.rs:9-138): typed metadata, tensor descriptors and payloads at aligned
offsets."""
import struct

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_FMT = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q", I64: "<q",
        F64: "<d"}


def put_str(out: bytearray, s) -> None:
    b = s.encode() if isinstance(s, str) else bytes(s)
    out += struct.pack("<Q", len(b)) + b


def put_value(out: bytearray, vtype: int, value, elem_type: int = None) -> None:
    if vtype == STR:
        put_str(out, value)
    elif vtype == ARR:
        out += struct.pack("<IQ", elem_type, len(value))
        for v in value:
            put_value(out, elem_type, v[1] if elem_type == ARR else v, v[0] if elem_type == ARR else None)
    else:
        out += struct.pack(_FMT[vtype], value)


def build(kvs, tensors, alignment: int = 32, version: int = 3) -> bytes:
    """kvs: [(key, type, value[, elem_type])]; tensors: [(name, shape, ggml_type, payload bytes)]; alignment also
    written as general.alignment when it is not 32."""
    offsets, cur = [], 0
    for _, _, _, payload in tensors:
        offsets.append(cur)
        cur = (cur + len(payload) + alignment - 1) // alignment * alignment
    out = bytearray(b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(kvs)))
    for kv in kvs:
        put_str(out, kv[0])
        out += struct.pack("<I", kv[1])
        put_value(out, kv[1], kv[2], kv[3] if len(kv) > 3 else None)
    for (name, shape, ty, _), off in zip(tensors, offsets):
        put_str(out, name)
        out += struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", ty, off)
    while len(out) % alignment:
        out.append(0)
    for _, _, _, payload in tensors:
        out += bytes(payload)
        while len(out) % alignment:
            out.append(0)
    return bytes(out)
