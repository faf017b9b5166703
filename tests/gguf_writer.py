"""A small GGUF (v2/v3) writer for the loader tests: header, typed metadata,
tensor infos and the aligned payload, written from the format's definition
(little-endian, 64-bit string / array lengths, tensor offsets relative to the
aligned start of the payload). Pieces can be overridden to build the malformed
files the loader must reject.
"""

from __future__ import annotations

import struct

import numpy as np

# GGUF metadata value type ids
U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARR, U64, I64, F64 = range(13)
_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f", BOOL: "<B", U64: "<Q",
           I64: "<q", F64: "<d"}


def gguf_string(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def value_bytes(vtype: int, value) -> bytes:
    if vtype == STR:
        return gguf_string(value)
    if vtype == ARR:
        etype, items = value
        return struct.pack("<IQ", etype, len(items)) + b"".join(value_bytes(etype, v) for v in items)
    return struct.pack(_SCALAR[vtype], value)


def kv_bytes(key: str, vtype: int, value) -> bytes:
    return gguf_string(key) + struct.pack("<I", vtype) + value_bytes(vtype, value)


def tensor_info_bytes(name: str, shape, ggml_type: int, offset: int) -> bytes:
    return (gguf_string(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<q", d) for d in shape) +
            struct.pack("<IQ", ggml_type, offset))


def build(metadata: list[tuple[str, int, object]], tensors: list[tuple[str, tuple, int, bytes]], *,
          version: int = 3, alignment: int = 32, magic: bytes = b"GGUF", offsets: list[int] | None = None,
          counts: tuple[int, int] | None = None, pad_byte: int = 0) -> bytes:
    """metadata: (key, type, value); tensors: (name, shape, ggml type, data
    bytes). Tensors are laid out in order, each at an `alignment` multiple
    (or at `offsets` when given)."""
    head = magic + struct.pack("<I", version)
    n_t, n_kv = counts if counts else (len(tensors), len(metadata))
    head += struct.pack("<QQ", n_t, n_kv)
    body = b"".join(kv_bytes(k, t, v) for k, t, v in metadata)
    offs, pos = [], 0
    for i, (_, _, _, data) in enumerate(tensors):
        if offsets is not None:
            offs.append(offsets[i])
        else:
            pos = (pos + alignment - 1) // alignment * alignment
            offs.append(pos)
            pos += len(data)
    infos = b"".join(tensor_info_bytes(n, s, t, o) for (n, s, t, _), o in zip(tensors, offs))
    meta_end = len(head) + len(body) + len(infos)
    payload_start = (meta_end + alignment - 1) // alignment * alignment
    end = max([o + len(d) for o, (_, _, _, d) in zip(offs, tensors)] + [0])
    payload = bytearray([pad_byte]) * end
    for o, (_, _, _, d) in zip(offs, tensors):
        payload[o:o + len(d)] = d
    return head + body + infos + bytes([pad_byte]) * (payload_start - meta_end) + bytes(payload)


def to_string_float(v: float) -> str:
    """C++ std::to_string of a float / double: printf("%f")."""
    return "%f" % v


def random_tensor_bytes(rng: np.random.Generator, ggml_type: int, num_elements: int) -> bytes:
    import ggml_blocks

    if ggml_type in ggml_blocks.BLOCK:
        return ggml_blocks.random_blocks(rng, ggml_type, num_elements // ggml_blocks.BLOCK[ggml_type][0]).tobytes()
    width = {0: 4, 1: 2, 30: 2}[ggml_type]
    return rng.integers(0, 256, num_elements * width, dtype=np.uint8).tobytes()
