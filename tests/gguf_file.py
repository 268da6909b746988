"""A GGUF (version 3) writer for the tests, from the published format:
a little-endian header ("GGUF", version, tensor count, metadata count),
typed metadata (strings and arrays as uint64 length + items), tensor infos
(name, rank, dimensions innermost first, ggml type, offset in the aligned
data section) and the tensors' bytes, each at a multiple of the
alignment. Test infrastructure: it writes the fixtures the reader is
checked against."""
from __future__ import annotations

import struct

import numpy as np

U8, I8, U16, I16, U32, I32, F32, BOOL, STRING, ARRAY, U64, I64, F64 = range(13)
GGML_F32, GGML_F16, GGML_Q8_0, GGML_I32, GGML_BF16 = 0, 1, 8, 26, 30

_SCALAR = {U8: "<B", I8: "<b", U16: "<H", I16: "<h", U32: "<I", I32: "<i", F32: "<f",
           BOOL: "<?", U64: "<Q", I64: "<q", F64: "<d"}


def _string(text: str | bytes) -> bytes:
    raw = text.encode() if isinstance(text, str) else text
    return struct.pack("<Q", len(raw)) + raw


def _value(kind: int, value) -> bytes:
    if kind == STRING:
        return _string(value)
    if kind == ARRAY:
        element, items = value
        if element == STRING:
            body = b"".join(_string(v) for v in items)
        else:
            body = np.asarray(items, dtype=np.dtype(_SCALAR[element][1:]).newbyteorder("<")) \
                .tobytes() if element != BOOL else bytes(int(bool(v)) for v in items)
        return struct.pack("<IQ", element, len(items)) + body
    return struct.pack(_SCALAR[kind], value)


def write(path, metadata: list, tensors: list, alignment: int = 32, version: int = 3,
          magic: bytes = b"GGUF", truncate: int | None = None) -> None:
    """metadata: [(key, kind, value)] (ARRAY values: (element kind, items));
    tensors: [(name, ggml type, dims innermost first, bytes)]."""
    head = magic + struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, kind, value in metadata:
        head += _string(key) + struct.pack("<I", kind) + _value(kind, value)
    offsets, offset = [], 0
    for _, _, _, data in tensors:
        offsets.append(offset)
        offset += (len(data) + alignment - 1) // alignment * alignment
    for (name, kind, dims, _), at in zip(tensors, offsets):
        head += _string(name) + struct.pack("<I", len(dims))
        head += b"".join(struct.pack("<Q", d) for d in dims)
        head += struct.pack("<IQ", kind, at)
    head += b"\0" * ((-len(head)) % alignment)
    body = b""
    for (_, _, _, data), at in zip(tensors, offsets):
        body += b"\0" * (at - len(body)) + data
    blob = head + body
    if truncate is not None:
        blob = blob[:truncate]
    with open(path, "wb") as f:
        f.write(blob)


def embedded_table(files: dict[str, str]) -> list:
    """audio.cpp's embedded-file metadata: names, offsets (one more than
    the files) and the bytes as one integer array."""
    names, offsets, data = [], [0], []
    for name, text in files.items():
        names.append(name)
        data.extend(text.encode())
        offsets.append(len(data))
    return [("audiocpp.embedded_files.names", ARRAY, (STRING, names)),
            ("audiocpp.embedded_files.offsets", ARRAY, (U64, offsets)),
            ("audiocpp.embedded_files.data", ARRAY, (U8, data))]
