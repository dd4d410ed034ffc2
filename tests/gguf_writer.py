"""Minimal GGUF v3 writer for the loader tests (test infrastructure, written from the public
GGUF layout: header, metadata, tensor infos, data section at the alignment boundary)."""
from __future__ import annotations

import struct

import numpy as np

from tinyserve_amd import gguf_reader as gr

_FMT = {gr.VT_UINT8: "<B", gr.VT_INT8: "<b", gr.VT_UINT16: "<H", gr.VT_INT16: "<h", gr.VT_UINT32: "<I",
        gr.VT_INT32: "<i", gr.VT_FLOAT32: "<f", gr.VT_BOOL: "<?", gr.VT_UINT64: "<Q", gr.VT_INT64: "<q",
        gr.VT_FLOAT64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, value) -> bytes:
    if vtype == gr.VT_STRING:
        return _string(value)
    if vtype == gr.VT_ARRAY:
        atype, items = value
        out = struct.pack("<IQ", atype, len(items))
        return out + b"".join(_string(v) if atype == gr.VT_STRING else struct.pack(_FMT[atype], v) for v in items)
    return struct.pack(_FMT[vtype], value)


def write_gguf(path, tensors: list[tuple[str, tuple[int, ...], int, np.ndarray]],
               metadata: dict[str, tuple[int, object]] | None = None, alignment: int | None = None,
               version: int = 3) -> None:
    """tensors: (name, ne (innermost first), ggml type, raw bytes); metadata: key -> (value type,
    value), arrays as (VT_ARRAY, (element type, [values])). Tensor data is placed at
    ``alignment``-multiple offsets (32 by default, general.alignment when given)."""
    meta = dict(metadata or {})
    if alignment is not None:
        meta["general.alignment"] = (gr.VT_UINT32, alignment)
    align = alignment or gr.DEFAULT_ALIGNMENT
    head = struct.pack("<IIQQ", gr.GGUF_MAGIC, version, len(tensors), len(meta))
    head += b"".join(_string(k) + struct.pack("<I", vt) + _value(vt, v) for k, (vt, v) in meta.items())
    data = b""
    infos = b""
    for name, ne, gtype, raw in tensors:
        raw = np.ascontiguousarray(raw).view(np.uint8).tobytes()
        data += b"\0" * ((-len(data)) % align)
        infos += _string(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        infos += struct.pack("<IQ", gtype, len(data))
        data += raw
    body = head + infos
    body += b"\0" * ((-len(body)) % align)
    with open(path, "wb") as f:
        f.write(body + data)
