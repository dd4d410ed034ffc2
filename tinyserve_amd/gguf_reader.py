"""GGUF file reader: header, metadata and tensor directory, tensor bytes without decoding.

Mirrors the reference's ``GGUFReader`` (tinyserve/gguf_reader.py:15-225): the same
``GGML_TYPES`` table, ``GGUFTensorInfo`` record and methods (``get_tensor_data``,
``get_tensor_data_by_offset``, ``list_expert_tensors``, ``list_fused_expert_tensors``,
``metadata``, ``tensors``, ``close``). Differences: the file is memory-mapped, so
``tensor_view`` hands out zero-copy uint8 views; the data section starts at the
``general.alignment`` boundary the file declares (32 when absent, which is what the
reference always assumes); truncated files raise ``ValueError``.

Format (GGUF v2 / v3, little-endian): magic "GGUF", u32 version, u64 tensor count, u64
metadata count; metadata entries (string key, u32 value type, value); tensor infos
(string name, u32 n_dims, n_dims x u64 ne with ne[0] the innermost dimension, u32 ggml
type, u64 offset into the data section); the data section. Strings are a u64 length
followed by UTF-8 bytes.
"""
from __future__ import annotations

import mmap
import re
import struct
from dataclasses import dataclass
from pathlib import Path

import numpy as np

# ggml type id -> (name, bytes per block, values per block)
GGML_TYPES: dict[int, tuple[str, int, int]] = {
    0: ("F32", 4, 1),
    1: ("F16", 2, 1),
    2: ("Q4_0", 18, 32),
    3: ("Q4_1", 20, 32),
    6: ("Q5_0", 22, 32),
    7: ("Q5_1", 24, 32),
    8: ("Q8_0", 34, 32),
    10: ("Q2_K", 256, 256),
    11: ("Q3_K", 256, 256),
    12: ("Q4_K", 144, 256),
    13: ("Q5_K", 176, 256),
    14: ("Q6_K", 210, 256),
    15: ("Q8_K", 256, 256),
}

GGUF_MAGIC = 0x46554747  # b"GGUF" read as a little-endian u32
DEFAULT_ALIGNMENT = 32

# metadata value types
VT_UINT8, VT_INT8, VT_UINT16, VT_INT16, VT_UINT32, VT_INT32, VT_FLOAT32, VT_BOOL = range(8)
VT_STRING, VT_ARRAY, VT_UINT64, VT_INT64, VT_FLOAT64 = range(8, 13)
_SCALAR = {
    VT_UINT8: "<B", VT_INT8: "<b", VT_UINT16: "<H", VT_INT16: "<h", VT_UINT32: "<I", VT_INT32: "<i",
    VT_FLOAT32: "<f", VT_BOOL: "<?", VT_UINT64: "<Q", VT_INT64: "<q", VT_FLOAT64: "<d",
}


@dataclass
class GGUFTensorInfo:
    name: str
    shape: tuple[int, ...]  # ggml ne: shape[0] is the innermost (contiguous) dimension
    ggml_type: int
    ggml_type_name: str
    offset: int  # relative to the data section
    nbytes: int
    block_size: int


def tensor_nbytes(ggml_type: int, shape: tuple[int, ...]) -> int:
    """Bytes of a tensor: whole blocks of its type (tinyserve/gguf_reader.py:150-156)."""
    _, bpb, bs = GGML_TYPES.get(ggml_type, ("UNKNOWN", 1, 1))
    n = 1
    for d in shape:
        n *= int(d)
    return (n + bs - 1) // bs * bpb


class GGUFReader:
    MAGIC = GGUF_MAGIC

    def __init__(self, path: str | Path):
        self.path = Path(path)
        self._file = open(self.path, "rb")
        try:
            size = self._file.seek(0, 2)
            if size < 24:
                raise ValueError(f"{self.path}: {size} bytes is too short for a GGUF header")
            self._mm = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        except Exception:
            self._file.close()
            raise
        self._pos = 0
        self._tensors: list[GGUFTensorInfo] = []
        self._metadata: dict = {}
        self._data_offset = 0
        self.version = 0
        try:
            self._parse()
        except (struct.error, UnicodeDecodeError, ValueError, IndexError) as e:
            self.close()
            if isinstance(e, ValueError):
                raise
            raise ValueError(f"{self.path}: malformed GGUF ({e})") from e

    # ---- parsing
    def _take(self, n: int) -> bytes:
        if self._pos + n > len(self._mm):
            raise ValueError(f"{self.path}: truncated GGUF (need {n} bytes at {self._pos})")
        b = self._mm[self._pos : self._pos + n]
        self._pos += n
        return b

    def _u32(self) -> int:
        return struct.unpack("<I", self._take(4))[0]

    def _u64(self) -> int:
        return struct.unpack("<Q", self._take(8))[0]

    def _string(self) -> str:
        return self._take(self._u64()).decode("utf-8")

    def _scalar(self, vtype: int):
        fmt = _SCALAR[vtype]
        return struct.unpack(fmt, self._take(struct.calcsize(fmt)))[0]

    def _value(self, vtype: int):
        if vtype == VT_STRING:
            return self._string()
        if vtype == VT_ARRAY:
            atype, n = self._u32(), self._u64()
            if atype == VT_STRING:
                return [self._string() for _ in range(n)]
            if atype in _SCALAR:
                fmt = _SCALAR[atype]
                sz = struct.calcsize(fmt)
                raw = self._take(sz * n)
                return list(struct.unpack("<" + fmt[1] * n, raw)) if n else []
            raise ValueError(f"{self.path}: metadata array of value type {atype}")
        if vtype in _SCALAR:
            return self._scalar(vtype)
        raise ValueError(f"{self.path}: metadata value type {vtype}")

    def _parse(self) -> None:
        if self._u32() != GGUF_MAGIC:
            self._pos = 0
            raise ValueError(f"Not a GGUF file: magic={struct.unpack('<I', self._mm[:4])[0]:#x}")
        self.version = self._u32()
        if self.version not in (2, 3):
            raise ValueError(f"{self.path}: GGUF version {self.version} (2 and 3 are supported)")
        n_tensors, n_kv = self._u64(), self._u64()
        for _ in range(n_kv):
            key = self._string()
            self._metadata[key] = self._value(self._u32())
        for _ in range(n_tensors):
            name = self._string()
            n_dims = self._u32()
            shape = tuple(self._u64() for _ in range(n_dims))
            ggml_type = self._u32()
            offset = self._u64()
            type_name, _, block_size = GGML_TYPES.get(ggml_type, ("UNKNOWN", 1, 1))
            self._tensors.append(GGUFTensorInfo(name, shape, ggml_type, type_name, offset,
                                                tensor_nbytes(ggml_type, shape), block_size))
        align = int(self._metadata.get("general.alignment", DEFAULT_ALIGNMENT))
        if align <= 0 or align & (align - 1):
            raise ValueError(f"{self.path}: general.alignment {align} is not a power of two")
        self._data_offset = (self._pos + align - 1) // align * align
        for t in self._tensors:
            if self._data_offset + t.offset + t.nbytes > len(self._mm):
                raise ValueError(f"{self.path}: tensor {t.name} ends past the end of the file")

    # ---- data
    @property
    def data_offset(self) -> int:
        return self._data_offset

    def tensor_view(self, info: GGUFTensorInfo, offset: int = 0, nbytes: int | None = None) -> np.ndarray:
        """Zero-copy uint8 view of a tensor's bytes (or a byte range of them)."""
        n = info.nbytes - offset if nbytes is None else nbytes
        if offset < 0 or n < 0 or offset + n > info.nbytes:
            raise ValueError(f"byte range [{offset}, {offset + n}) outside tensor {info.name} ({info.nbytes} bytes)")
        return np.frombuffer(self._mm, dtype=np.uint8, count=n, offset=self._data_offset + info.offset + offset)

    def get_tensor_data(self, info: GGUFTensorInfo) -> bytes:
        start = self._data_offset + info.offset
        return self._mm[start : start + info.nbytes]

    def get_tensor_data_by_offset(self, offset: int, nbytes: int) -> bytes:
        """Raw bytes at an offset of the data section (for slices of fused tensors)."""
        start = self._data_offset + offset
        if offset < 0 or start + nbytes > len(self._mm):
            raise ValueError(f"byte range [{offset}, {offset + nbytes}) outside the data section")
        return self._mm[start : start + nbytes]

    # ---- expert tensors
    def list_expert_tensors(self) -> dict[tuple[int, int], dict[str, GGUFTensorInfo]]:
        """Per-expert tensors ``blk.<L>.ffn_<gate|up|down>.<E>.weight`` grouped by (layer, expert)."""
        pattern = re.compile(r"blk\.(\d+)\.ffn_(gate|up|down)\.(\d+)\.weight$")
        groups: dict[tuple[int, int], dict[str, GGUFTensorInfo]] = {}
        for t in self._tensors:
            m = pattern.match(t.name)
            if m:
                groups.setdefault((int(m.group(1)), int(m.group(3))), {})[m.group(2)] = t
        return groups

    def list_fused_expert_tensors(self) -> dict[int, dict[str, GGUFTensorInfo]]:
        """Fused tensors ``blk.<L>.ffn_<gate|up|down>_exps.weight`` (ne = [in, out, experts]:
        expert e is one contiguous byte range) grouped by layer."""
        pattern = re.compile(r"blk\.(\d+)\.ffn_(gate|up|down)_exps\.weight$")
        groups: dict[int, dict[str, GGUFTensorInfo]] = {}
        for t in self._tensors:
            m = pattern.match(t.name)
            if m:
                groups.setdefault(int(m.group(1)), {})[m.group(2)] = t
        return groups

    @property
    def metadata(self) -> dict:
        return self._metadata

    @property
    def tensors(self) -> list[GGUFTensorInfo]:
        return self._tensors

    def close(self) -> None:
        mm = getattr(self, "_mm", None)
        if mm is not None:
            try:
                mm.close()
            except BufferError:  # views handed out by tensor_view keep the map alive
                pass
            self._mm = None
        self._file.close()

    def __enter__(self) -> "GGUFReader":
        return self

    def __exit__(self, *exc) -> None:
        self.close()
