"""A minimal safetensors reader and writer.

The format: an 8-byte little-endian header length, a JSON header mapping each
tensor name to ``{"dtype", "shape", "data_offsets": [start, end]}`` (offsets
relative to the end of the header), an optional ``"__metadata__"`` entry, then
the raw little-endian tensor bytes.  Reading maps the file and returns byte
views; nothing but the JSON header is parsed, so no file can execute code.
The reference inventories the same files itself
(``glm_tpu/model_loader/source_inventory.py``).
"""

from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from math import prod
from pathlib import Path
from typing import Mapping

import numpy as np

# bytes per element of the dtypes the MoE checkpoint uses
DTYPE_BYTES = {"F8_E4M3": 1, "U8": 1, "I8": 1, "BF16": 2, "F16": 2, "F32": 4, "I32": 4, "I64": 8, "F64": 8}
MAX_HEADER_BYTES = 100 << 20


@dataclass(frozen=True)
class TensorInfo:
    name: str
    dtype: str
    shape: tuple[int, ...]
    start: int  # absolute file offsets of the tensor's bytes
    end: int

    @property
    def byte_count(self) -> int:
        return self.end - self.start


class SafetensorsFile:
    """Tensor headers of one file and read-only byte views of their payloads."""

    def __init__(self, path: str | Path):
        self.path = Path(path)
        with open(self.path, "rb") as f:
            raw = f.read(8)
            if len(raw) != 8:
                raise ValueError(f"{self.path}: not a safetensors file (short header length)")
            (size,) = struct.unpack("<Q", raw)
            if size <= 0 or size > MAX_HEADER_BYTES:
                raise ValueError(f"{self.path}: implausible safetensors header length {size}")
            header = json.loads(f.read(size).decode("utf-8"))
        if not isinstance(header, dict):
            raise ValueError(f"{self.path}: safetensors header is not an object")
        file_size = self.path.stat().st_size
        base = 8 + size
        self.metadata = header.pop("__metadata__", None)
        self.tensors: dict[str, TensorInfo] = {}
        for name, entry in header.items():
            dtype, shape, offsets = entry["dtype"], tuple(int(d) for d in entry["shape"]), entry["data_offsets"]
            if dtype not in DTYPE_BYTES:
                raise ValueError(f"{self.path}: tensor {name!r} has unsupported dtype {dtype!r}")
            start, end = base + int(offsets[0]), base + int(offsets[1])
            if not (base <= start <= end <= file_size) or end - start != prod(shape) * DTYPE_BYTES[dtype]:
                raise ValueError(f"{self.path}: tensor {name!r} has inconsistent offsets")
            self.tensors[name] = TensorInfo(name, dtype, shape, start, end)
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r") if file_size > 0 else None

    def info(self, name: str) -> TensorInfo:
        return self.tensors[name]

    def raw(self, name: str) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view (no copy)."""
        t = self.tensors[name]
        return self._map[t.start:t.end]

    def array(self, name: str) -> np.ndarray:
        """The tensor as a numpy array of its storage type: uint8 for FP8,
        uint16 bit patterns for BF16/F16, else the matching numpy dtype."""
        t = self.tensors[name]
        storage = {"F8_E4M3": np.uint8, "U8": np.uint8, "I8": np.int8, "BF16": np.uint16, "F16": np.uint16,
                   "F32": np.float32, "I32": np.int32, "I64": np.int64, "F64": np.float64}[t.dtype]
        return self.raw(name).view(storage).reshape(t.shape)


def write_safetensors(path: str | Path, tensors: Mapping[str, tuple[str, np.ndarray]],
                      metadata: Mapping[str, str] | None = None) -> None:
    """Write ``{name: (dtype, array)}``; the array's bytes are written as they
    are (uint8 for F8_E4M3, uint16 bit patterns for BF16), C order."""
    header: dict[str, object] = {}
    blobs = []
    offset = 0
    for name, (dtype, array) in tensors.items():
        a = np.ascontiguousarray(array)
        if dtype not in DTYPE_BYTES or a.dtype.itemsize != DTYPE_BYTES[dtype]:
            raise ValueError(f"tensor {name!r}: {a.dtype} storage does not fit dtype {dtype!r}")
        data = a.tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [offset, offset + len(data)]}
        blobs.append(data)
        offset += len(data)
    if metadata:
        header["__metadata__"] = dict(metadata)
    text = json.dumps(header, separators=(",", ":")).encode("utf-8")
    text += b" " * (-len(text) % 8)  # payload starts 8-byte aligned
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(text)))
        f.write(text)
        for data in blobs:
            f.write(data)
