"""Memory-mapped safetensors reader (and a small writer for tests and tools).

Mirrors nnmetal/src/safetensors.zig:

* file = u64 little-endian header length, JSON header, data region
  (safetensors.zig:1-27, :226-262);
* limits MAX_TENSORS 1024, MAX_DIMS 4, MAX_HEADER_BYTES 16 MiB,
  MAX_NAME_LENGTH 256 (:28-39);
* dtypes U8, U32, F16, F32, BF16, anything else UnsupportedDtype (:46-77);
* ``__metadata__`` is skipped (:344);
* every tensor needs ``dtype``, ``shape`` (<= 4 non-negative ints) and
  ``data_offsets`` [start, end] with start <= end <= data size (:409-572).

The reference asserts on the header-length limit and on name length
(:255, :379); here both are errors like every other malformed input.  Each
error is a :class:`SafetensorsError` whose ``kind`` is the reference's error
name (``"DataOffsetOutOfBounds"``, ``"UnsupportedDtype"`` ...).

Tensor data are zero-copy numpy views into the mapping: they stay valid while
the :class:`SafetensorsFile` is open.
"""
from __future__ import annotations

import json
import mmap
import os
import struct
from dataclasses import dataclass

import numpy as np

MAX_TENSORS = 1024
MAX_DIMS = 4
MAX_HEADER_BYTES = 16 * 1024 * 1024
MAX_NAME_LENGTH = 256

# dtype string -> (bytes per element, numpy dtype of the raw view).  BF16 is
# returned as its raw uint16 bit pattern.
DTYPES = {
    "U8": (1, np.uint8),
    "U32": (4, np.uint32),
    "F16": (2, np.float16),
    "F32": (4, np.float32),
    "BF16": (2, np.uint16),
}


class SafetensorsError(ValueError):
    """Malformed or unsupported safetensors input; ``kind`` names the case."""

    def __init__(self, kind: str, msg: str):
        super().__init__(f"{kind}: {msg}")
        self.kind = kind


def dtype_from_string(s: str) -> str:
    """Dtype.fromString (safetensors.zig:65-77)."""
    if s not in DTYPES:
        raise SafetensorsError("UnsupportedDtype", f"unsupported dtype {s!r}")
    return s


def dtype_size(s: str) -> int:
    """Dtype.sizeBytes (safetensors.zig:54-62)."""
    return DTYPES[dtype_from_string(s)][0]


@dataclass
class TensorDescriptor:
    """One tensor: name, dtype string, shape and its raw bytes in the file."""

    name: str
    dtype: str
    shape: tuple
    data: memoryview

    @property
    def rank(self) -> int:
        return len(self.shape)

    def element_count(self) -> int:
        n = 1
        for d in self.shape:
            n *= d
        return n

    def size_bytes(self) -> int:
        return self.element_count() * dtype_size(self.dtype)

    def array(self) -> np.ndarray:
        """Zero-copy view with the tensor's shape (BF16 as raw uint16).
        Requires the byte range to hold exactly ``size_bytes()``."""
        if len(self.data) != self.size_bytes():
            raise SafetensorsError(
                "InvalidDataOffsets",
                f"tensor {self.name!r}: {len(self.data)} bytes for shape {self.shape} "
                f"{self.dtype} ({self.size_bytes()} expected)")
        dt = np.dtype(DTYPES[self.dtype][1]).newbyteorder("<")
        return np.frombuffer(self.data, dtype=dt).reshape(self.shape)


def _is_uint(v) -> bool:
    return isinstance(v, int) and not isinstance(v, bool) and v >= 0


class SafetensorsFile:
    """A parsed safetensors file (SafetensorsFile, safetensors.zig:119-222)."""

    def __init__(self):
        self._mm = None
        self._file = None
        self.tensors: list[TensorDescriptor] = []
        self._by_name: dict[str, TensorDescriptor] = {}
        self.metadata: dict | None = None

    # -- construction -------------------------------------------------------
    @classmethod
    def open(cls, path: str | os.PathLike) -> "SafetensorsFile":
        """``init``: mmap the file read-only and parse its header."""
        self = cls()
        f = open(path, "rb")
        try:
            size = os.fstat(f.fileno()).st_size
            if size < 10:
                raise SafetensorsError("InvalidHeader", f"{path}: {size} bytes is too short")
            self._mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
            self._file = f
            self._parse(memoryview(self._mm))
        except BaseException:
            self.close()
            f.close()
            raise
        return self

    @classmethod
    def from_bytes(cls, data: bytes | bytearray | memoryview) -> "SafetensorsFile":
        """``initFromBytes``: parse an in-memory file; views borrow ``data``."""
        self = cls()
        mv = memoryview(data).cast("B")
        if len(mv) < 10:
            raise SafetensorsError("InvalidHeader", f"{len(mv)} bytes is too short")
        self._parse(mv)
        return self

    def close(self) -> None:
        """``deinit``: drop every descriptor, then unmap."""
        self.tensors, self._by_name = [], {}
        if self._mm is not None:
            try:
                self._mm.close()
            except BufferError:
                # numpy views handed out by array() still reference the map;
                # it is released when the last of them goes.
                pass
            self._mm = None
        if self._file is not None:
            self._file.close()
            self._file = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def count(self) -> int:
        return len(self.tensors)

    def get_tensor(self, name: str) -> TensorDescriptor | None:
        """``getTensor`` (safetensors.zig:196-213): None when absent."""
        return self._by_name.get(name)

    def names(self) -> list[str]:
        return [t.name for t in self.tensors]

    # -- parsing (safetensors.zig:226-572) -----------------------------------
    def _parse(self, mv: memoryview) -> None:
        (hlen,) = struct.unpack_from("<Q", mv, 0)
        if hlen > MAX_HEADER_BYTES:
            raise SafetensorsError("InvalidHeader",
                                   f"header length {hlen} exceeds {MAX_HEADER_BYTES}")
        data_start = 8 + hlen
        if data_start > len(mv):
            raise SafetensorsError("InvalidHeader",
                                   f"header length ({hlen}) exceeds file size ({len(mv)})")
        try:
            root = json.loads(bytes(mv[8:data_start]).decode("utf-8"))
        except (UnicodeDecodeError, json.JSONDecodeError) as e:
            raise SafetensorsError("InvalidJson", str(e)) from None
        if not isinstance(root, dict):
            raise SafetensorsError("InvalidJson", "JSON root is not an object")
        data = mv[data_start:]
        for name, entry in root.items():
            if name == "__metadata__":
                self.metadata = entry if isinstance(entry, dict) else None
                continue
            if len(self.tensors) >= MAX_TENSORS:
                raise SafetensorsError("TooManyTensors",
                                       f"tensor count exceeds MAX_TENSORS ({MAX_TENSORS})")
            desc = _parse_entry(name, entry, data)
            self.tensors.append(desc)
            self._by_name[name] = desc


def _parse_entry(name: str, entry, data: memoryview) -> TensorDescriptor:
    """parseTensorEntry / parseDtype / parseShape / parseDataSlice."""
    if not name or len(name.encode("utf-8")) > MAX_NAME_LENGTH:
        raise SafetensorsError("InvalidTensorEntry",
                               f"tensor name length must be 1..{MAX_NAME_LENGTH}")
    if not isinstance(entry, dict):
        raise SafetensorsError("InvalidTensorEntry", f"tensor {name!r} value is not an object")
    if "dtype" not in entry:
        raise SafetensorsError("MissingDtype", f"tensor {name!r} missing 'dtype'")
    if not isinstance(entry["dtype"], str):
        raise SafetensorsError("InvalidDtype", f"tensor {name!r} dtype is not a string")
    dtype = dtype_from_string(entry["dtype"])
    if "shape" not in entry:
        raise SafetensorsError("MissingShape", f"tensor {name!r} missing 'shape'")
    shape = entry["shape"]
    if not isinstance(shape, list):
        raise SafetensorsError("InvalidShape", f"tensor {name!r} shape is not an array")
    if len(shape) > MAX_DIMS:
        raise SafetensorsError("TooManyDimensions",
                               f"tensor {name!r} has {len(shape)} dims, max is {MAX_DIMS}")
    for i, d in enumerate(shape):
        if not (isinstance(d, int) and not isinstance(d, bool)):
            raise SafetensorsError("InvalidShape", f"tensor {name!r} shape[{i}] not an int")
        if d < 0:
            raise SafetensorsError("InvalidShape", f"tensor {name!r} shape[{i}] is negative")
    if "data_offsets" not in entry:
        raise SafetensorsError("MissingDataOffsets", f"tensor {name!r} missing 'data_offsets'")
    offs = entry["data_offsets"]
    if not isinstance(offs, list) or len(offs) != 2 or not all(_is_uint(v) for v in offs):
        raise SafetensorsError("InvalidDataOffsets",
                               f"tensor {name!r} data_offsets must be two non-negative ints")
    start, end = offs
    if end < start:
        raise SafetensorsError("InvalidDataOffsets",
                               f"tensor {name!r} has end ({end}) < start ({start})")
    if end > len(data):
        raise SafetensorsError("DataOffsetOutOfBounds",
                               f"tensor {name!r} end offset ({end}) exceeds data ({len(data)})")
    return TensorDescriptor(name, dtype, tuple(shape), data[start:end])


def find_tensor(files, name: str) -> TensorDescriptor:
    """findTensorInFiles (nnmetal/src/model.zig:786-798): first shard that
    holds ``name``; TensorNotFound otherwise."""
    for f in files:
        d = f.get_tensor(name)
        if d is not None:
            return d
    raise SafetensorsError("TensorNotFound", f"tensor not found in any shard: {name}")


# -- writer -------------------------------------------------------------------

_NP_TO_DTYPE = {np.dtype(np.uint8): "U8", np.dtype(np.uint32): "U32",
                np.dtype(np.float16): "F16", np.dtype(np.float32): "F32"}


def save(path: str | os.PathLike, tensors: dict, metadata: dict | None = None) -> None:
    """Write a safetensors file.  ``tensors`` maps name -> numpy array, or
    name -> (dtype string, array) to force a dtype (``("BF16", uint16
    bits)``).  Data are laid out in insertion order, 8-byte aligned header."""
    header, blobs, off = {}, [], 0
    if metadata is not None:
        header["__metadata__"] = {str(k): str(v) for k, v in metadata.items()}
    for name, v in tensors.items():
        if isinstance(v, tuple):
            dt, arr = v
            dtype_from_string(dt)
        else:
            arr = v
            dt = _NP_TO_DTYPE.get(np.asarray(arr).dtype)
            if dt is None:
                raise SafetensorsError("UnsupportedDtype", f"{name}: numpy dtype {arr.dtype}")
        arr = np.ascontiguousarray(arr)
        raw = arr.astype(arr.dtype.newbyteorder("<"), copy=False).tobytes()
        header[name] = {"dtype": dt, "shape": list(arr.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    hjson = json.dumps(header, separators=(",", ":")).encode("utf-8")
    hjson += b" " * ((-len(hjson)) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hjson)))
        f.write(hjson)
        for b in blobs:
            f.write(b)
